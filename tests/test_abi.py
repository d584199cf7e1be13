"""The C ABI (include/asc_hip.h) without a GPU: the library loads, exports every
declared entry point, and rejects invalid arguments before touching the device."""
import ctypes
import os
import re

import pytest

from pyasc_amd import _native

HEADER = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include", "asc_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(asc_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = _native.load_library()
    names = declared_functions()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES or name in _native.STRING_FUNCS, name


def test_version_string():
    assert "gfx950" in _native.version()


@pytest.mark.parametrize("fn,args,code", [
    ("asc_vadd", (0, 0, 0, 0, -1, 128, 4, 16, None), _native.ERR_INVALID_ARG),
    ("asc_vadd", (0, 0, 0, 0, 16, 0, 4, 16, None), _native.ERR_INVALID_ARG),
    ("asc_vadd", (0, 0, 0, 0, 16, 4, 4, 16, None), _native.ERR_INVALID_ARG),  # null buffers
    ("asc_vadd", (9, 1, 1, 1, 16, 4, 4, 16, None), _native.ERR_UNSUPPORTED),
    ("asc_softmax_rows_f32", (0, 0, 4, 8, 16, 1, None), _native.ERR_INVALID_ARG),  # padded tile, null buffer
    ("asc_softmax_rows_f32", (0, 0, 4, 8, 0, 1, None), _native.ERR_INVALID_ARG),
    ("asc_softmax_blocks_f32", (0, 0, 4, 8, 1, 0, None), _native.ERR_INVALID_ARG),
    ("asc_unary", (18, 0, 1, 1, 8, None), _native.ERR_INVALID_ARG),           # unknown op
    ("asc_unary", (0, 3, 1, 1, 8, None), _native.ERR_UNSUPPORTED),           # int32 elements
    ("asc_unary", (0, 0, 0, 1, 8, None), _native.ERR_INVALID_ARG),           # null buffer
    ("asc_binary", (6, 0, 1, 1, 1, 8, 1, 0.0, 1, None), _native.ERR_UNSUPPORTED),  # float shift
    ("asc_binary", (6, 3, 1, 1, 1, 8, 1, 0.0, 32, None), _native.ERR_INVALID_ARG),  # shift >= 32
    ("asc_axpy", (3, 1, 1, 2.0, 8, None), _native.ERR_UNSUPPORTED),
    ("asc_axpy", (0, 1, 1, 2.0, -1, None), _native.ERR_INVALID_ARG),
    ("asc_transpose_batched", (2, 1, 1, 1, 16, 16, None), _native.ERR_INVALID_ARG),  # x aliases z
    ("asc_transpose_batched", (8, 1, 2, 1, 16, 16, None), _native.ERR_UNSUPPORTED),
    ("asc_quant_i8", (3, 1, 1, 2.0, 0.9, 8, None), _native.ERR_UNSUPPORTED),
    ("asc_atomic_tiles", (1, 0, 1, 1, 4, 8, 0.0, 0, None), _native.ERR_INVALID_ARG),  # sub is not atomic
    ("asc_atomic_tiles", (0, 0, 0, 1, 4, 8, 0.0, 0, None), _native.ERR_INVALID_ARG),  # null x
    ("asc_fill", (0, 0, 8, 1.0, 0, None), _native.ERR_INVALID_ARG),
    ("asc_rect_binary", (0, 0, 1, 1, 1, 8, 8, -1, 0, 2, 2, None), _native.ERR_INVALID_ARG),
    ("asc_broadcast_rows", (3, 1, 1, 2, 2, None), _native.ERR_UNSUPPORTED),
    ("asc_module_load", (None, None), _native.ERR_INVALID_ARG),
    ("asc_module_unload", (None,), _native.ERR_INVALID_ARG),
    ("asc_module_get_function", (None, b"k", None), _native.ERR_INVALID_ARG),
    ("asc_module_launch", (None, 1, 64, None, 0, None), _native.ERR_INVALID_ARG),  # null function
    ("asc_module_launch", (1, 0, 64, None, 0, None), _native.ERR_INVALID_ARG),  # empty grid
    ("asc_module_launch", (1, 1, 2048, None, 0, None), _native.ERR_INVALID_ARG),  # block too large
    ("asc_module_launch", (1, 1, 64, None, 8, None), _native.ERR_INVALID_ARG),  # null argument blob
    ("asc_module_launch", (1, 1 << 22, 1024, None, 0, None), _native.ERR_UNSUPPORTED),  # 2^32 threads
    ("asc_reduce_f32", (0, 1, 1, 1 << 26, 1, 1, 1 << 26, None), _native.ERR_UNSUPPORTED),  # 2^32 threads
    ("asc_rms_norm", (0, 1, 1, 1, 1 << 25, 4, 4, 1e-6, None), _native.ERR_UNSUPPORTED),  # 2^25 rows x 128
    ("asc_copy_bytes", (16, 32, -16, None), _native.ERR_INVALID_ARG),
    ("asc_copy_bytes", (0, 32, 16, None), _native.ERR_INVALID_ARG),  # null src
    ("asc_copy_bytes", (16, 32, 24, None), _native.ERR_ALIGNMENT),  # size not a multiple of 16
    ("asc_copy_bytes", (8, 32, 16, None), _native.ERR_ALIGNMENT),  # unaligned src
    # chained matmul: dtype codes 1 = float16, 0 = float32; N must equal K; the workspace
    # must hold M * N * 2 bytes and be non-null
    ("asc_matmul_chained", (0, 0, 16, 16, 16, 64, 64, 64, 32, 1 << 20, None), _native.ERR_UNSUPPORTED),
    ("asc_matmul_chained", (1, 0, 16, 16, 16, 64, 64, 32, 32, 1 << 20, None), _native.ERR_INVALID_ARG),
    ("asc_matmul_chained", (1, 0, 16, 16, 16, 64, 64, 64, 32, 64 * 64 * 2 - 1, None), _native.ERR_INVALID_ARG),
    ("asc_matmul_chained", (1, 0, 16, 16, 16, 64, 64, 64, None, 1 << 20, None), _native.ERR_INVALID_ARG),
    # the allocation-free form: same checks, and an intermediate above its 32 MiB scratch buffer
    ("asc_matmul_chained_noalloc", (0, 0, 16, 16, 16, 64, 64, 64, None), _native.ERR_UNSUPPORTED),
    ("asc_matmul_chained_noalloc", (1, 0, 16, 16, 16, 64, 64, 32, None), _native.ERR_INVALID_ARG),
    ("asc_matmul_chained_noalloc", (1, 0, 16, 16, 16, 4097, 4096, 4096, None), _native.ERR_UNSUPPORTED),
])
def test_argument_errors_are_reported(fn, args, code):
    lib = _native.load_library()
    rc = getattr(lib, fn)(*args)
    assert rc == code
    assert fn in _native.last_error()
    with pytest.raises(RuntimeError, match=f"Function {fn} returned {code}"):
        _native.check(rc, fn)


def test_zero_sized_launch_is_a_noop():
    lib = _native.load_library()
    # empty work returns before any launch, null buffers included
    assert lib.asc_unary(0, 0, None, None, 0, None) == 0
    assert lib.asc_axpy(0, None, None, 2.0, 0, None) == 0
    assert lib.asc_fill(0, None, 0, 1.0, 0, None) == 0
    assert lib.asc_atomic_tiles(0, 0, None, None, 0, 8, 0.0, 0, None) == 0
    assert lib.asc_transpose_batched(2, None, None, 0, 16, 16, None) == 0
    assert lib.asc_rect_binary(0, 0, None, None, None, 8, 8, 8, 0, 2, 2, None) == 0  # clipped to nothing
    assert lib.asc_vadd(0, None, None, None, 0, 128, 4, 16, None) == 0
    assert lib.asc_copy_bytes(None, None, 0, None) == 0
    assert lib.asc_matmul_chained(1, 0, None, None, None, 0, 64, 64, None, 0, None) == 0
    assert lib.asc_matmul_chained_noalloc(2, 0, None, None, None, 0, 64, 64, None) == 0
    assert lib.asc_vadd(0, None, None, None, 100, 128, 0, 16, None) == 0  # tile_per_block 0 covers nothing
