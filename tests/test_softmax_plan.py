"""asc_softmax_plan without a GPU: the launch the softmax entries make (kernel, grid, block,
arguments), which the asc2 code-object path replays through asc_module_launch.  The kernel
choice at every row-length boundary, the coverage arguments of both reference kernels
(python/test/asc2/kernels/test_softmax.py:16-27, test_softmax_fused.py:16-24), the
alignment flag, and the entries' own argument errors."""
import ctypes

import pytest

from pyasc_amd import _native
from pyasc_amd.launchers import SOFTMAX_CO_FUNCTIONS, SOFTMAX_ROWS_CODE_OBJECT

X, OUT = 0x10000, 0x20000  # 16-byte aligned stand-ins; the plan never dereferences them


def plan(dtype, fused, x, out, rows, cols, size, grid):
    p = _native.SoftmaxPlan()
    rc = _native.load_library().asc_softmax_plan(dtype, fused, x, out, rows, cols, size, grid, ctypes.byref(p))
    return rc, p


@pytest.mark.parametrize("length,kernel,block", [
    (1, "wave_1x2", 256), (256, "wave_1x2", 256), (257, "wave_2x2", 256), (512, "wave_2x2", 256),
    (513, "block_2x128", 128), (1024, "block_2x128", 128), (1025, "block_2x256", 256), (2048, "block_2x256", 256),
    (2049, "block_2x512", 512), (4096, "block_2x512", 512), (4097, "block_8x256", 256), (8192, "block_8x256", 256),
    (8193, "long", 256), (100000, "long", 256)])
def test_f32_kernel_per_row_length(length, kernel, block):
    rows = 1001
    rc, p = plan(_native.DT_FLOAT32, 0, X, OUT, rows, length, length, 16)
    assert rc == 0
    assert p.kernel.decode() == f"asc2_softmax_{kernel}" and p.block == block
    # a wave takes two rows (four waves per block); the block kernels take one row per block
    assert p.grid == ((rows + 7) // 8 if kernel.startswith("wave") else rows)
    assert (p.rows, p.stride, p.len, p.flag) == (rows, length, length, int(length % 4 == 0))


def test_rows_kernel_processes_tile_columns_of_each_row():
    # test_softmax.py: rows b, b + grid, ... all rows; each row's first tile_size columns
    rc, p = plan(_native.DT_FLOAT32, 0, X, OUT, 64, 1024, 1000, 16)
    assert rc == 0 and (p.rows, p.stride, p.len, p.flag) == (64, 1024, 1000, 1)
    assert p.kernel.decode() == "asc2_softmax_block_2x128"


@pytest.mark.parametrize("rows,block_size,grid,covered", [(64, 4, 16, 64), (100, 3, 16, 48), (10, 100, 16, 10)])
def test_fused_kernel_covers_grid_times_block_rows(rows, block_size, grid, covered):
    # test_softmax_fused.py: block b softmaxes rows [b*block_size, (b+1)*block_size)
    rc, p = plan(_native.DT_FLOAT32, 1, X, OUT, rows, 300, block_size, grid)
    assert rc == 0 and (p.rows, p.stride, p.len) == (covered, 300, 300)
    assert p.kernel.decode() == "asc2_softmax_wave_2x2" and p.grid == (covered + 7) // 8


def test_alignment_flag():
    assert plan(_native.DT_FLOAT32, 0, X + 4, OUT, 8, 64, 64, 1)[1].flag == 0  # x not 16-byte aligned
    assert plan(_native.DT_FLOAT32, 0, X, OUT + 8, 8, 64, 64, 1)[1].flag == 0
    assert plan(_native.DT_FLOAT32, 0, X, OUT, 8, 66, 64, 1)[1].flag == 0      # row stride not 4 floats
    assert plan(_native.DT_FLOAT32, 0, X, OUT, 8, 68, 63, 1)[1].flag == 1      # ragged length: per-lane tail
    assert plan(_native.DT_FLOAT16, 0, X, OUT, 8, 64, 64, 1)[1].flag == 1
    assert plan(_native.DT_FLOAT16, 0, X, OUT, 8, 64, 60, 1)[1].flag == 0      # f16 vectors need len % 8 == 0
    assert plan(_native.DT_FLOAT16, 0, X, OUT, 8, 60, 56, 1)[1].flag == 0      # and stride % 8 == 0


def test_f16_and_padded_kernels():
    rc, p = plan(_native.DT_FLOAT16, 0, X, OUT, 70000, 1024, 1024, 16)
    assert rc == 0 and p.kernel.decode() == "asc2_softmax_f16" and (p.grid, p.block) == (65536, 256)
    for dtype, name in ((_native.DT_FLOAT32, "padded_f32"), (_native.DT_FLOAT16, "padded_f16")):
        # tile_size > num_cols: flag is the count of padding zeros in each row's tile
        rc, p = plan(dtype, 0, X, OUT, 30, 100, 128, 16)
        assert rc == 0 and p.kernel.decode() == f"asc2_softmax_{name}"
        assert (p.grid, p.block, p.rows, p.stride, p.len, p.flag) == (30, 256, 30, 100, 100, 28)


def test_empty_launch_has_no_grid():
    for args in ((0, 1024, 1024, 16), (0, 100, 128, 16)):  # no rows (the second a padded tile)
        rc, p = plan(_native.DT_FLOAT32, 0, 0, 0, *args)
        assert rc == 0 and p.grid == 0 and p.kernel == b""
    rc, p = plan(_native.DT_FLOAT32, 1, 0, 0, 64, 0, 4, 16)
    assert rc == 0 and p.grid == 0


@pytest.mark.parametrize("dtype,fused,x,rows,cols,size,grid,code,who", [
    (0, 0, X, -1, 8, 8, 1, _native.ERR_INVALID_ARG, "asc_softmax_rows_f32"),
    (0, 0, X, 4, 8, 0, 1, _native.ERR_INVALID_ARG, "asc_softmax_rows_f32"),
    (1, 0, 0, 4, 8, 8, 1, _native.ERR_INVALID_ARG, "asc_softmax_rows_f16"),      # null buffer
    (0, 0, 0, 4, 8, 16, 1, _native.ERR_INVALID_ARG, "asc_softmax_rows_f32"),     # padded tile, null buffer
    (0, 1, X, 4, 8, 1, 0, _native.ERR_INVALID_ARG, "asc_softmax_blocks_f32"),
    (1, 1, X, 4, 1 << 31, 1, 1, _native.ERR_UNSUPPORTED, "asc_softmax_blocks_f16"),
    (2, 0, X, 4, 8, 8, 1, _native.ERR_UNSUPPORTED, "asc_softmax_plan"),          # bf16
    # one 128-thread block per row: more than 2^32 threads in one launch
    (0, 0, X, 40_000_000, 1024, 1024, 16, _native.ERR_UNSUPPORTED, "asc_softmax_rows_f32"),
])
def test_plan_errors_match_the_entries(dtype, fused, x, rows, cols, size, grid, code, who):
    rc, _ = plan(dtype, fused, x, OUT, rows, cols, size, grid)
    assert rc == code and who in _native.last_error()
    if dtype in (0, 1):  # the entry point itself reports the same error before any launch
        entry = getattr(_native.load_library(), f"asc_softmax_{'blocks' if fused else 'rows'}_"
                                                f"{'f16' if dtype else 'f32'}")
        assert entry(x, OUT, rows, cols, size, grid, None) == code


def test_every_planned_kernel_is_in_the_code_object():
    planned = set()
    for length in (100, 300, 1000, 2000, 4000, 8000, 9000):
        planned.add(plan(_native.DT_FLOAT32, 0, X, OUT, 8, length, length, 1)[1].kernel.decode())
    for dtype in (_native.DT_FLOAT32, _native.DT_FLOAT16):
        planned.add(plan(dtype, 0, X, OUT, 8, 100, 128, 1)[1].kernel.decode())
    planned.add(plan(_native.DT_FLOAT16, 0, X, OUT, 8, 128, 128, 1)[1].kernel.decode())
    assert planned == set(SOFTMAX_CO_FUNCTIONS)
    image = SOFTMAX_ROWS_CODE_OBJECT.path.read_bytes()
    for name in SOFTMAX_CO_FUNCTIONS:
        assert name.encode() + b"\0" in image, name
