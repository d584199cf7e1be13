"""asc_matmul_plan, asc_matmul_i8_plan, asc_flash_attention_plan (and, over random shapes,
asc_softmax_plan) without a GPU: the launch each library entry point makes, as a
code-object kernel name, grid, block and the kernel's argument struct as a blob.  The asc2 code-object path replays these plans; the GPU
tests compare its results with the library's bit for bit.  Here: the kernel choice, the
blob's fields, and that a plan fails exactly where its entry point does."""
import ctypes
import math
import struct

import pytest
from hypothesis import given, settings, strategies as st

from pyasc_amd import _native
from pyasc_amd.launchers import (ATTENTION_CODE_OBJECT, MATMUL_CO_FUNCTIONS, MATMUL_I8_CO_FUNCTIONS,
                                 SOFTMAX_CO_FUNCTIONS, _matmul_code_object, _mnblock_body)

A, B, C, BIAS = 0x100000, 0x200000, 0x300000, 0x400000  # 16-byte aligned stand-ins, never dereferenced
F32, F16, BF16 = _native.DT_FLOAT32, _native.DT_FLOAT16, _native.DT_BFLOAT16


def lib():
    return _native.load_library()


def mm_plan(in_dt, out_dt, M, N, K, lda=None, ldb=None, ldc=None, a=A, act=0, alpha=0.0, bias=0):
    p = _native.LaunchPlan()
    rc = lib().asc_matmul_plan(in_dt, out_dt, a, B, C, bias, M, N, K, lda or K, ldb or N, ldc or N, act, alpha,
                               ctypes.byref(p))
    return rc, p


# GemmArgs: a, b, c, M, N, K, (pad), lda, ldb, ldc, epilogue {bias, act, alpha}, tiles_m, tiles_n
GEMM_ARGS = struct.Struct("<QQQiii4xqqqQifii")


@pytest.mark.parametrize("in_dt,out_dt,M,N,K,kernel,grid,block", [
    (BF16, BF16, 8192, 8192, 8192, "mfma_bf16_fast_bf16", 1024, 512),   # tile-aligned: direct-to-LDS loop
    (F16, F16, 8192, 8192, 8192, "mfma_f16_fast_f16", 1024, 512),
    (BF16, F32, 512, 256, 64, "mfma_bf16_fast_f32", 2, 512),
    (F16, F32, 480, 224, 1344, "mfma_f16_checked_f32", 2, 256),          # ragged: bounds-checked loop
    (BF16, F16, 256, 256, 40, "mfma_bf16_checked_f16", 1, 256),          # K not a multiple of 32
    (F32, F32, 256, 256, 256, "f32_mfma_f32", 256, 256),                  # 16x16 blocks up to 2048^2 outputs
    (F32, F16, 2048, 2048, 64, "f32_mfma_f16", 16384, 256),
    (F32, BF16, 2049, 2048, 64, "f32_fma_bf16", 33 * 32, 256),            # 64x64 tiles above
])
def test_matmul_kernel_choice(in_dt, out_dt, M, N, K, kernel, grid, block):
    rc, p = mm_plan(in_dt, out_dt, M, N, K)
    assert rc == 0
    assert p.kernel.decode() == f"asc2_mm_{kernel}" and (p.grid, p.block) == (grid, block)
    assert p.kernel.decode() in MATMUL_CO_FUNCTIONS


def test_matmul_blob_is_the_argument_struct():
    rc, p = mm_plan(F16, F32, 300, 520, 72, lda=80, ldb=528, ldc=520, act=2, alpha=0.25, bias=BIAS)
    assert rc == 0 and p.args_size == GEMM_ARGS.size
    a, b, c, M, N, K, lda, ldb, ldc, bias, act, alpha, tm, tn = GEMM_ARGS.unpack(p.blob())
    assert (a, b, c, bias) == (A, B, C, BIAS)
    assert (M, N, K, lda, ldb, ldc, act, alpha) == (300, 520, 72, 80, 528, 520, 2, 0.25)
    assert (tm, tn) == (2, 3) and p.grid == tm * tn


def test_unaligned_operand_takes_the_checked_kernel():
    assert mm_plan(BF16, BF16, 256, 256, 256, a=A + 2)[1].kernel.decode() == "asc2_mm_mfma_bf16_checked_bf16"
    assert mm_plan(BF16, BF16, 256, 256, 256, lda=260)[1].kernel.decode() == "asc2_mm_mfma_bf16_checked_bf16"
    assert mm_plan(BF16, BF16, 256, 256, 256, lda=264)[1].kernel.decode() == "asc2_mm_mfma_bf16_fast_bf16"


@pytest.mark.parametrize("args,code", [
    ((F16, F16, 0, 0, 0, 0, -1, 8, 8, 8, 8, 8, 0, 0.0), _native.ERR_INVALID_ARG),        # negative shape
    ((F16, F16, A, B, C, 0, 8, 8, 8, 4, 8, 8, 0, 0.0), _native.ERR_INVALID_ARG),          # lda < K
    ((F16, F16, 0, 0, C, 0, 8, 8, 8, 8, 8, 8, 0, 0.0), _native.ERR_INVALID_ARG),          # null operands
    ((3, F16, A, B, C, 0, 8, 8, 8, 8, 8, 8, 0, 0.0), _native.ERR_UNSUPPORTED),            # int32 input
    ((F16, 3, A, B, C, 0, 8, 8, 8, 8, 8, 8, 0, 0.0), _native.ERR_UNSUPPORTED),            # int32 output
    ((F16, F16, A, B, C, 0, 8, 8, 8, 8, 8, 8, 3, 0.0), _native.ERR_INVALID_ARG),          # unknown activation
    ((F16, F16, A, B, C, 0, 1 << 29, 1 << 29, 32, 32, 1 << 29, 1 << 29, 0, 0.0),
     _native.ERR_UNSUPPORTED),                                                              # grid over 2^32 threads
])
def test_matmul_plan_errors_match_the_entry(args, code):
    p = _native.LaunchPlan()
    assert lib().asc_matmul_plan(*args, ctypes.byref(p)) == code
    assert lib().asc_matmul_bias_act(*args, None) == code


def test_empty_matmul_has_no_launch():
    rc, p = mm_plan(BF16, BF16, 0, 256, 256)
    assert rc == 0 and p.grid == 0 and p.kernel == b"" and p.args_size == 0


# I8Args: a, b, scale, c, M, N, K, trunc19, tiles_m, tiles_n
I8_ARGS = struct.Struct("<QQQQiiiiii")


def i8_plan(M, N, K, dequant, trunc19=0, scale=BIAS, a=A):
    p = _native.LaunchPlan()
    rc = lib().asc_matmul_i8_plan(a, B, scale, C, M, N, K, dequant, trunc19, ctypes.byref(p))
    return rc, p


@pytest.mark.parametrize("M,N,K,dequant,kernel,grid,block", [
    (4096, 11008, 4096, 1, "fast_f16", 688, 512), (4096, 11008, 4096, 0, "fast_i32", 688, 512),
    (100, 300, 64, 1, "checked_f16", 2, 256), (256, 256, 96, 0, "checked_i32", 1, 256)])
def test_int8_kernel_choice(M, N, K, dequant, kernel, grid, block):
    rc, p = i8_plan(M, N, K, dequant)
    assert rc == 0 and p.kernel.decode() == f"asc2_i8_{kernel}" and (p.grid, p.block) == (grid, block)
    assert p.kernel.decode() in MATMUL_I8_CO_FUNCTIONS


def test_int8_blob_is_the_argument_struct():
    rc, p = i8_plan(512, 768, 128, 1, trunc19=1)
    assert rc == 0 and p.args_size == I8_ARGS.size
    assert I8_ARGS.unpack(p.blob()) == (A, B, BIAS, C, 512, 768, 128, 1, 2, 3)
    rc, p = i8_plan(512, 768, 128, 0, trunc19=1)  # int32 output: no scale, no trunc19
    assert I8_ARGS.unpack(p.blob())[2] == 0 and I8_ARGS.unpack(p.blob())[7] == 0


def test_int8_plan_errors_match_the_entries():
    p = _native.LaunchPlan()
    assert lib().asc_matmul_i8_plan(A, B, 0, C, 8, 8, 8, 1, 0, ctypes.byref(p)) == _native.ERR_INVALID_ARG
    assert lib().asc_matmul_i8_dequant_f16(A, B, None, C, 8, 8, 8, 0, None) == _native.ERR_INVALID_ARG
    assert lib().asc_matmul_i8_plan(A, B, 0, C, 8, 8, (1 << 17) + 1, 0, 0, ctypes.byref(p)) == \
        _native.ERR_UNSUPPORTED
    assert lib().asc_matmul_i8_i32(A, B, C, 8, 8, (1 << 17) + 1, None) == _native.ERR_UNSUPPORTED


# FaArgs: q, k, v, o, lse, heads_total, seq, n_qblocks, head_group, scale_log2, causal
FA_ARGS = struct.Struct("<QQQQQqiiifi4x")


@pytest.mark.parametrize("B_,H,S,D,kernel,grid,block,blocks_per_head", [
    (4, 32, 4096, 128, "d128", 128 * 16, 512, 16), (2, 8, 1000, 64, "d64", 16 * 8, 256, 8),
    (1, 1, 1, 128, "d128", 1, 512, 1)])
def test_attention_plan(B_, H, S, D, kernel, grid, block, blocks_per_head):
    p = _native.LaunchPlan()
    scale = 1 / math.sqrt(D)
    rc = lib().asc_flash_attention_plan(A, B, C, BIAS, 0, B_, H, S, D, scale, 0, ctypes.byref(p))
    assert rc == 0 and p.kernel.decode() == f"asc2_fa_fwd_{kernel}" and (p.grid, p.block) == (grid, block)
    assert p.kernel.decode() in ATTENTION_CODE_OBJECT.functions
    assert p.args_size == FA_ARGS.size
    q, k, v, o, lse, heads_total, seq, nqb, group, scale_log2, causal = FA_ARGS.unpack(p.blob())
    assert (q, k, v, o, lse, heads_total, seq, nqb, group, causal) == (A, B, C, BIAS, 0, B_ * H, S, blocks_per_head,
                                                                         1, 0)
    assert scale_log2 == pytest.approx(scale * 1.4426950408889634, rel=1e-7)


def test_attention_plan_errors_match_the_entry():
    p = _native.LaunchPlan()
    for args, code in (((A, B, C, BIAS, 0, 1, 1, 64, 96, 0.1, 0), _native.ERR_UNSUPPORTED),    # head_dim 96
                       ((A, B, C, BIAS, 0, 1, 1, 64, 64, -1.0, 0), _native.ERR_INVALID_ARG),  # sm_scale <= 0
                       ((A + 8, B, C, BIAS, 0, 1, 1, 64, 64, 0.1, 0), _native.ERR_ALIGNMENT),
                       ((0, B, C, BIAS, 0, 1, 1, 64, 64, 0.1, 0), _native.ERR_INVALID_ARG)):
        assert lib().asc_flash_attention_plan(*args, ctypes.byref(p)) == code
        assert lib().asc_flash_attention_fwd_bf16(*args, None) == code


def test_code_object_images_hold_the_planned_kernels():
    for co, names in ((_matmul_code_object(_mnblock_body), MATMUL_CO_FUNCTIONS),
                      (ATTENTION_CODE_OBJECT, ATTENTION_CODE_OBJECT.functions)):
        data = co.path.read_bytes()
        for name in names:
            assert name.encode() + b".kd" in data, name


# ------------------------------------------------------------------ properties over random shapes

@settings(max_examples=400, deadline=None)
@given(half=st.booleans(), fused=st.booleans(), rows=st.integers(0, 3_000_000), cols=st.integers(0, 40000),
       size=st.integers(1, 50000), grid=st.integers(1, 128), x_off=st.sampled_from([0, 2, 4, 8, 16]))
def test_softmax_plan_properties(half, fused, rows, cols, size, grid, x_off):
    """Every successful plan names a code-object kernel, covers exactly the rows the
    reference kernel writes, and fits one launch (grid x block < 2^32)."""
    p = _native.SoftmaxPlan()
    rc = lib().asc_softmax_plan(F16 if half else F32, int(fused), A + x_off, C, rows, cols, size, grid,
                                ctypes.byref(p))
    if rc != 0:
        assert rc in (_native.ERR_UNSUPPORTED, _native.ERR_INVALID_ARG)
        return
    covered = min(rows, grid * size) if fused else rows
    padded = not fused and size > cols
    if p.grid == 0:
        assert covered == 0 or (not padded and cols == 0 and fused)
        return
    assert p.kernel.decode() in SOFTMAX_CO_FUNCTIONS and p.grid * p.block < 2 ** 32
    assert (p.rows, p.stride) == (covered, cols)
    assert p.len == (cols if fused or padded else size)
    if padded:
        assert p.flag == size - cols and p.kernel.decode().startswith("asc2_softmax_padded")
    else:
        assert p.len <= cols
        kind = p.kernel.decode()
        # every row is launched: one workgroup per row, or four waves of two rows
        if "wave" in kind:
            assert p.grid * 8 >= covered and p.block == 256
        elif half:
            assert p.grid == min(covered, 65536)  # grid-stride rows
        else:
            assert p.grid == covered
        if x_off % 16:
            assert p.flag == 0  # unaligned rows never take 16-byte vectors


@settings(max_examples=400, deadline=None)
@given(in_dt=st.sampled_from([F32, F16, BF16]), out_dt=st.sampled_from([F32, F16, BF16]),
       M=st.integers(0, 20000), N=st.integers(0, 20000), K=st.integers(0, 20000), pad=st.integers(0, 64),
       a_off=st.sampled_from([0, 2, 16]))
def test_matmul_plan_properties(in_dt, out_dt, M, N, K, pad, a_off):
    """The direct-to-LDS kernels are only planned for shapes and buffers they can take
    without bounds checks; every plan's blob carries the call's shape and fits one launch."""
    rc, p = mm_plan(in_dt, out_dt, M, N, K, lda=K + pad, ldb=N, ldc=N, a=A + a_off)
    if rc != 0:
        assert rc == _native.ERR_UNSUPPORTED  # only a grid over 2^32 threads is refused here
        return
    if M == 0 or N == 0:
        assert p.grid == 0
        return
    name = p.kernel.decode()
    assert name in MATMUL_CO_FUNCTIONS and p.grid * p.block < 2 ** 32
    a, b, c, m, n, k, lda, ldb, ldc, bias, act, alpha, tm, tn = GEMM_ARGS.unpack(p.blob())
    assert (a, m, n, k, lda) == (A + a_off, M, N, K, K + pad)
    if "_fast_" in name:
        assert in_dt != F32 and M % 256 == 0 and N % 256 == 0 and K % 32 == 0 and K > 0
        assert a_off % 16 == 0 and (K + pad) % 8 == 0
    if in_dt == F32:
        assert name.startswith("asc2_mm_f32_")
    assert name.endswith({F32: "_f32", F16: "_f16", BF16: "_bf16"}[out_dt])


@settings(max_examples=300, deadline=None)
@given(M=st.integers(0, 30000), N=st.integers(0, 30000), K=st.integers(0, 1 << 17), dequant=st.booleans(),
       c_off=st.sampled_from([0, 8, 16]))
def test_int8_plan_properties(M, N, K, dequant, c_off):
    p = _native.LaunchPlan()
    rc = lib().asc_matmul_i8_plan(A, B, BIAS, C + c_off, M, N, K, int(dequant), 0, ctypes.byref(p))
    assert rc == 0
    if M == 0 or N == 0:
        assert p.grid == 0
        return
    name = p.kernel.decode()
    assert name in MATMUL_I8_CO_FUNCTIONS and p.grid * p.block < 2 ** 32
    assert name.endswith("_f16" if dequant else "_i32")
    if "_fast_" in name:
        assert M % 256 == 0 and N % 256 == 0 and K % 64 == 0 and K > 0 and c_off % 16 == 0
    assert p.grid == ((M + 255) // 256) * ((N + 255) // 256)
