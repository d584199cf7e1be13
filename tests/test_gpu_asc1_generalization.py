"""asc1 generalization kernels on the GPU (python/test/generalization/basic): vadd and
its bits / l0 / sw variants (one signature), vadds, vsqrt, duplicate, axpy, copy and
transpose, with each test's parameter list, launch helper and golden; then the same
kernels at larger sizes against exact expectations (bit-exact adds, fills, copies and
transposes; sqrt correctly rounded; axpy within one rounding of the fp64 value)."""
import numpy as np
import pytest
import torch

import asc
import asc.lib.runtime as rt
import asc.runtime.config as config

pytestmark = pytest.mark.gpu

PARAMS = [(torch.float32, (1000,)), (torch.float32, (1,)), (torch.float32, (9999,)), (torch.float16, (2048,)),
          (torch.int32, (8192,)), (torch.int16, (8192,)), (torch.int32, (153, 834))]  # test_vadd.py:88-96


def _inputs(dtype, size):
    if dtype in {torch.float16, torch.float32}:
        return torch.randn(size, dtype=dtype)
    return torch.randint(-100, 99, size, dtype=dtype)


def _launch_shape(total, cores, tile_length):
    block_length = (total + cores - 1) // cores
    return block_length, (block_length + tile_length - 1) // tile_length


def fp32_matmul_close(c, a, b, bias=None, alpha=None):
    """c against a @ b (+ bias, then leaky relu with slope alpha) computed in fp64, within the
    error bound of an fp32 sum of K products (K * 2^-24 * (|a| @ |b| + |bias|)); leaky relu is
    1-Lipschitz, so the bound holds after it.  (An absolute tolerance against torch's own fp32
    product, as the reference's test_matmul*.py use, fails for a few percent of random draws:
    both sides round, in different orders.)"""
    a64, b64 = a.double(), b.double()
    ref = a64 @ b64
    mag = a64.abs() @ b64.abs()
    if bias is not None:
        ref = ref + bias.double()
        mag = mag + bias.double().abs()
    if alpha is not None:
        ref = torch.where(ref >= 0, ref, ref * alpha)
    bound = a.shape[1] * 2.0 ** -24 * mag + 1e-6
    return bool(((c.double() - ref).abs() <= bound).all())


@asc.jit
def vadd_kernel(x: asc.GlobalAddress, y: asc.GlobalAddress, z: asc.GlobalAddress, block_length: asc.ConstExpr[int],
                buffer_num: asc.ConstExpr[int], tile_length: asc.ConstExpr[int], tile_num: asc.ConstExpr[int]):
    ...  # declaration: binds the registered native kernel by signature


@pytest.mark.parametrize("tile_length", [512, 64])  # test_vadd.py / test_vadd_sw.py: 512; _bits / _l0: 64
@pytest.mark.parametrize("dtype, size", PARAMS, ids=str)
def test_vadd_family(device, dtype, size, tile_length):
    x, y = _inputs(dtype, size), _inputs(dtype, size)
    z = torch.zeros_like(x)
    block_length, tile_num = _launch_shape(z.numel(), 16, tile_length)
    vadd_kernel[16, rt.current_stream()](x, y, z, block_length, 1, tile_length, tile_num)
    assert torch.allclose(z, x + y)
    assert torch.equal(z, x + y)


@asc.jit
def vadds_kernel(x: asc.GlobalAddress, scalar, z: asc.GlobalAddress, block_length: asc.ConstExpr[int],
                 buffer_num: asc.ConstExpr[int], tile_length: asc.ConstExpr[int], tile_num: asc.ConstExpr[int]):
    ...  # declaration: binds the registered native kernel by signature


@pytest.mark.parametrize("dtype, size", PARAMS, ids=str)
def test_vadds(device, dtype, size):
    # test_vadds.py:93-106
    x = _inputs(dtype, size)
    scalar = (torch.randn((), dtype=dtype) if dtype.is_floating_point else torch.randint(-100, 99, (), dtype=dtype))
    scalar = scalar.item()
    z = torch.zeros_like(x)
    block_length, tile_num = _launch_shape(z.numel(), 16, 512)
    vadds_kernel[16, rt.current_stream()](x, scalar, z, block_length, 1, 512, tile_num)
    assert torch.allclose(z, x + scalar)
    assert torch.equal(z, x + torch.tensor(scalar, dtype=dtype))


@asc.jit
def vsqrt_kernel(x: asc.GlobalAddress, z: asc.GlobalAddress, block_length: asc.ConstExpr[int],
                 buffer_num: asc.ConstExpr[int], tile_length: asc.ConstExpr[int], tile_num: asc.ConstExpr[int]):
    ...  # declaration: binds the registered native kernel by signature


@pytest.mark.parametrize("dtype, size", [(torch.float16, (2048,)), (torch.float32, (5000,)), (torch.float32, (9999,)),
                                         (torch.float32, (8192,)), (torch.bfloat16, (4097,))], ids=str)
def test_vsqrt(device, dtype, size):
    # test_vsqrt.py:90-106 (bfloat16 added); sqrt is correctly rounded: equal to torch's
    x = torch.abs(torch.randn(size, dtype=dtype) + 10.0)
    z = torch.zeros_like(x)
    block_length, tile_num = _launch_shape(z.numel(), 16, 512)
    vsqrt_kernel[16, rt.current_stream()](x, z, block_length, 1, 512, tile_num)
    assert torch.allclose(z, torch.sqrt(x), rtol=1e-3 if dtype != torch.float32 else 1e-5)
    assert torch.equal(z, torch.sqrt(x.double()).to(dtype))


@asc.jit
def duplicate_kernel(scalar, z: asc.GlobalAddress, block_length: asc.ConstExpr[int], buffer_num: asc.ConstExpr[int],
                     tile_length: asc.ConstExpr[int], tile_num: asc.ConstExpr[int]):
    ...  # declaration: binds the registered native kernel by signature


@pytest.mark.parametrize("dtype, size", [(torch.float32, (1000,)), (torch.float32, (1,)), (torch.float16, (2048,)),
                                         (torch.int32, (8192,)), (torch.int16, (8192,))], ids=str)
def test_duplicate(device, dtype, size):
    # test_duplicate.py:76-90: z is float32 whatever the scalar's dtype
    scalar = (torch.randn((), dtype=dtype) if dtype.is_floating_point else torch.randint(1, 99, (), dtype=dtype))
    scalar = scalar.item()
    z = torch.zeros(size)
    block_length, tile_num = _launch_shape(z.numel(), 16, 512)
    duplicate_kernel[16, rt.current_stream()](scalar, z, block_length, 1, 512, tile_num)
    assert torch.allclose(z, torch.full(size, scalar, dtype=z.dtype))
    assert torch.equal(z, torch.full(size, scalar, dtype=z.dtype))


@asc.jit
def axpy_kernel(x: asc.GlobalAddress, y: asc.GlobalAddress, z: asc.GlobalAddress, scalar: float,
                block_length: asc.ConstExpr[int], buffer_num: asc.ConstExpr[int], tile_length: asc.ConstExpr[int],
                tile_num: asc.ConstExpr[int]):
    ...  # declaration: binds the registered native kernel by signature


@pytest.mark.parametrize("dtype, size", [(torch.float32, (4096,)), (torch.float32, (8192,)), (torch.float16, (8192,)),
                                         (torch.float16, (2048,))], ids=str)
def test_axpy(device, dtype, size):
    # test_axpy.py:107-121: z starts at 0, so z = y * scalar
    x = torch.randn(size, dtype=dtype) * 10.0
    y = torch.randn(size, dtype=dtype) * 10.0
    z = torch.zeros_like(x)
    n = z.numel()
    axpy_kernel[1, rt.current_stream()](x, y, z, 2.5, n, 1, n, 1)
    expected = y * 2.5
    assert torch.allclose(z, expected, rtol=1e-3 if dtype == torch.float16 else 1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_axpy_accumulates_vs_fp64(device, dtype):
    g = torch.Generator().manual_seed(5)
    n = (1 << 20) + 3
    y = (torch.randn(n, generator=g) * 10).to(dtype)
    z0 = (torch.randn(n, generator=g) * 10).to(dtype)
    z = z0.clone()
    axpy_kernel[4, rt.current_stream()](torch.zeros(n, dtype=dtype), y, z, -0.75, (n + 3) // 4, 1, 4096,
                                        ((n + 3) // 4 + 4095) // 4096)
    prod = y.double() * -0.75
    ref = prod + z0.double()
    if dtype == torch.float32:
        # product and sum each rounded in fp32: half an ulp of each
        bound = 2.0 ** -24 * (prod.abs() + ref.abs() * (1 + 2.0 ** -23))
    else:
        # the 16-bit product and sum are exact or nearly so in fp32; one rounding to the
        # element type: within one ulp of the result
        bound = ref.abs() * {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}[dtype]
    assert bool(((z.double() - ref).abs() <= bound + 1e-30).all())


@asc.jit
def copy_kernel(x: asc.GlobalAddress, z: asc.GlobalAddress, data_size: asc.ConstExpr[int]):
    ...  # declaration: binds the registered native kernel by signature


@pytest.mark.parametrize("dtype, size", [(torch.float32, (1000,)), (torch.float32, (1,)), (torch.float32, (9999,)),
                                         (torch.float16, (2048,)), (torch.int32, (8192,)), (torch.int16, (8192,)),
                                         (torch.int32, (1000,))], ids=str)
def test_copy(device, dtype, size):
    # test_copy.py:100-122: mask 64 elements, 4 repeats of 8 32-byte blocks
    x = _inputs(dtype, size)
    z = torch.zeros_like(x)
    copy_kernel[1, rt.current_stream()](x, z, x.numel())
    expected = torch.zeros_like(x)
    stride = 8 * (32 // x.dtype.itemsize)
    for i in range(4):
        if i * stride + 64 > size[0]:
            break
        expected[i * stride:i * stride + 64] = x[i * stride:i * stride + 64]
    assert torch.equal(z, expected)


@asc.jit
def transpose_kernel(x: asc.GlobalAddress, z: asc.GlobalAddress, block_length: asc.ConstExpr[int],
                     buffer_num: asc.ConstExpr[int], tile_length: asc.ConstExpr[int], tile_num: asc.ConstExpr[int]):
    ...  # declaration: binds the registered native kernel by signature


@pytest.mark.parametrize("dtype", [torch.float16, torch.int16])
def test_transpose(device, dtype):
    # test_transpose.py:95-108: one 16x16 tile
    x = torch.randn((16, 16), dtype=dtype) if dtype.is_floating_point else torch.randint(0, 99, (16, 16), dtype=dtype)
    z = torch.zeros_like(x)
    transpose_kernel[1, rt.current_stream()](x, z, 256, 1, 256, 1)
    assert torch.equal(z, x.T)


def test_transpose_many_tiles(device):
    # 8 blocks of 4 tiles: each 256-element tile transposed on its own
    x = torch.arange(8 * 4 * 256, dtype=torch.int16)
    z = torch.zeros_like(x)
    transpose_kernel[8](x, z, 1024, 1, 256, 4)
    assert torch.equal(z, x.reshape(-1, 16, 16).transpose(1, 2).reshape(-1))


# ------------------------------------------------------------------- python/test/generalization/adv

def _adv_tiling(m, n, k, dtype, bias=False, batch=None):
    # generate_tiling of test_matmul.py:94-113 / test_matmul_iterate_all.py:70-87 /
    # test_matmul_iterate_batch.py:73-95
    import asc.lib.host as host
    t = host.MultiCoreMatmulTiling(host.get_ascendc_platform())
    host_dtype = host.DataType.DT_FLOAT if dtype == torch.float32 else host.DataType.DT_FLOAT16
    t.set_a_type(host.TPosition.GM, host.CubeFormat.ND, host_dtype, False)
    t.set_b_type(host.TPosition.GM, host.CubeFormat.ND, host_dtype, False)
    t.set_c_type(host.TPosition.VECCALC, host.CubeFormat.ND, host.DataType.DT_FLOAT)
    t.set_bias_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT)
    t.set_dim(16)
    t.set_org_shape(m, n, k)
    t.set_shape(m, n, k)
    if bias:
        t.enable_bias(True)
    t.set_traverse(host.MatrixTraverse.FIRSTM)
    t.set_buffer_space(-1, -1, -1)
    if batch:
        t.set_a_layout(batch, m, 1, 1, k)
        t.set_b_layout(batch, k, 1, 1, n)
        t.set_c_layout(batch, m, 1, 1, n)
        t.set_batch_num(batch)
    tiling = asc.adv.TCubeTiling()
    t.get_tiling(tiling)
    return tiling


@asc.jit
def matmul_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress, alpha: float,
                  tiling: asc.adv.TCubeTiling, bias: asc.GlobalAddress, workspace: asc.GlobalAddress):
    ...  # declaration: binds the registered native kernel by signature


def test_adv_matmul(device):
    # test_matmul.py:126-145: fp32 1024x256x512 (m, k, n), bias, leaky relu 0.01
    m, k, n = 1024, 256, 512
    a = (torch.rand((m, k)) - .5) * 10
    b = (torch.rand((k, n)) - .5) * 10
    bias = (torch.rand((1, n)) - .5) * 10
    c = torch.zeros((m, n))
    workspace = torch.zeros(16 * 1024 * 1024, dtype=torch.uint8)
    tiling = _adv_tiling(m, n, k, torch.float32, bias=True)
    matmul_kernel[tiling.used_core_num, rt.current_stream()](a, b, c, 0.01, tiling, bias, workspace)
    assert fp32_matmul_close(c, a, b, bias=bias, alpha=0.01)


@asc.jit
def iterate_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress, tiling: asc.adv.TCubeTiling,
                   workspace: asc.GlobalAddress):
    ...  # declaration: binds the registered native kernel by signature


iterate_kernel.fn_name = "matmul_kernel"  # test_matmul_iterate_all.py:24, test_matmul_iterate_batch.py:29


@pytest.mark.parametrize("dtype, size", [(torch.float16, (256, 64, 128)), (torch.int8, (256, 64, 128)),
                                         (torch.int8, (300, 96, 200))], ids=str)
def test_adv_matmul_iterate_all(device, dtype, size):
    # test_matmul_iterate_all.py:100-120 (its body also takes int8 -> int32)
    m, k, n = size
    if dtype == torch.float16:
        a = (torch.rand((m, k), dtype=dtype) - 0.5) * 10
        b = (torch.rand((k, n), dtype=dtype) - 0.5) * 10
        c = torch.zeros((m, n), dtype=torch.float32)
        matmul = a.to(torch.float32) @ b.to(torch.float32)
    else:
        a = torch.randint(-5, 5, (m, k), dtype=dtype)
        b = torch.randint(-5, 5, (k, n), dtype=dtype)
        c = torch.zeros((m, n), dtype=torch.int32)
        matmul = a.to(torch.int32) @ b.to(torch.int32)
    workspace = torch.zeros(16 * 1024 * 1024, dtype=torch.uint8)
    tiling = _adv_tiling(m, n, k, dtype)
    iterate_kernel[tiling.used_core_num, rt.current_stream()](a, b, c, tiling, workspace)
    assert torch.allclose(c, matmul, atol=1e-3)
    if dtype == torch.int8:
        assert torch.equal(c, matmul)


@pytest.mark.parametrize("dtype, size", [(torch.float32, (64, 64, 64)), (torch.float16, (32, 32, 32))], ids=str)
def test_adv_matmul_iterate_batch(device, dtype, size):
    # test_matmul_iterate_batch.py:109-150, BATCH_A = BATCH_B = BATCH = 2
    m, k, n = size
    a = torch.vstack([(torch.rand((m, k), dtype=dtype) - .5) * 10 for _ in range(2)])
    b = torch.vstack([(torch.rand((k, n), dtype=dtype) - .5) * 10 for _ in range(2)])
    matmul = torch.vstack([a[i * m:(i + 1) * m].float() @ b[i * k:(i + 1) * k].float() for i in range(2)])
    c = torch.zeros((2 * m, n), dtype=torch.float32)
    workspace = torch.zeros(16 * 1024 * 1024, dtype=torch.uint8)
    tiling = _adv_tiling(m, n, k, dtype, batch=2)
    iterate_kernel[tiling.used_core_num, rt.current_stream()](a, b, c, tiling, workspace)
    assert torch.allclose(c, matmul, atol=1e-3)


@asc.jit(kernel_type=config.KernelType.AIV_ONLY)
def quant_kernel(src_gm: asc.GlobalAddress, dst_gm: asc.GlobalAddress, size: int, tmp_min_bytes: int,
                 use_config: asc.ConstExpr[bool]):
    ...  # declaration: binds the registered native kernel by signature


@pytest.mark.parametrize("use_config", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_adv_quant(device, dtype, use_config):
    # test_quant.py:94-104
    src = torch.rand((32,), dtype=dtype) * 8.0 - 4.0
    dst = torch.zeros_like(src, dtype=torch.int8)
    quant_kernel[1, rt.current_stream()](src, dst, src.numel(), 512, use_config)
    assert torch.allclose(dst, torch.round((src * 2.0) + 0.9).to(torch.int8))


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_quant_vs_oracle(device, dtype):
    from pyasc_amd import kernels
    from oracle import asc2_oracle as O
    g = torch.Generator().manual_seed(9)
    n = (1 << 20) + 11
    src = (torch.randn(n, generator=g) * 60).to(getattr(torch, dtype))
    src[:6] = torch.tensor([float("nan"), float("inf"), -float("inf"), 0.05, -0.45, 63.2])
    dst = torch.empty(n, dtype=torch.int8, device=device)
    kernels.quant_i8(src.to(device), dst, 2.0, 0.9)
    torch.cuda.synchronize()
    host = src.view(torch.int16).numpy().view(np.uint16) if dtype == "bfloat16" else src.numpy()
    np.testing.assert_array_equal(dst.cpu().numpy(), O.quant_i8(host, 2.0, 0.9, dtype))
