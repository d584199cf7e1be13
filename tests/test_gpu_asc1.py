"""asc1 kernels on the GPU: the kernels of the reference's python/test/kernels/test_vadd.py,
test_matmul.py and test_matmul_torch.py (the two kernels behind the reference's only
published task durations, test/all_task_durations_golden.csv) and of tutorials 01_add and
02_add_framework, launched as those files launch them (``kernel[grid, rt.current_stream()]``
with numpy arrays or CPU tensors, which the launch copies to the device and back).

Assertions: the reference tests' own (assert_allclose / allclose), plus bit-exact
comparisons of the vadd results with x + y and with the oracle's block coverage."""
import numpy as np
import pytest
import torch

import asc
import asc.lib.runtime as rt
from oracle import asc2_oracle as O

pytestmark = pytest.mark.gpu


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
def vadd_kernel(x: asc.GlobalAddress, y: asc.GlobalAddress, z: asc.GlobalAddress, BLOCK_LENGTH: asc.ConstExpr[int],
                BUFFER_NUM: asc.ConstExpr[int], TILE_LENGTH: asc.ConstExpr[int], TILE_NUM: asc.ConstExpr[int]):
    ...  # declaration: binds the registered native kernel by signature


def vadd_launch(x: np.ndarray, y: np.ndarray, use_core_num: int = 16, tile_num: int = 8) -> np.ndarray:
    # the launch helper of python/test/kernels/test_vadd.py:72-82
    z = np.zeros_like(x)
    block_length = (z.size + use_core_num - 1) // use_core_num
    tile_length = (block_length + tile_num - 1) // tile_num
    vadd_kernel[use_core_num, rt.current_stream()](x, y, z, block_length, 1, tile_length, tile_num)
    return z


def test_asc1_vadd_reference_case(device):
    # test_vadd.py:85-92
    rng = np.random.default_rng(seed=2025)
    x = rng.random(8192, dtype=np.float32)
    y = rng.random(8192, dtype=np.float32)
    z = vadd_launch(x, y)
    np.testing.assert_allclose(z, x + y)
    np.testing.assert_array_equal(z, x + y)


@pytest.mark.parametrize("size, cores, tile_num", [(8191, 16, 8), (1 << 20, 16, 8), (100003, 7, 3), (5, 16, 8)])
def test_asc1_vadd_coverage_vs_oracle(device, size, cores, tile_num):
    rng = np.random.default_rng(size)
    x = rng.random(size, dtype=np.float32) * 100
    y = rng.random(size, dtype=np.float32) * 100
    z = vadd_launch(x, y, cores, tile_num)
    block_length = (size + cores - 1) // cores
    cover = tile_num * ((block_length + tile_num - 1) // tile_num)
    np.testing.assert_array_equal(z, O.block_add(x, y, np.zeros_like(x), cores, block_length, cover))


@pytest.mark.parametrize("grid, stride, cover, size", [(4, 100, 64, 400), (4, 100, 64, 350), (3, 1000, 999, 2500)])
def test_asc1_vadd_blocks_with_gaps(device, grid, stride, cover, size):
    # TILE_NUM * TILE_LENGTH below BLOCK_LENGTH: each block leaves a gap before the next
    x = torch.randn(size)
    y = torch.randn(size)
    z = torch.full((size,), -5.0)
    tile_num = 4
    vadd_kernel[grid](x, y, z, stride, 1, cover // tile_num, tile_num)
    exp = O.block_add(x.numpy(), y.numpy(), np.full(size, -5.0, np.float32), grid, stride,
                      tile_num * (cover // tile_num))
    np.testing.assert_array_equal(z.numpy(), exp)


@asc.jit
def tutorial_add_kernel(x: asc.GlobalAddress, y: asc.GlobalAddress, z: asc.GlobalAddress, block_length: int):
    ...  # declaration: binds the registered native kernel by signature


tutorial_add_kernel.fn_name = "vadd_kernel"  # python/tutorials/01_add/add.py:29


@asc.jit
def tutorial_add_framework_kernel(x: asc.GlobalAddress, y: asc.GlobalAddress, z: asc.GlobalAddress, block_length: int,
                                  tile_length: asc.ConstExpr[int]):
    ...  # declaration: binds the registered native kernel by signature


tutorial_add_framework_kernel.fn_name = "vadd_kernel"  # python/tutorials/02_add_framework/add_framework.py:29


@pytest.mark.parametrize("on_device", [False, True])
def test_tutorial_add(device, on_device):
    # add.py:73-90: USE_CORE_NUM 8, size 8 * 2048, torch.allclose(z, x + y)
    dev = device if on_device else "cpu"
    x = torch.rand(8 * 2048, dtype=torch.float32, device=dev)
    y = torch.rand(8 * 2048, dtype=torch.float32, device=dev)
    z = torch.zeros_like(x)
    tutorial_add_kernel[8, rt.current_stream()](x, y, z, z.numel() // 8)
    if on_device:
        rt.synchronize()
    assert torch.allclose(z, x + y)
    assert torch.equal(z, x + y)


@pytest.mark.parametrize("size", [8 * 2048, 8 * 2048 + 13])
def test_tutorial_add_framework(device, size):
    # add_framework.py:83-101: block_length rounded up, tile_length = block_length // 16
    x = torch.rand(size, dtype=torch.float32)
    y = torch.rand(size, dtype=torch.float32)
    z = torch.zeros_like(x)
    block_length = (size + 8 - 1) // 8
    tile_length = block_length // 8 // 2
    tutorial_add_framework_kernel[8, rt.current_stream()](x, y, z, block_length, tile_length)
    exp = O.block_add(x.numpy(), y.numpy(), np.zeros(size, np.float32), 8, block_length, 16 * tile_length)
    np.testing.assert_array_equal(z.numpy(), exp)
    if size == 8 * 2048:
        assert torch.allclose(z, x + y)


@asc.jit
def matmul_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress, alpha: float,
                  tiling: asc.adv.TCubeTiling, bias: asc.GlobalAddress, workspace: asc.GlobalAddress):
    ...  # declaration: binds the registered native kernel by signature


def matmul_launch(a: np.ndarray, b: np.ndarray, bias: np.ndarray, alpha: float, cores=None) -> np.ndarray:
    # the launch helper of python/test/kernels/test_matmul.py:82-99 (64x64 blocks, full K)
    size_m, size_k = a.shape
    _, size_n = b.shape
    c = np.empty((size_m, size_n), dtype=a.dtype)
    used_core_num = asc.ceildiv(size_m, 64) * asc.ceildiv(size_n, 64)
    tiling = asc.adv.TCubeTiling(used_core_num=used_core_num, m=size_m, k_a=size_k, k_b=size_k, n=size_n,
                                 base_m=64, base_k=64, base_n=64, single_core_m=64, single_core_k=size_k,
                                 single_core_n=64, depth_a1=1, depth_b1=1, step_m=1, step_n=1, share_mode=0, is_bias=1)
    workspace = np.zeros(16 * 1024 * 1024, dtype="uint8")
    matmul_kernel[cores or used_core_num, rt.current_stream()](a, b, c, alpha, tiling, bias, workspace)
    return c


@pytest.mark.parametrize("m, k, n", [(256, 256, 256), (200, 72, 130)])
def test_asc1_matmul_reference_case(device, m, k, n):
    # test_matmul.py:102-113
    rng = np.random.default_rng(seed=2025)
    a = (rng.random((m, k), dtype="float32") - .5) * 10
    b = (rng.random((k, n), dtype="float32") - .5) * 10
    bias = (rng.random((1, n), dtype="float32") - .5) * 10
    alpha = 0.01
    matmul = a @ b + bias
    c = matmul_launch(a, b, bias, alpha)
    np.testing.assert_allclose(c, np.where(matmul >= 0, matmul, matmul * alpha), atol=1e-3)
    # against the float64 product: fp32 accumulation over k terms of |a b| <= 25
    ref = a.astype(np.float64) @ b.astype(np.float64) + bias
    ref = np.where(ref >= 0, ref, ref * alpha)
    assert np.abs(c - ref).max() <= 1e-6 * 25 * k + 1e-5


def test_asc1_matmul_partial_launch_is_rejected(device):
    # four 64x64 tiles; a mixed kernel runs two instances per block, so one block misses two
    a = np.ones((128, 64), np.float32)
    b = np.ones((64, 128), np.float32)
    with pytest.raises(NotImplementedError, match="cover every tile"):
        matmul_launch(a, b, np.zeros((1, 128), np.float32), 0.1, cores=1)
    c = matmul_launch(a, b, np.zeros((1, 128), np.float32), 0.1, cores=2)  # 4 instances: complete
    np.testing.assert_array_equal(c, np.full((128, 128), 64, np.float32))


@asc.jit
def matmul_torch_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress, alpha: float,
                        size_m: asc.ConstExpr[int], size_k: asc.ConstExpr[int], size_n: asc.ConstExpr[int],
                        size_base_m: asc.ConstExpr[int], size_base_k: asc.ConstExpr[int],
                        size_base_n: asc.ConstExpr[int], size_single_m: asc.ConstExpr[int],
                        size_single_k: asc.ConstExpr[int], size_single_n: asc.ConstExpr[int],
                        used_core_num: asc.ConstExpr[int], workspace: asc.GlobalAddress):
    ...  # declaration: binds the registered native kernel by signature


matmul_torch_kernel.fn_name = "matmul_kernel"  # python/test/kernels/test_matmul_torch.py:21


def test_asc1_matmul_torch_reference_case(device):
    # test_matmul_torch.py:88-121
    m, k, n = 256, 256, 256
    a = (torch.randn((m, k), dtype=torch.float32) - .5) * 10
    b = (torch.randn((k, n), dtype=torch.float32) - .5) * 10
    alpha = 0.01
    c = torch.empty((m, n), dtype=a.dtype)
    used_core_num = asc.ceildiv(m, 64) * asc.ceildiv(n, 64)
    workspace = torch.zeros(16 * 1024 * 1024, dtype=torch.uint8)
    matmul_torch_kernel[used_core_num, rt.current_stream()](
        a, b, c, alpha, size_m=m, size_k=k, size_n=n, size_base_m=64, size_base_k=64, size_base_n=64,
        size_single_m=64, size_single_k=k, size_single_n=64, used_core_num=used_core_num, workspace=workspace)
    assert fp32_matmul_close(c, a, b, alpha=alpha)


def test_runtime_streams(device):
    s = rt.create_stream()
    x = torch.ones(1 << 20, device=device)
    with torch.cuda.stream(s):
        y = x * 2
    rt.synchronize(s, timeout=10_000)
    assert float(y.sum()) == 2 * (1 << 20)
    assert rt.current_platform() == "gfx950" and rt.device_count() >= 1 and rt.current_device() == 0
    rt.destroy_stream(s)
    rt.synchronize_device()


@asc.jit(always_compile=True)
def matmul_mix_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress, tiling: asc.adv.TCubeTiling,
                      workspace: asc.GlobalAddress):
    ...  # declaration: binds the registered native kernel by signature


matmul_mix_kernel.fn_name = "matmul_kernel"  # python/tutorials/03_matmul_mix/matmul_mix.py:32


@asc.jit(matmul_cube_only=True, always_compile=True)
def matmul_cube_only_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress,
                            bias: asc.GlobalAddress, tiling: asc.adv.TCubeTiling, workspace: asc.GlobalAddress):
    ...  # declaration: binds the registered native kernel by signature


matmul_cube_only_kernel.fn_name = "matmul_kernel"  # python/tutorials/04_matmul_cube_only/matmul_cube_only.py:33


def _generate_tiling(m, n, k, cores, bias):
    # generate_tiling of the tutorials (matmul_mix.py:90-106, matmul_cube_only.py:97-115)
    import asc.lib.host as host
    t = host.MultiCoreMatmulTiling(host.get_ascendc_platform())
    t.set_a_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT16, False)
    t.set_b_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT16, False)
    t.set_c_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT)
    t.set_bias_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT)
    t.set_dim(cores)
    t.set_org_shape(m, n, k)
    t.set_shape(m, n, k)
    t.enable_bias(bias)
    t.set_buffer_space(-1, -1, -1)
    tiling = asc.adv.TCubeTiling()
    t.get_tiling(tiling)
    return tiling


def test_tutorial_matmul_mix(device):
    # matmul_mix.py:109-121: USE_CORE_NUM 48, launched on USE_CORE_NUM // 2 blocks
    m, k, n = 512, 512, 1024
    a = torch.randint(-5, 5, (m, k)).to(torch.float16)
    b = torch.randint(-5, 5, (k, n)).to(torch.float16)
    matmul = torch.matmul(a.to(torch.float32), b.to(torch.float32)).to(torch.float32)
    tiling = _generate_tiling(m, n, k, 48, False)
    c = torch.zeros((m, n), dtype=torch.float32)
    workspace = torch.zeros(16 * 1024 * 1024, dtype=torch.uint8)
    matmul_mix_kernel[48 // 2, rt.current_stream()](a, b, c, tiling, workspace)
    assert torch.allclose(c, matmul, rtol=1e-3, atol=1e-3)
    assert torch.equal(c, matmul)  # integer-valued products: exact


@pytest.mark.parametrize("enable_bias", [False, True])
def test_tutorial_matmul_cube_only(device, enable_bias):
    # matmul_cube_only.py:118-135: USE_CORE_NUM 24, launched on tiling.used_core_num blocks
    m, k, n = 128, 64, 30720
    a = torch.randint(-5, 5, (m, k)).to(torch.float16)
    b = torch.randint(-5, 5, (k, n)).to(torch.float16)
    bias = torch.randint(-5, 5, (1, n)).to(torch.float32)
    matmul = torch.matmul(a.to(torch.float32), b.to(torch.float32)).to(torch.float32)
    if enable_bias:
        matmul = matmul + bias
    tiling = _generate_tiling(m, n, k, 24, enable_bias)
    c = torch.zeros((m, n), dtype=torch.float32)
    workspace = torch.zeros(16 * 1024 * 1024, dtype=torch.uint8)
    matmul_cube_only_kernel[tiling.used_core_num, rt.current_stream()](a, b, c, bias, tiling, workspace)
    assert torch.allclose(c, matmul, rtol=1e-3, atol=1e-3)
    assert torch.equal(c, matmul)


def test_tutorial_matmul_too_few_blocks(device):
    # a mixed kernel runs two instances per block: (used_core_num - 1) // 2 blocks miss a tile
    tiling = _generate_tiling(512, 1024, 64, 48, False)
    assert tiling.used_core_num >= 4
    a, b = torch.ones(512, 64, dtype=torch.float16), torch.ones(64, 1024, dtype=torch.float16)
    with pytest.raises(NotImplementedError, match="cover every tile"):
        matmul_mix_kernel[(tiling.used_core_num - 1) // 2](a, b, torch.zeros(512, 1024), tiling, torch.zeros(16))


@asc.jit
def matmul_leakyrelu_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress,
                            bias: asc.GlobalAddress, alpha: float, tiling: asc.adv.TCubeTiling,
                            workspace: asc.GlobalAddress):
    ...  # declaration: binds the registered native kernel by signature


def test_tutorial_matmul_leakyrelu_host_tiling(device):
    # matmul_leakyrelu.py:86-131 as written: host tiling with set_dim(2), FIRSTM traverse,
    # fix split 256x128, launched on used_core_num // 2 blocks
    import asc.lib.host as host
    m, k, n = 1024, 256, 640
    a = torch.randint(-5, 5, (m, k)).to(torch.float16)
    b = torch.randint(-5, 5, (k, n)).to(torch.float16)
    bias = torch.randint(-5, 5, (1, n)).to(torch.float32)
    alpha = 0.001
    matmul = (torch.matmul(a.to(torch.float32), b.to(torch.float32)).to(torch.float32) + bias).to(torch.float32)
    mt = host.MultiCoreMatmulTiling(host.get_ascendc_platform())
    mt.set_a_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT16, False)
    mt.set_b_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT16, False)
    mt.set_c_type(host.TPosition.VECCALC, host.CubeFormat.ND, host.DataType.DT_FLOAT)
    mt.set_bias_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT)
    mt.set_dim(2)
    mt.set_org_shape(m, n, k)
    mt.set_shape(m, n, k)
    mt.enable_bias(True)
    mt.set_traverse(host.MatrixTraverse.FIRSTM)
    mt.set_fix_split(256, 128, -1)
    mt.set_buffer_space(-1, -1, -1)
    tiling = asc.adv.TCubeTiling()
    mt.get_tiling(tiling)
    assert (tiling.base_m, tiling.base_n) == (256, 128) and tiling.used_core_num == 2
    c = torch.zeros((m, n), dtype=torch.float32)
    workspace = torch.zeros(16 * 1024 * 1024, dtype=torch.uint8)
    matmul_leakyrelu_kernel[tiling.used_core_num // 2, rt.current_stream()](a, b, c, bias, alpha, tiling, workspace)
    assert torch.allclose(c, torch.where(matmul >= 0, matmul, matmul * alpha), rtol=1e-3, atol=1e-3)
