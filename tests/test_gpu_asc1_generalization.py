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


@asc.jit
def vadd_kernel(x: asc.GlobalAddress, y: asc.GlobalAddress, z: asc.GlobalAddress, block_length: asc.ConstExpr[int],
                buffer_num: asc.ConstExpr[int], tile_length: asc.ConstExpr[int], tile_num: asc.ConstExpr[int]):
    raise AssertionError("kernel bodies are not executed")


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
    raise AssertionError("kernel bodies are not executed")


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
    raise AssertionError("kernel bodies are not executed")


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
    raise AssertionError("kernel bodies are not executed")


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
    raise AssertionError("kernel bodies are not executed")


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
    raise AssertionError("kernel bodies are not executed")


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
    raise AssertionError("kernel bodies are not executed")


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
