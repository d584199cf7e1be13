"""leaky_relu, vmuladd and gelu on the GPU.

The reference tests' launch forms first (python/test/asc2/kernels/test_leaky_relu.py,
test_vmuladd.py, test_gelu.py): kernels declared with @asc2.jit, launched as
kernel[grid](...) on CPU torch tensors / numpy arrays, compared with the same golden
expressions (oracle/cpu_golden.py).  Then the kernel API against the oracle: leaky_relu and vmuladd
bit-exact for every dtype, gelu within rtol 1e-5 / atol 1e-6 of the oracle's float64
evaluation of the same expression (the reference test's own bar vs torch is rtol 1e-3,
atol 1e-5)."""
import numpy as np
import pytest
import torch

import asc
import asc2
from oracle import asc2_oracle as O
from oracle import cpu_golden
from pyasc_amd import kernels

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def _np(t, dtype):
    return _bits(t) if dtype == torch.bfloat16 else t.cpu().numpy()


_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}


# ------------------------------------------------------------------------ reference-style launches
# Declared by signature (the declaration body binds the registered native kernel) and
# launched as kernel[grid](...) with the grid and tile arguments each reference test's
# launch helper derives, on its recipe and golden expression.

@asc2.jit(always_compile=True)
def leaky_relu_kernel(x_ptr: asc.GlobalAddress, alpha: float, out_ptr: asc.GlobalAddress, size: int,
                      tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
    """out = x where x >= 0, else x * alpha, over the tiles of block b (store clipped to size)."""


def test_leaky_relu_reference_recipe(device):
    # test_leaky_relu.py:40-47 (CPU tensors: copied in and back by the launcher); 16 blocks
    # of 128-element tiles, alpha a 0-dim bf16 tensor passed by value
    x = torch.rand(8192, dtype=torch.bfloat16) * 10.0 - 5.0
    alpha = torch.tensor(0.1, dtype=torch.bfloat16)
    out = torch.empty_like(x)
    leaky_relu_kernel[16](x, alpha, out, x.numel(), 128, asc.ceildiv(asc.ceildiv(x.numel(), 128), 16))
    golden = cpu_golden.leaky_relu(x, alpha)
    torch.testing.assert_close(out, golden)
    assert torch.equal(out.view(torch.int16), golden.view(torch.int16))  # bit-exact


@asc2.jit(always_compile=True, vf_fusion=True)
def vmuladd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, z_ptr: asc.GlobalAddress,
                   out_ptr: asc.GlobalAddress, size: int, tile_size: asc.ConstExpr[int],
                   tile_per_block: asc.ConstExpr[int], buffer_factor: asc.ConstExpr[int]):
    """out = x * y + z (multiply rounded, then add) over the tiles of block b."""


def test_vmuladd_reference_recipe(device):
    # test_vmuladd.py:43-52: 16 blocks of 32-element tiles, buffer_factor 2
    rng = np.random.default_rng(seed=2026)
    x, y, z = (rng.random(8192, dtype=np.float32) * 10 for _ in range(3))
    out = np.empty_like(x)
    vmuladd_kernel[16](x, y, z, out, x.size, 32, asc.ceildiv(asc.ceildiv(x.size, 32), 16), buffer_factor=2)
    np.testing.assert_allclose(out, x * y + z)
    np.testing.assert_array_equal(out, x * y + z)  # bit-exact: no fused multiply-add


@asc2.jit(always_compile=True)
def gelu_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: asc.ConstExpr,
                num_columns: asc.ConstExpr, tile_size: asc.ConstExpr, approximate: asc.ConstExpr):
    """Rows b, b+grid, ...: gelu of the first tile_size columns (tanh form when approximate)."""


@pytest.mark.parametrize("approximate", [True, False])
def test_gelu_reference_recipe(device, approximate):
    # test_gelu.py:52-59: 30 rows of 1024 fp32, 16 blocks, tile 1024
    x = torch.rand((30, 1024), dtype=torch.float32)
    out = torch.empty_like(x)
    gelu_kernel[16](x, out, 30, 1024, 1024, approximate)
    torch.testing.assert_close(out, cpu_golden.gelu(x, approximate), rtol=1e-3, atol=1e-5)
    expected = O.gelu_rows(x.numpy(), np.zeros((30, 1024)), 30, 1024, 1024, approximate)
    np.testing.assert_allclose(out.numpy(), expected, rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------------------- kernel API

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("size,tile,tpb,grid", [(8192, 128, 4, 16), (1000, 32, 2, 8), (3001, 7, 5, 11),
                                                (1 << 20, 128, 512, 16)])
def test_leaky_relu_vs_oracle(device, dtype, size, tile, tpb, grid):
    g = torch.Generator().manual_seed(size + tile)
    x = (torch.randn(size, generator=g) * 4).to(dtype)
    x[::97] = -0.0
    out = torch.full((size,), 3.0, dtype=dtype, device=device)
    alpha = 0.1 if dtype == torch.float32 else float(torch.tensor(0.1, dtype=dtype).item())
    kernels.leaky_relu(x.to(device), alpha, out, size, tile, tpb, grid)
    torch.cuda.synchronize()
    expected = O.leaky_relu(_np(x, dtype), alpha, _np(torch.full((size,), 3.0, dtype=dtype), dtype), size, tile,
                            tpb, grid, _NAMES[dtype])
    np.testing.assert_array_equal(_np(out, dtype).view(np.uint8), np.asarray(expected).view(np.uint8))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("size,tile,tpb,grid", [(8192, 32, 16, 16), (1000, 32, 2, 8), (3001, 7, 5, 11),
                                                (1 << 20, 128, 512, 16)])
def test_vmuladd_vs_oracle(device, dtype, size, tile, tpb, grid):
    g = torch.Generator().manual_seed(size + 2 * tile)
    x, y, z = ((torch.randn(size, generator=g) * 3).to(dtype) for _ in range(3))
    out = torch.full((size,), -1.0, dtype=dtype, device=device)
    kernels.vmuladd(x.to(device), y.to(device), z.to(device), out, size, tile, tpb, grid)
    torch.cuda.synchronize()
    expected = O.vmuladd(_np(x, dtype), _np(y, dtype), _np(z, dtype),
                         _np(torch.full((size,), -1.0, dtype=dtype), dtype), size, tile, tpb, grid, _NAMES[dtype])
    np.testing.assert_array_equal(_np(out, dtype).view(np.uint8), np.asarray(expected).view(np.uint8))
    if dtype != torch.float32:
        n = O.vadd_covered(size, tile, tpb, grid)
        golden = x[:n] * y[:n] + z[:n]  # torch's own mul-then-add in that dtype
        assert torch.equal(out[:n].cpu().view(torch.int16), golden.view(torch.int16))


def test_elementwise_unaligned_views(device):
    # offset views are not 16-byte aligned: the element-wise path must give the same bits
    base = torch.randn(4099, device=device)
    x, y, z = base[1:4097], base[2:4098], base[3:4099]
    out = torch.empty(4097, device=device)[1:]
    kernels.vmuladd(x, y, z, out, 4096, 128, 2, 16)
    kernels.leaky_relu(x, 0.3, out, 4096, 128, 2, 16)
    torch.cuda.synchronize()
    expected = O.leaky_relu_elements(x.cpu().numpy(), 0.3, "float32")
    np.testing.assert_array_equal(out.cpu().numpy(), expected)


@pytest.mark.parametrize("approximate", [True, False])
@pytest.mark.parametrize("rows,cols,tile", [(37, 1000, 1000), (64, 4096, 3000), (5, 7, 7), (16384, 1024, 1024),
                                           (9, 100, 128), (3, 5, 64)])
def test_gelu_vs_oracle(device, approximate, rows, cols, tile):
    g = torch.Generator().manual_seed(rows * cols)
    x = torch.randn(rows, cols, generator=g) * 3
    out = torch.full((rows, cols), 5.0, device=device)
    kernels.gelu_rows(x.to(device), out, rows, cols, tile, approximate, 16)
    torch.cuda.synchronize()
    expected = O.gelu_rows(x.numpy(), np.full((rows, cols), 5.0), rows, cols, tile, approximate)
    np.testing.assert_allclose(out.cpu().numpy(), expected, rtol=1e-5, atol=1e-6)


def test_elementwise_argument_errors(device):
    x = torch.randn(100, device=device)
    with pytest.raises(ValueError):
        kernels.leaky_relu(x, 0.1, torch.empty(50, device=device), 100, 32, 4, 1)
    with pytest.raises(TypeError):
        kernels.vmuladd(x, x.half(), x, x, 100, 32, 4, 1)
    with pytest.raises(ValueError):  # the launch touches 20 x 10 elements of a 100-element tensor
        kernels.gelu_rows(x, torch.empty_like(x), 20, 10, 11, True, 1)
    with pytest.raises(ValueError):
        kernels.gelu_rows(x, torch.empty_like(x), 10, 10, 0, True, 1)
