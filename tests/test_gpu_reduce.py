"""Reductions and RMS norm on the GPU (row reductions and rms_norm).

First the reference's reduction tests (python/test/asc2/operations/
test_reduce_ops.py) in launch form: the kernels declared by signature, on the same
parametrisation and goldens (torch sum /
amax / amin / prod, default assert_close tolerances).  Then the kernel API at
bandwidth sizes against the oracle: max / min exact, sums within 1e-5 of the sum of
absolute values per result (an fp32 summation-error bound), products on values near
one within 1e-5 relative; rms_norm within 2e-6 relative (fp32) or fp16 rounding."""
import numpy as np
import pytest
import torch

import asc
import asc2
from oracle import asc2_oracle as O
from pyasc_amd import kernels

pytestmark = pytest.mark.gpu


@asc2.jit(always_compile=True)
def kernel(input_ptr: asc.GlobalAddress, output_ptr: asc.GlobalAddress, reduce_dim: asc.ConstExpr,
           input_shape: asc.ConstExpr, input_offsets: asc.ConstExpr, output_shape: asc.ConstExpr,
           output_offsets: asc.ConstExpr, op: asc.ConstExpr, keep_dims: asc.ConstExpr) -> None:
    """output = op(input tile, reduce_dim, keep_dims) for one of the asc2.reduce_* ops."""


@asc2.jit(always_compile=True)
def kernel_all(input_ptr: asc.GlobalAddress, output_ptr: asc.GlobalAddress, input_shape: asc.ConstExpr,
               input_offsets: asc.ConstExpr, output_shape: asc.ConstExpr, output_offsets: asc.ConstExpr,
               op: asc.ConstExpr) -> None:
    """output filled with op(input tile), the reduction over the whole tile."""


# asc2 reduction -> the torch golden the reference test compares it with
_OPS = {"prod": (asc2.reduce_prod, torch.prod), "min": (asc2.reduce_min, torch.amin),
        "sum": (asc2.reduce_sum, torch.sum), "max": (asc2.reduce_max, torch.amax)}
# test_reduce_ops.py's 2-D parametrisation: each op along each dim of a 64x32 fp32 input,
# prod with keep_dims, and whole-tile reductions of sum (64x32), max and min (32x32)
# (the reference runs the whole-tile rows through kernel_all)
REFERENCE_CASES = ([(op, [64, 32], False, dim) for op in ("prod", "min", "sum", "max") for dim in (0, 1)] +
                   [("prod", [64, 32], True, 0), ("sum", [64, 32], None, None), ("max", [32, 32], None, None),
                    ("min", [32, 32], None, None)])


@pytest.mark.parametrize("name, shape, keep_dims, dim", REFERENCE_CASES)
def test_reduce_reference_cases(device, name, shape, keep_dims, dim):
    # test_reduce_ops.py:55-82: randn * 2 fp32, one block, default assert_close tolerances
    op, golden = _OPS[name]
    x = torch.randn(shape, dtype=torch.float32) * 2.0
    if dim is None:
        out_shape = [32]
    else:
        out_shape = [1 if (i == dim and keep_dims) else s for i, s in enumerate(shape) if i != dim or keep_dims]
    out = torch.zeros(out_shape, dtype=torch.float32)
    in_offsets, out_offsets = [0] * len(shape), [0] * len(out_shape)
    if dim is None:
        kernel_all[1](x, out, shape, in_offsets, out_shape, out_offsets, op)
        expected = torch.full(out_shape, golden(x).item())
    else:
        kernel[1](x, out, dim, shape, in_offsets, out_shape, out_offsets, op, keep_dims)
        expected = golden(x, dim, keepdim=keep_dims)
    torch.testing.assert_close(out, expected)


@asc2.jit(always_compile=True)
def reduce_tile_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int, tile_size: asc.ConstExpr[int]):
    """out[0] = the max of the first tile_size elements of x."""


@pytest.mark.parametrize("tile_size", [1, 7, 17])
def test_reduce_partial_tile(device, tile_size):
    # test_reduce_ops.py:95-107
    torch.manual_seed(0)
    tensor_size = 32
    x = torch.rand(tensor_size, dtype=torch.float32) * -10.0
    x[tile_size:] = 1000.0
    out = torch.empty(1, dtype=torch.float32)
    reduce_tile_kernel[1](x, out, tensor_size, tile_size=tile_size)
    expected = torch.amax(x[:tile_size]).unsqueeze(0)
    torch.testing.assert_close(out, expected)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (1000, 333), (3, 100003), (16384, 1024)])
@pytest.mark.parametrize("dim", [0, 1])
def test_reduce_large_vs_oracle(device, rows, cols, dim):
    if dim == 0 and rows * cols > 5_000_000:
        rows = 512  # the column kernel walks rows serially; keep the test short
    g = torch.Generator().manual_seed(rows + cols)
    x = torch.randn(rows, cols, generator=g) * 3
    xd = x.to(device)
    n = cols if dim == 0 else rows
    for op in ("sum", "max", "min"):
        out = torch.empty(n, device=device)
        kernels.reduce_f32(xd, out, op, dim)
        torch.cuda.synchronize()
        expected = O.reduce(x.numpy(), op, dim)
        if op == "sum":
            bound = 1e-5 * np.abs(x.numpy()).sum(axis=dim) + 1e-30
            assert (np.abs(out.cpu().numpy().astype(np.float64) - expected) <= bound).all()
        else:
            np.testing.assert_array_equal(out.cpu().numpy(), expected)


def test_reduce_prod_and_all(device):
    g = torch.Generator().manual_seed(9)
    x = 1.0 + 0.001 * torch.randn(256, 1024, generator=g)
    out = torch.empty(256, device=device)
    kernels.reduce_f32(x.to(device), out, "prod", 1)
    torch.cuda.synchronize()
    np.testing.assert_allclose(out.cpu().numpy(), O.reduce(x.numpy(), "prod", 1), rtol=1e-5)
    big = torch.randn(1 << 20, generator=g)
    allout = torch.full((7,), -1.0, device=device)
    kernels.reduce_f32(big.to(device), allout, "max", None)
    torch.cuda.synchronize()
    assert (allout.cpu() == big.max()).all()


@asc2.jit(always_compile=True)
def rms_norm_kernel(x_ptr: asc.GlobalAddress, gamma_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress,
                    num_rows: int, num_cols: int, epsilon: float, tile_size: asc.ConstExpr[int]):
    """Build-defined kernel (no reference body), declared by signature: for every row i,
    out[i, :tile_size] = asc2.rms_norm(x[i, :tile_size], gamma[:tile_size], epsilon)."""


def test_rms_norm_kernel_surface(device):
    x = torch.randn(64, 1024) * 2
    gamma = torch.rand(1024) + 0.5
    out = torch.zeros(64, 1024)
    rms_norm_kernel[16](x, gamma, out, 64, 1024, 1e-6, 1024)
    ref = torch.nn.functional.rms_norm(x.double(), [1024], gamma.double(), eps=1e-6)
    np.testing.assert_allclose(out.numpy(), ref.numpy(), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
# row lengths reach every launch shape: 128 threads x 1 or 2 vectors, 256 / 512 / 1024 x 2
# (fp32 2000, 4096, 8192; fp16 4096, 8192, 12000), and the two-pass kernel (20000)
@pytest.mark.parametrize("rows,cols,tile", [(4096, 4096, 4096), (37, 1000, 1000), (5, 7, 7), (64, 3000, 2000),
                                            (8, 20000, 20000), (128, 8192, 8192), (16, 12000, 12000)])
def test_rms_norm_vs_oracle(device, dtype, rows, cols, tile):
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = (torch.randn(rows, cols, generator=g) * 2).to(dtype)
    gamma = torch.rand(tile, generator=g) + 0.5
    out = torch.full((rows, cols), 9.0, dtype=dtype, device=device)
    kernels.rms_norm(x.to(device), gamma.to(device), out, rows, cols, 1e-5, tile)
    torch.cuda.synchronize()
    expected = O.rms_norm_rows(x.float().numpy(), gamma.numpy(), 1e-5, tile)
    got = out.cpu().float().numpy()
    if dtype == torch.float32:
        np.testing.assert_allclose(got[:, :tile], expected[:, :tile], rtol=2e-6, atol=1e-7)
    else:
        np.testing.assert_allclose(got[:, :tile], expected[:, :tile], rtol=1e-3, atol=1e-4)
    assert (got[:, tile:] == 9.0).all()
