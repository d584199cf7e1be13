"""Reductions and RMS norm on the GPU (row reductions and rms_norm).

First the reference's own reduction tests (python/test/asc2/operations/
test_reduce_ops.py): the same kernels, parametrisation and goldens (torch sum /
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
    g_input = asc2.tensor(input_ptr, input_shape)
    g_output = asc2.tensor(output_ptr, output_shape)
    input = asc2.load(g_input, input_shape, offsets=input_offsets)
    output = op(input, reduce_dim, keep_dims=keep_dims)
    asc2.store(output, g_output, offsets=output_offsets)


@asc2.jit(always_compile=True)
def kernel_all(input_ptr: asc.GlobalAddress, output_ptr: asc.GlobalAddress, input_shape: asc.ConstExpr,
               input_offsets: asc.ConstExpr, output_shape: asc.ConstExpr, output_offsets: asc.ConstExpr,
               op: asc.ConstExpr) -> None:
    g_input = asc2.tensor(input_ptr, input_shape)
    g_output = asc2.tensor(output_ptr, output_shape)
    input = asc2.load(g_input, input_shape, offsets=input_offsets)
    scalar = op(input)
    output = asc2.full(output_shape, scalar, dtype=input.dtype)
    asc2.store(output, g_output, offsets=output_offsets)


# test_reduce_ops.py:16-29 (the 2-D cases; the dim=None rows are commented out there and
# are exercised through kernel_all below)
REFERENCE_CASES = [
    [asc2.reduce_prod, torch.prod, [64, 32], torch.float32, False, 0],
    [asc2.reduce_prod, torch.prod, [64, 32], torch.float32, False, 1],
    [asc2.reduce_min, torch.amin, [64, 32], torch.float32, False, 0],
    [asc2.reduce_min, torch.amin, [64, 32], torch.float32, False, 1],
    [asc2.reduce_sum, torch.sum, [64, 32], torch.float32, False, 0],
    [asc2.reduce_sum, torch.sum, [64, 32], torch.float32, False, 1],
    [asc2.reduce_max, torch.amax, [64, 32], torch.float32, False, 0],
    [asc2.reduce_max, torch.amax, [64, 32], torch.float32, False, 1],
    [asc2.reduce_prod, torch.prod, [64, 32], torch.float32, True, 0],
    [asc2.reduce_sum, torch.sum, [64, 32], torch.float32, None, None],
    [asc2.reduce_max, torch.amax, [32, 32], torch.float32, None, None],
    [asc2.reduce_min, torch.amin, [32, 32], torch.float32, None, None],
]


@pytest.mark.parametrize("op, torch_op, shape, dtype, keep_dims, dim", REFERENCE_CASES)
def test_reduce_reference_cases(device, op, torch_op, shape, dtype, keep_dims, dim):
    # test_reduce_ops.py:55-82
    input = torch.randn(shape, dtype=dtype) * 2.0
    if dim is None:
        output_shape = [32]
    else:
        output_shape = list(shape)
        if keep_dims:
            output_shape[dim] = 1
        else:
            del output_shape[dim]
    output = torch.zeros(output_shape, dtype=dtype)
    input_offsets = [0] * len(shape)
    output_offsets = [0] * len(output_shape)
    if dim is None:
        kernel_all[1](input, output, shape, input_offsets, output_shape, output_offsets, op)
        expected = torch.ones(output_shape, dtype=dtype) * torch_op(input).item()
    else:
        kernel[1](input, output, dim, shape, input_offsets, output_shape, output_offsets, op, keep_dims)
        expected = torch_op(input, dim, keepdim=keep_dims)
    torch.testing.assert_close(output, expected)


@asc2.jit(always_compile=True)
def reduce_tile_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int, tile_size: asc.ConstExpr[int]):
    x_gm = asc2.tensor(x_ptr, [size])
    out_gm = asc2.tensor(out_ptr, [1])
    tile = asc2.load(x_gm, [tile_size], offsets=[0])
    max_val = asc2.reduce_max(tile)
    result = asc2.full([1], max_val, dtype=tile.dtype)
    asc2.store(result, out_gm, offsets=[0])


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
