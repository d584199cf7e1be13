"""Row softmax parity on the GPU: within 1e-6 relative of torch.softmax on the CPU
(the reference's golden, python/test/asc2/kernels/test_softmax.py:43) and of the
oracle; untouched columns/rows are bit-identical."""
import os

import numpy as np
import pytest
import torch

from oracle import asc2_oracle as O
from pyasc_amd import kernels

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
RTOL = 1e-6  # north-star tolerance for softmax (relative, no absolute slack)


def _rand(rows, cols, seed, scale=2.0):
    return torch.randn(rows, cols, generator=torch.Generator().manual_seed(seed)) * scale


def test_fixture_64x1024(device):
    f = np.load(os.path.join(GOLDEN, "softmax_64x1024.npz"))
    x = torch.from_numpy(f["x"]).to(device)
    out = torch.empty_like(x)
    kernels.softmax_rows(x, out, 64, 1024, 1024, 16)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu(), torch.from_numpy(f["expected"]), rtol=RTOL, atol=0)


@pytest.mark.parametrize("rows,cols", [(4096, 4096), (16384, 1024)])
def test_config_shapes_vs_torch_cpu(device, rows, cols):
    x = _rand(rows, cols, 1)
    out = torch.empty(rows, cols, device=device)
    kernels.softmax_rows(x.to(device), out, rows, cols, cols, 16)
    torch.cuda.synchronize()
    ref = torch.softmax(x, dim=1)
    torch.testing.assert_close(out.cpu(), ref, rtol=RTOL, atol=0)
    sums = out.double().sum(1).cpu()
    assert (sums - 1).abs().max() < cols * 2**-24


@pytest.mark.parametrize("cols", [1, 7, 64, 100, 255, 256, 300, 512, 700, 1000, 1024, 1500, 2048, 3000, 4096,
                                  6000, 8192, 10000, 20000])
def test_row_lengths_vs_oracle(device, cols):
    rows = 37
    x = _rand(rows, cols, cols)
    out = torch.empty(rows, cols, device=device)
    kernels.softmax_rows(x.to(device), out, rows, cols, cols, 16)
    torch.cuda.synchronize()
    expected = O.softmax_rows(x.numpy(), np.zeros((rows, cols), np.float32), rows, cols, cols, 16)
    np.testing.assert_allclose(out.cpu().numpy(), expected, rtol=RTOL, atol=0)
    torch.testing.assert_close(out.cpu(), torch.softmax(x, 1), rtol=RTOL, atol=0)


def test_partial_tile_leaves_columns(device):
    rows, cols, tile = 50, 1000, 640
    x = _rand(rows, cols, 3)
    out = torch.full((rows, cols), 9.0, device=device)
    kernels.softmax_rows(x.to(device), out, rows, cols, tile, 5)
    torch.cuda.synchronize()
    expected = O.softmax_rows(x.numpy(), np.full((rows, cols), 9.0, np.float32), rows, cols, tile, 5)
    np.testing.assert_array_equal(out.cpu().numpy()[:, tile:], 9.0)
    np.testing.assert_allclose(out.cpu().numpy(), expected, rtol=RTOL, atol=0)


@pytest.mark.parametrize("rows,cols,tile", [(64, 1024, 2048), (37, 1000, 1024), (5, 3, 64), (300, 1, 2),
                                            (9, 4096, 5000)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_tile_wider_than_row_vs_oracle(device, rows, cols, tile, dtype):
    # the reference's padded load and whole-tile reductions: each row's max and sum include
    # tile - cols zeros; the row's own cols outputs are written
    x = (_rand(rows, cols, cols, scale=0.5)).to(dtype)
    out = torch.full((rows, cols), 7.0, dtype=dtype, device=device)
    kernels.softmax_rows(x.to(device), out, rows, cols, tile, 16)
    torch.cuda.synchronize()
    expected = O.softmax_rows(x.numpy(), np.zeros((rows, cols), x.numpy().dtype), rows, cols, tile, 16)
    if dtype == torch.float32:
        np.testing.assert_allclose(out.cpu().numpy(), expected, rtol=RTOL, atol=0)
    else:  # within one float16 ulp of the exact padded softmax
        np.testing.assert_allclose(out.cpu().float().numpy(), expected.astype(np.float32), rtol=2 ** -10, atol=0)
    assert (out.double().sum(1).cpu() < 1).all()


@pytest.mark.parametrize("rows,cols,block,grid", [(64, 1024, 4, 16), (100, 333, 7, 10), (10, 4096, 3, 2),
                                                  (16384, 1024, 1024, 16)])
def test_fused_blocks_coverage(device, rows, cols, block, grid):
    x = _rand(rows, cols, rows + cols)
    out = torch.full((rows, cols), -2.0, device=device)
    kernels.softmax_blocks(x.to(device), out, rows, cols, block, grid)
    torch.cuda.synchronize()
    expected = O.softmax_blocks(x.numpy(), np.full((rows, cols), -2.0, np.float32), rows, cols, block, grid)
    np.testing.assert_allclose(out.cpu().numpy(), expected, rtol=RTOL, atol=0)


def test_extreme_rows(device):
    x = torch.tensor([[0.0] * 8, [1e4] + [0.0] * 7, [-1e30] * 8, [3.0, -90.0, 1.0, -200.0, 0.5, 0.25, 88.0, 88.0]])
    out = torch.empty(4, 8, device=device)
    kernels.softmax_rows(x.to(device), out, 4, 8, 8, 2)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu(), torch.softmax(x, 1), rtol=RTOL, atol=0)


# ---------------------------------------------------------------------------------------- float16
# asc2.softmax on float16 tiles: the reference's operation test
# (python/test/asc2/operations/test_softmax.py) unchanged in form, then the two kernel
# signatures on float16 tensors against the oracle (within one float16 ulp: the kernel
# rounds its fp32 result, the oracle the exact value).

import asc  # noqa: E402
import asc2  # noqa: E402


@asc2.jit(always_compile=True)
def softmax_1d_kernel(dst_ptr, src_ptr, length: asc.ConstExpr) -> None:
    ...  # declaration: binds the registered native kernel by signature


@asc2.jit(always_compile=True)
def softmax_2d_kernel(dst_ptr, src_ptr, shape: asc.ConstExpr) -> None:
    ...  # declaration: binds the registered native kernel by signature


@pytest.mark.parametrize("dtype, shape", [(torch.float16, [1, 16]), (torch.float16, [4, 1024]),
                                          (torch.float32, [1, 8]), (torch.float32, [4, 256])])
def test_operations_softmax_2d(device, dtype, shape):
    # test_softmax.py:35-45
    src = torch.rand(shape, dtype=dtype)
    dst = torch.zeros_like(src)
    softmax_2d_kernel[1](dst, src, shape)
    torch.testing.assert_close(dst, torch.softmax(src, dim=1))


@pytest.mark.parametrize("dtype, length", [(torch.float16, 16), (torch.float16, 1024), (torch.float32, 8),
                                           (torch.float32, 1024)])
def test_operations_softmax_1d(device, dtype, length):
    # test_softmax.py:48-58
    src = torch.rand(length, dtype=dtype)
    dst = torch.zeros_like(src)
    softmax_1d_kernel[1](dst, src, length)
    torch.testing.assert_close(dst, torch.softmax(src, dim=0))


def _within_one_f16_ulp(got: np.ndarray, expected: np.ndarray):
    diff = np.abs(got.astype(np.float64) - expected.astype(np.float64))
    ulp = np.spacing(np.maximum(np.abs(got), np.abs(expected)).astype(np.float16)).astype(np.float64)
    assert (diff <= ulp).all(), float((diff / ulp).max())


@pytest.mark.parametrize("rows,cols,tile", [(4096, 4096, 4096), (37, 1000, 1000), (64, 1000, 993), (3, 100003, 100003),
                                            (200, 8, 8), (5, 1, 1)])
def test_f16_rows_vs_oracle(device, rows, cols, tile):
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g) * 4).half()
    out = torch.full((rows, cols), 7.0, dtype=torch.float16, device=device)
    kernels.softmax_rows(x.to(device), out, rows, cols, tile, 16)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    expected = np.stack([O.softmax_row(r) for r in x.numpy()[:, :tile]])
    _within_one_f16_ulp(got[:, :tile], expected)
    assert (got[:, tile:] == np.float16(7.0)).all()


def test_f16_blocks_coverage(device):
    rows, cols, block, grid = 100, 333, 7, 10  # covers rows [0, 70)
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(rows, cols, generator=g) * 2).half()
    out = torch.full((rows, cols), 3.0, dtype=torch.float16, device=device)
    kernels.softmax_blocks(x.to(device), out, rows, cols, block, grid)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    _within_one_f16_ulp(got[:70], np.stack([O.softmax_row(r) for r in x.numpy()[:70]]))
    assert (got[70:] == np.float16(3.0)).all()
