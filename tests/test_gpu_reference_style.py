"""The reference's asc2 kernel tests, unchanged in form: kernels defined with
@asc2.jit and launched as kernel[grid](...) on numpy arrays / CPU torch tensors,
compared with the same golden expressions
(python/test/asc2/kernels/test_vadd.py, test_softmax.py, test_softmax_fused.py)."""
import numpy as np
import pytest
import torch

import asc
import asc2

pytestmark = pytest.mark.gpu


@asc2.jit(always_compile=True)
def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
    x_gm = asc2.tensor(x_ptr, [size])
    y_gm = asc2.tensor(y_ptr, [size])
    out_gm = asc2.tensor(out_ptr, [size])
    base_offset = asc2.block_idx() * tile_size * tile_per_block
    for i in range(tile_per_block):
        tile_offset = base_offset + i * tile_size
        x = asc2.load(x_gm, [tile_size], offsets=[tile_offset])
        y = asc2.load(y_gm, [tile_size], offsets=[tile_offset])
        asc2.store(x + y, out_gm, offsets=[tile_offset])


def vadd_launch(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    out = np.empty_like(x)
    size = out.size
    core_num = 16
    tile_size = 128
    num_tiles = asc.ceildiv(size, tile_size)
    vadd_kernel[core_num](x, y, out, size, tile_size, asc.ceildiv(num_tiles, core_num))
    return out


def test_vadd(device):
    rng = np.random.default_rng(seed=2026)
    size = 8192
    x = rng.random(size, dtype=np.float32) * 10
    y = rng.random(size, dtype=np.float32) * 10
    out = vadd_launch(x, y)
    np.testing.assert_array_equal(out, x + y)


def test_vadd_device_tensors_and_stream(device):
    x = torch.rand(8192, device=device)
    y = torch.rand(8192, device=device)
    out = torch.empty_like(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    vadd_kernel[16, s](x, y, out, 8192, 128, 4)
    s.synchronize()
    assert torch.equal(out.cpu(), x.cpu() + y.cpu())


@asc2.jit(always_compile=True, vf_fusion=True)
def softmax_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: int, num_cols: int,
                   tile_size: asc.ConstExpr[int]):
    x_gm = asc2.tensor(x_ptr, [num_rows, num_cols])
    out_gm = asc2.tensor(out_ptr, [num_rows, num_cols])
    for i in range(asc2.block_idx(), num_rows, asc2.block_num(), parallel=True):
        row = asc2.load(x_gm, [1, tile_size], offsets=[i, 0])
        row_minus_max = row - asc2.reduce_max(row)
        numerator = asc2.exp(row_minus_max)
        denominator = asc2.reduce_sum(numerator)
        asc2.store(numerator / denominator, out_gm, offsets=[i, 0])


def test_softmax(device):
    x = torch.rand((64, 1024), dtype=torch.float32)
    out = torch.empty_like(x)
    softmax_kernel[16](x, out, 64, 1024, tile_size=1024)
    torch.testing.assert_close(out, torch.softmax(x, dim=1))


def test_softmax_fused(device):
    @asc2.jit(always_compile=True)
    def softmax_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: int,
                       num_cols: asc.ConstExpr[int], block_size: asc.ConstExpr[int]):
        x_gm = asc2.tensor(x_ptr, [num_rows, num_cols])
        out_gm = asc2.tensor(out_ptr, [num_rows, num_cols])
        start_rows = asc2.block_idx() * block_size
        rows = asc2.load(x_gm, [block_size, num_cols], offsets=[start_rows, 0])
        asc2.store(asc2.softmax(rows), out_gm, offsets=[start_rows, 0])

    core_num = 16
    x = torch.rand((64, 1024), dtype=torch.float32)
    out = torch.empty_like(x)
    block_size = (64 + core_num - 1) // core_num
    softmax_kernel[core_num](x, out, 64, 1024, block_size)
    torch.testing.assert_close(out, torch.softmax(x, dim=1))
