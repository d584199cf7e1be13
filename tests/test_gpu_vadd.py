"""vadd parity on the GPU through the C ABI: bit-exact against the oracle and the
reference's golden ``x + y`` (python/test/asc2/kernels/test_vadd.py:41-48)."""
import os

import numpy as np
import pytest
import torch

from oracle import asc2_oracle as O
from pyasc_amd import kernels

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _np(t):
    """numpy view of a tensor: bfloat16 as uint16 bit patterns, other dtypes as themselves."""
    t = t.cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def _bits(a):
    """Bit patterns for a bit-exact comparison (NaN-safe)."""
    return a.view(np.uint16) if a.dtype in (np.float16, np.uint16) else a.view(np.uint32)


def test_reference_recipe_fixture(device):
    f = np.load(os.path.join(GOLDEN, "vadd_rng2026.npz"))
    x, y = torch.from_numpy(f["x"]).to(device), torch.from_numpy(f["y"]).to(device)
    out = torch.empty_like(x)
    kernels.vadd(x, y, out, 8192, 128, 4, 16)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), f["expected"])


def test_coverage_fixture(device):
    f = np.load(os.path.join(GOLDEN, "vadd_coverage.npz"))
    x, y = torch.from_numpy(f["x"]).to(device), torch.from_numpy(f["y"]).to(device)
    out = torch.full_like(x, -1.0)
    kernels.vadd(x, y, out, int(f["size"]), int(f["tile_size"]), int(f["tile_per_block"]), int(f["grid"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), f["expected"])


@pytest.mark.parametrize("size,tile,tpb,grid", [(8192, 128, 4, 16), (8191, 128, 4, 16), (1, 128, 1, 1),
                                                (10000, 100, 3, 7), (3, 1, 1, 2), (1 << 20, 128, 512, 16),
                                                ((1 << 22) + 5, 256, 1025, 16)])
@pytest.mark.parametrize("dtype", ["float32", "int32", "float16", "bfloat16"])
def test_vadd_vs_oracle(device, size, tile, tpb, grid, dtype):
    g = torch.Generator().manual_seed(size)
    if dtype == "int32":
        x = torch.randint(-2**31, 2**31, (size,), dtype=torch.int32, generator=g)
        y = torch.randint(-2**31, 2**31, (size,), dtype=torch.int32, generator=g)
        sentinel = torch.full((size,), 77, dtype=torch.int32)
    else:
        td = getattr(torch, dtype)
        x = (torch.randn(size, generator=g) * 10).to(td)
        y = (torch.randn(size, generator=g) * 10).to(td)
        sentinel = torch.full((size,), -1.0).to(td)
    out = sentinel.to(device)
    kernels.vadd(x.to(device), y.to(device), out, size, tile, tpb, grid)
    torch.cuda.synchronize()
    expected = O.vadd(_np(x), _np(y), _np(sentinel), size, tile, tpb, grid, dtype)
    np.testing.assert_array_equal(_bits(_np(out)), _bits(expected))


def test_unaligned_views(device):
    size = 4099
    g = torch.Generator().manual_seed(1)
    base_x = torch.rand(size + 3, generator=g)
    base_y = torch.rand(size + 3, generator=g)
    x, y = base_x.to(device)[1:1 + size], base_y.to(device)[3:3 + size]
    out_base = torch.zeros(size + 2, device=device)
    out = out_base[2:]
    kernels.vadd(x, y, out, size, 64, 8, 9)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), (base_x[1:1 + size] + base_y[3:3 + size]).numpy())


def test_full_size_against_numpy(device):
    n = 1 << 26  # the bandwidth shape of the bench is 1 << 28; same kernel, same path
    g = torch.Generator().manual_seed(0)
    x = torch.rand(n, generator=g)
    y = torch.rand(n, generator=g)
    out = torch.empty(n, device=device)
    tpb = (n // 128 + 15) // 16
    kernels.vadd(x.to(device), y.to(device), out, n, 128, tpb, 16)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), x.numpy() + y.numpy())


def test_host_checks_reject_short_buffers(device):
    x = torch.zeros(100, device=device)
    with pytest.raises(ValueError, match="touches"):
        kernels.vadd(x, x, torch.zeros(50, device=device), 100, 10, 10, 1)
