"""Seeded random shapes on both sides of each kernel's path boundaries, against the oracle.

The fixed parametrisations elsewhere pin the reference tests' cases and chosen edges. These
draws add shapes around each kernel's fast-path conditions. For the GEMMs those are
multiples of the 256 x 256 output tile and of the k-tile, the same plus or minus 1 or 31,
tiny dimensions, and anything in between. For softmax they are the row lengths where the
row body changes (256, 512, 1024, 2048, 4096, 8192 columns). A planner or bounds mistake
that only one shape class shows fails here. Each test also checks that its draws reached
every kernel they were meant to reach, using the launch plan's kernel name.

Bars: int8 accumulators and dequant bit-exact; fp16/bf16 GEMM atol/rtol 1e-2 against the
fp64-accumulated oracle; fp32 softmax rtol 1e-6, atol 0; attention atol/rtol 1e-2."""
import numpy as np
import pytest
import torch

from oracle import asc2_oracle as O
from pyasc_amd import kernels

pytestmark = pytest.mark.gpu


def _dim(rng, unit: int, kind: int, top: int) -> int:
    """kind 0: a multiple of ``unit``; 1: a multiple plus or minus 1 or 31; 2: anywhere
    in [1, top]; 3: tiny."""
    if kind == 0:
        return unit * int(rng.integers(1, top // unit + 1))
    if kind == 1:
        return max(1, unit * int(rng.integers(1, top // unit + 1)) + int(rng.choice([-31, -1, 1, 31])))
    if kind == 2:
        return int(rng.integers(1, top + 1))
    return int(rng.integers(1, 40))


def _gemm_shapes(seed: int, n: int, units, tops):
    """Every third draw is aligned in all dimensions (the fast path), every third is aligned
    but for one dimension moved by 1 or 31 (the checked path next to it), the rest random."""
    rng = np.random.default_rng(seed)
    shapes = []
    for i in range(n):
        kinds = [0, 0, 0]
        if i % 3 == 1:
            kinds[int(rng.integers(3))] = 1
        elif i % 3 == 2:
            kinds = [int(rng.integers(1, 4)) for _ in range(3)]
        shapes.append(tuple(_dim(rng, u, k, t) for u, k, t in zip(units, kinds, tops)))
    return shapes


GEMM_SHAPES = _gemm_shapes(2026, 18, units=(256, 256, 32), tops=(768, 768, 1024))
I8_SHAPES = _gemm_shapes(2027, 12, units=(256, 256, 64), tops=(768, 768, 512))


def test_gemm_shapes_reach_both_loops():
    # the draws hit the fast (tile-aligned, direct-to-LDS) and the checked loop alike
    fast = [s for s in GEMM_SHAPES if s[0] % 256 == 0 and s[1] % 256 == 0 and s[2] % 32 == 0]
    assert 5 <= len(fast) <= len(GEMM_SHAPES) - 5
    fast8 = [s for s in I8_SHAPES if s[0] % 256 == 0 and s[1] % 256 == 0 and s[2] % 64 == 0]
    assert 3 <= len(fast8) <= len(I8_SHAPES) - 3


@pytest.mark.parametrize("idx", range(len(GEMM_SHAPES)))
def test_matmul_random_shape(device, idx):
    M, N, K = GEMM_SHAPES[idx]
    rng = np.random.default_rng(idx)
    dtype = [torch.bfloat16, torch.float16][idx % 2]
    out_dtype = [torch.float32, torch.float16, torch.bfloat16][idx % 3]
    g = torch.Generator().manual_seed(1000 + idx)
    a = (torch.randn(M, K, generator=g) / np.sqrt(K)).to(dtype)
    b = torch.randn(K, N, generator=g).to(dtype)
    c = torch.full((M, N), float(rng.integers(-9, 9)), dtype=out_dtype, device=device)
    ad, bd = a.to(device), b.to(device)
    plan = kernels.matmul_plan(ad, bd, c).kernel.decode()
    aligned = M % 256 == 0 and N % 256 == 0 and K % 32 == 0
    assert ("_fast_" in plan) == aligned, (plan, M, N, K)
    kernels.matmul(ad, bd, c)
    torch.cuda.synchronize()
    ref = torch.from_numpy(O.matmul(a.float().numpy(), b.float().numpy()))
    torch.testing.assert_close(c.cpu().float(), ref.to(out_dtype).float(), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("idx", range(len(I8_SHAPES)))
def test_matmul_i8_random_shape(device, idx):
    M, N, K = I8_SHAPES[idx]
    g = torch.Generator().manual_seed(2000 + idx)
    a = torch.randint(-127, 128, (M, K), dtype=torch.int8, generator=g)
    b = torch.randint(-127, 128, (K, N), dtype=torch.int8, generator=g)
    scale = torch.rand(N, generator=g) * 0.009 + 0.001
    ad, bd = a.to(device), b.to(device)
    acc = torch.full((M, N), -5, dtype=torch.int32, device=device)
    out = torch.full((M, N), 3.0, dtype=torch.float16, device=device)
    plan = kernels.matmul_i8_plan(ad, bd, acc).kernel.decode()
    aligned = M % 256 == 0 and N % 256 == 0 and K % 64 == 0
    assert ("_fast_" in plan) == aligned, (plan, M, N, K)
    kernels.matmul_i8(ad, bd, acc)
    kernels.matmul_i8(ad, bd, out, scale=scale.to(device))
    torch.cuda.synchronize()
    expect = O.matmul_i8_acc(a.numpy(), b.numpy())
    np.testing.assert_array_equal(acc.cpu().numpy(), expect)
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16),
                                  O.dequant_f16(expect, scale.numpy()).view(np.uint16))


def _softmax_draws(seed: int, n: int):
    rng = np.random.default_rng(seed)
    draws = []
    for i in range(n):
        edge = int(rng.choice([256, 512, 1024, 2048, 4096, 8192]))
        cols = [edge, edge + int(rng.choice([-4, -1, 1, 4])), int(rng.integers(1, 20000))][i % 3]
        rows = int(rng.integers(1, 200))
        pad = int(rng.choice([0, 0, 0, 16, 300]))  # some tiles wider than the row
        draws.append((rows, max(1, cols), pad))
    return draws


SOFTMAX_DRAWS = _softmax_draws(2030, 18)  # a seed whose draws reach all eight fp32 bodies


@pytest.mark.parametrize("idx", range(len(SOFTMAX_DRAWS)))
def test_softmax_random_shape(device, idx):
    rows, cols, pad = SOFTMAX_DRAWS[idx]
    tile = cols + pad
    x = torch.randn(rows, cols, generator=torch.Generator().manual_seed(3000 + idx)) * 2.0
    out = torch.full((rows, cols), 9.0, device=device)
    kernels.softmax_rows(x.to(device), out, rows, cols, tile, 16)
    torch.cuda.synchronize()
    expected = O.softmax_rows(x.numpy(), np.zeros((rows, cols), np.float32), rows, cols, tile, 16)
    np.testing.assert_allclose(out.cpu().numpy(), expected, rtol=1e-6, atol=0)


def test_softmax_draws_reach_every_row_body(device):
    # the row-length draws, and the padded form, cover each fp32 softmax kernel
    seen = set()
    for rows, cols, pad in SOFTMAX_DRAWS:
        x = torch.empty(rows, cols, device=device)
        seen.add(kernels.softmax_plan(x, x, rows, cols, cols + pad, 16, False).kernel.decode())
    body = {"wave_1x2", "wave_2x2", "block_2x128", "block_2x256", "block_2x512", "block_8x256", "long",
            "padded_f32"}
    assert {s.split("asc2_softmax_")[-1] for s in seen} == body


def _attention_draws(seed: int, n: int):
    rng = np.random.default_rng(seed)
    # S: anywhere below 600, or a multiple of the 64-key tile plus -1, 0 or 1
    return [(int(rng.integers(1, 3)), int(rng.integers(1, 4)),
             [int(rng.integers(1, 600)), 64 * int(rng.integers(1, 9)) + int(rng.choice([-1, 0, 1]))][i % 2],
             [64, 128][(i // 2) % 2], bool(i % 3)) for i in range(n)]


ATTENTION_DRAWS = _attention_draws(2029, 10)


@pytest.mark.parametrize("idx", range(len(ATTENTION_DRAWS)))
def test_attention_random_shape(device, idx):
    B, H, S, D, causal = ATTENTION_DRAWS[idx]
    g = torch.Generator().manual_seed(4000 + idx)
    q, k, v = (torch.randn(B, H, S, D, generator=g).to(torch.bfloat16) for _ in range(3))
    o = torch.full(q.shape, 7.0, dtype=torch.bfloat16, device=device)
    kernels.flash_attention_fwd(q.to(device), k.to(device), v.to(device), o, D ** -0.5, causal)
    torch.cuda.synchronize()
    out = o.cpu().float().numpy()
    for bb in range(B):
        for hh in range(H):
            exact = O.attention(q[bb, hh].float().numpy(), k[bb, hh].float().numpy(), v[bb, hh].float().numpy(),
                                D ** -0.5, causal)
            np.testing.assert_allclose(out[bb, hh], exact, atol=1e-2, rtol=1e-2)


def _np(t: torch.Tensor) -> np.ndarray:
    # bfloat16 travels to the oracle as its uint16 bit patterns
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.int32])
def test_vadd_random_launches(device, dtype):
    # random sizes, tiles, blocks and grids, some covering less than the tensor, some with
    # an offset view (unaligned: the element kernel only)
    rng = np.random.default_rng(2030)
    for i in range(12):
        size = int(rng.integers(1, 300000))
        tile = int(rng.choice([8, 64, 128, 256, 1000]))
        grid = int(rng.integers(1, 64))
        tpb = int(rng.integers(0, -(-size // (tile * grid)) + 2))
        offset = int(rng.integers(0, 3))
        g = torch.Generator().manual_seed(5000 + i)
        if dtype == torch.int32:
            x, y = (torch.randint(-2 ** 31, 2 ** 31 - 1, (size + offset,), generator=g, dtype=torch.int32)
                    for _ in range(2))
        else:
            x, y = ((torch.rand(size + offset, generator=g) * 10).to(dtype) for _ in range(2))
        x, y = x[offset:], y[offset:]
        out = torch.full((size + offset,), 5, dtype=dtype, device=device)[offset:]
        kernels.vadd(x.to(device), y.to(device), out, size, tile, tpb, grid)
        torch.cuda.synchronize()
        names = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16",
                 torch.int32: "int32"}
        init = torch.full((size,), 5, dtype=dtype)
        expect = O.vadd(*(_np(t) for t in (x, y, init)), size, tile, tpb, grid, names[dtype])
        np.testing.assert_array_equal(_np(out.cpu()).view(np.uint8), np.asarray(expect).view(np.uint8),
                                      err_msg=f"size={size} tile={tile} tpb={tpb} grid={grid} offset={offset}")
