"""Pins the CPU oracle (oracle/asc2_oracle.py) before anything is compared with it.

Each check is chosen so a plausible mistake in the oracle (a dropped term, a wrong
index, a transposed operand, a wrong rounding) fails it: hand-derived fixtures,
literal loops of the reference kernel bodies, closed forms, and library routines
(torch CPU) standing for the reference tests' own golden expressions.
"""
import os
import struct

import numpy as np
import pytest
import torch

from oracle import asc2_oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name))


# ---------------------------------------------------------------------------------------------- vadd

def test_vadd_coverage_fixture():
    f = load("vadd_coverage.npz")
    out = np.full_like(f["x"], -1.0)
    got = O.vadd(f["x"], f["y"], out, int(f["size"]), int(f["tile_size"]), int(f["tile_per_block"]), int(f["grid"]))
    np.testing.assert_array_equal(got, f["expected"])


def test_vadd_reference_recipe_fixture():
    f = load("vadd_rng2026.npz")
    out = np.zeros_like(f["x"])
    got = O.vadd(f["x"], f["y"], out, 8192, 128, 4, 16)
    np.testing.assert_array_equal(got, f["expected"])


def _kernel_body_loop(x, y, out, size, tile, tpb, grid):
    """Literal per-element walk of test_vadd.py:22-28 with Python float32 scalars."""
    res = list(out)
    for b in range(grid):
        base = b * tile * tpb
        for i in range(tpb):
            off = base + i * tile
            for j in range(off, min(off + tile, size)):
                s = struct.unpack("f", struct.pack("f", float(x[j]) + float(y[j])))[0]
                res[j] = s
    return np.array(res, dtype=np.float32)


@pytest.mark.parametrize("size,tile,tpb,grid", [(300, 16, 3, 4), (1000, 128, 2, 3), (64, 8, 0, 5), (50, 7, 2, 2),
                                                (129, 128, 1, 1)])
def test_vadd_matches_kernel_body_loop(size, tile, tpb, grid):
    rng = np.random.default_rng(size + tile)
    x = rng.random(size, dtype=np.float32) * 10
    y = rng.random(size, dtype=np.float32) * 10
    out = np.full(size, -7.0, dtype=np.float32)
    np.testing.assert_array_equal(O.vadd(x, y, out, size, tile, tpb, grid), _kernel_body_loop(x, y, out, size,
                                                                                               tile, tpb, grid))


def test_vadd_int32_wraparound_known_answers():
    x = np.array([2**31 - 1, -2**31, -1, 123456789], dtype=np.int32)
    y = np.array([1, -1, 1, 987654321], dtype=np.int32)
    got = O.add_elements(x, y, "int32")
    np.testing.assert_array_equal(got, np.array([-2**31, 2**31 - 1, 0, 1111111110], dtype=np.int32))


def test_vadd_bf16_matches_torch_and_ties():
    g = torch.Generator().manual_seed(3)
    a = torch.randn(4096, generator=g).to(torch.bfloat16)
    b = torch.randn(4096, generator=g).to(torch.bfloat16)
    got = O.add_elements(a.view(torch.int16).numpy().view(np.uint16), b.view(torch.int16).numpy().view(np.uint16),
                         "bfloat16")
    np.testing.assert_array_equal(got, (a + b).view(torch.int16).numpy().view(np.uint16))
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7 in bfloat16: RNE keeps the even 1.0 (0x3F80)
    one = np.array([0x3F80], dtype=np.uint16)
    tiny = O.f32_to_bf16_bits(np.array([2.0**-8], dtype=np.float32))
    assert O.add_elements(one, tiny, "bfloat16")[0] == 0x3F80
    # 1 + 3*2^-8 ties upward to the even 1 + 2^-6 (0x3F82)
    assert O.f32_to_bf16_bits(np.array([1 + 3 * 2.0**-8], dtype=np.float32))[0] == 0x3F82


def test_vadd_f16_matches_torch():
    g = torch.Generator().manual_seed(4)
    a = (torch.randn(4096, generator=g) * 100).to(torch.float16)
    b = (torch.randn(4096, generator=g) * 100).to(torch.float16)
    np.testing.assert_array_equal(O.add_elements(a.numpy(), b.numpy(), "float16"), (a + b).numpy())


# ------------------------------------------------------------------------------------------- softmax

def test_softmax_closed_forms():
    np.testing.assert_array_equal(O.softmax_row(np.full(1024, 3.25, np.float32)), np.full(1024, 1 / 1024,
                                                                                          np.float32))
    # [0, ln 3] -> [1/4, 3/4]
    got = O.softmax_row(np.array([0.0, np.log(3.0)], dtype=np.float32))
    np.testing.assert_allclose(got, [0.25, 0.75], rtol=2e-7)
    # a row with one dominant entry: exp(-200) underflows to 0 in fp32
    got = O.softmax_row(np.array([0.0, -200.0, -200.0], dtype=np.float32))
    np.testing.assert_array_equal(got, np.array([1.0, 0.0, 0.0], dtype=np.float32))


def test_softmax_shift_invariance_and_sum():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(4096) * 2).astype(np.float32)
    a = O.softmax_row(x)
    b = O.softmax_row(x + np.float32(8.0))  # exact shift for |x| < 2^20
    np.testing.assert_allclose(a, b, rtol=2e-6)
    assert abs(float(a.astype(np.float64).sum()) - 1.0) < 4096 * 2**-24


@pytest.mark.parametrize("rows,cols", [(64, 1024), (16, 4096), (8, 777)])
def test_softmax_matches_torch_golden(rows, cols):
    g = torch.Generator().manual_seed(rows * cols)
    x = torch.randn(rows, cols, generator=g) * 2
    out = np.zeros((rows, cols), np.float32)
    got = O.softmax_rows(x.numpy(), out, rows, cols, cols, 16)
    torch.testing.assert_close(torch.from_numpy(got), torch.softmax(x, dim=1), rtol=1e-6, atol=0)


def test_softmax_fixture_and_partial_columns():
    f = load("softmax_64x1024.npz")
    got = O.softmax_rows(f["x"], np.zeros_like(f["x"]), 64, 1024, 1024, 16)
    np.testing.assert_allclose(got, f["expected"], rtol=1e-6, atol=0)
    # tile_size < num_cols: columns >= tile_size keep their old values
    out = np.full_like(f["x"], 5.0)
    got = O.softmax_rows(f["x"], out, 64, 1024, 512, 3)
    np.testing.assert_array_equal(got[:, 512:], 5.0)
    np.testing.assert_allclose(got[:, :512], torch.softmax(torch.from_numpy(f["x"][:, :512]), 1).numpy(),
                               rtol=1e-6, atol=0)


@pytest.mark.parametrize("rows,cols,tile", [(64, 1024, 2048), (7, 1000, 1024), (3, 5, 64), (5, 1, 2)])
def test_softmax_tile_wider_than_row(rows, cols, tile):
    # the padded load + whole-tile reductions: torch.softmax of the explicitly zero-padded row
    # (a library routine on the tile the reference's load builds), first num_cols values kept
    x = (torch.randn(rows, cols, generator=torch.Generator().manual_seed(cols)) * 0.5).numpy()
    got = O.softmax_rows(x, np.zeros_like(x), rows, cols, tile, 16)
    padded = torch.nn.functional.pad(torch.from_numpy(x), (0, tile - cols))
    np.testing.assert_allclose(got, torch.softmax(padded, dim=1)[:, :cols].numpy(), rtol=3e-6, atol=1e-30)
    np.testing.assert_allclose(got, torch.softmax(padded.double(), dim=1)[:, :cols].numpy(), rtol=1e-6, atol=0)
    # the padding takes part in the sum: the row's own outputs sum to less than 1
    assert (got.astype(np.float64).sum(1) < 1 - 1e-3).all()


def test_softmax_tile_wider_than_row_closed_forms():
    # a zero row padded to the tile: every element of the tile is 0, each output 1/tile
    got = O.softmax_rows(np.zeros((2, 6), np.float32), np.zeros((2, 6), np.float32), 2, 6, 8, 1)
    np.testing.assert_array_equal(got, np.full((2, 6), 1 / 8, np.float32))
    # a row far below zero: the padding zeros hold the maximum, exp(x - 0) underflows to 0
    got = O.softmax_rows(np.full((1, 3), -200.0, np.float32), np.zeros((1, 3), np.float32), 1, 3, 5, 1)
    np.testing.assert_array_equal(got, np.zeros((1, 3), np.float32))
    # float16 rows take the same padded path
    x = np.array([[0.5, -1.0, 2.0]], np.float16)
    got = O.softmax_rows(x, np.zeros_like(x), 1, 3, 4, 1)
    e = np.exp(np.array([0.5, -1.0, 2.0, 0.0]) - 2.0)
    np.testing.assert_array_equal(got, (e / e.sum())[:3].astype(np.float16)[None])


def test_softmax_blocks_coverage():
    x = np.random.default_rng(0).standard_normal((10, 32)).astype(np.float32)
    out = np.full_like(x, -3.0)
    got = O.softmax_blocks(x, out, 10, 32, 3, 2)  # rows [0, 6) written
    np.testing.assert_array_equal(got[6:], -3.0)
    np.testing.assert_allclose(got[:6], torch.softmax(torch.from_numpy(x[:6]), 1).numpy(), rtol=1e-6, atol=0)
    got = O.softmax_blocks(x, out, 10, 32, 4, 16)  # last block clipped at row 10
    np.testing.assert_allclose(got, torch.softmax(torch.from_numpy(x), 1).numpy(), rtol=1e-6, atol=0)


# -------------------------------------------------------------------------------------------- matmul

def _loop_matmul(a, b):
    M, K = a.shape
    N = b.shape[1]
    c = np.zeros((M, N))
    for i in range(M):
        for j in range(N):
            c[i, j] = sum(float(a[i, k]) * float(b[k, j]) for k in range(K))
    return c


def test_matmul_identity_permutation_and_loop():
    rng = np.random.default_rng(2)
    a = rng.standard_normal((12, 20)).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(O.matmul(a, np.eye(20, dtype=np.float32)), a)
    perm = np.eye(20, dtype=np.float32)[::-1]
    np.testing.assert_array_equal(O.matmul(a, perm), a[:, ::-1])
    b = rng.standard_normal((20, 7)).astype(np.float16).astype(np.float32)
    np.testing.assert_allclose(O.matmul(a, b), _loop_matmul(a, b), rtol=1e-6, atol=1e-6)
    # the transposed product is not accepted as the product
    sq = rng.standard_normal((8, 8)).astype(np.float32)
    sq2 = rng.standard_normal((8, 8)).astype(np.float32)
    assert not np.allclose(O.matmul(sq, sq2), O.matmul(sq2, sq))


def test_matmul_relu_cast_matches_torch_fixpipe_golden():
    g = torch.Generator().manual_seed(5)
    for dtype, out in ((torch.float16, "float16"), (torch.bfloat16, "float16")):
        a = (torch.rand((64, 128), generator=g, dtype=dtype) - .5) * 10
        b = (torch.rand((128, 256), generator=g, dtype=dtype) - .5) * 10
        ref = (a.to(torch.float32) @ b.to(torch.float32)).relu().to(torch.float16)
        got = O.matmul(a.float().numpy(), b.float().numpy(), relu=True, out_dtype=out)
        torch.testing.assert_close(torch.from_numpy(got), ref, atol=1e-3, rtol=1e-3)
    bits = O.matmul(np.array([[1.0, 2.0 ** -8]], np.float32), np.array([[1.0], [1.0]], np.float32),
                    out_dtype="bfloat16")
    assert bits[0, 0] == 0x3F80  # 1 + 2^-8 rounds to even 1.0 in bfloat16


def test_matmul_mnblock_fixture():
    f = load("matmul_mnblock_f16.npz")
    for idx in range(len(f["cases"])):
        got = O.matmul(f[f"a{idx}"].astype(np.float32), f[f"b{idx}"].astype(np.float32))
        np.testing.assert_allclose(got, f[f"c{idx}"], rtol=1e-5, atol=1e-5)


def test_mnblock_rectangles():
    cases = [(16, 16, 16, 1, 16, 16, 1), (16, 160, 16, 1, 16, 16, 1), (32, 16, 16, 2, 16, 16, 1),
             (16, 16, 32, 2, 16, 16, 1), (32, 16, 32, 2, 16, 16, 1), (32, 16, 32, 2, 16, 16, 2),
             (32, 16, 32, 4, 16, 16, 1), (480, 224, 1344, 30, 48, 32, 7)]
    for m, k, n, core_num, m_tile, n_tile, ntpb in cases:
        tiles_per_core = (m // m_tile) * (n // n_tile) // core_num
        mtpb = tiles_per_core // ntpb
        rects = O.mnblock_rectangles(m, n, core_num, m_tile, mtpb, n_tile, ntpb)
        cover = np.zeros((m, n), dtype=int)
        for m0, m1, n0, n1 in rects:
            cover[m0:m1, n0:n1] += 1
        assert (cover == 1).all(), (m, k, n)
    # hand-derived partial grid: M=32, N=32, 16x16 tiles, 1 tile per block, 2 blocks
    # block 0 -> (0, 0), block 1 -> (16, 0): only the left column of tiles
    assert O.mnblock_rectangles(32, 32, 2, 16, 1, 16, 1) == [(0, 16, 0, 16), (16, 32, 0, 16)]


# ---------------------------------------------------------------------------------------- int8 matmul

def test_matmul_i8_loop_and_extremes():
    rng = np.random.default_rng(3)
    a = rng.integers(-127, 128, (9, 33), dtype=np.int8)
    b = rng.integers(-127, 128, (33, 5), dtype=np.int8)
    np.testing.assert_array_equal(O.matmul_i8_acc(a, b), _loop_matmul(a.astype(np.int64), b.astype(np.int64)))
    K = 4096
    a = np.full((2, K), -128, dtype=np.int8)
    b = np.full((K, 3), -128, dtype=np.int8)
    np.testing.assert_array_equal(O.matmul_i8_acc(a, b), np.full((2, 3), 128 * 128 * K, dtype=np.int32))
    a[0] = 127
    np.testing.assert_array_equal(O.matmul_i8_acc(a, b)[0], np.full(3, -127 * 128 * K, dtype=np.int32))


def test_dequant_known_answers():
    acc = np.array([[1, -3, 70000, 2049]], dtype=np.int32)
    scale = np.array([0.5, 0.25, 1.0, 1.0], dtype=np.float32)
    got = O.dequant_f16(acc, scale)
    # 70000 overflows fp16 to inf; 2049 is a tie between 2048 and 2050 -> even 2048
    np.testing.assert_array_equal(got, np.array([[0.5, -0.75, np.inf, 2048.0]], dtype=np.float16))
    assert O.trunc19(np.array([1.0 + 2.0**-11], np.float32))[0] == np.float32(1.0)
    assert O.trunc19(np.array([1.0 + 2.0**-10], np.float32))[0] == np.float32(1.0 + 2.0**-10)


def test_dequant_reference_golden_fixture():
    f = load("matmul_quant.npz")
    for idx in range(3):
        acc = O.matmul_i8_acc(f[f"a{idx}"], f[f"b{idx}"])
        np.testing.assert_array_equal(acc, f[f"acc{idx}"])
        gold = O.dequant_reference_golden(acc, f[f"scale{idx}"])
        np.testing.assert_array_equal(gold, f[f"golden{idx}"])
        assert np.abs(acc).max() <= 2048
        np.testing.assert_array_equal(O.dequant_f16(acc, f[f"scale{idx}"], use_trunc19=True), gold)


# --------------------------------------------------------------------------------- flash attention

def test_attention_closed_forms():
    rng = np.random.default_rng(4)
    S, D = 37, 16
    q, k, v = (rng.standard_normal((S, D)) for _ in range(3))
    out = O.attention(q, k, v, 0.3, causal=True)
    np.testing.assert_allclose(out[0], v[0], rtol=1e-12)  # row 0 sees only key 0
    z = np.zeros((S, D))
    np.testing.assert_allclose(O.attention(z, k, v, 1.0, causal=False), np.tile(v.mean(0), (S, 1)), rtol=1e-12)
    prefix = np.cumsum(v, axis=0) / np.arange(1, S + 1)[:, None]
    np.testing.assert_allclose(O.attention(z, k, v, 1.0, causal=True), prefix, rtol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_matches_torch_sdpa(causal):
    g = torch.Generator().manual_seed(6)
    q, k, v = (torch.randn(1, 2, 64, 32, generator=g) for _ in range(3))
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal, scale=0.2)
    for h in range(2):
        got = O.attention(q[0, h].numpy(), k[0, h].numpy(), v[0, h].numpy(), 0.2, causal)
        np.testing.assert_allclose(got, ref[0, h].numpy(), rtol=1e-4, atol=1e-5)


# ------------------------------------------------------------------ leaky_relu / vmuladd / gelu

def _leaky_body_loop(x, alpha, size, tile, tpb, grid):
    """Literal per-element loop of test_leaky_relu.py:19-26 in float32."""
    out = np.full(x.shape, 7.0, np.float32)
    for b in range(grid):
        for i in range(tpb):
            off = (b * tpb + i) * tile
            for j in range(off, min(off + tile, size)):
                v = np.float32(x[j])
                out[j] = v if v >= 0 else np.float32(v * np.float32(alpha))
    return out


@pytest.mark.parametrize("size,tile,tpb,grid", [(1000, 32, 2, 8), (300, 7, 3, 4), (64, 128, 1, 1)])
def test_leaky_relu_matches_kernel_body_loop(size, tile, tpb, grid):
    x = np.random.default_rng(size).standard_normal(size).astype(np.float32) * 3
    got = O.leaky_relu(x, 0.1, np.full(size, 7.0, np.float32), size, tile, tpb, grid)
    np.testing.assert_array_equal(got, _leaky_body_loop(x, 0.1, size, tile, tpb, grid))


def test_leaky_relu_known_answers_and_torch_bf16_golden():
    x = np.array([2.0, -2.0, -0.0, 0.0, np.nan, -np.inf], np.float32)
    got = O.leaky_relu_elements(x, 0.25, "float32")
    assert got[0] == 2.0 and got[1] == -0.5 and got[4] != got[4] and got[5] == -np.inf
    assert np.signbit(got[2]) and not np.signbit(got[3])  # -0 >= 0 passes through unchanged
    # the reference test's recipe and golden (test_leaky_relu.py:41-47), bfloat16
    g = torch.Generator().manual_seed(0)
    xt = torch.rand(8192, dtype=torch.bfloat16, generator=g) * 10.0 - 5.0
    alpha = torch.tensor(0.1, dtype=torch.bfloat16)
    golden = torch.where(xt >= 0, xt, xt * alpha)
    bits = xt.view(torch.int16).numpy().view(np.uint16)
    ours = O.leaky_relu_elements(bits, float(alpha.item()), "bfloat16")
    np.testing.assert_array_equal(ours, golden.view(torch.int16).numpy().view(np.uint16))


def test_vmuladd_unfused_known_answer_and_goldens():
    one = np.float32(1.0 + 2.0 ** -12)
    # x*y = 1 + 2^-11 + 2^-24 rounds (tie to even) to 1 + 2^-11, so the sum is 0; a fused
    # multiply-add would give 2^-24
    got = O.muladd_elements(np.array([one]), np.array([one]), np.array([-(1.0 + 2.0 ** -11)], np.float32),
                            "float32")
    assert got[0] == 0.0
    rng = np.random.default_rng(seed=2026)  # test_vmuladd.py:43-52
    x, y, z = (rng.random(8192, dtype=np.float32) * 10 for _ in range(3))
    np.testing.assert_array_equal(O.muladd_elements(x, y, z, "float32"), x * y + z)
    for dt, name in ((torch.float16, "float16"), (torch.bfloat16, "bfloat16")):
        g = torch.Generator().manual_seed(3)
        xt, yt, zt = (torch.randn(4096, generator=g).to(dt) * 4 for _ in range(3))
        golden = xt * yt + zt
        if name == "bfloat16":
            conv = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
        else:
            conv = lambda t: t.numpy()  # noqa: E731
        ours = O.muladd_elements(conv(xt), conv(yt), conv(zt), name)
        np.testing.assert_array_equal(np.asarray(ours).view(np.uint16), conv(golden).view(np.uint16))


@pytest.mark.parametrize("approximate", [True, False])
def test_gelu_matches_torch_and_identities(approximate):
    x = np.linspace(-8, 8, 2001).astype(np.float32)
    ours = O.gelu_values(x, approximate)
    ref = torch.nn.functional.gelu(torch.from_numpy(x).double(), approximate="tanh" if approximate else "none")
    np.testing.assert_allclose(ours, ref.numpy(), rtol=1e-12, atol=1e-14)
    assert O.gelu_values(np.zeros(1, np.float32), approximate)[0] == 0.0
    # gelu(x) - gelu(-x) = x for both forms (x*Phi(x) and x*sigmoid(2u) are odd-complemented)
    np.testing.assert_allclose(ours - O.gelu_values(-x, approximate), x.astype(np.float64), rtol=0, atol=1e-12)
    out = O.gelu_rows(np.tile(x[:64], 3), np.full(192, 5.0), 3, 64, 40, approximate)
    assert (out[:, 40:] == 5.0).all()
    # a tile wider than the row: the row zero-padded to the tile, gelu over the padded row,
    # the row's own columns kept (the padding's values are gelu(0) = 0, written nowhere)
    rows = np.tile(x[:50], 3).reshape(3, 50)
    padded = np.concatenate([rows, np.zeros((3, 14), np.float32)], axis=1)
    wide = O.gelu_rows(rows, np.full((3, 50), 5.0), 3, 50, 64, approximate)
    full = O.gelu_rows(padded, np.full((3, 64), 5.0), 3, 64, 64, approximate)
    np.testing.assert_array_equal(wide, full[:, :50])
    assert (full[:, 50:] == 0.0).all()


def test_matmul_bias_leaky_relu_known_answer_and_tutorial_golden():
    a = np.array([[1.0, 2.0], [3.0, -4.0]], np.float32)
    b = np.array([[1.0, -1.0], [1.0, 1.0]], np.float32)
    # a @ b = [[3, 1], [-1, -7]]; + bias [0.5, -2] = [[3.5, -1], [-0.5, -9]]; leaky 0.25
    got = O.matmul_bias_leaky_relu(a, b, np.array([0.5, -2.0], np.float32), 0.25)
    np.testing.assert_array_equal(got, np.array([[3.5, -0.25], [-0.125, -2.25]], np.float32))
    # the tutorial's recipe and golden (matmul_leakyrelu.py:121-128)
    g = torch.Generator().manual_seed(5)
    m, k, n = 1024, 256, 640
    at = torch.randint(-5, 5, (m, k), generator=g).to(torch.float16)
    bt = torch.randint(-5, 5, (k, n), generator=g).to(torch.float16)
    bias = torch.randint(-5, 5, (1, n), generator=g).to(torch.float32)
    mm = (torch.matmul(at.to(torch.float32), bt.to(torch.float32)).to(torch.float32) + bias).to(torch.float32)
    golden = torch.where(mm >= 0, mm, mm * 0.001)
    ours = O.matmul_bias_leaky_relu(at.float().numpy(), bt.float().numpy(), bias.numpy(), 0.001)
    np.testing.assert_array_equal(ours, golden.numpy())


# ---------------------------------------------------------------------------- reductions, rms_norm

@pytest.mark.parametrize("op,torch_op", [("sum", torch.sum), ("max", torch.amax), ("min", torch.amin),
                                         ("prod", torch.prod)])
def test_reduce_matches_torch_goldens(op, torch_op):
    # test_reduce_ops.py:55-82: randn * 2.0 on [64, 32], dims 0 and 1, and all elements
    x = torch.randn(64, 32, generator=torch.Generator().manual_seed(1)) * 2.0
    for dim in (0, 1):
        torch.testing.assert_close(torch.from_numpy(O.reduce(x.numpy(), op, dim)), torch_op(x, dim))
    torch.testing.assert_close(torch.from_numpy(O.reduce(x.numpy(), op, None)), torch_op(x))


def test_reduce_exact_cases():
    ints = np.arange(-50, 50, dtype=np.float32).reshape(10, 10)
    np.testing.assert_array_equal(O.reduce(ints, "sum", 1), ints.sum(1))
    np.testing.assert_array_equal(O.reduce(ints, "max", 0), ints[-1])
    np.testing.assert_array_equal(O.reduce(ints, "min", None), np.float32(-50))
    pw = np.array([[2.0, 0.5, 4.0], [-1.0, 8.0, 0.25]], np.float32)
    np.testing.assert_array_equal(O.reduce(pw, "prod", 1), np.array([4.0, -2.0], np.float32))
    nan = np.array([[1.0, np.nan, 3.0]], np.float32)
    assert O.reduce(nan, "max", 1)[0] == 3.0  # maxNum: the non-NaN operand


def test_rms_norm_matches_torch_and_closed_forms():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(37, 300, generator=g, dtype=torch.float64) * 3
    gamma = torch.randn(300, generator=g, dtype=torch.float64)
    ours = O.rms_norm_rows(x.numpy(), gamma.numpy(), 1e-6, 300)
    ref = torch.nn.functional.rms_norm(x, [300], gamma, eps=float(np.float32(1e-6)))
    np.testing.assert_allclose(ours, ref.numpy(), rtol=1e-12, atol=1e-14)
    c = np.full((1, 8), 3.0)
    np.testing.assert_allclose(O.rms_norm_rows(c, np.full(8, 2.0), 0.5, 8),
                               np.full((1, 8), 3.0 / np.sqrt(9.0 + 0.5) * 2.0), rtol=1e-15)
    # scale invariance with eps = 0, and untouched columns past tile_size
    y1 = O.rms_norm_rows(x.numpy(), gamma.numpy(), 0.0, 200)
    y2 = O.rms_norm_rows(7.0 * x.numpy(), gamma.numpy(), 0.0, 200)
    np.testing.assert_allclose(y1[:, :200], y2[:, :200], rtol=1e-13)
    np.testing.assert_array_equal(y1[:, 200:], x.numpy()[:, 200:])


# ------------------------------------------------------------------ element-wise tile operations
# Pinned against torch's CPU ops (the operation tests' goldens,
# python/test/asc2/operations/test_{unary_ops,binary_ops,where}.py) and hand-derived
# known answers for what torch does not define the same way (integer x / 0).

def _bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.numpy().view(np.uint32)
    return t.numpy()


def _as_oracle(t: torch.Tensor, dtype: str) -> np.ndarray:
    return t.view(torch.int16).numpy().view(np.uint16) if dtype == "bfloat16" else t.numpy()


_EDGE_F = [0.0, -0.0, 1.0, -1.0, float("nan"), float("inf"), float("-inf"), 3.5, -2.25, 65504.0, 1e-8]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "maximum", "minimum"])
def test_binary_float_matches_torch(op, dtype):
    g = torch.Generator().manual_seed(21)
    td = getattr(torch, dtype)
    x = torch.cat([torch.randn(400, generator=g) * 5, torch.tensor(_EDGE_F * len(_EDGE_F))]).to(td)
    y = torch.cat([torch.randn(400, generator=g) * 5,
                   torch.tensor([v for v in _EDGE_F for _ in _EDGE_F])]).to(td)  # every pair of edge values
    expected = getattr(torch, op)(x, y)
    got = O.binary_elements(_as_oracle(x, dtype), _as_oracle(y, dtype), op, dtype)
    # bit-exact except the NaN payload, which torch's vector paths choose freely
    got_f = torch.from_numpy(got.view(np.int16)).view(torch.bfloat16).float() if dtype == "bfloat16" else \
        torch.from_numpy(got).float()
    nan = torch.isnan(expected.float())
    assert torch.equal(torch.isnan(got_f), nan)
    keep = ~nan
    if op in ("maximum", "minimum"):
        # torch returns either operand of a -0 / +0 tie depending on its code path;
        # those ties are pinned below by the IEEE 754-2019 definition
        keep &= ~((x.float() == 0) & (y.float() == 0))
    np.testing.assert_array_equal(got.view(np.uint16 if dtype != "float32" else np.uint32)[keep.numpy()],
                                  _bits(expected)[keep.numpy()])


def test_binary_signed_zero_and_nan_ties():
    # IEEE 754-2019 maximum / minimum (arith.maximumf / minimumf): -0 < +0, NaN propagates
    z = np.array([-0.0, 0.0, -0.0, 0.0], np.float32)
    w = np.array([0.0, -0.0, -0.0, 0.0], np.float32)
    assert O.binary_elements(z, w, "maximum", "float32").view(np.uint32).tolist() == [0, 0, 0x80000000, 0]
    assert O.binary_elements(z, w, "minimum", "float32").view(np.uint32).tolist() == \
        [0x80000000, 0x80000000, 0x80000000, 0]
    assert np.isnan(O.binary_elements(np.array([np.nan, 1], np.float32), np.array([1, np.nan], np.float32),
                                      "maximum", "float32")).all()


@pytest.mark.parametrize("dtype", ["int32", "int16"])
def test_binary_int_matches_torch(dtype):
    td = getattr(torch, dtype)
    info = torch.iinfo(td)
    g = torch.Generator().manual_seed(22)
    edge = [0, 1, -1, info.max, info.min, info.max - 1, info.min + 1, 7, -7]
    x = torch.cat([torch.randint(info.min, info.max, (500,), generator=g, dtype=torch.int64),
                   torch.tensor(edge * len(edge))]).to(td)
    y = torch.cat([torch.randint(info.min, info.max, (500,), generator=g, dtype=torch.int64),
                   torch.tensor([v for v in edge for _ in edge])]).to(td)
    for op in ("add", "sub", "mul", "maximum", "minimum"):
        np.testing.assert_array_equal(O.binary_elements(x.numpy(), y.numpy(), op, dtype),
                                      getattr(torch, op)(x, y).numpy(), err_msg=op)
    # torch traps on x / 0 and on min / -1 (x86 idiv); both are pinned by known answers below
    nz = (y != 0) & ~((x == info.min) & (y == -1))
    np.testing.assert_array_equal(O.binary_elements(x.numpy(), y.numpy(), "div", dtype)[nz.numpy()],
                                  torch.div(x[nz], y[nz], rounding_mode="trunc").numpy())
    for amount in (0, 1, 5, info.bits - 1):
        s = torch.full_like(x, amount)
        np.testing.assert_array_equal(O.binary_elements(x.numpy(), s.numpy(), "left_shift", dtype),
                                      torch.bitwise_left_shift(x, s).numpy())
        np.testing.assert_array_equal(O.binary_elements(x.numpy(), s.numpy(), "right_shift", dtype),
                                      torch.bitwise_right_shift(x, s).numpy())


def test_binary_int_known_answers():
    i32 = np.int32
    f = O.binary_elements
    assert f(np.array([7, -7, 0, -(2**31)], i32), np.array([0, 0, 0, -1], i32), "div", "int32").tolist() == \
        [0, 0, 0, -(2**31)]  # x / 0 = 0 (build-defined), INT_MIN / -1 wraps
    assert f(np.array([-7, 7], i32), np.array([2, -2], i32), "div", "int32").tolist() == [-3, -3]  # truncation
    assert f(np.array([2**31 - 1], i32), np.array([1], i32), "add", "int32").tolist() == [-(2**31)]
    assert f(np.array([-8, 1], i32), np.array([1, 31], i32), "right_shift", "int32").tolist() == [-4, 0]
    assert f(np.array([1], i32), np.array([31], i32), "left_shift", "int32").tolist() == [-(2**31)]


@pytest.mark.parametrize("op", ["abs", "ceil", "cos", "cosh", "erf", "exp", "exp2", "floor", "log", "log2", "negative",
                                "relu", "rsqrt", "sin", "sinh", "sqrt", "tan", "tanh"])
def test_unary_matches_torch(op):
    g = torch.Generator().manual_seed(23)
    x = torch.cat([torch.randn(2000, generator=g).clamp(1, 100), torch.randn(2000, generator=g) * 4])
    if op in ("log", "log2", "rsqrt", "sqrt"):
        x = x.abs() + 1e-3
    if op in ("cosh", "sinh", "exp", "exp2"):
        x = x.clamp(-20, 20)
    torch_op = {"negative": torch.neg}.get(op) or getattr(torch, op)
    expected = torch_op(x.double()).float()  # the exact value, rounded once
    got = O.unary_f32(x.numpy(), op)
    np.testing.assert_allclose(got, expected.numpy(), rtol=2e-7, atol=0)
    # and the float32 torch op the reference test compares with, at its own tolerance
    np.testing.assert_allclose(got, torch_op(x).numpy(), rtol=1e-5, atol=1e-3)


def test_unary_special_values():
    x = np.array([-3.0, -0.0, 0.0, np.nan, 2.0, -0.5], np.float32)
    assert O.unary_f32(x, "relu").view(np.uint32).tolist() == \
        torch.relu(torch.from_numpy(x)).numpy().view(np.uint32).tolist()  # +0, -0, +0, NaN, 2, +0
    assert O.unary_f32(np.array([-0.5, 0.5], np.float32), "ceil").view(np.uint32).tolist() == [0x80000000, 0x3F800000]
    assert O.unary_f32(np.array([-0.0], np.float32), "negative").view(np.uint32).tolist() == [0]


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32", "int16", "int32"])
@pytest.mark.parametrize("cmp, torch_op", [("equal", torch.eq), ("not_equal", torch.ne), ("greater", torch.gt),
                                           ("greater_equal", torch.ge), ("less", torch.lt), ("less_equal", torch.le)])
def test_where_matches_reference_golden(cmp, torch_op, dtype):
    # test_where.py:46 / :77 goldens, on the tests' input recipes plus ties
    td = getattr(torch, dtype)
    g = torch.Generator().manual_seed(24)
    if td.is_floating_point:
        x, y = torch.rand(300, generator=g).to(td), torch.rand(300, generator=g).to(td)
    else:
        x, y = torch.randint(-100, 100, (300,), generator=g).to(td), torch.randint(-100, 100, (300,), generator=g).to(td)
    y[:50] = x[:50]
    expected = torch.where(torch_op(x, y), x, y)
    got = O.where_compare(_as_oracle(x, dtype), _as_oracle(y, dtype), cmp, dtype)
    np.testing.assert_array_equal(got, _as_oracle(expected, dtype))
    s = torch.tensor(0 if td.is_signed else 0.5, dtype=td)
    expected = torch.where(torch_op(x, s), torch.tensor(0, dtype=td), torch.tensor(1, dtype=td))
    got = O.where_scalar(_as_oracle(x, dtype), s.item(), cmp, dtype, 0, 1)
    np.testing.assert_array_equal(got, _as_oracle(expected, dtype))


# ---------------------------------------------------------------------------------- softmax float16

def test_softmax_f16_matches_torch():
    g = torch.Generator().manual_seed(31)
    x = (torch.randn(64, 1000, generator=g) * 3).half()
    expected = torch.softmax(x, dim=1)  # float16 in, float16 out (fp32 math inside)
    got = np.stack([O.softmax_row(r) for r in x.numpy()])
    assert got.dtype == np.float16
    # one float16 ulp apart at most: torch rounds its fp32 result, the oracle the exact value
    diff = np.abs(got.astype(np.float64) - expected.numpy().astype(np.float64))
    ulp = np.spacing(np.maximum(np.abs(got), np.abs(expected.numpy())).astype(np.float16)).astype(np.float64)
    assert (diff <= ulp).all()


def test_softmax_f16_closed_forms():
    assert (O.softmax_row(np.full(7, 2.5, np.float16)) == np.float16(1 / 7)).all()
    got = O.softmax_row(np.array([0.0, np.log(3)], np.float16))
    # ln 3 in float16 is 1.0986328125; the exact softmax of the rounded input, rounded
    e = np.exp(np.float64(np.float16(np.log(3))))
    assert got.tolist() == [np.float16(1 / (1 + e)), np.float16(e / (1 + e))]


# --------------------------------------------------------------------- tile load / store, shape ops

MEMORY_CASES = [  # test_memory_ops.py:8-48 (dim, tensor_shape, tile_shape, tile_id, offsets)
    (1, [64], [16], [3], None), (2, [128, 128], [32, 32], [3, 3], None), (2, [1024, 512], [128, 64], [1, 2], None),
    (1, [37], [8], [3], None), (2, [123, 456], [13, 16], [2, 5], None), (1, [53], [16], None, [22]),
    (2, [257, 511], [19, 24], None, [40, 64]), (2, [1000, 1000], [33, 40], [1, 1], None),
    (2, [150, 300], [21, 40], None, [10, 20]), (2, [512, 512], None, None, [0, 0]), (1, [1024], None, None, [0]),
]


@pytest.mark.parametrize("dim, tensor_shape, tile_shape, tile_id, offsets", MEMORY_CASES, ids=str)
def test_tile_binary_matches_memory_test_golden(dim, tensor_shape, tile_shape, tile_id, offsets):
    from pyasc_amd.kernels import tile_offsets
    g = torch.Generator().manual_seed(41)
    x, y = [torch.randn(tensor_shape, generator=g) for _ in range(2)]
    z = torch.zeros(tensor_shape)
    offs = tile_offsets(tensor_shape, tile_shape, tile_id, offsets)
    got = O.tile_binary(x.numpy(), y.numpy(), z.numpy(), "add", tile_shape, offs, "float32")
    # test_memory_ops.py:104-114
    actual = [i * s for i, s in zip(tile_id, tile_shape)] if tile_id is not None else offsets
    slices = tuple(slice(o, o + s) for o, s in zip(actual, tile_shape)) if tile_shape is not None else tuple(actual)
    expected = torch.zeros_like(z)
    expected[slices] = x[slices] + y[slices]
    np.testing.assert_array_equal(got, expected.numpy())


def test_tile_binary_clips_and_offsets_rules():
    from pyasc_amd.kernels import tile_offsets
    x = np.arange(10, dtype=np.float32)
    got = O.tile_binary(x, x, np.zeros(10, np.float32), "add", [4], [8], "float32")
    assert got.tolist() == [0] * 8 + [16, 18]  # a tile past the end is clipped by the store
    with pytest.raises(ValueError):
        tile_offsets([10], [4], [1], [4])  # exactly one of tile_id / offsets
    with pytest.raises(ValueError):
        tile_offsets([10], [4], None, None)
    assert tile_offsets([64, 64], [8, 16], [2, 3], None) == [16, 48]


@pytest.mark.parametrize("rows, cols", [(4, 32), (50, 32), (1, 64)])
def test_broadcast_rows_matches_torch(rows, cols):
    x = torch.randn(1, cols)
    np.testing.assert_array_equal(O.broadcast_rows(x.numpy(), rows, cols), torch.broadcast_to(x, (rows, cols)).numpy())
    np.testing.assert_array_equal(O.broadcast_rows(x.numpy(), 1, cols).reshape(-1), torch.ravel(x).numpy())


@pytest.mark.parametrize("dtype", ["float32", "float16", "int32"])
@pytest.mark.parametrize("op, torch_op", [("add", torch.add), ("maximum", torch.maximum), ("minimum", torch.minimum)])
def test_atomic_tiles_matches_atomic_test_golden(op, torch_op, dtype):
    # test_atomic_ops.py:45-68: 4 blocks of 32 over a 128-element x, +10 in the body
    td = getattr(torch, dtype)
    g = torch.Generator().manual_seed(11)
    if td.is_floating_point:
        x = torch.randn(128, generator=g).clamp(1, 100).to(td)
        z = torch.randn(32, generator=g).clamp(1, 100).to(td)
    else:
        x = torch.randint(1, 100, (128,), generator=g, dtype=td)
        z = torch.randint(1, 100, (32,), generator=g, dtype=td)
    expected = z.clone()
    for i in range(4):
        expected = torch_op(expected, x[i * 32:(i + 1) * 32] + 10)
    got = O.atomic_tiles(x.numpy(), z.numpy(), op, 4, 32, 10, dtype)
    np.testing.assert_allclose(got, expected.numpy(), atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("dtype", ["int32", "int16", "float16", "bfloat16", "float32"])
def test_atomic_tiles_closed_forms(dtype):
    # integer-valued data with every partial sum below 256 in magnitude: each combine is
    # exact (bfloat16 too), so the result is a column reduction
    rng = np.random.default_rng(5)
    xv = rng.integers(-2, 3, size=(37, 53))
    zv = rng.integers(-30, 31, size=53)

    def enc(v):
        return O.f32_to_bf16_bits(v.astype(np.float32)) if dtype == "bfloat16" else v.astype(np.dtype(dtype))

    def dec(v):
        return O.bf16_bits_to_f32(v) if dtype == "bfloat16" else v
    x, z = enc(xv).reshape(-1), enc(zv)
    np.testing.assert_array_equal(dec(O.atomic_tiles(x, z, "add", 37, 53, 3, dtype)), zv + xv.sum(0) + 37 * 3)
    np.testing.assert_array_equal(dec(O.atomic_tiles(x, z, "maximum", 37, 53, 3, dtype)),
                                  np.maximum(zv, xv.max(0) + 3))
    np.testing.assert_array_equal(dec(O.atomic_tiles(x, z, "minimum", 37, 53, -4, dtype)),
                                  np.minimum(zv, xv.min(0) - 4))
    # no tiles: z unchanged
    np.testing.assert_array_equal(O.atomic_tiles(x, z, "add", 0, 53, 3, dtype), z)


def test_atomic_tiles_int_wraps():
    x = np.array([2**31 - 1, 5], dtype=np.int32)
    z = np.array([1, 0], dtype=np.int32)
    np.testing.assert_array_equal(O.atomic_tiles(x, z, "add", 1, 2, 0, "int32"), np.array([-2**31, 5], np.int32))


@pytest.mark.parametrize("dtype", ["float16", "float32", "int16", "int32", "bfloat16"])
def test_fill_matches_torch_full(dtype):
    td = getattr(torch, dtype)
    ref = torch.full((3, 32), 777, dtype=td).reshape(-1)
    ref_np = ref.view(torch.int16).numpy().view(np.uint16) if dtype == "bfloat16" else ref.numpy()
    np.testing.assert_array_equal(O.fill(96, 777, dtype), ref_np)


def _asc1_body_walk(x, y, z, grid, block_length, tile_length, tile_num):
    """Literal walk of python/test/kernels/test_vadd.py:19-35: per block, TILE_NUM tiles of
    TILE_LENGTH from the block's start, with Python float32 scalars, clipped at len(z)."""
    res = list(z)
    for b in range(grid):
        for i in range(tile_num):
            for j in range(tile_length):
                e = b * block_length + i * tile_length + j
                if e < len(res):
                    res[e] = np.float32(x[e]) + np.float32(y[e])
    return np.array(res, dtype=np.float32)


@pytest.mark.parametrize("size, grid, tile_num", [(8192, 16, 8), (8191, 16, 8), (100, 3, 4), (37, 5, 2)])
def test_block_add_matches_asc1_body_walk(size, grid, tile_num):
    rng = np.random.default_rng(size)
    x, y = rng.random(size, dtype=np.float32), rng.random(size, dtype=np.float32)
    z = np.full(size, -3.0, dtype=np.float32)
    block_length = (size + grid - 1) // grid          # the test's launch helper (test_vadd.py:72-80)
    tile_length = (block_length + tile_num - 1) // tile_num
    np.testing.assert_array_equal(O.block_add(x, y, z, grid, block_length, tile_num * tile_length),
                                  _asc1_body_walk(x, y, z, grid, block_length, tile_length, tile_num))


def test_block_add_reference_golden_and_gaps():
    # test_vadd.py:85-92: the launch covers everything, golden x + y
    rng = np.random.default_rng(seed=2025)
    x, y = rng.random(8192, dtype=np.float32), rng.random(8192, dtype=np.float32)
    np.testing.assert_array_equal(O.block_add(x, y, np.zeros(8192, np.float32), 16, 512, 8 * 64), x + y)
    # two blocks of stride 4 adding 3 elements each over 10: elements 3, 7, 8, 9 untouched
    x, y = np.arange(10, dtype=np.float32), np.full(10, 100, dtype=np.float32)
    got = O.block_add(x, y, np.zeros(10, np.float32), 2, 4, 3)
    np.testing.assert_array_equal(got, [100, 101, 102, 0, 104, 105, 106, 0, 0, 0])


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_quant_matches_quant_test_golden(dtype):
    # test_quant.py:79-104: src = rand * 8 - 4, golden torch.round(src * 2.0 + 0.9).to(int8)
    td = getattr(torch, dtype)
    g = torch.Generator().manual_seed(21)
    src = (torch.rand(4096, generator=g) * 8.0 - 4.0).to(td)
    golden = torch.round((src * 2.0) + 0.9).to(torch.int8).numpy()
    np.testing.assert_array_equal(O.quant_i8(src.numpy(), 2.0, 0.9, dtype), golden)


def test_quant_known_answers():
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 127.4, 127.6, 1000.0, -128.4, -1000.0, np.nan, np.inf, -np.inf],
                 np.float32)
    np.testing.assert_array_equal(O.quant_i8(x, 1.0, 0.0, "float32"),
                                  np.array([0, 2, 2, 0, -2, 127, 127, 127, -128, -128, 0, 127, -128], np.int8))
    # the offset is rounded to the source dtype first: fp16(0.1) = 0.0999755859375
    np.testing.assert_array_equal(O.quant_i8(np.array([2.4], np.float16), 1.0, 0.1, "float16"), [2])
    bits = O.f32_to_bf16_bits(np.array([3.0, -3.0], np.float32))
    np.testing.assert_array_equal(O.quant_i8(bits, 0.5, 0.0, "bfloat16"), [2, -2])  # 1.5 -> 2, -1.5 -> -2


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("op", ["abs", "ceil", "cos", "exp", "floor", "log", "negative", "relu", "rsqrt", "sin",
                                "sqrt", "tanh", "erf"])
def test_unary_16bit_matches_torch(op, dtype):
    td = getattr(torch, dtype)
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(20000, generator=g) * 3).to(td)
    if op in ("log", "rsqrt", "sqrt"):
        x = x.abs() + 0.01
    fn = {"negative": torch.neg, "relu": torch.relu}.get(op, getattr(torch, op, None))
    ref = fn(x).float().numpy()
    host = x.view(torch.int16).numpy().view(np.uint16) if dtype == "bfloat16" else x.numpy()
    got = O.unary(host, op, dtype)
    got = O.bf16_bits_to_f32(got) if dtype == "bfloat16" else got.astype(np.float32)
    ulp = 2.0 ** -10 if dtype == "float16" else 2.0 ** -7
    if op in ("abs", "ceil", "floor", "negative", "relu", "sqrt"):
        np.testing.assert_array_equal(got, ref)
    else:
        np.testing.assert_allclose(got, ref, rtol=ulp, atol=1e-6)
