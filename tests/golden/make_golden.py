"""Writes the small golden fixtures under tests/golden/.

The reference ships no stored vectors: each of its tests regenerates inputs and
compares with a torch/numpy CPU expression.  These fixtures freeze exactly those
recipes (seeds, distributions, shapes) together with the reference tests' own
golden expressions, evaluated here with numpy/torch CPU, so the oracle and the
GPU kernels are checked against the same data without the reference:

  vadd_rng2026.npz        python/test/asc2/kernels/test_vadd.py:41-48
                          (rng 2026, size 8192, x*10, golden x + y)
  vadd_coverage.npz       hand-derived: size 1000, tile 128, tpb 2, grid 3 ->
                          elements [0, 768) written, the rest keep the sentinel
  softmax_64x1024.npz     python/test/asc2/kernels/test_softmax.py:38-43
                          (torch.rand 64x1024, golden torch.softmax(x, dim=1))
  matmul_mnblock_f16.npz  python/test/asc2/kernels/test_matmul_mnblock.py:73-92
                          (the seven small shapes of the parametrisation, golden
                          a.float() @ b.float())
  matmul_quant.npz        python/test/generalization/adv/test_matmul_quant.py:94-136
                          (randint(-5, 5) int8, scale (rand-0.5)*10, golden gen_golden)

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def save(name: str, **arrays) -> None:
    np.savez_compressed(os.path.join(HERE, name), **arrays)


def vadd() -> None:
    rng = np.random.default_rng(seed=2026)
    size = 8192
    x = rng.random(size, dtype=np.float32) * 10
    y = rng.random(size, dtype=np.float32) * 10
    save("vadd_rng2026.npz", x=x, y=y, expected=x + y)

    rng = np.random.default_rng(seed=7)
    n = 1000
    x = rng.random(n, dtype=np.float32)
    y = rng.random(n, dtype=np.float32)
    expected = np.full(n, -1.0, dtype=np.float32)
    expected[:768] = x[:768] + y[:768]  # 3 blocks x 2 tiles x 128 elements
    save("vadd_coverage.npz", x=x, y=y, expected=expected, size=n, tile_size=128, tile_per_block=2, grid=3)


def softmax() -> None:
    g = torch.Generator().manual_seed(2026)
    x = torch.rand((64, 1024), dtype=torch.float32, generator=g)
    save("softmax_64x1024.npz", x=x.numpy(), expected=torch.softmax(x, dim=1).numpy())


def matmul_mnblock() -> None:
    cases = [
        (16, 16, 16, 1, 16, 16, 1),
        (16, 160, 16, 1, 16, 16, 1),
        (32, 16, 16, 2, 16, 16, 1),
        (16, 16, 32, 2, 16, 16, 1),
        (32, 16, 32, 2, 16, 16, 1),
        (32, 16, 32, 2, 16, 16, 2),
        (32, 16, 32, 4, 16, 16, 1),
    ]  # the 480x224x1344 case is regenerated in the GPU test (its C alone is 2.5 MB)
    g = torch.Generator().manual_seed(2027)
    out = {"cases": np.array(cases, dtype=np.int64)}
    for idx, (m, k, n, *_rest) in enumerate(cases):
        a = torch.rand((m, k), dtype=torch.float16, generator=g)
        b = torch.rand((k, n), dtype=torch.float16, generator=g)
        out[f"a{idx}"] = a.numpy()
        out[f"b{idx}"] = b.numpy()
        out[f"c{idx}"] = (a.to(torch.float32) @ b.to(torch.float32)).numpy()
    save("matmul_mnblock_f16.npz", **out)


def matmul_quant() -> None:
    g = torch.Generator().manual_seed(2028)
    out = {}
    for idx, (m, k, n) in enumerate([(256, 256, 256), (256, 128, 64), (64, 128, 256)]):
        a = torch.randint(-5, 5, (m, k), dtype=torch.int8, generator=g)
        b = torch.randint(-5, 5, (k, n), dtype=torch.int8, generator=g)
        quant = (torch.rand((1, n), dtype=torch.float32, generator=g) - .5) * 10
        acc = a.to(torch.int32) @ b.to(torch.int32)
        # gen_golden: fp16(acc), then each row times the trunc-19 quant vector
        golden = acc.to(torch.float16)
        mask = 0xFFFFE000 - (1 << 32)  # the bit pattern 0xFFFFE000 as a signed int32
        q = (quant.view(torch.int32) & mask).view(torch.float32)
        for i in range(m):
            golden[i, :] = golden[i, :] * q
        out[f"a{idx}"] = a.numpy()
        out[f"b{idx}"] = b.numpy()
        out[f"scale{idx}"] = quant.numpy().reshape(-1)
        out[f"acc{idx}"] = acc.numpy()
        out[f"golden{idx}"] = golden.numpy()
    save("matmul_quant.npz", **out)


if __name__ == "__main__":
    vadd()
    softmax()
    matmul_mnblock()
    matmul_quant()
    print("fixtures written to", HERE)
