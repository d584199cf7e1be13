"""The reference tests' CPU golden expressions, used as the timed CPU baseline
(``cpu_baseline`` in bench.py) -- TEST/MEASUREMENT INFRASTRUCTURE ONLY.

Each function is the expression a reference test asserts against, evaluated
with torch on the host cores:
  vadd        x + y                                   README.md:53; python/test/asc2/kernels/test_vadd.py:48
  softmax     torch.softmax(x, dim=1)                 python/test/asc2/kernels/test_softmax.py:43
  matmul      a.to(float32) @ b.to(float32)           python/test/asc2/kernels/test_matmul_tiled.py:49
  int8        a.to(int32) @ b.to(int32)               python/test/generalization/adv/test_matmul_iterate_all.py:116
  dequant     (acc.float() * scale).half()            build definition of DEQF16 (test_matmul_quant.py:94-106)
  attention   softmax(q k^T * scale + mask) v in fp32 (no reference golden; build-defined)
  leaky_relu  torch.where(x >= 0, x, x * alpha)       python/test/asc2/kernels/test_leaky_relu.py:47
  vmuladd     x * y + z                               python/test/asc2/kernels/test_vmuladd.py:52
  gelu        0.5 x (1 + tanh(...)) / 0.5 x (1 + erf(x / sqrt 2))   python/test/asc2/kernels/test_gelu.py:44-48
"""
from __future__ import annotations

import math

import torch


def vadd(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    return x + y


def softmax(x: torch.Tensor) -> torch.Tensor:
    return torch.softmax(x, dim=1)


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return a.to(torch.float32) @ b.to(torch.float32)


def matmul_i8(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return a.to(torch.int32) @ b.to(torch.int32)


def dequant(acc: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return (acc.float() * scale).half()


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sm_scale: float, causal: bool,
              rows: torch.Tensor | None = None) -> torch.Tensor:
    """One (batch, head) slice [S, D] in fp32; with ``rows`` (query indices) only those
    output rows, each with the same keys and causal mask as in the full computation."""
    qr = q if rows is None else q[rows]
    s = (qr.float() @ k.float().T) * sm_scale
    if causal:
        qi = torch.arange(q.shape[0]) if rows is None else rows
        s = s.masked_fill(torch.arange(k.shape[0])[None, :] > qi[:, None], float("-inf"))
    return torch.softmax(s, dim=-1) @ v.float()


def leaky_relu(x: torch.Tensor, alpha: torch.Tensor) -> torch.Tensor:
    return torch.where(x >= 0, x, x * alpha)


def vmuladd(x, y, z):
    return x * y + z


def gelu(x: torch.Tensor, approximate: bool) -> torch.Tensor:
    if approximate:
        return 0.5 * x * (1 + torch.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * torch.pow(x, 3))))
    return 0.5 * x * (1 + torch.erf(x / math.sqrt(2)))
