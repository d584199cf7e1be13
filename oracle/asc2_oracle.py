"""CPU oracle for the asc2 hot-path kernels -- TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, what each reference kernel computes.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker (or the timed CPU baseline);
the product path (pyasc_amd) never calls it and has no CPU fallback.

How each function is pinned (tests/test_oracle.py):
  vadd            hand-derived coverage fixture, a literal per-element loop of the
                  kernel body, IEEE/two's-complement known answers, torch's own
                  float16/bfloat16 add.
  softmax_*       closed forms (constant row -> 1/n, two-point rows), shift
                  invariance, row sums, torch.softmax (the reference's golden);
                  tiles wider than the row: torch.softmax of the explicitly
                  zero-padded row, a zero row -> 1/tile, tile == cols unchanged.
  matmul          identity / permutation products, a pure-Python fp64 loop on
                  tiny shapes, torch fp32 matmul (the reference's golden).
  mnblock cover   hand-derived rectangles, full coverage of the reference test's
                  parametrisations.
  matmul_i8       pure-Python integer loop, extreme-value closed forms.
  dequant         hand-computed RNE cases, the reference golden formula
                  (gen_golden) where |acc| <= 2048.
  attention       causal row 0 == v[0], q = 0 -> (prefix) means of v, torch's
                  scaled_dot_product_attention in fp32.
  leaky_relu      a literal per-element loop of the kernel body, sign / -0 / NaN
                  known answers, torch.where(x >= 0, x, x * alpha) in bfloat16
                  (the reference's golden).
  vmuladd         per-element fp32 known answers (rounding of the product shows),
                  numpy's unfused x * y + z (the reference's golden), torch float16
                  / bfloat16 mul-then-add.
  gelu            torch.nn.functional.gelu in float64 (both forms; same function,
                  different expression), gelu(0) = 0, gelu(x) - gelu(-x) = x.
  matmul + bias   the tutorial's golden (torch fp32 matmul + bias, then where) on
  + leaky_relu    its integer-valued recipe (exact), a hand-computed 2x2 case.
  reduce          torch sum / amax / amin / prod (the reduction tests' goldens),
                  integer-valued sums (exact), products of powers of two (exact).
  tile add        the memory test's own golden (z[slices] = x[slices] + y[slices],
  (memory ops)    test_memory_ops.py:104-114) on all its cases; clipping by hand.
  broadcast_rows  torch.broadcast_to / reshape (test_shape_ops.py's goldens).
  block_add       the asc1 vadd test's golden (x + y, test_vadd.py:85-92) at its launch
                  parameters, a literal walk of the body's tile loop, hand-worked gaps.
  unary (16-bit)  torch's float16 / bfloat16 ops (fp32 math, one rounding) within one ulp;
                  the exact ops (abs, neg, floor, ceil, sqrt, relu) bit for bit.
  atomic tiles    the atomic test's golden (torch add / maximum / minimum folded over
                  the blocks, test_atomic_ops.py:62-67); closed forms: the column sum
                  plus n_tiles * addend (integers), the column max / min plus addend.
  fill            torch.full (test_shape_ops.py:75-78).
  quant_i8        the quant test's golden torch.round(src * 2.0 + 0.9).to(int8) on its
                  recipe (test_quant.py:79-104; fp32 exact by construction), ties to even,
                  saturation and NaN by hand.
  softmax f16     torch.softmax on float16 (within one float16 ulp), constant row
                  -> 1/n rounded, two-point rows.
  rms_norm        torch.nn.functional.rms_norm in float64, constant rows (closed
                  form c / sqrt(c^2 + eps) * gamma), scale invariance.
  tile ops        torch's add / sub / mul / div / maximum / minimum / shifts on
  (binary,        every dtype with signed-zero, NaN, infinity and integer-extreme
  unary, where)   pairs (bit-exact; NaN compared as NaN); hand known answers for
                  integer x / 0, min / -1, shifts and IEEE 754-2019 max/min ties;
                  torch's unary functions in float64 rounded once; torch.where over
                  torch's comparisons (the where tests' goldens).
Every function here has at least one such check; none is "parity unpinned".
"""
from __future__ import annotations

from typing import List, Tuple

import numpy as np

# ------------------------------------------------------------------------------------ bfloat16 bits


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (NaN -> quiet NaN)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


# ---------------------------------------------------------------------------------------------- vadd

def vadd_covered(size: int, tile_size: int, tile_per_block: int, grid: int) -> int:
    """python/test/asc2/kernels/test_vadd.py:22-28: block b writes tiles
    (b*tpb + i)*tile for i < tpb; the store clips at ``size``
    (lib/Conversion/LowerToAsc/LowerAscTileDataTransfer.cpp:255-268)."""
    return max(0, min(size, grid * tile_per_block * tile_size))


def add_elements(x: np.ndarray, y: np.ndarray, dtype: str) -> np.ndarray:
    """Elementwise ``x + y`` of one asc2 ``add`` (python/asc/language/tile/binary_ops.py:110-114):
    float32/float16 IEEE RNE, int32 two's-complement wraparound, bfloat16 given as
    uint16 bit patterns (fp32 add then RNE)."""
    if dtype == "bfloat16":
        return f32_to_bf16_bits(bf16_bits_to_f32(x) + bf16_bits_to_f32(y))
    if dtype == "int32":
        return (x.astype(np.int64) + y.astype(np.int64)).astype(np.uint64).astype(np.uint32).view(np.int32)
    with np.errstate(over="ignore"):
        return (x + y).astype(x.dtype)


def vadd(x: np.ndarray, y: np.ndarray, out: np.ndarray, size: int, tile_size: int, tile_per_block: int, grid: int,
         dtype: str = "float32") -> np.ndarray:
    """Returns a copy of ``out`` after the kernel body ran for every logical block."""
    res = out.copy()
    n = vadd_covered(size, tile_size, tile_per_block, grid)
    res[:n] = add_elements(x[:n], y[:n], dtype)
    return res


def block_add(x: np.ndarray, y: np.ndarray, z: np.ndarray, grid: int, block_stride: int, block_cover: int,
              dtype: str = "float32") -> np.ndarray:
    """The asc1 vadd bodies (python/test/kernels/test_vadd.py:16-35; python/tutorials/01_add/
    add.py:29-70, 02_add_framework/add_framework.py:29-80): block b < grid views x, y, z from
    b * block_stride and adds ``block_cover`` elements (TILE_NUM tiles of TILE_LENGTH).
    Returns a copy of z with the union of the blocks written, clipped at z's length."""
    res = np.asarray(z).copy()
    n = res.size
    starts = np.arange(grid, dtype=np.int64) * block_stride
    idx = (starts[:, None] + np.arange(block_cover, dtype=np.int64)[None, :]).reshape(-1)
    idx = np.unique(idx[idx < n])
    res[idx] = add_elements(np.asarray(x)[idx], np.asarray(y)[idx], dtype)
    return res


# -------------------------------------------------------------------------- leaky_relu / vmuladd / gelu

def _to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    return bf16_bits_to_f32(x) if dtype == "bfloat16" else np.asarray(x).astype(np.float32)


def _from_f32(v: np.ndarray, dtype: str) -> np.ndarray:
    """RNE from float32 to the element type (bfloat16 as uint16 bit patterns)."""
    if dtype == "bfloat16":
        return f32_to_bf16_bits(v)
    with np.errstate(over="ignore"):  # beyond the float16 range rounds to inf
        return np.asarray(v, dtype=np.float32).astype(np.float16 if dtype == "float16" else np.float32)


def leaky_relu_elements(x: np.ndarray, alpha: float, dtype: str) -> np.ndarray:
    """python/test/asc2/kernels/test_leaky_relu.py:24 ``where(x >= 0, x, x * alpha)``: the
    product in float32, rounded once to the element type; x >= 0 (also -0) passes unchanged."""
    xf = _to_f32(x, dtype)
    with np.errstate(over="ignore", invalid="ignore"):
        prod = _from_f32(xf * np.float32(alpha), dtype)
    return np.where(xf >= 0, x, prod)


def leaky_relu(x: np.ndarray, alpha: float, out: np.ndarray, size: int, tile_size: int, tile_per_block: int,
               grid: int, dtype: str = "float32") -> np.ndarray:
    """test_leaky_relu.py:16-26: vadd-style tiles, coverage [0, min(size, grid*tpb*tile))."""
    res = out.copy()
    n = vadd_covered(size, tile_size, tile_per_block, grid)
    res[:n] = leaky_relu_elements(x[:n], alpha, dtype)
    return res


def muladd_elements(x: np.ndarray, y: np.ndarray, z: np.ndarray, dtype: str) -> np.ndarray:
    """python/test/asc2/kernels/test_vmuladd.py:29 ``x * y + z``: two tile ops, each rounded to
    the element type (the golden at :52 is numpy's unfused ``x * y + z``)."""
    with np.errstate(over="ignore", invalid="ignore"):
        prod = _from_f32(_to_f32(x, dtype) * _to_f32(y, dtype), dtype)
        return _from_f32(_to_f32(prod, dtype) + _to_f32(z, dtype), dtype)


def vmuladd(x: np.ndarray, y: np.ndarray, z: np.ndarray, out: np.ndarray, size: int, tile_size: int,
            tile_per_block: int, grid: int, dtype: str = "float32") -> np.ndarray:
    """test_vmuladd.py:16-31: vadd-style tiles, coverage [0, min(size, grid*tpb*tile))."""
    res = out.copy()
    n = vadd_covered(size, tile_size, tile_per_block, grid)
    res[:n] = muladd_elements(x[:n], y[:n], z[:n], dtype)
    return res


def gelu_values(x: np.ndarray, approximate: bool) -> np.ndarray:
    """python/test/asc2/kernels/test_gelu.py:24-31 in float64 on float32 inputs:
    tanh form x - x / (exp(x*(x*x*k2 + k1)) + 1) with k1 = 2*sqrt(2/pi), k2 = k1*0.044715;
    erf form x * (erf(x*sqrt(0.5)) + 1) * 0.5."""
    xd = np.asarray(x, dtype=np.float32).astype(np.float64)
    if approximate:
        k1 = 2.0 * np.sqrt(2.0 / np.pi)
        k2 = k1 * 0.044715
        with np.errstate(over="ignore"):
            return xd - xd / (np.exp(xd * (xd * xd * k2 + k1)) + 1.0)
    from scipy.special import erf
    return xd * (erf(xd * np.sqrt(0.5)) + 1.0) * 0.5


def gelu_rows(x: np.ndarray, out: np.ndarray, num_rows: int, num_cols: int, tile_size: int,
              approximate: bool) -> np.ndarray:
    """test_gelu.py:19-33: every row's first ``tile_size`` columns (grid-stride rows cover all
    rows).  With ``tile_size > num_cols`` the [1, tile] load pads the row with zeros
    (LowerAscTileDataTransfer.cpp:181-222); gelu is element-wise, so the row's own columns
    are gelu(x) whatever the padding, and only the row's own columns are written (the
    reference's tile store would also write the padding's gelu(0) = 0 into the next row,
    racing with that row's own store)."""
    tile_size = min(tile_size, num_cols)
    x2 = np.asarray(x, dtype=np.float32).reshape(num_rows, num_cols)
    res = np.array(out, dtype=np.float64).reshape(num_rows, num_cols)
    res[:, :tile_size] = gelu_values(x2[:, :tile_size], approximate)
    return res


# --------------------------------------------------------------------------------- reductions, rms_norm

def reduce(x: np.ndarray, op: str, dim) -> np.ndarray:
    """asc2.reduce_{sum,max,min,prod} (python/asc/language/tile/reduction_ops.py:61-126) of a
    float32 tile along ``dim`` (None: all elements).  Sums and products in float64, rounded
    once to float32; max / min exact (the non-NaN operand, IEEE maxNum / minNum)."""
    xd = np.asarray(x, dtype=np.float32).astype(np.float64)
    axis = None if dim is None else int(dim)
    if op == "sum":
        r = xd.sum(axis=axis)
    elif op == "prod":
        r = xd.prod(axis=axis)
    elif op == "max":
        r = np.fmax.reduce(xd, axis=axis) if axis is not None else np.fmax.reduce(xd.reshape(-1))
    elif op == "min":
        r = np.fmin.reduce(xd, axis=axis) if axis is not None else np.fmin.reduce(xd.reshape(-1))
    else:
        raise ValueError(op)
    with np.errstate(over="ignore"):  # products of many elements overflow to +-inf, as in fp32
        return np.asarray(r).astype(np.float32)


def rms_norm_rows(x: np.ndarray, gamma: np.ndarray, eps: float, tile_size: int) -> np.ndarray:
    """asc2.rms_norm (unary_ops.py:225-237, AscendC RmsNorm) over each row's first
    ``tile_size`` columns, in float64: y = x / sqrt(mean(x^2) + eps) * gamma; other columns
    keep x's values (the caller's output buffer is untouched there)."""
    xd = np.asarray(x, dtype=np.float64)
    head = xd[:, :tile_size]
    r = 1.0 / np.sqrt((head * head).mean(axis=1, keepdims=True) + np.float64(np.float32(eps)))
    out = xd.copy()
    out[:, :tile_size] = head * r * np.asarray(gamma, dtype=np.float64)[:tile_size]
    return out


# ------------------------------------------------------------------------------------------- softmax

def softmax_row(row: np.ndarray) -> np.ndarray:
    """One row of test_softmax.py:22-26: r = x - max(x); e = exp(r); out = e / sum(e).

    Each step is the correctly rounded fp32 result: the subtraction in fp32, exp
    and the sum evaluated in fp64 and rounded once, the division in fp32.  The
    reference's Ascend ExpL2/ReduceSumL2 rounding is not observable (no NPU); this
    is the fp32-exact statement both the GPU kernel and torch.softmax approximate.
    """
    if np.asarray(row).dtype == np.float16:
        return softmax_row_f16(row)
    row = np.asarray(row, dtype=np.float32)
    r = (row - row.max()).astype(np.float32)
    e = np.exp(r.astype(np.float64)).astype(np.float32)
    s = np.float32(e.astype(np.float64).sum())
    return (e / s).astype(np.float32)


def softmax_row_f16(row: np.ndarray) -> np.ndarray:
    """asc2.softmax of a float16 row (python/asc/language/tile/unary_ops.py:213-222;
    python/test/asc2/operations/test_softmax.py): the exact softmax of the float16
    values (fp64 exp, sum and division; x - max is exact) rounded once to float16."""
    row = np.asarray(row, dtype=np.float16).astype(np.float64)
    e = np.exp(row - row.max())
    return (e / e.sum()).astype(np.float16)


def softmax_rows(x: np.ndarray, out: np.ndarray, num_rows: int, num_cols: int, tile_size: int,
                 grid: int) -> np.ndarray:
    """test_softmax.py:16-27: rows i = b, b+grid, ... for b < grid; the first ``tile_size``
    columns of each row are replaced.  With ``tile_size > num_cols`` the [1, tile] load
    right-pads the row with the pad value 0 (LowerAscTileDataTransfer.cpp:181-222) and the
    reductions run over the whole tile (LowerAscTile.cpp:428-459): the softmax of the
    padded row, whose first num_cols values are the row's result.  (The reference's store
    also spills the padded values into the next row, where they race with that row's own
    store across blocks; the row's own values are what an in-order run leaves, and what
    is written here.)"""
    x2 = x.reshape(-1)[:num_rows * num_cols].reshape(num_rows, num_cols)
    res = out.copy().reshape(-1)
    res2 = res[:num_rows * num_cols].reshape(num_rows, num_cols)
    pad = max(0, tile_size - num_cols)
    for b in range(grid):
        for i in range(b, num_rows, grid):
            tile = x2[i, :tile_size]
            if pad:
                tile = np.concatenate([tile, np.zeros(pad, dtype=tile.dtype)])
            res2[i, :min(tile_size, num_cols)] = softmax_row(tile)[:min(tile_size, num_cols)]
    return res.reshape(out.shape)


def softmax_blocks(x: np.ndarray, out: np.ndarray, num_rows: int, num_cols: int, block_size: int,
                   grid: int) -> np.ndarray:
    """test_softmax_fused.py:16-24: block b handles rows [b*bs, (b+1)*bs) clipped to num_rows."""
    x2 = x.reshape(-1)[:num_rows * num_cols].reshape(num_rows, num_cols)
    res = out.copy().reshape(-1)
    res2 = res[:num_rows * num_cols].reshape(num_rows, num_cols)
    for b in range(grid):
        for i in range(b * block_size, min(num_rows, (b + 1) * block_size)):
            res2[i] = softmax_row(x2[i])
    return res.reshape(out.shape)


# -------------------------------------------------------------------------------------------- matmul

def matmul(a: np.ndarray, b: np.ndarray, relu: bool = False, out_dtype: str = "float32") -> np.ndarray:
    """asc2 ``a @ b`` (binary_ops.py:180-200) with an fp32 L0C result, optional fixpipe relu
    and cast (TransformStoreFixpipe.cpp:55-86).  Inputs are the fp16/bf16 values as
    float32 arrays (bf16 callers convert bits first); products are exact in fp64 and
    the fp64 sum stands in for the fp32 accumulator.  Returns float32, or float16 /
    bfloat16 bits (uint16) after RNE rounding of the fp32 value."""
    acc = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    if relu:
        acc = np.maximum(acc, np.float32(0))
    if out_dtype == "float32":
        return acc
    if out_dtype == "float16":
        return acc.astype(np.float16)
    if out_dtype == "bfloat16":
        return f32_to_bf16_bits(acc)
    raise ValueError(out_dtype)


def matmul_bias_leaky_relu(a: np.ndarray, b: np.ndarray, bias: np.ndarray, alpha: float) -> np.ndarray:
    """python/tutorials/05_matmul_leakyrelu/matmul_leakyrelu.py:27-70: the Matmul API's fp32
    result with set_bias (bias[n] added to the fp32 accumulator), then asc.leaky_relu
    (vec_binary_scalar.py:63-66, v >= 0 ? v : v * alpha in fp32).  Products exact in fp64,
    the fp64 sum standing in for the fp32 accumulator as in ``matmul``."""
    acc = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    v = (acc + np.asarray(bias, dtype=np.float32).reshape(1, -1)).astype(np.float32)
    return np.where(v >= 0, v, (v * np.float32(alpha)).astype(np.float32))


def mnblock_rectangles(M: int, N: int, grid: int, m_tile: int, m_tiles_per_block: int, n_tile: int,
                       n_tiles_per_block: int) -> List[Tuple[int, int, int, int]]:
    """C rectangles (m0, m1, n0, n1) one block of test_matmul_mnblock.py:23-36 writes:
    m_base = (m_tile*mtpb*b) % M, n_base = ((m_tile*mtpb*b) // M) * n_tile*ntpb,
    walked tile by tile exactly as the kernel's two loops do."""
    rects = set()
    for blk in range(grid):
        m_elems = m_tile * m_tiles_per_block
        m_base = (m_elems * blk) % M
        n_base = ((m_elems * blk) // M) * (n_tile * n_tiles_per_block)
        for j in range(n_tiles_per_block):
            n0 = n_base + j * n_tile
            for i in range(m_tiles_per_block):
                m0 = m_base + i * m_tile
                m1, n1 = min(M, m0 + m_tile), min(N, n0 + n_tile)
                if m0 < m1 and n0 < n1:
                    rects.add((m0, m1, n0, n1))
    return sorted(rects)


# ---------------------------------------------------------------------------------------- int8 matmul

def matmul_i8_acc(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """int32 accumulators of an int8 x int8 product (test_matmul_iterate_all.py:116:
    ``a.to(int32) @ b.to(int32)``), computed exactly in int64."""
    acc = a.astype(np.int64) @ b.astype(np.int64)
    if np.abs(acc).max(initial=0) >= 2**31:
        raise OverflowError("int32 accumulator overflow")
    return acc.astype(np.int32)


def trunc19(scale: np.ndarray) -> np.ndarray:
    """Clears the low 13 mantissa bits (1 sign + 8 exponent + 10 mantissa bits kept),
    test_matmul_quant.py:94-101."""
    return (np.asarray(scale, dtype=np.float32).view(np.uint32) & np.uint32(0xFFFFE000)).view(np.float32)


def dequant_f16(acc: np.ndarray, scale: np.ndarray, use_trunc19: bool = False) -> np.ndarray:
    """Build definition of the DEQF16 store: fp16_rne(fp32(acc) *_rne s[n])."""
    s = trunc19(scale) if use_trunc19 else np.asarray(scale, dtype=np.float32)
    with np.errstate(over="ignore"):  # fp16 overflow to inf is part of the definition
        return (acc.astype(np.float32) * s.reshape(1, -1)).astype(np.float16)


def dequant_reference_golden(acc: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """The reference test's golden (test_matmul_quant.py:94-106): fp16(acc) first, then
    each row times trunc19(scale) in fp32 and stored back to fp16.  Equal to
    ``dequant_f16(acc, scale, True)`` whenever |acc| <= 2048 (fp16-exact integers)."""
    with np.errstate(over="ignore"):
        g = acc.astype(np.float16)
        return (g.astype(np.float32) * trunc19(scale).reshape(1, -1)).astype(np.float16)


# ---------------------------------------------------------------------- element-wise tile operations

def _erf64(v: np.ndarray) -> np.ndarray:
    from scipy.special import erf
    return erf(v)


_UNARY_F64 = {
    "abs": np.abs, "ceil": np.ceil, "cos": np.cos, "cosh": np.cosh, "erf": _erf64, "exp": np.exp, "exp2": np.exp2,
    "floor": np.floor, "log": np.log, "log2": np.log2, "negative": np.negative,
    "relu": lambda v: np.where(v < 0, 0.0, v),  # negative -> +0; -0 and NaN pass through (torch.relu)
    "rsqrt": lambda v: 1.0 / np.sqrt(v), "sin": np.sin, "sinh": np.sinh, "sqrt": np.sqrt, "tan": np.tan,
    "tanh": np.tanh,
}


def unary_f32(x: np.ndarray, op: str) -> np.ndarray:
    """One asc2 unary op on a float32 tile (python/asc/language/tile/unary_ops.py;
    python/test/asc2/operations/test_unary_ops.py:9-28): the exact value (fp64)
    rounded once to float32."""
    with np.errstate(all="ignore"):
        return _UNARY_F64[op](np.asarray(x, dtype=np.float32).astype(np.float64)).astype(np.float32)


def unary(x: np.ndarray, op: str, dtype: str) -> np.ndarray:
    """The same op on a float32 / float16 / bfloat16 tile: the 16-bit elements widen
    exactly to float32, the op's float32 value (the exact value rounded to float32) is
    rounded (RNE) to the element type (bfloat16 as uint16 bits)."""
    return _from_f32(unary_f32(_to_f32(x, dtype), op), dtype)


_INT_BITS = {"int32": 32, "int16": 16}


def _wrap(v: np.ndarray, dtype: str) -> np.ndarray:
    bits = _INT_BITS[dtype]
    u = np.asarray(v, dtype=np.int64).astype(np.uint64) & np.uint64((1 << bits) - 1)
    signed = u.astype(np.int64) - ((u >> np.uint64(bits - 1)) & np.uint64(1)).astype(np.int64) * (1 << bits)
    return signed.astype(np.int32 if bits == 32 else np.int16)


def binary_elements(x: np.ndarray, y: np.ndarray, op: str, dtype: str) -> np.ndarray:
    """One asc2 binary op on equal-shape operands of one element type
    (python/asc/language/tile/binary_ops.py:110-175; a scalar operand is broadcast
    by the caller after conversion to the tile's dtype, utils.py:73-94).
    Floats: computed in float32, rounded once (RNE) to the element type (bfloat16
    as uint16 bit patterns); maximum/minimum are IEEE 754-2019 maximum/minimum
    (arith.maximumf/minimumf): NaN propagates, -0 < +0.  Integers: two's-complement wrap,
    div truncates toward zero with x / 0 = 0, shifts are shl / arithmetic shr."""
    if dtype in _INT_BITS:
        a, b = np.asarray(x).astype(np.int64), np.asarray(y).astype(np.int64)
        if op == "add":
            r = a + b
        elif op == "sub":
            r = a - b
        elif op == "mul":
            r = a * b  # |a*b| < 2^62: exact before the wrap
        elif op == "div":
            safe = np.where(b == 0, 1, b)
            q = np.abs(a) // np.abs(safe)
            r = np.where(b == 0, 0, np.where((a < 0) ^ (safe < 0), -q, q))
        elif op == "maximum":
            r = np.maximum(a, b)
        elif op == "minimum":
            r = np.minimum(a, b)
        elif op == "left_shift":
            r = a << b
        elif op == "right_shift":
            r = a >> b  # arithmetic on signed values
        else:
            raise ValueError(op)
        return _wrap(r, dtype)
    fa, fb = _to_f32(x, dtype), _to_f32(y, dtype)
    with np.errstate(all="ignore"):
        if op == "add":
            r = fa + fb
        elif op == "sub":
            r = fa - fb
        elif op == "mul":
            r = fa * fb
        elif op == "div":
            r = fa / fb
        elif op == "maximum":
            tie = np.where(np.signbit(fa), fb, fa)  # equal operands: +0 over -0
            r = np.where(np.isnan(fa), fa, np.where(np.isnan(fb), fb, np.where(fa == fb, tie, np.maximum(fa, fb))))
        elif op == "minimum":
            tie = np.where(np.signbit(fa), fa, fb)  # equal operands: -0 over +0
            r = np.where(np.isnan(fa), fa, np.where(np.isnan(fb), fb, np.where(fa == fb, tie, np.minimum(fa, fb))))
        else:
            raise ValueError(op)
    return _from_f32(np.asarray(r, dtype=np.float32), dtype)


def _compare(a: np.ndarray, b: np.ndarray, cmp: str) -> np.ndarray:
    return {"equal": np.equal, "not_equal": np.not_equal, "greater": np.greater, "greater_equal": np.greater_equal,
            "less": np.less, "less_equal": np.less_equal}[cmp](a, b)


def where_compare(x: np.ndarray, y: np.ndarray, cmp: str, dtype: str) -> np.ndarray:
    """python/test/asc2/operations/test_where.py:24-26: where(cmp(x, y), x, y); 16-bit
    floats compare exactly in float32 (bfloat16 as uint16 bit patterns)."""
    if dtype in _INT_BITS:
        return np.where(_compare(x, y, cmp), x, y)
    return np.where(_compare(_to_f32(x, dtype), _to_f32(y, dtype), cmp), x, y)


def where_scalar(x: np.ndarray, s, cmp: str, dtype: str, true_value, false_value) -> np.ndarray:
    """python/test/asc2/operations/test_where.py:53-54: where(cmp(x, s), t, f) with s, t,
    f converted to x's dtype (bfloat16 as uint16 bit patterns)."""
    shape = np.asarray(x).shape

    def full(v):
        if dtype in _INT_BITS:
            return _wrap(np.full(shape, int(v), dtype=np.int64), dtype)
        return _from_f32(np.full(shape, v, dtype=np.float32), dtype)

    if dtype in _INT_BITS:
        c = _compare(np.asarray(x), full(s), cmp)
    else:
        c = _compare(_to_f32(x, dtype), _to_f32(full(s), dtype), cmp)
    return np.where(c, full(true_value), full(false_value))


# ------------------------------------------------------------------ tile load / store, shape ops

def tile_binary(x: np.ndarray, y: np.ndarray, z: np.ndarray, op: str, tile_shape, offsets,
                dtype: str) -> np.ndarray:
    """asc2.load of the same tile of x and y, op, asc2.store to z (python/asc/language/
    tile/memory_ops.py:65-114; python/test/asc2/operations/test_memory_ops.py:58-92):
    returns a copy of z with the tile at ``offsets`` (shape ``tile_shape``, None for
    one element) replaced, clipped at the tensor bounds as the store clips."""
    res = z.copy()
    shape = tile_shape if tile_shape is not None else [1] * len(offsets)
    sl = tuple(slice(o, min(o + s, d)) for o, s, d in zip(offsets, shape, z.shape))
    res[sl] = binary_elements(x[sl], y[sl], op, dtype)
    return res


def broadcast_rows(x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """asc2.broadcast_to from [1, cols] to [rows, cols] (rows = 1: the unchanged data of
    reshape / ravel / squeeze / expand_dims; python/asc/language/tile/shape_ops.py)."""
    return np.tile(np.asarray(x).reshape(-1)[:cols], rows).reshape(rows, cols)


def atomic_tiles(x: np.ndarray, z: np.ndarray, op: str, n_tiles: int, tile_len: int, addend,
                 dtype: str) -> np.ndarray:
    """asc2.atomic_add / atomic_max / atomic_min of tile b of x plus ``addend`` into
    z[0:tile_len] for b < n_tiles (python/asc/language/tile/atomic_ops.py:19-33, a store in
    atomic mode, lib/Conversion/LowerToAsc/LowerAtomic.cpp:44-70; the kernel and golden of
    python/test/asc2/operations/test_atomic_ops.py:33-68): the tiles combine in block
    order, each combine being the element type's binary op."""
    x = np.asarray(x).reshape(-1)
    res = np.asarray(z).reshape(-1)[:tile_len].copy()
    c = np.full(tile_len, addend).astype(res.dtype) if dtype != "bfloat16" else \
        f32_to_bf16_bits(np.full(tile_len, addend, dtype=np.float32))
    for b in range(n_tiles):
        tile = binary_elements(x[b * tile_len:(b + 1) * tile_len], c, "add", dtype)
        res = binary_elements(res, tile, op, dtype)
    return res


def quant_i8(src: np.ndarray, scale: float, offset: float, dtype: str) -> np.ndarray:
    """asc.adv.quant (python/asc/language/adv/quantization.py:18-36; test_quant.py's kernel):
    scale and offset materialized in the source dtype (quantization.py:28-29), the multiply
    and the add each rounded to that dtype, then rint (ties to even), clamped to the int8
    range; NaN gives 0 (build-defined).  bfloat16 as uint16 bit patterns."""
    def rnd(v):
        return _to_f32(_from_f32(v, dtype), dtype)
    sc = rnd(np.full(1, scale, np.float32))[0]
    of = rnd(np.full(1, offset, np.float32))[0]
    with np.errstate(invalid="ignore"):
        v = rnd(rnd(_to_f32(src, dtype) * sc) + of)
        r = np.clip(np.rint(v), -128, 127)
        return np.where(np.isnan(v), 0, r).astype(np.int8)


def fill(n: int, value, dtype: str) -> np.ndarray:
    """asc2.full([1], value, dtype) broadcast to n elements and stored
    (python/asc/language/tile/creation_ops.py:20-31; test_shape_ops.py:64-78)."""
    if dtype == "bfloat16":
        return f32_to_bf16_bits(np.full(n, value, dtype=np.float32))
    with np.errstate(over="ignore"):  # float16 overflow rounds to inf, as the device conversion does
        return np.full(n, value).astype(np.dtype(dtype))


# --------------------------------------------------------------------------------- flash attention

def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, sm_scale: float, causal: bool) -> np.ndarray:
    """softmax(q k^T * scale + mask) v for one [S, D] head, in fp64 (mask: key j > query i)."""
    q64, k64, v64 = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    s = (q64 @ k64.T) * sm_scale
    if causal:
        S = s.shape[0]
        s = np.where(np.triu(np.ones((S, s.shape[1]), dtype=bool), 1), -np.inf, s)
    s = s - s.max(axis=1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=1, keepdims=True)
    return p @ v64
