"""Typed host API over libasc_hip.so: torch device tensors in, kernels launched.

Every function checks on the host that the buffers hold everything the kernel
will touch (shape, dtype, device, layout) before it reaches the C ABI, so an
inconsistent call raises ValueError/TypeError here instead of faulting on the
GPU.  Launches are asynchronous on ``stream`` (default: torch's current stream).
"""
from __future__ import annotations

import ctypes
from typing import Any, Optional

import torch

from . import _native

_DTYPE_CODES = {
    torch.float32: _native.DT_FLOAT32,
    torch.float16: _native.DT_FLOAT16,
    torch.bfloat16: _native.DT_BFLOAT16,
    torch.int32: _native.DT_INT32,
    torch.int8: _native.DT_INT8,
    torch.int16: _native.DT_INT16,
}


def _stream(stream: Any) -> int:
    if stream is None:
        return _native.current_stream_handle()
    if isinstance(stream, int):
        return stream
    return int(stream.cuda_stream)


def _device_tensor(t: Any, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"'{name}' must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"'{name}' must be on the HIP device, got {t.device}")
    return t


def _contiguous(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_contiguous():
        raise ValueError(f"'{name}' must be contiguous")
    return t


def _code(t: torch.Tensor, name: str, allowed) -> int:
    if t.dtype not in allowed:
        raise TypeError(f"'{name}' has unsupported dtype {t.dtype}; expected one of {sorted(map(str, allowed))}")
    return _DTYPE_CODES[t.dtype]


# ---------------------------------------------------------------------------------------------- vadd

def vadd_covered(size: int, tile_size: int, tile_per_block: int, grid: int) -> int:
    """Elements written by asc2 vadd_kernel: [0, min(size, grid*tpb*tile))
    (python/test/asc2/kernels/test_vadd.py:22-28 with the store clipped at ``size``)."""
    return max(0, min(size, grid * tile_per_block * tile_size))


def vadd_check(x: torch.Tensor, y: torch.Tensor, out: torch.Tensor, size: int, tile_size: int, tile_per_block: int,
               grid: int) -> int:
    """Host checks of a vadd launch; returns the covered element count."""
    for t, n in ((x, "x"), (y, "y"), (out, "out")):
        _contiguous(_device_tensor(t, n), n)
    allowed = (torch.float32, torch.float16, torch.bfloat16, torch.int32)
    _code(x, "x", allowed)
    if y.dtype != x.dtype or out.dtype != x.dtype:
        raise TypeError(f"vadd operands must share one dtype, got {x.dtype}, {y.dtype}, {out.dtype}")
    if tile_size <= 0 or tile_per_block < 0 or grid <= 0 or size < 0:
        raise ValueError(f"invalid vadd launch: size={size}, tile_size={tile_size}, "
                         f"tile_per_block={tile_per_block}, grid={grid}")
    covered = vadd_covered(size, tile_size, tile_per_block, grid)
    for t, n in ((x, "x"), (y, "y"), (out, "out")):
        if t.numel() < covered:
            raise ValueError(f"'{n}' holds {t.numel()} elements but the launch touches {covered}")
    return covered


def vadd(x: torch.Tensor, y: torch.Tensor, out: torch.Tensor, size: int, tile_size: int, tile_per_block: int,
         grid: int, stream: Any = None) -> None:
    vadd_check(x, y, out, size, tile_size, tile_per_block, grid)
    code = _DTYPE_CODES[x.dtype]
    _native.call("asc_vadd", code, x.data_ptr(), y.data_ptr(), out.data_ptr(), size, tile_size, tile_per_block,
                 grid, _stream(stream))


# -------------------------------------------------------------------------- leaky_relu / vmuladd / gelu

def _check_stream_operands(tensors, covered: int) -> int:
    """Common checks of the tiled elementwise kernels: contiguous device tensors of one
    float dtype, each holding at least the covered elements.  Returns the dtype code."""
    for t, n in tensors:
        _contiguous(_device_tensor(t, n), n)
    first = tensors[0][0]
    code = _code(first, tensors[0][1], (torch.float32, torch.float16, torch.bfloat16))
    for t, n in tensors:
        if t.dtype != first.dtype:
            raise TypeError(f"operands must share one dtype, got {first.dtype} and {t.dtype} ('{n}')")
        if t.numel() < covered:
            raise ValueError(f"'{n}' holds {t.numel()} elements but the launch touches {covered}")
    return code


def _check_tiling(size: int, tile_size: int, tile_per_block: int, grid: int, what: str) -> None:
    if tile_size <= 0 or tile_per_block < 0 or grid <= 0 or size < 0:
        raise ValueError(f"invalid {what} launch: size={size}, tile_size={tile_size}, "
                         f"tile_per_block={tile_per_block}, grid={grid}")


def leaky_relu_check(x: torch.Tensor, out: torch.Tensor, size: int, tile_size: int, tile_per_block: int,
                     grid: int) -> int:
    """Host checks of a leaky_relu launch; returns the covered element count."""
    _check_tiling(size, tile_size, tile_per_block, grid, "leaky_relu")
    covered = vadd_covered(size, tile_size, tile_per_block, grid)
    _check_stream_operands(((x, "x"), (out, "out")), covered)
    return covered


def leaky_relu(x: torch.Tensor, alpha: float, out: torch.Tensor, size: int, tile_size: int, tile_per_block: int,
               grid: int, stream: Any = None) -> None:
    """asc2 leaky_relu_kernel (python/test/asc2/kernels/test_leaky_relu.py:16-26):
    out = where(x >= 0, x, x * alpha) over the vadd-style covered range; ``alpha`` is
    used at its float value (a 0-dim bf16 tensor's exact value)."""
    leaky_relu_check(x, out, size, tile_size, tile_per_block, grid)
    _native.call("asc_leaky_relu", _DTYPE_CODES[x.dtype], x.data_ptr(), float(alpha), out.data_ptr(), size,
                 tile_size, tile_per_block, grid, _stream(stream))


def vmuladd_check(x: torch.Tensor, y: torch.Tensor, z: torch.Tensor, out: torch.Tensor, size: int, tile_size: int,
                  tile_per_block: int, grid: int) -> int:
    """Host checks of a vmuladd launch; returns the covered element count."""
    _check_tiling(size, tile_size, tile_per_block, grid, "vmuladd")
    covered = vadd_covered(size, tile_size, tile_per_block, grid)
    _check_stream_operands(((x, "x"), (y, "y"), (z, "z"), (out, "out")), covered)
    return covered


def vmuladd(x: torch.Tensor, y: torch.Tensor, z: torch.Tensor, out: torch.Tensor, size: int, tile_size: int,
            tile_per_block: int, grid: int, stream: Any = None) -> None:
    """asc2 vmuladd_kernel (python/test/asc2/kernels/test_vmuladd.py:16-31): out = x * y + z,
    multiply and add rounded separately."""
    vmuladd_check(x, y, z, out, size, tile_size, tile_per_block, grid)
    _native.call("asc_vmuladd", _DTYPE_CODES[x.dtype], x.data_ptr(), y.data_ptr(), z.data_ptr(), out.data_ptr(),
                 size, tile_size, tile_per_block, grid, _stream(stream))


def gelu_rows_check(x: torch.Tensor, out: torch.Tensor, num_rows: int, num_cols: int, tile_size: int,
                    grid: int) -> None:
    """Host checks of a gelu launch."""
    if tile_size <= 0 or grid <= 0 or num_rows < 0 or num_cols < 0:
        raise ValueError(f"invalid gelu launch: rows={num_rows}, cols={num_cols}, tile={tile_size}, grid={grid}")
    for t, n in ((x, "x"), (out, "out")):
        _contiguous(_device_tensor(t, n), n)
        if t.dtype != torch.float32:
            raise TypeError(f"gelu supports float32 only, '{n}' is {t.dtype}")
        if t.numel() < num_rows * num_cols:
            raise ValueError(f"'{n}' holds {t.numel()} elements but the launch touches {num_rows}x{num_cols}")


def gelu_rows(x: torch.Tensor, out: torch.Tensor, num_rows: int, num_cols: int, tile_size: int, approximate: bool,
              grid: int, stream: Any = None) -> None:
    """asc2 gelu_kernel (python/test/asc2/kernels/test_gelu.py:19-33) on fp32 rows.  A tile
    wider than the row computes the row's own columns (the padding is zeros and gelu is
    element-wise) and writes nothing past them."""
    gelu_rows_check(x, out, num_rows, num_cols, tile_size, grid)
    _native.call("asc_gelu_rows_f32", x.data_ptr(), out.data_ptr(), num_rows, num_cols, tile_size,
                 int(bool(approximate)), grid, _stream(stream))


# ------------------------------------------------------------------------------------------- softmax

def _check_softmax(x: torch.Tensor, out: torch.Tensor, rows: int, num_cols: int) -> str:
    """Checks the buffers; returns the entry-point suffix of their dtype ("f32" / "f16")."""
    for t, n in ((x, "x"), (out, "out")):
        _contiguous(_device_tensor(t, n), n)
        if t.dtype not in (torch.float32, torch.float16):
            raise TypeError(f"softmax supports float32 and float16, '{n}' is {t.dtype}")
        if t.numel() < rows * num_cols:
            raise ValueError(f"'{n}' holds {t.numel()} elements but the launch touches {rows}x{num_cols}")
    if out.dtype != x.dtype:
        raise TypeError(f"'out' must be {x.dtype}, got {out.dtype}")
    return "f32" if x.dtype == torch.float32 else "f16"


def _softmax_launch(x: torch.Tensor, out: torch.Tensor, num_rows: int, num_cols: int, size: int, grid: int,
                    fused: bool) -> str:
    """Checks a softmax launch (size is tile_size, or block_size when fused); returns the
    dtype suffix ("f32" / "f16")."""
    if size <= 0 or grid <= 0 or num_rows < 0 or num_cols < 0:
        raise ValueError(f"invalid softmax launch: rows={num_rows}, cols={num_cols}, "
                         f"{'block' if fused else 'tile'}={size}, grid={grid}")
    rows = softmax_blocks_covered(num_rows, size, grid) if fused else num_rows
    return _check_softmax(x, out, rows, num_cols)


def softmax_rows(x: torch.Tensor, out: torch.Tensor, num_rows: int, num_cols: int, tile_size: int, grid: int,
                 stream: Any = None) -> None:
    """asc2 softmax_kernel(x, out, num_rows, num_cols, tile_size) of
    python/test/asc2/kernels/test_softmax.py:16-27.  With tile_size > num_cols each row's
    statistics include the tile's tile_size - num_cols zero padding (the reference's padded
    load and whole-tile reductions) and each row writes its own num_cols outputs."""
    suffix = _softmax_launch(x, out, num_rows, num_cols, tile_size, grid, False)
    _native.call(f"asc_softmax_rows_{suffix}", x.data_ptr(), out.data_ptr(), num_rows, num_cols, tile_size, grid,
                 _stream(stream))


def softmax_blocks_covered(num_rows: int, block_size: int, grid: int) -> int:
    """Rows written by the fused asc2 softmax_kernel: [0, min(num_rows, grid*block_size))."""
    return max(0, min(num_rows, grid * block_size))


def softmax_blocks(x: torch.Tensor, out: torch.Tensor, num_rows: int, num_cols: int, block_size: int, grid: int,
                   stream: Any = None) -> None:
    """asc2 softmax_kernel(x, out, num_rows, num_cols, block_size) of
    python/test/asc2/kernels/test_softmax_fused.py:16-24."""
    suffix = _softmax_launch(x, out, num_rows, num_cols, block_size, grid, True)
    _native.call(f"asc_softmax_blocks_{suffix}", x.data_ptr(), out.data_ptr(), num_rows, num_cols, block_size,
                 grid, _stream(stream))


def softmax_plan(x: torch.Tensor, out: torch.Tensor, num_rows: int, num_cols: int, size: int, grid: int,
                 fused: bool) -> "_native.SoftmaxPlan":
    """The launch softmax_rows (fused False, size = tile_size) or softmax_blocks (fused True,
    size = block_size) makes for these buffers, as a kernel of the asc2_softmax code object
    with its grid, block and arguments (asc_softmax_plan); plan.grid == 0 when there is
    nothing to launch.  Same checks and errors as those two calls."""
    suffix = _softmax_launch(x, out, num_rows, num_cols, size, grid, fused)
    plan = _native.SoftmaxPlan()
    _native.call("asc_softmax_plan", _native.DT_FLOAT32 if suffix == "f32" else _native.DT_FLOAT16, int(fused),
                 x.data_ptr(), out.data_ptr(), num_rows, num_cols, size, grid, ctypes.byref(plan))
    return plan


# ---------------------------------------------------------------------------------- reductions, rms_norm

REDUCE_OPS = {"sum": 0, "max": 1, "min": 2, "prod": 3}


def reduce_f32(x: torch.Tensor, out: torch.Tensor, op: str, dim: Optional[int], stream: Any = None) -> None:
    """asc2.reduce_{sum,max,min,prod} of a 1-D or 2-D float32 tensor along ``dim`` (0 or 1 of
    a 2-D tensor) or over all elements (``dim=None``: the scalar is written to every element
    of ``out``, as asc2.full does in test_reduce_ops.py's kernel_all)."""
    if op not in REDUCE_OPS:
        raise ValueError(f"unknown reduction {op!r}; expected one of {sorted(REDUCE_OPS)}")
    for t, n in ((x, "x"), (out, "out")):
        _contiguous(_device_tensor(t, n), n)
        if t.dtype != torch.float32:
            raise TypeError(f"reductions support float32, '{n}' is {t.dtype}")
    if x.dim() == 1:
        rows, cols = 1, x.shape[0]
    elif x.dim() == 2:
        rows, cols = x.shape
    else:
        raise ValueError("x must be 1-D or 2-D")
    if dim is None:
        _native.call("asc_reduce_f32", REDUCE_OPS[op], x.data_ptr(), out.data_ptr(), rows, cols, -1, out.numel(),
                     _stream(stream))
        return
    if x.dim() != 2 or dim not in (0, 1):
        raise ValueError(f"dim must be 0 or 1 of a 2-D tensor, got dim={dim} for shape {tuple(x.shape)}")
    need = rows if dim == 1 else cols
    if out.numel() != need:
        raise ValueError(f"out must hold {need} elements, holds {out.numel()}")
    _native.call("asc_reduce_f32", REDUCE_OPS[op], x.data_ptr(), out.data_ptr(), rows, cols, dim, need,
                 _stream(stream))


def rms_norm(x: torch.Tensor, gamma: torch.Tensor, out: torch.Tensor, num_rows: int, num_cols: int,
             epsilon: float, tile_size: Optional[int] = None, stream: Any = None) -> None:
    """asc2.rms_norm over the first ``tile_size`` (default: all) columns of each row:
    y = x / sqrt(mean(x^2) + epsilon) * gamma, fp32 or fp16 rows, fp32 gamma."""
    tile = num_cols if tile_size is None else int(tile_size)
    if num_rows < 0 or num_cols < 0 or not 0 < tile <= num_cols:
        raise ValueError(f"invalid rms_norm launch: rows={num_rows}, cols={num_cols}, tile={tile}")
    for t, n in ((x, "x"), (out, "out")):
        _contiguous(_device_tensor(t, n), n)
        if t.numel() < num_rows * num_cols:
            raise ValueError(f"'{n}' holds {t.numel()} elements but the launch touches {num_rows}x{num_cols}")
    code = _code(x, "x", (torch.float32, torch.float16))
    if out.dtype != x.dtype:
        raise TypeError(f"out must be {x.dtype}, got {out.dtype}")
    _contiguous(_device_tensor(gamma, "gamma"), "gamma")
    if gamma.dtype != torch.float32 or gamma.numel() < tile:
        raise ValueError(f"gamma must be float32 with at least {tile} elements")
    _native.call("asc_rms_norm", code, x.data_ptr(), gamma.data_ptr(), out.data_ptr(), num_rows, num_cols, tile,
                 float(epsilon), _stream(stream))


# -------------------------------------------------------------------------------------------- matmul

def _row_major_2d(t: torch.Tensor, name: str) -> int:
    """Leading dimension of a 2-D row-major (unit inner stride) tensor.  Rows must not
    overlap: a row stride below the row length (an expanded or as_strided view) would
    make the kernel read or write past the tensor's storage, and is refused."""
    if t.dim() != 2:
        raise ValueError(f"'{name}' must be 2-D, got shape {tuple(t.shape)}")
    if t.stride(1) != 1 and t.shape[1] > 1:
        raise ValueError(f"'{name}' must have unit stride along its last dimension")
    if t.shape[0] > 1 and t.stride(0) < t.shape[1]:
        raise ValueError(f"'{name}' has row stride {t.stride(0)} below its row length {t.shape[1]}: "
                         "overlapping or expanded rows are not supported")
    return max(t.stride(0), t.shape[1], 1)


ACT_NONE, ACT_RELU, ACT_LEAKY_RELU = 0, 1, 2


def _matmul_args(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, relu: bool, bias: Optional[torch.Tensor],
                 leaky_alpha: Optional[float]) -> tuple:
    """Checks a matmul and returns the C arguments of asc_matmul_bias_act (and of
    asc_matmul_plan) without the stream: in/out dtype codes, pointers, M, N, K, the leading
    dimensions, the activation code and alpha."""
    for t, n in ((a, "a"), (b, "b"), (c, "c")):
        _device_tensor(t, n)
    in_code = _code(a, "a", (torch.float32, torch.float16, torch.bfloat16))
    if b.dtype != a.dtype:
        raise TypeError(f"a and b must share a dtype, got {a.dtype} and {b.dtype}")
    out_code = _code(c, "c", (torch.float32, torch.float16, torch.bfloat16))
    lda, ldb, ldc = _row_major_2d(a, "a"), _row_major_2d(b, "b"), _row_major_2d(c, "c")
    M, K = a.shape
    K2, N = b.shape
    if K2 != K:
        raise ValueError(f"inner dimensions differ: a is {tuple(a.shape)}, b is {tuple(b.shape)}")
    if tuple(c.shape) != (M, N):
        raise ValueError(f"c must be {(M, N)}, got {tuple(c.shape)}")
    if relu and leaky_alpha is not None:
        raise ValueError("relu and leaky_alpha are exclusive")
    bias_ptr = 0
    if bias is not None:
        _contiguous(_device_tensor(bias, "bias"), "bias")
        if bias.dtype != torch.float32 or bias.numel() != N:
            raise ValueError(f"bias must be float32 with {N} elements, got {bias.dtype} with {bias.numel()}")
        bias_ptr = bias.data_ptr()
    act = ACT_LEAKY_RELU if leaky_alpha is not None else (ACT_RELU if relu else ACT_NONE)
    return (in_code, out_code, a.data_ptr(), b.data_ptr(), c.data_ptr(), bias_ptr, M, N, K, lda, ldb, ldc, act,
            float(leaky_alpha or 0.0))


def matmul(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, relu: bool = False, stream: Any = None,
           bias: Optional[torch.Tensor] = None, leaky_alpha: Optional[float] = None) -> None:
    """c = cast(act(a @ b + bias)) with fp32 accumulation; the cast is chosen by c's dtype
    (float32: no cast; float16/bfloat16: RNE).  ``bias``: float32 with N elements (added
    per column), ``relu``: max(v, 0), ``leaky_alpha``: v >= 0 ? v : v * alpha (excludes relu)."""
    args = _matmul_args(a, b, c, relu, bias, leaky_alpha)
    if bias is None and leaky_alpha is None:
        in_code, out_code, ap, bp, cp, _, M, N, K, lda, ldb, ldc, _, _ = args
        _native.call("asc_matmul", in_code, out_code, ap, bp, cp, M, N, K, lda, ldb, ldc, int(bool(relu)),
                     _stream(stream))
        return
    _native.call("asc_matmul_bias_act", *args, _stream(stream))


def matmul_chained(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, workspace: Optional[torch.Tensor] = None,
                   stream: Any = None) -> None:
    """The asc2 chained matmul (python/test/asc2/kernels/test_matmul_l0c_to_l1.py:17-30):
    t = (a @ b) cast to a's dtype, c = cast(t @ b) to c's dtype, fp32 accumulation, N == K.
    ``workspace`` (a contiguous device tensor of at least M * N * 2 bytes) holds t; without
    one it is taken from torch's allocator on the launch stream."""
    for t, n in ((a, "a"), (b, "b"), (c, "c")):
        _contiguous(_device_tensor(t, n), n)
    in_code = _code(a, "a", (torch.float16, torch.bfloat16))
    if b.dtype != a.dtype:
        raise TypeError(f"a and b must share a dtype, got {a.dtype} and {b.dtype}")
    out_code = _code(c, "c", (torch.float32, torch.float16, torch.bfloat16))
    if a.dim() != 2 or b.dim() != 2:
        raise ValueError(f"a and b must be 2-D, got {tuple(a.shape)} and {tuple(b.shape)}")
    M, K = a.shape
    K2, N = b.shape
    if K2 != K or N != K:
        raise ValueError(f"the chained matmul needs b square and a's columns equal to its rows: a {tuple(a.shape)}, "
                         f"b {tuple(b.shape)}")
    if tuple(c.shape) != (M, N):
        raise ValueError(f"c must be {(M, N)}, got {tuple(c.shape)}")
    handle = _stream(stream)
    if workspace is None:
        workspace = torch.empty(M * N, dtype=a.dtype, device=a.device)
        # freed on return: on a stream other than torch's current one the caching
        # allocator must not hand its memory out again before these launches have run
        if handle != torch.cuda.current_stream(a.device).cuda_stream:
            workspace.record_stream(torch.cuda.ExternalStream(handle, device=a.device))
    else:
        _contiguous(_device_tensor(workspace, "workspace"), "workspace")
    nbytes = workspace.numel() * workspace.element_size()
    _native.call("asc_matmul_chained", in_code, out_code, a.data_ptr(), b.data_ptr(), c.data_ptr(), M, N, K,
                 workspace.data_ptr(), nbytes, handle)


def matmul_plan(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, relu: bool = False,
                bias: Optional[torch.Tensor] = None, leaky_alpha: Optional[float] = None) -> "_native.LaunchPlan":
    """The launch matmul(...) makes, as a kernel of the asc2_matmul code object with its
    grid, block and argument blob (asc_matmul_plan); plan.grid == 0 when there is nothing
    to launch.  Same checks and errors as matmul."""
    plan = _native.LaunchPlan()
    _native.call("asc_matmul_plan", *_matmul_args(a, b, c, relu, bias, leaky_alpha), ctypes.byref(plan))
    return plan


def _matmul_i8_args(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, scale: Optional[torch.Tensor],
                    trunc19: bool) -> tuple:
    """Checks an int8 matmul and returns the C arguments of asc_matmul_i8_plan: pointers
    a, b, scale (0 for int32 output), c, then M, N, K, the dequant flag and trunc19."""
    for t, n in ((a, "a"), (b, "b"), (c, "c")):
        _contiguous(_device_tensor(t, n), n)
    _code(a, "a", (torch.int8,))
    _code(b, "b", (torch.int8,))
    if a.dim() != 2 or b.dim() != 2 or c.dim() != 2:
        raise ValueError("a, b and c must be 2-D")
    M, K = a.shape
    K2, N = b.shape
    if K2 != K or tuple(c.shape) != (M, N):
        raise ValueError(f"shape mismatch: a {tuple(a.shape)}, b {tuple(b.shape)}, c {tuple(c.shape)}")
    if c.dtype == torch.int32:
        return (a.data_ptr(), b.data_ptr(), 0, c.data_ptr(), M, N, K, 0, 0)
    if c.dtype != torch.float16:
        raise TypeError(f"c must be int32 (accumulators) or float16 (dequantised), got {c.dtype}")
    if scale is None:
        raise ValueError("a float16 output needs the per-channel scale vector")
    _contiguous(_device_tensor(scale, "scale"), "scale")
    if scale.dtype != torch.float32 or scale.numel() != N:
        raise ValueError(f"scale must be float32 with {N} elements, got {scale.dtype} with {scale.numel()}")
    return (a.data_ptr(), b.data_ptr(), scale.data_ptr(), c.data_ptr(), M, N, K, 1, int(bool(trunc19)))


def matmul_i8(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, scale: Optional[torch.Tensor] = None,
              trunc19: bool = False, stream: Any = None) -> None:
    """int8 GEMM with exact int32 accumulation.  c int32: raw accumulators.  c float16:
    c = fp16(fp32(acc) * scale[n]) (scale required, fp32 of length N)."""
    ap, bp, sp, cp, M, N, K, dequant, t19 = _matmul_i8_args(a, b, c, scale, trunc19)
    if not dequant:
        _native.call("asc_matmul_i8_i32", ap, bp, cp, M, N, K, _stream(stream))
        return
    _native.call("asc_matmul_i8_dequant_f16", ap, bp, sp, cp, M, N, K, t19, _stream(stream))


def matmul_i8_plan(a: torch.Tensor, b: torch.Tensor, c: torch.Tensor, scale: Optional[torch.Tensor] = None,
                   trunc19: bool = False) -> "_native.LaunchPlan":
    """The launch matmul_i8(...) makes, as a kernel of the asc2_matmul_i8 code object with
    its grid, block and argument blob (asc_matmul_i8_plan).  Same checks as matmul_i8."""
    plan = _native.LaunchPlan()
    _native.call("asc_matmul_i8_plan", *_matmul_i8_args(a, b, c, scale, trunc19), ctypes.byref(plan))
    return plan


# --------------------------------------------------------------------------------------- attention

FA_HEAD_DIMS = (64, 128)


def _attention_args(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, sm_scale: float,
                    causal: bool, lse: Optional[torch.Tensor]) -> tuple:
    """Checks an attention call and returns the C arguments of
    asc_flash_attention_fwd_bf16 without the stream."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (o, "o")):
        _contiguous(_device_tensor(t, n), n)
        if t.dtype != torch.bfloat16:
            raise TypeError(f"'{n}' must be bfloat16, got {t.dtype}")
        if t.dim() != 4 or tuple(t.shape) != tuple(q.shape):
            raise ValueError(f"'{n}' must be [batch, heads, seq_len, head_dim] like q {tuple(q.shape)}")
    batch, heads, seq_len, head_dim = q.shape
    if not sm_scale > 0:
        raise ValueError(f"sm_scale must be positive, got {sm_scale}")
    if head_dim not in FA_HEAD_DIMS:
        raise ValueError(f"head_dim {head_dim} not supported (supported: {FA_HEAD_DIMS})")
    lse_ptr = 0
    if lse is not None:
        _contiguous(_device_tensor(lse, "lse"), "lse")
        if lse.dtype != torch.float32 or lse.numel() != batch * heads * seq_len:
            raise ValueError("lse must be float32 [batch, heads, seq_len]")
        lse_ptr = lse.data_ptr()
    return (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse_ptr, batch, heads, seq_len, head_dim,
            float(sm_scale), int(bool(causal)))


def flash_attention_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, sm_scale: float,
                        causal: bool, lse: Optional[torch.Tensor] = None, stream: Any = None) -> None:
    """o = softmax(q k^T * sm_scale + causal mask) v for bf16 [batch, heads, seq, head_dim]."""
    _native.call("asc_flash_attention_fwd_bf16", *_attention_args(q, k, v, o, sm_scale, causal, lse),
                 _stream(stream))


def flash_attention_plan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor, sm_scale: float,
                         causal: bool, lse: Optional[torch.Tensor] = None) -> "_native.LaunchPlan":
    """The launch flash_attention_fwd(...) makes, as a kernel of the asc2_flash_attention
    code object with its grid, block and argument blob (asc_flash_attention_plan)."""
    plan = _native.LaunchPlan()
    _native.call("asc_flash_attention_plan", *_attention_args(q, k, v, o, sm_scale, causal, lse),
                 ctypes.byref(plan))
    return plan


# ------------------------------------------------------------------ element-wise tile operations

UNARY_OPS = ("abs", "ceil", "cos", "cosh", "erf", "exp", "exp2", "floor", "log", "log2", "negative", "relu",
             "rsqrt", "sin", "sinh", "sqrt", "tan", "tanh")
BINARY_OPS = ("add", "sub", "mul", "div", "maximum", "minimum", "left_shift", "right_shift")
COMPARE_OPS = ("equal", "not_equal", "greater", "greater_equal", "less", "less_equal")
_TILE_DTYPES = (torch.float32, torch.float16, torch.bfloat16, torch.int32, torch.int16)


def _flat(t: torch.Tensor, name: str, n: int) -> torch.Tensor:
    _contiguous(_device_tensor(t, name), name)
    if t.numel() < n:
        raise ValueError(f"'{name}' holds {t.numel()} elements, {n} needed")
    return t


def _scalar_parts(value: Any, dtype: torch.dtype):
    """(scalar_f, scalar_i) transport of a scalar operand for an element type."""
    if isinstance(value, torch.Tensor):
        if value.dim() != 0:
            raise ValueError("a scalar operand must be a 0-dim tensor or a python number")
        value = value.item()
    if dtype.is_floating_point:
        return float(value), 0
    if isinstance(value, float) and not value.is_integer():
        raise TypeError(f"an integer tile takes an integer scalar, got {value}")
    return 0.0, int(value)


def unary_f32(x: torch.Tensor, out: torch.Tensor, op: str, n: Optional[int] = None, stream=None) -> None:
    """out[:n] = op(x[:n]), fp32 (asc2 unary ops, python/asc/language/tile/unary_ops.py)."""
    if op not in UNARY_OPS:
        raise ValueError(f"unknown unary op {op!r}; expected one of {UNARY_OPS}")
    n = x.numel() if n is None else int(n)
    for t, name in ((x, "x"), (out, "out")):
        _flat(t, name, n)
        if t.dtype != torch.float32:
            raise TypeError(f"'{name}' must be float32, got {t.dtype}")
    _native.call("asc_unary_f32", UNARY_OPS.index(op), x.data_ptr(), out.data_ptr(), n, _stream(stream))


_FLOAT_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def unary(x: torch.Tensor, out: torch.Tensor, op: str, n: Optional[int] = None, stream=None) -> None:
    """out[:n] = op(x[:n]) on float32 / float16 / bfloat16 (16-bit: fp32 op, one RNE rounding)."""
    if op not in UNARY_OPS:
        raise ValueError(f"unknown unary op {op!r}; expected one of {UNARY_OPS}")
    n = x.numel() if n is None else int(n)
    code = _code(x, "x", _FLOAT_DTYPES)
    if out.dtype != x.dtype:
        raise TypeError(f"'out' must be {x.dtype}, got {out.dtype}")
    _flat(x, "x", n)
    _flat(out, "out", n)
    _native.call("asc_unary", UNARY_OPS.index(op), code, x.data_ptr(), out.data_ptr(), n, _stream(stream))


def axpy(src: torch.Tensor, dst: torch.Tensor, scalar: float, n: Optional[int] = None, stream=None) -> None:
    """dst[:n] = src[:n] * scalar + dst[:n] (asc.axpy): float32 / float16 / bfloat16, the
    scalar rounded to the element type, fp32 math, one rounding of the result."""
    n = src.numel() if n is None else int(n)
    code = _code(src, "src", _FLOAT_DTYPES)
    if dst.dtype != src.dtype:
        raise TypeError(f"'dst' must be {src.dtype}, got {dst.dtype}")
    _flat(src, "src", n)
    _flat(dst, "dst", n)
    _native.call("asc_axpy", code, src.data_ptr(), dst.data_ptr(), float(_scalar_parts(scalar, src.dtype)[0]), n,
                 _stream(stream))


def transpose_batched(x: torch.Tensor, z: torch.Tensor, batch: int, rows: int, cols: int, stream=None) -> None:
    """z[b, c, r] = x[b, r, c] for row-major [batch, rows, cols] of 2- or 4-byte elements."""
    n = int(batch) * int(rows) * int(cols)
    _flat(x, "x", n)
    _flat(z, "z", n)
    if z.dtype != x.dtype:
        raise TypeError(f"'z' must be {x.dtype}, got {z.dtype}")
    _native.call("asc_transpose_batched", x.element_size(), x.data_ptr(), z.data_ptr(), int(batch), int(rows),
                 int(cols), _stream(stream))


def quant_i8(src: torch.Tensor, dst: torch.Tensor, scale: float, offset: float, n: Optional[int] = None,
             stream=None) -> None:
    """dst[:n] = saturate_int8(rint(src * scale + offset)) (asc.adv.quant): scale and offset
    in src's dtype, each operation rounded to it, ties to even, NaN -> 0."""
    n = src.numel() if n is None else int(n)
    code = _code(src, "src", _FLOAT_DTYPES)
    if dst.dtype != torch.int8:
        raise TypeError(f"'dst' must be int8, got {dst.dtype}")
    _flat(src, "src", n)
    _flat(dst, "dst", n)
    _native.call("asc_quant_i8", code, src.data_ptr(), dst.data_ptr(), float(scale), float(offset), n,
                 _stream(stream))


def binary(x: Any, y: Any, out: torch.Tensor, op: str, n: Optional[int] = None, stream=None) -> None:
    """out[:n] = op(x, y) with either operand a tensor or a scalar (asc2 binary ops,
    python/asc/language/tile/binary_ops.py); the result dtype is the tensor operand's."""
    if op not in BINARY_OPS:
        raise ValueError(f"unknown binary op {op!r}; expected one of {BINARY_OPS}")
    x_t, y_t = isinstance(x, torch.Tensor) and x.dim() > 0, isinstance(y, torch.Tensor) and y.dim() > 0
    if not (x_t or y_t):
        raise TypeError("at least one operand must be a tensor")
    ref = x if x_t else y
    n = ref.numel() if n is None else int(n)
    code = _code(ref, "x" if x_t else "y", _TILE_DTYPES)
    if out.dtype != ref.dtype:
        raise TypeError(f"'out' must be {ref.dtype}, got {out.dtype}")
    _flat(out, "out", n)
    mode, scalar = 0, None
    if x_t and y_t:
        if y.dtype != x.dtype:
            raise TypeError(f"operand dtypes differ: {x.dtype} and {y.dtype}")
        _flat(x, "x", n)
        _flat(y, "y", n)
    elif x_t:
        mode, scalar = 1, y
        _flat(x, "x", n)
    else:
        mode, scalar = 2, x
        _flat(y, "y", n)
    if op in ("left_shift", "right_shift"):
        if mode != 1 or ref.dtype.is_floating_point:
            raise TypeError(f"{op} takes an integer tensor and a scalar shift amount")
        bits = torch.iinfo(ref.dtype).bits
        shift = int(scalar.item()) if isinstance(scalar, torch.Tensor) else int(scalar)
        if not 0 <= shift < bits:
            raise ValueError(f"{op} amount {shift} is outside [0, {bits}) for {ref.dtype}")
    s_f, s_i = _scalar_parts(scalar, ref.dtype) if scalar is not None else (0.0, 0)
    # an unused operand slot gets the output buffer (valid for n elements), never NULL
    _native.call("asc_binary", BINARY_OPS.index(op), code, x.data_ptr() if x_t else out.data_ptr(),
                 y.data_ptr() if y_t else out.data_ptr(), out.data_ptr(), n, mode, s_f, s_i, _stream(stream))


def where_compare(x: torch.Tensor, y: Any, out: torch.Tensor, cmp: str, true_value=None, false_value=None,
                  n: Optional[int] = None, stream=None) -> None:
    """out = where(cmp(x, y), x, y) for a tensor y, or where(cmp(x, s), true_value,
    false_value) for a scalar s (asc2.where over a comparison, test_where.py)."""
    if cmp not in COMPARE_OPS:
        raise ValueError(f"unknown comparison {cmp!r}; expected one of {COMPARE_OPS}")
    n = x.numel() if n is None else int(n)
    code = _code(x, "x", _TILE_DTYPES)
    _flat(x, "x", n)
    _flat(out, "out", n)
    if out.dtype != x.dtype:
        raise TypeError(f"'out' must be {x.dtype}, got {out.dtype}")
    if isinstance(y, torch.Tensor) and y.dim() > 0:
        if y.dtype != x.dtype:
            raise TypeError(f"operand dtypes differ: {x.dtype} and {y.dtype}")
        _flat(y, "y", n)
        _native.call("asc_where_cmp", COMPARE_OPS.index(cmp), code, x.data_ptr(), y.data_ptr(), out.data_ptr(), n,
                     0, 0.0, 0, 0.0, 0.0, _stream(stream))
        return
    if true_value is None or false_value is None:
        raise ValueError("a scalar comparison needs true_value and false_value")
    s_f, s_i = _scalar_parts(y, x.dtype)
    _native.call("asc_where_cmp", COMPARE_OPS.index(cmp), code, x.data_ptr(), x.data_ptr(), out.data_ptr(), n, 1, s_f,
                 s_i, float(true_value), float(false_value), _stream(stream))


# ------------------------------------------------------------------- tile load / store, shape ops

def tile_offsets(tensor_shape, tile_shape, tile_id=None, offsets=None):
    """Offsets of a tile: exactly one of ``tile_id`` (-> tile_id * tile_shape) or
    ``offsets`` (python/asc/language/tile/memory_ops.py:24-31, 65-80)."""
    if (tile_id is None) == (offsets is None):
        raise ValueError("Exactly one of 'tile_id' or 'offsets' must be provided")
    if tile_shape is not None and len(tile_shape) != len(tensor_shape):
        raise RuntimeError("rank of 'tensor_shape' must match rank of 'shape'")
    if tile_id is not None:
        return [int(i) * int(s) for i, s in zip(tile_id, tile_shape)]
    if len(offsets) != len(tensor_shape):
        raise ValueError(f"{len(offsets)} offsets for a rank-{len(tensor_shape)} tensor")
    return [int(o) for o in offsets]


def tile_binary(x: torch.Tensor, y: torch.Tensor, z: torch.Tensor, op: str, tensor_shape, tile_shape, offsets,
                stream=None) -> None:
    """z[tile] = op(x[tile], y[tile]) for the tile at ``offsets`` of shape ``tile_shape``
    (None: one element) in 1-D / 2-D row-major tensors of ``tensor_shape``; the store
    clips at the tensor bounds (asc2.load, op, asc2.store)."""
    if op not in BINARY_OPS[:6]:
        raise ValueError(f"op {op!r} is not an element-wise binary op")
    shape = [int(v) for v in tensor_shape]
    if len(shape) not in (1, 2):
        raise NotImplementedError("tiles of 1-D and 2-D tensors")
    tile = [1] * len(shape) if tile_shape is None else [int(v) for v in tile_shape]
    if len(tile) != len(shape) or len(offsets) != len(shape):
        raise RuntimeError("rank of 'tensor_shape' must match rank of the tile and of 'offsets'")
    rows, cols = (1, shape[0]) if len(shape) == 1 else shape
    r0, c0 = (0, int(offsets[0])) if len(shape) == 1 else (int(offsets[0]), int(offsets[1]))
    h, w = (1, tile[0]) if len(shape) == 1 else tile
    if r0 < 0 or c0 < 0:
        raise ValueError(f"negative tile offsets {list(offsets)}")
    code = _code(x, "x", _TILE_DTYPES)
    for t, name in ((x, "x"), (y, "y"), (z, "z")):
        _flat(t, name, rows * cols)
        if t.dtype != x.dtype:
            raise TypeError(f"'{name}' must be {x.dtype}, got {t.dtype}")
    _native.call("asc_rect_binary", BINARY_OPS.index(op), code, x.data_ptr(), y.data_ptr(), z.data_ptr(), rows, cols,
                 r0, c0, h, w, _stream(stream))


def broadcast_rows(x: torch.Tensor, z: torch.Tensor, rows: int, cols: int, stream=None) -> None:
    """z[r, c] = x[c] for r < rows (asc2.broadcast_to from [1, cols]; rows = 1 copies)."""
    _flat(x, "x", cols)
    _flat(z, "z", rows * cols)
    if z.dtype != x.dtype:
        raise TypeError(f"'z' must be {x.dtype}, got {z.dtype}")
    _native.call("asc_broadcast_rows", x.element_size(), x.data_ptr(), z.data_ptr(), rows, cols, _stream(stream))


ATOMIC_OPS = ("add", "maximum", "minimum")


def atomic_tiles(x: torch.Tensor, z: torch.Tensor, op: str, n_tiles: int, tile_len: int, addend=0,
                 stream=None) -> None:
    """z[j] = op(z[j], x[b * tile_len + j] + addend) for b < n_tiles, each combine atomic
    (asc2.atomic_add / atomic_max / atomic_min, python/asc/language/tile/atomic_ops.py:19-33;
    the kernel of python/test/asc2/operations/test_atomic_ops.py:33-40).  The order in which
    the tiles' float sums land is unspecified."""
    if op not in ATOMIC_OPS:
        raise ValueError(f"unknown atomic op {op!r}; expected one of {ATOMIC_OPS}")
    n_tiles, tile_len = int(n_tiles), int(tile_len)
    if n_tiles < 0 or tile_len < 0:
        raise ValueError("n_tiles and tile_len must be non-negative")
    code = _code(x, "x", _TILE_DTYPES)
    _flat(x, "x", n_tiles * tile_len)
    _flat(z, "z", tile_len)
    if z.dtype != x.dtype:
        raise TypeError(f"'z' must be {x.dtype}, got {z.dtype}")
    c_f, c_i = _scalar_parts(addend, x.dtype)
    _native.call("asc_atomic_tiles", BINARY_OPS.index(op), code, x.data_ptr(), z.data_ptr(), n_tiles, tile_len, c_f,
                 c_i, _stream(stream))


def fill(z: torch.Tensor, value, n: Optional[int] = None, stream=None) -> None:
    """z[:n] = value in z's element type (asc2.full broadcast to the tensor and stored)."""
    n = z.numel() if n is None else int(n)
    code = _code(z, "z", _TILE_DTYPES)
    _flat(z, "z", n)
    c_f, c_i = _scalar_parts(value, z.dtype)
    _native.call("asc_fill", code, z.data_ptr(), n, c_f, c_i, _stream(stream))
