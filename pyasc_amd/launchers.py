"""Registered kernel signatures: each maps one asc2 kernel of the reference (or a
build-defined asc2-style kernel where the reference has none) onto pyasc_amd.kernels.

Coverage rules follow the reference kernel bodies: the logical grid decides which
elements a launch writes, the physical HIP grid is the library's own choice.
"""
from __future__ import annotations

from typing import List, Tuple

import torch

from . import kernels
from .asc.core import as_torch_dtype, ceildiv
from .asc.runtime import module
from .registry import KernelCall, register


def _shape2(v, name: str) -> Tuple[int, int]:
    shape = tuple(int(s) for s in v)
    if len(shape) != 2:
        raise ValueError(f"'{name}' must be a 2-D shape, got {v}")
    return shape


def _check_shapes(call: KernelCall) -> Tuple[int, int, int]:
    a, b, c = call.args["a_ptr"], call.args["b_ptr"], call.args["c_ptr"]
    M, K = _shape2(call.consts["a_shape"], "a_shape")
    K2, N = _shape2(call.consts["b_shape"], "b_shape")
    if K2 != K:
        raise ValueError(f"a_shape {M, K} and b_shape {K2, N} do not chain")
    if tuple(_shape2(call.consts["c_shape"], "c_shape")) != (M, N):
        raise ValueError(f"c_shape must be {(M, N)}")
    for t, n, shp in ((a, "a_ptr", (M, K)), (b, "b_ptr", (K, N)), (c, "c_ptr", (M, N))):
        if t.numel() < shp[0] * shp[1]:
            raise ValueError(f"'{n}' holds {t.numel()} elements, {shp} needed")
    return M, N, K


def _as2d(t: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    return t.reshape(-1)[:rows * cols].view(rows, cols)


def _asc2_matmul_dtype(t: torch.Tensor) -> None:
    # asc2 matmul accepts f32/f16/bf16 tiles only (python/asc/language/tile/utils.py:129-139)
    if t.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TypeError(f"asc2 matmul supports float32, float16 and bfloat16 operands, got {t.dtype}")


# ------------------------------------------------ vadd / leaky_relu / vmuladd / gelu code objects

STREAM_THREADS, STREAM_UNROLL = 256, 4  # kThreads, kUnroll of vadd_kernels.h and elementwise_kernels.h
ELEM_MAX_GRID = 4096   # the elementwise element kernels are grid-stride (elementwise_kernels.h)
GELU_MAX_GRID = 8192   # so are gelu's rows
_CO_SUFFIX = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16", torch.int32: "i32"}


def _stream_code_object(functions, vec: str, elem: str, tensors, covered: int, extra, stream: int,
                        elem_max_grid: int = 0) -> None:
    """The library's streaming launch (csrc/vadd.hip, csrc/elementwise.hip) through a code
    object: kernel ``vec`` over the 16-byte vectors of [0, covered) when every tensor is
    16-byte aligned, kernel ``elem`` over the rest; the kernels take the tensors'
    pointers, then the range, then ``extra``."""
    ptrs = [("ptr", t.data_ptr()) for t in tensors]
    per_vec = 16 // tensors[0].element_size()
    done = 0
    if all(t.data_ptr() % 16 == 0 for t in tensors):
        n_vec = covered // per_vec
        if n_vec:
            module.launch(functions[vec], ceildiv(n_vec, STREAM_THREADS * STREAM_UNROLL), STREAM_THREADS,
                          ptrs + [("i64", n_vec)] + extra, stream)
        done = n_vec * per_vec
    if done < covered:
        grid = ceildiv(covered - done, STREAM_THREADS)
        if elem_max_grid:
            grid = min(grid, elem_max_grid)
        module.launch(functions[elem], grid, STREAM_THREADS, ptrs + [("i64", done), ("i64", covered)] + extra,
                      stream)


def _vadd_code_object_launch(call: KernelCall, functions) -> None:
    """vadd_kernel through the asc2_vadd code object (the device bodies of vadd_kernels.h);
    its element kernel takes one element per thread."""
    x, y, out = call.args["x_ptr"], call.args["y_ptr"], call.args["out_ptr"]
    covered = kernels.vadd_check(x, y, out, int(call.args["size"]), int(call.consts["tile_size"]),
                                 int(call.consts["tile_per_block"]), call.grid)
    if covered:
        sfx = _CO_SUFFIX[x.dtype]
        _stream_code_object(functions, f"asc2_vadd_vec_{sfx}", f"asc2_vadd_elem_{sfx}", (x, y, out), covered, [],
                            call.stream)


VADD_CODE_OBJECT = module.CodeObject(
    "asc2_vadd", tuple(f"asc2_vadd_{kind}_{sfx}" for sfx in ("f32", "f16", "bf16", "i32") for kind in ("vec", "elem")),
    _vadd_code_object_launch, "pyasc_amd/csrc/co/asc2_vadd.hip")


@register("vadd_kernel", ("x_ptr", "y_ptr", "out_ptr", "size", "tile_size", "tile_per_block"),
          "python/test/asc2/kernels/test_vadd.py:16-28", code_object=VADD_CODE_OBJECT)
def _vadd(call: KernelCall) -> None:
    kernels.vadd(call.args["x_ptr"], call.args["y_ptr"], call.args["out_ptr"], int(call.args["size"]),
                 int(call.consts["tile_size"]), int(call.consts["tile_per_block"]), call.grid, call.stream)


def _scalar(v) -> float:
    """A by-value float argument: a python number or a 0-dim tensor (its exact value)."""
    if isinstance(v, torch.Tensor):
        if v.dim() != 0:
            raise TypeError("a scalar argument must be a python number or a 0-dim tensor")
        return float(v.item())
    return float(v)


# The kernels of the asc2_elementwise code object (csrc/co/asc2_elementwise.hip).
ELEMENTWISE_CO_FUNCTIONS = tuple(
    f"asc2_{op}_{kind}_{sfx}" for op in ("leaky_relu", "vmuladd") for kind in ("vec", "elem")
    for sfx in ("f32", "f16", "bf16")) + ("asc2_gelu_rows_f32",)


def _leaky_relu_code_object_launch(call: KernelCall, functions) -> None:
    x, out = call.args["x_ptr"], call.args["out_ptr"]
    covered = kernels.leaky_relu_check(x, out, int(call.args["size"]), int(call.consts["tile_size"]),
                                       int(call.consts["tile_per_block"]), call.grid)
    if covered:
        sfx = _CO_SUFFIX[x.dtype]
        _stream_code_object(functions, f"asc2_leaky_relu_vec_{sfx}", f"asc2_leaky_relu_elem_{sfx}", (x, out),
                            covered, [("f32", _scalar(call.args["alpha"]))], call.stream, ELEM_MAX_GRID)


def _vmuladd_code_object_launch(call: KernelCall, functions) -> None:
    x, y, z, out = (call.args[n] for n in ("x_ptr", "y_ptr", "z_ptr", "out_ptr"))
    covered = kernels.vmuladd_check(x, y, z, out, int(call.args["size"]), int(call.consts["tile_size"]),
                                    int(call.consts["tile_per_block"]), call.grid)
    if covered:
        sfx = _CO_SUFFIX[x.dtype]
        _stream_code_object(functions, f"asc2_vmuladd_vec_{sfx}", f"asc2_vmuladd_elem_{sfx}", (x, y, z, out),
                            covered, [], call.stream, ELEM_MAX_GRID)


def _gelu_code_object_launch(call: KernelCall, functions) -> None:
    """gelu_kernel through the code object with asc_gelu_rows_f32's geometry: rows b, b +
    grid, ... of min(rows, GELU_MAX_GRID) workgroups, the row's first min(tile, cols)
    columns, 16-byte vectors when both buffers are aligned and rows are whole vectors."""
    x, out = call.args["x_ptr"], call.args["out_ptr"]
    rows, cols, tile = int(call.get("num_rows")), int(call.get("num_columns")), int(call.get("tile_size"))
    kernels.gelu_rows_check(x, out, rows, cols, tile, call.grid)
    if rows == 0:
        return
    vec_ok = x.data_ptr() % 16 == 0 and out.data_ptr() % 16 == 0 and cols % 4 == 0
    module.launch(functions["asc2_gelu_rows_f32"], min(rows, GELU_MAX_GRID), STREAM_THREADS,
                  [("ptr", x.data_ptr()), ("ptr", out.data_ptr()), ("i64", rows), ("i64", cols),
                   ("i32", min(tile, cols)), ("i32", int(bool(call.get("approximate")))), ("i32", int(vec_ok))],
                  call.stream)


def _elementwise_code_object(launch) -> module.CodeObject:
    return module.CodeObject("asc2_elementwise", ELEMENTWISE_CO_FUNCTIONS, launch,
                             "pyasc_amd/csrc/co/asc2_elementwise.hip")


@register("leaky_relu_kernel", ("x_ptr", "alpha", "out_ptr", "size", "tile_size", "tile_per_block"),
          "python/test/asc2/kernels/test_leaky_relu.py:16-26",
          code_object=_elementwise_code_object(_leaky_relu_code_object_launch))
def _leaky_relu(call: KernelCall) -> None:
    kernels.leaky_relu(call.args["x_ptr"], _scalar(call.args["alpha"]), call.args["out_ptr"],
                       int(call.args["size"]), int(call.consts["tile_size"]), int(call.consts["tile_per_block"]),
                       call.grid, call.stream)


@register("vmuladd_kernel", ("x_ptr", "y_ptr", "z_ptr", "out_ptr", "size", "tile_size", "tile_per_block",
                             "buffer_factor"),
          "python/test/asc2/kernels/test_vmuladd.py:16-31",
          code_object=_elementwise_code_object(_vmuladd_code_object_launch))
def _vmuladd(call: KernelCall) -> None:
    # buffer_factor is the reference loop's unroll/double-buffer hint; it does not change the result
    kernels.vmuladd(call.args["x_ptr"], call.args["y_ptr"], call.args["z_ptr"], call.args["out_ptr"],
                    int(call.args["size"]), int(call.consts["tile_size"]), int(call.consts["tile_per_block"]),
                    call.grid, call.stream)


@register("gelu_kernel", ("x_ptr", "out_ptr", "num_rows", "num_columns", "tile_size", "approximate"),
          "python/test/asc2/kernels/test_gelu.py:19-33", code_object=_elementwise_code_object(_gelu_code_object_launch))
def _gelu(call: KernelCall) -> None:
    kernels.gelu_rows(call.args["x_ptr"], call.args["out_ptr"], int(call.get("num_rows")),
                      int(call.get("num_columns")), int(call.get("tile_size")), bool(call.get("approximate")),
                      call.grid, call.stream)


# ------------------------------------------------------------------------------------------- softmax

# The kernels of the asc2_softmax code object (csrc/co/asc2_softmax.hip), one per row body.
SOFTMAX_CO_FUNCTIONS = tuple(f"asc2_softmax_{body}" for body in (
    "wave_1x2", "wave_2x2", "block_2x128", "block_2x256", "block_2x512", "block_8x256", "long", "f16", "padded_f32",
    "padded_f16"))


def _softmax_code_object_launch(fused: bool):
    """softmax_kernel through the asc2_softmax code object: asc_softmax_plan picks the
    kernel, grid, block and arguments the library entry (asc_softmax_rows_* /
    asc_softmax_blocks_*) would launch, and the code object's kernel of that name runs
    them (the same device body)."""
    size_name = "block_size" if fused else "tile_size"

    def launch(call: KernelCall, functions) -> None:
        x, out = call.args["x_ptr"], call.args["out_ptr"]
        plan = kernels.softmax_plan(x, out, int(call.get("num_rows")), int(call.get("num_cols")),
                                    int(call.get(size_name)), call.grid, fused)
        if plan.grid:
            module.launch(functions[plan.kernel.decode()], plan.grid, plan.block,
                          [("ptr", x.data_ptr()), ("ptr", out.data_ptr()), ("i64", plan.rows),
                           ("i64", plan.stride), ("i32", plan.len), ("i32", plan.flag)], call.stream)

    return launch


SOFTMAX_ROWS_CODE_OBJECT = module.CodeObject("asc2_softmax", SOFTMAX_CO_FUNCTIONS, _softmax_code_object_launch(False),
                                             "pyasc_amd/csrc/co/asc2_softmax.hip")
SOFTMAX_BLOCKS_CODE_OBJECT = module.CodeObject("asc2_softmax", SOFTMAX_CO_FUNCTIONS, _softmax_code_object_launch(True),
                                               "pyasc_amd/csrc/co/asc2_softmax.hip")


@register("softmax_kernel", ("x_ptr", "out_ptr", "num_rows", "num_cols", "tile_size"),
          "python/test/asc2/kernels/test_softmax.py:16-27", code_object=SOFTMAX_ROWS_CODE_OBJECT)
def _softmax_rows(call: KernelCall) -> None:
    kernels.softmax_rows(call.args["x_ptr"], call.args["out_ptr"], int(call.get("num_rows")),
                         int(call.get("num_cols")), int(call.get("tile_size")), call.grid, call.stream)


@register("softmax_kernel", ("x_ptr", "out_ptr", "num_rows", "num_cols", "block_size"),
          "python/test/asc2/kernels/test_softmax_fused.py:16-24", code_object=SOFTMAX_BLOCKS_CODE_OBJECT)
def _softmax_blocks(call: KernelCall) -> None:
    kernels.softmax_blocks(call.args["x_ptr"], call.args["out_ptr"], int(call.get("num_rows")),
                           int(call.get("num_cols")), int(call.get("block_size")), call.grid, call.stream)


# ---------------------------------------------------------------------------------- reductions, rms_norm

def _reduce_name(op) -> str:
    """The asc2 reduction passed as a ConstExpr (asc2.reduce_sum ...) -> its kernel op name."""
    name = getattr(op, "__name__", str(op))
    for k in ("sum", "max", "min", "prod"):
        if name == f"reduce_{k}":
            return k
    raise NotImplementedError(f"no native reduction for op {name!r}")


def _zero_offsets(offsets, what: str) -> None:
    if any(int(o) != 0 for o in offsets):
        raise NotImplementedError(f"{what} must be all zero (the reference tests load the whole tensor)")


@register("kernel", ("input_ptr", "output_ptr", "reduce_dim", "input_shape", "input_offsets", "output_shape",
                     "output_offsets", "op", "keep_dims"),
          "python/test/asc2/operations/test_reduce_ops.py:33-41")
def _reduce_dim(call: KernelCall) -> None:
    x, out = call.args["input_ptr"], call.args["output_ptr"]
    shape = [int(v) for v in call.consts["input_shape"]]
    _zero_offsets(call.consts["input_offsets"], "input_offsets")
    _zero_offsets(call.consts["output_offsets"], "output_offsets")
    if len(shape) != 2:
        raise NotImplementedError("reductions along a dim are implemented for 2-D tiles")
    kernels.reduce_f32(_as2d(x, shape[0], shape[1]), out.reshape(-1), _reduce_name(call.consts["op"]),
                       int(call.consts["reduce_dim"]), call.stream)


@register("kernel_all", ("input_ptr", "output_ptr", "input_shape", "input_offsets", "output_shape", "output_offsets",
                         "op"),
          "python/test/asc2/operations/test_reduce_ops.py:44-52")
def _reduce_all(call: KernelCall) -> None:
    x, out = call.args["input_ptr"], call.args["output_ptr"]
    shape = [int(v) for v in call.consts["input_shape"]]
    _zero_offsets(call.consts["input_offsets"], "input_offsets")
    _zero_offsets(call.consts["output_offsets"], "output_offsets")
    n = 1
    for d in shape:
        n *= d
    out_n = 1
    for d in call.consts["output_shape"]:
        out_n *= int(d)
    for t, name, need in ((x, "input_ptr", n), (out, "output_ptr", out_n)):
        if t.numel() < need:
            raise ValueError(f"'{name}' holds {t.numel()} elements, its shape needs {need}")
    kernels.reduce_f32(x.reshape(-1)[:n], out.reshape(-1)[:out_n], _reduce_name(call.consts["op"]), None,
                       call.stream)


@register("reduce_tile_kernel", ("x_ptr", "out_ptr", "size", "tile_size"),
          "python/test/asc2/operations/test_reduce_ops.py:85-92")
def _reduce_tile(call: KernelCall) -> None:
    # max over the first tile_size elements, stored as a [1] tile
    tile = int(call.consts["tile_size"])
    x = call.args["x_ptr"]
    if tile > int(call.args["size"]) or tile > x.numel():
        raise ValueError("tile_size exceeds the tensor")
    kernels.reduce_f32(x.reshape(-1)[:tile], call.args["out_ptr"].reshape(-1)[:1], "max", None, call.stream)


@register("rms_norm_kernel", ("x_ptr", "gamma_ptr", "out_ptr", "num_rows", "num_cols", "epsilon", "tile_size"),
          "python/asc/language/tile/unary_ops.py:225-237 (asc2.rms_norm; build-defined kernel)")
def _rms_norm(call: KernelCall) -> None:
    kernels.rms_norm(call.args["x_ptr"], call.args["gamma_ptr"], call.args["out_ptr"], int(call.get("num_rows")),
                     int(call.get("num_cols")), _scalar(call.args["epsilon"]), int(call.consts["tile_size"]),
                     call.stream)


# -------------------------------------------------------------------------------------------- matmul

def mnblock_rectangles(M: int, N: int, grid: int, m_tile: int, m_tiles_per_block: int, n_tile: int,
                       n_tiles_per_block: int) -> List[Tuple[int, int, int, int]]:
    """C rectangles (m0, m1, n0, n1) written by the mnblock kernel body for a logical grid
    (python/test/asc2/kernels/test_matmul_mnblock.py:23-36): block b starts at
    m = (m_tile*mtpb*b) % M, n = ((m_tile*mtpb*b) // M) * n_tile*ntpb and covers
    m_tile*mtpb rows and n_tile*ntpb columns, clipped to C."""
    m_span, n_span = m_tile * m_tiles_per_block, n_tile * n_tiles_per_block
    rects = set()
    for blk in range(grid):
        m0 = (m_span * blk) % M
        n0 = ((m_span * blk) // M) * n_span
        m1, n1 = min(M, m0 + m_span), min(N, n0 + n_span)
        if m0 < m1 and n0 < n1:
            rects.add((m0, m1, n0, n1))
    return sorted(rects)


def _merge_full(rects: List[Tuple[int, int, int, int]], M: int, N: int) -> List[Tuple[int, int, int, int]]:
    covered = torch.zeros(M, N, dtype=torch.bool)
    for m0, m1, n0, n1 in rects:
        covered[m0:m1, n0:n1] = True
    return [(0, M, 0, N)] if bool(covered.all()) else rects


# The asc2 matmul bodies take the matmul they launch: kernels.matmul (the library's
# asc_matmul) or, for a code-object launch, the same call replayed from asc_matmul_plan
# through the asc2_matmul code object.  Either way the same kernels run with the same
# arguments.

def _matmul_through(functions, stream):
    """kernels.matmul's call form, launched through the asc2_matmul code object."""
    def mm(a, b, c, relu=False, stream=stream, bias=None, leaky_alpha=None):
        module.launch_plan(functions, kernels.matmul_plan(a, b, c, relu=relu, bias=bias, leaky_alpha=leaky_alpha),
                           stream)
    return mm


def _mnblock_body(call: KernelCall, mm) -> None:
    M, N, K = _check_shapes(call)
    a, b, c = _as2d(call.args["a_ptr"], M, K), _as2d(call.args["b_ptr"], K, N), _as2d(call.args["c_ptr"], M, N)
    _asc2_matmul_dtype(a)
    rects = mnblock_rectangles(M, N, call.grid, int(call.consts["m_tile"]), int(call.consts["m_tiles_per_block"]),
                               int(call.consts["n_tile"]), int(call.consts["n_tiles_per_block"]))
    for m0, m1, n0, n1 in _merge_full(rects, M, N):
        mm(a[m0:m1], b[:, n0:n1], c[m0:m1, n0:n1], stream=call.stream)


def _ktiled_body(call: KernelCall, mm) -> None:
    M, N, K = _check_shapes(call)
    k_tiles = int(call.consts["k_tiles"])
    if k_tiles <= 0:
        raise ValueError("k_tiles must be positive")
    # acc = sum_{i<k_tiles} A[:, i*ko:(i+1)*ko] @ B[i*ko:(i+1)*ko, :] with ko = K // k_tiles
    k_used = (K // k_tiles) * k_tiles
    a, b, c = _as2d(call.args["a_ptr"], M, K), _as2d(call.args["b_ptr"], K, N), _as2d(call.args["c_ptr"], M, N)
    _asc2_matmul_dtype(a)
    if k_used == 0:
        c.zero_()
        return
    mm(a[:, :k_used], b[:k_used], c, stream=call.stream)


def _fixpipe_body(call: KernelCall, mm) -> None:
    # c = relu(a @ b).to(c's dtype), relu and cast fused into the store
    M, N, K = _check_shapes(call)
    a, b, c = _as2d(call.args["a_ptr"], M, K), _as2d(call.args["b_ptr"], K, N), _as2d(call.args["c_ptr"], M, N)
    _asc2_matmul_dtype(a)
    mm(a, b, c, relu=True, stream=call.stream)


def _chained_body(call: KernelCall, mm, chained=None) -> None:
    # t = (a @ b).to(dtype); c = t @ b  (needs N == K).  ``chained``: one call that runs both
    # matmuls with its own intermediate (the library's asc_matmul_chained); else two ``mm``.
    M, N, K = _check_shapes(call)
    if N != K:
        raise ValueError(f"the chained matmul multiplies (a@b) by b again and needs N == K, got N={N}, K={K}")
    a, b, c = _as2d(call.args["a_ptr"], M, K), _as2d(call.args["b_ptr"], K, N), _as2d(call.args["c_ptr"], M, N)
    _asc2_matmul_dtype(a)
    mid_dtype = as_torch_dtype(call.consts["dtype"])
    if mid_dtype != b.dtype:
        raise TypeError(f"the intermediate dtype {mid_dtype} must match b's dtype {b.dtype} for the second matmul")
    if chained is not None and a.dtype in (torch.float16, torch.bfloat16):
        chained(a, b, c, stream=call.stream)
        return
    t = torch.empty((M, N), dtype=mid_dtype, device=a.device)
    mm(a, b, t, stream=call.stream)
    mm(t, b, c, stream=call.stream)
    # t is freed on return; on a stream other than torch's current one the caching
    # allocator must not hand its memory out again before these launches have run
    if call.stream != torch.cuda.current_stream(a.device).cuda_stream:
        t.record_stream(torch.cuda.ExternalStream(call.stream, device=a.device))


# The kernels of the asc2_matmul code object (csrc/co/asc2_matmul.hip).
MATMUL_CO_FUNCTIONS = tuple(
    f"asc2_mm_{kind}_{out}" for out in ("f32", "f16", "bf16")
    for kind in ("mfma_bf16_fast", "mfma_bf16_checked", "mfma_f16_fast", "mfma_f16_checked", "f32_mfma", "f32_fma"))


def _matmul_code_object(body) -> module.CodeObject:
    return module.CodeObject("asc2_matmul", MATMUL_CO_FUNCTIONS,
                             lambda call, functions: body(call, _matmul_through(functions, call.stream)),
                             "pyasc_amd/csrc/co/asc2_matmul.hip")


@register("matmul_kernel", ("a_ptr", "b_ptr", "c_ptr", "a_shape", "b_shape", "c_shape", "m_tile",
                            "m_tiles_per_block", "n_tile", "n_tiles_per_block"),
          "python/test/asc2/kernels/test_matmul_mnblock.py:17-36", code_object=_matmul_code_object(_mnblock_body))
def _matmul_mnblock(call: KernelCall) -> None:
    _mnblock_body(call, kernels.matmul)


@register("matmul_kernel", ("a_ptr", "b_ptr", "c_ptr", "a_shape", "b_shape", "c_shape", "k_tiles"),
          "python/test/asc2/kernels/test_matmul_tiled.py:17-31", code_object=_matmul_code_object(_ktiled_body))
def _matmul_ktiled(call: KernelCall) -> None:
    _ktiled_body(call, kernels.matmul)


@register("matmul_kernel", ("a_ptr", "b_ptr", "c_ptr", "a_shape", "b_shape", "c_shape"),
          "python/test/asc2/kernels/test_matmul_fixpipe.py:17-27", code_object=_matmul_code_object(_fixpipe_body))
def _matmul_fixpipe(call: KernelCall) -> None:
    _fixpipe_body(call, kernels.matmul)


@register("matmul_kernel", ("a_ptr", "b_ptr", "c_ptr", "a_shape", "b_shape", "c_shape", "dtype"),
          "python/test/asc2/kernels/test_matmul_l0c_to_l1.py:17-30", code_object=_matmul_code_object(_chained_body))
def _matmul_chained(call: KernelCall) -> None:
    _chained_body(call, kernels.matmul, kernels.matmul_chained)


# ------------------------------------------------------------- int8 matmul (build-defined asc2 style)

def _int8_body(call: KernelCall, mm8) -> None:
    M, N, K = _check_shapes(call)
    a, b, c = _as2d(call.args["a_ptr"], M, K), _as2d(call.args["b_ptr"], K, N), _as2d(call.args["c_ptr"], M, N)
    mm8(a, b, c)


def _dequant_body(call: KernelCall, mm8, trunc19: bool) -> None:
    M, N, K = _check_shapes(call)
    a, b, c = _as2d(call.args["a_ptr"], M, K), _as2d(call.args["b_ptr"], K, N), _as2d(call.args["c_ptr"], M, N)
    mm8(a, b, c, scale=call.args["quant_ptr"].reshape(-1), trunc19=trunc19)


def _trunc_scale(call: KernelCall) -> bool:
    return bool(call.consts["trunc_scale"]) if "trunc_scale" in call.consts else False


# The kernels of the asc2_matmul_i8 code object (csrc/co/asc2_matmul_i8.hip).
MATMUL_I8_CO_FUNCTIONS = tuple(f"asc2_i8_{path}_{out}" for path in ("fast", "checked") for out in ("i32", "f16"))


def _i8_code_object(launch) -> module.CodeObject:
    def run(call: KernelCall, functions) -> None:
        def mm8(a, b, c, scale=None, trunc19=False):
            module.launch_plan(functions, kernels.matmul_i8_plan(a, b, c, scale=scale, trunc19=trunc19),
                               call.stream)
        launch(call, mm8)
    return module.CodeObject("asc2_matmul_i8", MATMUL_I8_CO_FUNCTIONS, run, "pyasc_amd/csrc/co/asc2_matmul_i8.hip")


def _library_i8(call: KernelCall):
    def mm8(a, b, c, scale=None, trunc19=False):
        kernels.matmul_i8(a, b, c, scale=scale, trunc19=trunc19, stream=call.stream)
    return mm8


@register("matmul_int8_kernel", ("a_ptr", "b_ptr", "c_ptr", "a_shape", "b_shape", "c_shape"),
          "python/test/generalization/adv/test_matmul_iterate_all.py:106-120 (int8 -> int32 case)",
          code_object=_i8_code_object(_int8_body))
def _matmul_int8(call: KernelCall) -> None:
    _int8_body(call, _library_i8(call))


@register("matmul_dequant_kernel", ("a_ptr", "b_ptr", "c_ptr", "quant_ptr", "a_shape", "b_shape", "c_shape"),
          "python/test/generalization/adv/test_matmul_quant.py:23-51",
          code_object=_i8_code_object(lambda call, mm8: _dequant_body(call, mm8, False)))
def _matmul_dequant(call: KernelCall) -> None:
    _dequant_body(call, _library_i8(call), False)


@register("matmul_dequant_kernel",
          ("a_ptr", "b_ptr", "c_ptr", "quant_ptr", "a_shape", "b_shape", "c_shape", "trunc_scale"),
          "python/test/generalization/adv/test_matmul_quant.py:23-51,94-106",
          code_object=_i8_code_object(lambda call, mm8: _dequant_body(call, mm8, _trunc_scale(call))))
def _matmul_dequant_trunc(call: KernelCall) -> None:
    _dequant_body(call, _library_i8(call), _trunc_scale(call))


# -------------------------------------------------------- flash attention (build-defined asc2 style)

def _attention_views(call: KernelCall):
    batch, heads, seq = int(call.get("batch")), int(call.get("heads")), int(call.get("seq_len"))
    head_dim = int(call.get("head_dim"))
    if int(call.get("block_m")) <= 0 or int(call.get("block_n")) <= 0:
        raise ValueError("block_m and block_n must be positive")
    shape = (batch, heads, seq, head_dim)
    n = batch * heads * seq * head_dim
    views = []
    for name in ("q_ptr", "k_ptr", "v_ptr", "o_ptr"):
        t = call.args[name]
        if t.numel() < n:
            raise ValueError(f"'{name}' holds {t.numel()} elements, {shape} needed")
        views.append(t.reshape(-1)[:n].view(shape))
    return views


def _attention_code_object_launch(call: KernelCall, functions) -> None:
    q, k, v, o = _attention_views(call)
    module.launch_plan(functions, kernels.flash_attention_plan(q, k, v, o, float(call.get("sm_scale")),
                                                               bool(call.get("causal"))), call.stream)


ATTENTION_CODE_OBJECT = module.CodeObject("asc2_flash_attention", ("asc2_fa_fwd_d64", "asc2_fa_fwd_d128"),
                                          _attention_code_object_launch,
                                          "pyasc_amd/csrc/co/asc2_flash_attention.hip")


@register("flash_attention_fwd_kernel",
          ("q_ptr", "k_ptr", "v_ptr", "o_ptr", "batch", "heads", "seq_len", "head_dim", "sm_scale", "causal",
           "block_m", "block_n"), "none (the reference has no attention kernel)", code_object=ATTENTION_CODE_OBJECT)
def _flash_attention(call: KernelCall) -> None:
    q, k, v, o = _attention_views(call)
    kernels.flash_attention_fwd(q, k, v, o, float(call.get("sm_scale")), bool(call.get("causal")),
                                stream=call.stream)


# --------------------------------------------------------- element-wise tile operations (operation tests)

def _op_name(op, allowed, what: str) -> str:
    """The asc2 function passed as a ConstExpr (asc2.add ...) -> its name, checked."""
    name = getattr(op, "__name__", str(op))
    if name not in allowed:
        raise NotImplementedError(f"no native {what} for op {name!r}")
    return name


@register("kernel", ("x_ptr", "z_ptr", "block_length", "op"), "python/test/asc2/operations/test_unary_ops.py:35-40")
def _unary(call: KernelCall) -> None:
    # float32 as the reference test runs it; float16 / bfloat16 tiles as asc2 allows them
    n = int(call.consts["block_length"])
    kernels.unary(call.args["x_ptr"].reshape(-1), call.args["z_ptr"].reshape(-1),
                  _op_name(call.consts["op"], kernels.UNARY_OPS, "unary op"), n, call.stream)


@register("kernel", ("x_ptr", "y_ptr", "z_ptr", "block_length", "fmt", "op"),
          "python/test/asc2/operations/test_binary_ops.py:24-38")
def _binary(call: KernelCall) -> None:
    # fmt "VV" / "VS" / "SV": which operand is a tile (test_binary_ops.py:8-9, 25-35);
    # by-value operands arrive as python scalars
    fmt = str(call.consts["fmt"])
    x, y = call.args["x_ptr"], call.args["y_ptr"]
    x_vec, y_vec = isinstance(x, torch.Tensor), isinstance(y, torch.Tensor)
    if (x_vec, y_vec) != {"VV": (True, True), "VS": (True, False), "SV": (False, True)}.get(fmt, (None, None)):
        raise ValueError(f"operands do not match fmt {fmt!r}")
    n = int(call.consts["block_length"])
    kernels.binary(x.reshape(-1) if x_vec else x, y.reshape(-1) if y_vec else y, call.args["z_ptr"].reshape(-1),
                   _op_name(call.consts["op"], kernels.BINARY_OPS, "binary op"), n, call.stream)


@register("where_kernel", ("x_ptr", "y_ptr", "z_ptr", "op"), "python/test/asc2/operations/test_where.py:18-27")
def _where(call: KernelCall) -> None:
    # the body's tiles span the tensors (SIZE elements in the reference test)
    x = call.args["x_ptr"].reshape(-1)
    kernels.where_compare(x, call.args["y_ptr"].reshape(-1), call.args["z_ptr"].reshape(-1),
                          _op_name(call.consts["op"], kernels.COMPARE_OPS, "comparison"), n=x.numel(),
                          stream=call.stream)


@register("where_scalar_kernel", ("x_ptr", "scalar", "z_ptr", "op"),
          "python/test/asc2/operations/test_where.py:48-55")
def _where_scalar(call: KernelCall) -> None:
    # where(op(x, scalar), 0, 1) in x's dtype
    x = call.args["x_ptr"].reshape(-1)
    kernels.where_compare(x, call.args["scalar"], call.args["z_ptr"].reshape(-1),
                          _op_name(call.consts["op"], kernels.COMPARE_OPS, "comparison"), true_value=0,
                          false_value=1, n=x.numel(), stream=call.stream)



# ------------------------------------------------------ asc2.softmax on a whole tile (operation tests)

@register("softmax_1d_kernel", ("dst_ptr", "src_ptr", "length"), "python/test/asc2/operations/test_softmax.py:15-22")
def _softmax_1d(call: KernelCall) -> None:
    # one row of `length`; the body also stores src back unchanged
    n = int(call.consts["length"])
    src, dst = call.args["src_ptr"], call.args["dst_ptr"]
    kernels.softmax_blocks(src.reshape(-1), dst.reshape(-1), 1, n, 1, 1, call.stream)


@register("softmax_2d_kernel", ("dst_ptr", "src_ptr", "shape"), "python/test/asc2/operations/test_softmax.py:25-32")
def _softmax_2d(call: KernelCall) -> None:
    # softmax along the last dim of the [rows, cols] tile; the body also stores src back unchanged
    rows, cols = _shape2(call.consts["shape"], "shape")
    src, dst = call.args["src_ptr"], call.args["dst_ptr"]
    kernels.softmax_blocks(src.reshape(-1), dst.reshape(-1), rows, cols, rows, 1, call.stream)


# ------------------------------------------------ tile load / add / store (test_memory_ops.py)
# Each kernel body loads the same tile of x and y (offsets, or tile_id * tile_shape),
# adds them and stores the sum to the same tile of z (test_memory_ops.py:58-92).

def _memory_tile(call: KernelCall, tensor_shape) -> None:
    tile_shape = call.consts.get("tile_shape")
    offsets = kernels.tile_offsets(tensor_shape, tile_shape, call.consts.get("tile_id"), call.consts.get("offsets"))
    kernels.tile_binary(call.args["x_ptr"].reshape(-1), call.args["y_ptr"].reshape(-1), call.args["z_ptr"].reshape(-1),
                        "add", tensor_shape, tile_shape, offsets, call.stream)


@register("kernel_static", ("x_ptr", "y_ptr", "z_ptr", "tensor_shape", "tile_shape", "tile_id", "offsets"),
          "python/test/asc2/operations/test_memory_ops.py:58-64")
def _memory_static(call: KernelCall) -> None:
    _memory_tile(call, [int(v) for v in call.consts["tensor_shape"]])


@register("kernel_dynamic_1D", ("x_ptr", "y_ptr", "z_ptr", "ts0", "tile_shape", "tile_id", "offsets"),
          "python/test/asc2/operations/test_memory_ops.py:67-73")
def _memory_dynamic_1d(call: KernelCall) -> None:
    _memory_tile(call, [int(call.args["ts0"])])


@register("kernel_dynamic_2D", ("x_ptr", "y_ptr", "z_ptr", "ts0", "ts1", "tile_shape", "tile_id", "offsets"),
          "python/test/asc2/operations/test_memory_ops.py:76-82")
def _memory_dynamic_2d(call: KernelCall) -> None:
    _memory_tile(call, [int(call.args["ts0"]), int(call.args["ts1"])])


@register("kernel_scalar_load_store", ("x_ptr", "y_ptr", "z_ptr", "tensor_shape", "offsets"),
          "python/test/asc2/operations/test_memory_ops.py:85-90")
def _memory_scalar(call: KernelCall) -> None:
    # shape-less loads read one element at `offsets` (memory_ops.py:70-74)
    shape = [int(v) for v in call.consts["tensor_shape"]]
    offsets = kernels.tile_offsets(shape, None, None, call.consts["offsets"])
    kernels.tile_binary(call.args["x_ptr"].reshape(-1), call.args["y_ptr"].reshape(-1), call.args["z_ptr"].reshape(-1),
                        "add", shape, None, offsets, call.stream)


@register("kernel", ("x_ptr", "y_ptr", "tensor_shape", "offsets"),
          "python/test/asc2/operations/test_memory_ops.py:131-137")
def _store_one_element(call: KernelCall) -> None:
    # y[offsets] = x[offsets]: a scalar load stored through a 1-element tile
    shape = [int(v) for v in call.consts["tensor_shape"]]
    offsets = kernels.tile_offsets(shape, None, None, call.consts["offsets"])
    if len(shape) not in (1, 2) or any(o < 0 or o >= d for o, d in zip(offsets, shape)):
        raise ValueError(f"offsets {offsets} outside the tensor {shape}")
    flat = offsets[0] if len(shape) == 1 else offsets[0] * shape[1] + offsets[1]
    x, y = call.args["x_ptr"].reshape(-1), call.args["y_ptr"].reshape(-1)
    kernels.broadcast_rows(x[flat:flat + 1], y[flat:flat + 1], 1, 1, call.stream)


# --------------------------------------------------------------- shape operations (test_shape_ops.py)

@register("kernel", ("x_ptr", "z_ptr", "input_shape", "output_shape", "in_offsets", "out_offsets", "op", "op_param"),
          "python/test/asc2/operations/test_shape_ops.py:47-55")
def _shape_op(call: KernelCall) -> None:
    name = _op_name(call.consts["op"], ("broadcast_to", "reshape", "ravel", "expand_dims", "squeeze"), "shape op")
    in_shape = [int(v) for v in call.consts["input_shape"]]
    out_shape = [int(v) for v in call.consts["output_shape"]]
    _zero_offsets(call.consts["in_offsets"], "in_offsets")
    _zero_offsets(call.consts["out_offsets"], "out_offsets")
    x, z = call.args["x_ptr"].reshape(-1), call.args["z_ptr"].reshape(-1)
    n_in = 1
    for d in in_shape:
        n_in *= d
    n_out = 1
    for d in out_shape:
        n_out *= d
    if name == "broadcast_to":
        # [.., 1, C] -> [.., R, C]: every leading dim of the input is 1 (shape_ops broadcast rules)
        if any(d != 1 for d in in_shape[:-1]) or in_shape[-1] != out_shape[-1]:
            raise NotImplementedError(f"broadcast_to from {in_shape} to {out_shape}: rows of one row only")
        kernels.broadcast_rows(x, z, n_out // out_shape[-1], out_shape[-1], call.stream)
        return
    if n_in != n_out:
        raise ValueError(f"{name}: {in_shape} and {out_shape} hold different element counts")
    kernels.broadcast_rows(x, z, 1, n_out, call.stream)  # a view change: the data are copied as they are


# ------------------------------------------------------------------ atomic ops (test_atomic_ops.py)

@register("kernel", ("x_ptr", "z_ptr", "tensor_shape", "tile_length", "op"),
          "python/test/asc2/operations/test_atomic_ops.py:33-40")
def _atomic_op(call: KernelCall) -> None:
    # block b loads x[b*tile_length : (b+1)*tile_length], adds full_like(.., 10) and combines
    # the tile into z[0:tile_length] with the atomic op
    name = _op_name(call.consts["op"], ("atomic_add", "atomic_max", "atomic_min"), "atomic op")
    size = 1
    for d in call.consts["tensor_shape"]:
        size *= int(d)
    tile_length = int(call.consts["tile_length"])
    if call.grid * tile_length > size:
        raise ValueError(f"{call.grid} blocks of {tile_length} elements read past the {size}-element tensor")
    op = {"atomic_add": "add", "atomic_max": "maximum", "atomic_min": "minimum"}[name]
    kernels.atomic_tiles(call.args["x_ptr"].reshape(-1), call.args["z_ptr"].reshape(-1), op, call.grid, tile_length,
                         10, call.stream)


@register("kernel", ("out_ptr", "shape", "offsets"), "python/test/asc2/operations/test_shape_ops.py:68-72")
def _broadcast_dup(call: KernelCall) -> None:
    # asc2.full([1], 777, dtype).broadcast_to(*shape), stored over the whole tensor
    _zero_offsets(call.consts["offsets"], "offsets")
    n = 1
    for d in call.consts["shape"]:
        n *= int(d)
    kernels.fill(call.args["out_ptr"].reshape(-1), 777, n, call.stream)
