"""Native launchers of the asc1 kernels: python/test/kernels, the tutorials and
python/test/generalization.  asc1 kernels address the Ascend pipeline explicitly
(GlobalTensor views, TQue queues, data_copy, adv.Matmul); what they compute is registered
here by signature, like the asc2 kernels in launchers.py."""
from __future__ import annotations

from typing import List, Tuple

import torch

from . import kernels
from .asc.core import ceildiv
from .launchers import _scalar
from .registry import KernelCall, register


def _block_ranges(n: int, grid: int, block_stride: int, block_cover: int) -> List[Tuple[int, int]]:
    """[start, end) ranges written by asc1 blocks b < grid that each process ``block_cover``
    elements from b * block_stride (TILE_NUM tiles of TILE_LENGTH), clipped at n (the NPU
    copy does not clip).  One range when the blocks tile the data without gaps."""
    if block_stride <= 0 or block_cover < 0:
        raise ValueError(f"invalid block length {block_stride} / elements per block {block_cover}")
    if grid <= 0 or block_cover == 0:
        return []
    if block_cover >= block_stride:
        end = min(n, (grid - 1) * block_stride + block_cover)
        return [(0, end)] if end > 0 else []
    return [(b * block_stride, min(n, b * block_stride + block_cover)) for b in range(grid) if b * block_stride < n]


def _block_add(call: KernelCall, block_stride: int, block_cover: int) -> None:
    """z = x + y over the blocks' ranges (the asc1 vadd bodies)."""
    x, y, z = (call.args[k].reshape(-1) for k in ("x", "y", "z"))
    for s, e in _block_ranges(z.numel(), call.grid, block_stride, block_cover):
        if x.dtype in (torch.float32, torch.float16, torch.bfloat16, torch.int32):
            tile = min(e - s, 1 << 30)
            kernels.vadd(x[s:e], y[s:e], z[s:e], e - s, tile, ceildiv(e - s, tile), 1, call.stream)
        else:
            kernels.binary(x[s:e], y[s:e], z[s:e], "add", stream=call.stream)


@register("vadd_kernel", ("x", "y", "z", "BLOCK_LENGTH", "BUFFER_NUM", "TILE_LENGTH", "TILE_NUM"),
          "python/test/kernels/test_vadd.py:16-35")
def _asc1_vadd(call: KernelCall) -> None:
    # TILE_NUM tiles of TILE_LENGTH from each block's start (BUFFER_NUM only sizes the queues)
    _block_add(call, int(call.consts["BLOCK_LENGTH"]), int(call.consts["TILE_NUM"]) * int(call.consts["TILE_LENGTH"]))


@register("vadd_kernel", ("x", "y", "z", "block_length"), "python/tutorials/01_add/add.py:29-70")
def _tutorial_add(call: KernelCall) -> None:
    # TILE_NUM * BUFFER_NUM = 8 * 2 tiles of block_length // 16 elements (add.py:21-23, 40)
    bl = int(call.args["block_length"])
    _block_add(call, bl, 16 * (bl // 16))


@register("vadd_kernel", ("x", "y", "z", "block_length", "tile_length"),
          "python/tutorials/02_add_framework/add_framework.py:29-80")
def _tutorial_add_framework(call: KernelCall) -> None:
    # TILE_NUM * BUFFER_NUM = 8 * 2 tiles of tile_length elements (add_framework.py:21-23, 47-50)
    _block_add(call, int(call.args["block_length"]), 16 * int(call.consts["tile_length"]))


def _matmul_instances(call: KernelCall) -> int:
    """Kernel instances a launch of ``grid`` blocks runs for an asc1 Matmul kernel: a mixed
    cube + vector kernel runs as MIX_AIC_1_2, one cube core and two vector cores per block,
    and get_block_idx counts the vector cores; with matmul_cube_only it runs as AIC_ONLY,
    one instance per block (python/asc/runtime/compiler.py:291-299).  An explicit
    kernel_type option decides instead."""
    options = call.extra.get("options", {})
    kernel_type = options.get("kernel_type")
    if kernel_type is not None:
        return call.grid * (2 if getattr(kernel_type, "name", str(kernel_type)) == "MIX_AIC_1_2" else 1)
    return call.grid * (1 if options.get("matmul_cube_only") else 2)


def _asc1_matmul(call: KernelCall, tiles_m: int, tiles_n: int, bias, alpha=None, used_core_num=None) -> None:
    """c = act(a @ b + bias) over the whole output, for asc1 kernels whose instance i computes
    one single_core_m x single_core_n tile when i < used_core_num: the launch must cover
    every tile (min(instances, used_core_num) >= the tile count), as the reference's
    launches do."""
    a, b, c = call.args["a"], call.args["b"], call.args["c"]
    if a.dim() != 2 or b.dim() != 2 or c.dim() != 2:
        raise ValueError("a, b and c must be 2-D")
    blocks = _matmul_instances(call)
    if used_core_num is not None:
        blocks = min(blocks, int(used_core_num))
    if blocks < tiles_m * tiles_n:
        raise NotImplementedError(f"{blocks} computing blocks for {tiles_m * tiles_n} output tiles: only launches "
                                  "that cover every tile are provided")
    kernels.matmul(a, b, c, bias=None if bias is None else bias.reshape(-1),
                   leaky_alpha=None if alpha is None else _scalar(alpha), stream=call.stream)


def _tiles_of(call: KernelCall):
    t = call.args["tiling"]
    M, N = call.args["a"].shape[0], call.args["b"].shape[1]
    return ceildiv(M, int(t.single_core_m)), ceildiv(N, int(t.single_core_n))


@register("matmul_kernel", ("a", "b", "c", "alpha", "tiling", "bias", "workspace"),
          "python/test/kernels/test_matmul.py:17-79")
def _asc1_matmul_bias(call: KernelCall) -> None:
    """c = leaky_relu(a @ b + bias, alpha), fp32 accumulation.  Block b computes the
    single_core_m x single_core_n tile of calc_offsets (test_matmul.py:67-79); a launch
    must cover every tile, as the test's used_core_num does."""
    _asc1_matmul(call, *_tiles_of(call), call.args["bias"], call.args["alpha"])


@register("matmul_kernel", ("a", "b", "c", "alpha", "size_m", "size_k", "size_n", "size_base_m", "size_base_k",
                            "size_base_n", "size_single_m", "size_single_k", "size_single_n", "used_core_num",
                            "workspace"),
          "python/test/kernels/test_matmul_torch.py:20-85")
def _asc1_matmul_torch(call: KernelCall) -> None:
    """c = leaky_relu(a @ b, alpha), fp32 accumulation (the same kernel without bias, tiling
    given as ConstExprs)."""
    k = call.consts
    if (int(k["size_m"]), int(k["size_k"])) != tuple(call.args["a"].shape) or \
            (int(k["size_k"]), int(k["size_n"])) != tuple(call.args["b"].shape):
        raise ValueError(f"size_m/size_k/size_n ({k['size_m']}, {k['size_k']}, {k['size_n']}) do not match a "
                         f"{tuple(call.args['a'].shape)} and b {tuple(call.args['b'].shape)}")
    _asc1_matmul(call, ceildiv(int(k["size_m"]), int(k["size_single_m"])),
                 ceildiv(int(k["size_n"]), int(k["size_single_n"])), None, call.args["alpha"],
                 int(k["used_core_num"]))


@register("matmul_kernel", ("a", "b", "c", "tiling", "workspace"),
          "python/tutorials/03_matmul_mix/matmul_mix.py:31-77; python/test/generalization/adv/"
          "test_matmul_iterate_all.py:23-47 and test_matmul_iterate_batch.py:28-51")
def _matmul_tiling(call: KernelCall) -> None:
    """Matmul.iterate_all without bias (the tutorial and iterate_all test): c = a @ b with fp32
    accumulation and output, or int8 a, b -> exact int32 c; instances below
    tiling.used_core_num compute one tile each (matmul_mix.py:47-52).  A tiling that carries
    a batch (batch_num and the A/B layouts, as test_matmul_iterate_batch.py's generate_tiling
    sets them) selects that test's Matmul.iterate_batch body instead."""
    t = call.args["tiling"]
    if int(getattr(t, "batch_num", -1)) > 0:
        _matmul_batched(call, t)
        return
    a, b, c = call.args["a"], call.args["b"], call.args["c"]
    if a.dtype == torch.int8:
        tiles_m, tiles_n = _tiles_of(call)
        if min(_matmul_instances(call), int(t.used_core_num)) < tiles_m * tiles_n:
            raise NotImplementedError("the launch does not cover every tile")
        kernels.matmul_i8(a, b, c, stream=call.stream)
        return
    _asc1_matmul(call, *_tiles_of(call), None, None, t.used_core_num)


def _matmul_batched(call: KernelCall, t) -> None:
    """Matmul.iterate_batch (test_matmul_iterate_batch.py:47-49, golden :116-141): A holds
    batch_a [m, k] matrices stacked by rows, B batch_b [k, n], C batch_num [m, n]; output
    matrix i is A[i // (batch / batch_a)] @ B[i // (batch / batch_b)] in fp32."""
    a, b, c = (call.args[k].reshape(-1) for k in ("a", "b", "c"))
    batch = int(t.batch_num)
    ba, m, k = int(t.a_layout_info_b), int(t.a_layout_info_s), int(t.a_layout_info_d)
    bb, k2, n = int(t.b_layout_info_b), int(t.b_layout_info_s), int(t.b_layout_info_d)
    if min(ba, bb, m, k, n) <= 0 or k2 != k or batch % ba or batch % bb:
        raise ValueError(f"inconsistent batch layout: batch {batch}, A {ba}x[{m},{k}], B {bb}x[{k2},{n}]")
    if a.numel() < ba * m * k or b.numel() < bb * k * n or c.numel() < batch * m * n:
        raise ValueError("a, b or c holds fewer elements than the batch layout describes")
    for i in range(batch):
        ia, ib = i // (batch // ba), i // (batch // bb)
        kernels.matmul(a[ia * m * k:(ia + 1) * m * k].view(m, k), b[ib * k * n:(ib + 1) * k * n].view(k, n),
                       c[i * m * n:(i + 1) * m * n].view(m, n), stream=call.stream)


@register("matmul_kernel", ("a", "b", "c", "bias", "tiling", "workspace"),
          "python/tutorials/04_matmul_cube_only/matmul_cube_only.py:32-85")
def _tutorial_matmul_cube_only(call: KernelCall) -> None:
    """c = a @ b (+ bias when tiling.is_bias), fp32 accumulation and output
    (matmul_cube_only.py:53-60)."""
    t = call.args["tiling"]
    _asc1_matmul(call, *_tiles_of(call), call.args["bias"] if int(getattr(t, "is_bias", 0)) else None, None,
                 t.used_core_num)


# ------------------------------------------- asc1 generalization tests (python/test/generalization/basic)
# Each kernel body processes tile_num tiles of tile_length from b * block_length (block b).

def _gen_ranges(call: KernelCall, out: torch.Tensor):
    c = call.consts
    return _block_ranges(out.numel(), call.grid, int(c["block_length"]), int(c["tile_num"]) * int(c["tile_length"]))


@register("vadd_kernel", ("x", "y", "z", "block_length", "buffer_num", "tile_length", "tile_num"),
          "python/test/generalization/basic/test_vadd.py:21-70 (also test_vadd_bits.py, test_vadd_l0.py, "
          "test_vadd_sw.py, whose one-repeat adds cover their 64-element tiles)")
def _gen_vadd(call: KernelCall) -> None:
    _block_add(call, int(call.consts["block_length"]), int(call.consts["tile_num"]) * int(call.consts["tile_length"]))


@register("vadds_kernel", ("x", "scalar", "z", "block_length", "buffer_num", "tile_length", "tile_num"),
          "python/test/generalization/basic/test_vadds.py:21-61")
def _gen_vadds(call: KernelCall) -> None:
    # asc.adds: z = x + scalar, the scalar in x's element type
    x, z = call.args["x"].reshape(-1), call.args["z"].reshape(-1)
    for s, e in _gen_ranges(call, z):
        kernels.binary(x[s:e], call.args["scalar"], z[s:e], "add", stream=call.stream)


@register("vsqrt_kernel", ("x", "z", "block_length", "buffer_num", "tile_length", "tile_num"),
          "python/test/generalization/basic/test_vsqrt.py:21-61")
def _gen_vsqrt(call: KernelCall) -> None:
    x, z = call.args["x"].reshape(-1), call.args["z"].reshape(-1)
    for s, e in _gen_ranges(call, z):
        kernels.unary(x[s:e], z[s:e], "sqrt", stream=call.stream)


@register("duplicate_kernel", ("scalar", "z", "block_length", "buffer_num", "tile_length", "tile_num"),
          "python/test/generalization/basic/test_duplicate.py:21-46")
def _gen_duplicate(call: KernelCall) -> None:
    # asc.duplicate: every element takes the scalar, in z's element type
    z = call.args["z"].reshape(-1)
    scalar = call.args["scalar"]
    scalar = scalar.item() if isinstance(scalar, torch.Tensor) else scalar
    for s, e in _gen_ranges(call, z):
        kernels.fill(z[s:e], scalar, stream=call.stream)


@register("axpy_kernel", ("x", "y", "z", "scalar", "block_length", "buffer_num", "tile_length", "tile_num"),
          "python/test/generalization/basic/test_axpy.py:21-76")
def _gen_axpy(call: KernelCall) -> None:
    # asc.axpy(z_local, y_local, scalar): z = y * scalar + z (x is loaded and unused)
    y, z = call.args["y"].reshape(-1), call.args["z"].reshape(-1)
    for s, e in _gen_ranges(call, z):
        kernels.axpy(y[s:e], z[s:e], _scalar(call.args["scalar"]), stream=call.stream)


@register("copy_kernel", ("x", "z", "data_size"), "python/test/generalization/basic/test_copy.py:21-67")
def _gen_copy(call: KernelCall) -> None:
    """z[0:data_size] = 0, then asc.copy with mask 64, 4 repeats of 8 blocks (256 bytes):
    repeat r copies 64 elements from r * (256 / element size), for the repeats that fit
    in data_size (the test's golden, test_copy.py:107-122)."""
    x, z = call.args["x"].reshape(-1), call.args["z"].reshape(-1)
    n = int(call.consts["data_size"])
    if n > min(x.numel(), z.numel()):
        raise ValueError(f"data_size {n} exceeds the tensors ({x.numel()}, {z.numel()} elements)")
    kernels.fill(z, 0, n, call.stream)
    stride = 256 // z.element_size()
    for r in range(4):
        s = r * stride
        if s + 64 > n:
            break
        kernels.broadcast_rows(x[s:s + 64], z[s:s + 64], 1, 64, call.stream)


@register("transpose_kernel", ("x", "z", "block_length", "buffer_num", "tile_length", "tile_num"),
          "python/test/generalization/basic/test_transpose.py:21-67")
def _gen_transpose(call: KernelCall) -> None:
    """asc.transpose of each 16 x 16 tile of 2-byte elements (tile_length 256)."""
    x, z = call.args["x"].reshape(-1), call.args["z"].reshape(-1)
    if int(call.consts["tile_length"]) != 256 or z.element_size() != 2:
        raise NotImplementedError("asc.transpose takes 16x16 tiles of 2-byte elements (tile_length 256)")
    if int(call.consts["block_length"]) % 256:
        raise NotImplementedError("block_length must be a multiple of 256 so that every tile is a whole 16x16 tile")
    for s, e in _gen_ranges(call, z):
        if (e - s) % 256:
            raise ValueError(f"elements [{s}, {e}) do not hold whole 16x16 tiles")
        kernels.transpose_batched(x[s:e], z[s:e], (e - s) // 256, 16, 16, call.stream)



@register("quant_kernel", ("src_gm", "dst_gm", "size", "tmp_min_bytes", "use_config"),
          "python/test/generalization/adv/test_quant.py:22-57")
def _gen_quant(call: KernelCall) -> None:
    """asc.adv.quant with the body's scale 2.0 and offset 0.9 on the first ``size`` elements;
    the temporary buffer size and the QuantConfig do not change the result."""
    n = int(call.args["size"])
    kernels.quant_i8(call.args["src_gm"].reshape(-1), call.args["dst_gm"].reshape(-1), 2.0, 0.9, n, call.stream)


# ------------------------------------------------------- tutorial 05 (matmul + bias + leaky relu)

@register("matmul_leakyrelu_kernel", ("a", "b", "c", "bias", "alpha", "tiling", "workspace"),
          "python/tutorials/05_matmul_leakyrelu/matmul_leakyrelu.py:27-70")
def _matmul_leakyrelu(call: KernelCall) -> None:
    """c = leaky_relu(a @ b + bias, alpha) in fp32 (the tutorial's Matmul + set_bias + asc.leaky_relu).
    Shapes come from the tensors: a [M, K], b [K, N], c [M, N], bias N elements.  The
    MI355X kernel picks its own tiles; a tiling that carries a per-core split
    (single_core_m / single_core_n, as asc.lib.host fills it) must describe a launch that
    covers the whole output.  The workspace is not used."""
    a, b, c, bias = call.args["a"], call.args["b"], call.args["c"], call.args["bias"]
    if a.dim() != 2 or b.dim() != 2 or c.dim() != 2:
        raise ValueError("a, b and c must be 2-D")
    t = call.args["tiling"]
    if hasattr(t, "single_core_m") and hasattr(t, "single_core_n"):
        # a tiling with a split (asc.lib.host): the launch must cover every tile
        _asc1_matmul(call, *_tiles_of(call), bias, call.args["alpha"], getattr(t, "used_core_num", None))
        return
    kernels.matmul(a, b, c, bias=bias.reshape(-1), leaky_alpha=_scalar(call.args["alpha"]), stream=call.stream)
