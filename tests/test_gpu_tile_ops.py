"""Element-wise asc2 tile operations on the GPU: the generic kernels of the
reference's operation tests (python/test/asc2/operations/test_unary_ops.py,
test_binary_ops.py, test_where.py).

First the reference tests themselves: the same kernel signatures, parametrisation,
input recipes (size 32) and assertions (allclose atol 1e-3 for float32,
torch.equal otherwise; assert_close for where).  Then the kernel API at a
million elements against the oracle, with edge values (signed zeros, NaN,
infinities, integer extremes): bit-exact for binary and where (NaN compared as
NaN), within a few float32 ulps (rtol 1e-6, atol 1e-7) for the libm unary ops."""
import numpy as np
import pytest
import torch

import asc
import asc2
from oracle import asc2_oracle as O
from pyasc_amd import kernels

pytestmark = pytest.mark.gpu

VV, VS, SV = "VV", "VS", "SV"


@asc2.jit(always_compile=True)
def kernel(x_ptr, y_ptr, z_ptr, block_length: asc.ConstExpr, fmt: asc.ConstExpr, op: asc.ConstExpr) -> None:
    ...  # declaration: binds the registered native kernel by signature


# test_binary_ops.py:11-20
BINARY_OPS = [
    (asc2.add, torch.add, [VV, VS, SV], [torch.bfloat16, torch.float32, torch.int32]),
    (asc2.div, torch.div, [VV, VS, SV], [torch.float32]),
    (asc2.mul, torch.mul, [VV, VS, SV], [torch.bfloat16, torch.float32, torch.int32]),
    (asc2.sub, torch.sub, [VV, VS, SV], [torch.bfloat16, torch.float32, torch.int32]),
    (asc2.left_shift, torch.bitwise_left_shift, [VS], [torch.int32]),
    (asc2.right_shift, torch.bitwise_right_shift, [VS], [torch.int32]),
    (asc2.maximum, torch.maximum, [VV, VS, SV], [torch.bfloat16, torch.float32, torch.int32]),
    (asc2.minimum, torch.minimum, [VV, VS, SV], [torch.bfloat16, torch.float32, torch.int32]),
]


@pytest.mark.parametrize("asc_op, torch_op, fmt, dtype", [(a, t, f, d) for a, t, fmts, dtypes in BINARY_OPS
                                                          for f in fmts for d in dtypes],
                         ids=lambda v: getattr(v, "__name__", str(v)))
def test_binary_reference_cases(device, asc_op, torch_op, fmt, dtype):
    # test_binary_ops.py:46-87
    size = 32

    def create_input(is_vector):
        if is_vector:
            if dtype.is_floating_point:
                return torch.randn((size,), dtype=dtype).clamp(1, 100)
            return torch.randint(1, 100, (size,), dtype=dtype)
        return torch.tensor(2, dtype=dtype)

    x = create_input(fmt in (VV, VS))
    y = create_input(fmt in (VV, SV))
    z = torch.zeros(size, dtype=dtype)
    kernel[1](x, y, z, size, fmt, asc_op)
    if dtype == torch.float32:
        assert torch.allclose(z, torch_op(x, y), atol=1e-3)
    else:
        assert torch.equal(z, torch_op(x, y))


@asc2.jit(always_compile=True)
def unary_kernel(x_ptr: asc.GlobalAddress, z_ptr: asc.GlobalAddress, block_length: asc.ConstExpr,
                 op: asc.ConstExpr) -> None:
    ...  # declaration: binds the registered native kernel by signature


# the reference names this kernel `kernel` too (test_unary_ops.py:35); dispatch is by
# name and parameter names, so the same registered entry serves it under either name
unary_kernel.fn_name = "kernel"

UNARY_OPS = [(asc2.abs, torch.abs), (asc2.ceil, torch.ceil), (asc2.cos, torch.cos), (asc2.cosh, torch.cosh),
             (asc2.erf, torch.erf), (asc2.exp, torch.exp), (asc2.exp2, torch.exp2), (asc2.floor, torch.floor),
             (asc2.log, torch.log), (asc2.negative, torch.neg), (asc2.relu, torch.relu), (asc2.rsqrt, torch.rsqrt),
             (asc2.sin, torch.sin), (asc2.sinh, torch.sinh), (asc2.sqrt, torch.sqrt), (asc2.tan, torch.tan),
             (asc2.tanh, torch.tanh)]  # test_unary_ops.py:10-28


@pytest.mark.parametrize("asc_op, torch_op", UNARY_OPS, ids=lambda v: getattr(v, "__name__", str(v)))
def test_unary_reference_cases(device, asc_op, torch_op):
    # test_unary_ops.py:43-69
    x = torch.randn((32,), dtype=torch.float32).clamp(1, 100)
    z = torch.zeros(32, dtype=torch.float32)
    unary_kernel[1](x, z, 32, asc_op)
    assert torch.allclose(z, torch_op(x), atol=1e-3)


@asc2.jit(always_compile=True)
def where_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, z_ptr: asc.GlobalAddress, op: asc.ConstExpr):
    ...  # declaration: binds the registered native kernel by signature


@asc2.jit(always_compile=True)
def where_scalar_kernel(x_ptr: asc.GlobalAddress, scalar, z_ptr: asc.GlobalAddress, op: asc.ConstExpr):
    ...  # declaration: binds the registered native kernel by signature


WHERE_DTYPES = [torch.float16, torch.bfloat16, torch.float32, torch.int16, torch.int32]
COMPARES = [(asc2.equal, torch.eq), (asc2.not_equal, torch.ne), (asc2.greater, torch.gt),
            (asc2.greater_equal, torch.ge), (asc2.less, torch.lt), (asc2.less_equal, torch.le)]


def _where_input(dtype):
    # test_where.py:11-15
    if dtype.is_floating_point:
        return torch.rand(32, dtype=dtype)
    return torch.randint(-100, 100, (32,), dtype=dtype)


@pytest.mark.parametrize("dtype", WHERE_DTYPES, ids=str)
@pytest.mark.parametrize("asc_op, torch_op", COMPARES, ids=lambda v: getattr(v, "__name__", str(v)))
def test_where_reference_cases(device, asc_op, torch_op, dtype):
    # test_where.py:39-46 and 70-77
    x, y = _where_input(dtype), _where_input(dtype)
    result = torch.zeros_like(x)
    where_kernel[1](x, y, result, asc_op)
    torch.testing.assert_close(result, torch.where(torch_op(x, y), x, y))
    s = torch.tensor(0 if dtype.is_signed else 0.5, dtype=dtype)
    result = torch.zeros_like(x)
    where_scalar_kernel[1](x, s, result, asc_op)
    torch.testing.assert_close(result, torch.where(torch_op(x, s), torch.tensor(0, dtype=dtype),
                                                   torch.tensor(1, dtype=dtype)))


# ------------------------------------------------------------- kernel API at size, against the oracle

N = (1 << 20) + 37
_EDGE_F = [0.0, -0.0, 1.0, -1.0, float("nan"), float("inf"), float("-inf"), 3.5, -2.25, 65504.0, 1e-8, 1e30]


def _float_data(dtype, seed):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(N, generator=g) * 8
    v[:len(_EDGE_F) ** 2] = torch.tensor(_EDGE_F * len(_EDGE_F)) if seed % 2 else \
        torch.tensor([e for e in _EDGE_F for _ in _EDGE_F])
    return v.to(dtype)


def _int_data(dtype, seed):
    info = torch.iinfo(dtype)
    g = torch.Generator().manual_seed(seed)
    v = torch.randint(info.min, info.max, (N,), generator=g, dtype=torch.int64)
    edge = [0, 1, -1, info.max, info.min, 7, -7]
    v[:len(edge) ** 2] = torch.tensor(edge * len(edge)) if seed % 2 else torch.tensor([e for e in edge for _ in edge])
    return v.to(dtype)


def _np(t: torch.Tensor, dtype: str) -> np.ndarray:
    return t.view(torch.int16).numpy().view(np.uint16) if dtype == "bfloat16" else t.numpy()


def _assert_same(got: torch.Tensor, expected: np.ndarray, dtype: str):
    g = _np(got, dtype)
    if dtype in ("int32", "int16"):
        np.testing.assert_array_equal(g, expected)
        return
    as_f = (lambda a: O.bf16_bits_to_f32(a)) if dtype == "bfloat16" else (lambda a: a.astype(np.float32))
    nan = np.isnan(as_f(expected))
    assert np.array_equal(np.isnan(as_f(g)), nan)
    view = np.uint32 if dtype == "float32" else np.uint16
    np.testing.assert_array_equal(g.view(view)[~nan], expected.view(view)[~nan])


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16", "int32", "int16"])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "maximum", "minimum"])
def test_binary_vs_oracle(device, op, dtype):
    td = getattr(torch, dtype)
    make = _float_data if td.is_floating_point else _int_data
    x, y = make(td, 1), make(td, 2)
    out = torch.empty(N, dtype=td, device=device)
    kernels.binary(x.to(device), y.to(device), out, op)
    torch.cuda.synchronize()
    _assert_same(out.cpu(), O.binary_elements(_np(x, dtype), _np(y, dtype), op, dtype), dtype)
    # scalar operands on either side (VS and SV), converted to the tile's dtype
    s = torch.tensor(-2.5 if td.is_floating_point else -3, dtype=td)
    s_np = _np(s.reshape(1), dtype)
    for mode, (a, b) in (("VS", (x, s)), ("SV", (s, x))):
        kernels.binary(a.to(device) if a.dim() else a, b.to(device) if b.dim() else b, out, op)
        torch.cuda.synchronize()
        full = np.repeat(s_np, N)
        expected = O.binary_elements(_np(x, dtype), full, op, dtype) if mode == "VS" else \
            O.binary_elements(full, _np(x, dtype), op, dtype)
        _assert_same(out.cpu(), expected, dtype)


@pytest.mark.parametrize("dtype", ["int32", "int16"])
def test_shifts_vs_oracle(device, dtype):
    td = getattr(torch, dtype)
    x = _int_data(td, 3)
    out = torch.empty(N, dtype=td, device=device)
    for op in ("left_shift", "right_shift"):
        for amount in (0, 1, 7, torch.iinfo(td).bits - 1):
            kernels.binary(x.to(device), amount, out, op)
            torch.cuda.synchronize()
            expected = O.binary_elements(x.numpy(), np.full(N, amount, dtype=x.numpy().dtype), op, dtype)
            np.testing.assert_array_equal(out.cpu().numpy(), expected)


@pytest.mark.parametrize("op", kernels.UNARY_OPS)
def test_unary_vs_oracle(device, op):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(N, generator=g) * 6
    if op in ("log", "log2", "rsqrt", "sqrt"):
        x = x.abs() + 1e-6
    if op in ("cosh", "sinh", "exp", "exp2"):
        x = x.clamp(-60, 60)
    x[:6] = torch.tensor([-0.0, 0.0, float("nan"), 1.0, 0.5, -0.5])
    out = torch.empty(N, device=device)
    kernels.unary_f32(x.to(device), out, op)
    torch.cuda.synchronize()
    expected = O.unary_f32(x.numpy(), op)
    np.testing.assert_allclose(out.cpu().numpy(), expected, rtol=1e-6, atol=1e-7, equal_nan=True)
    if op in ("abs", "ceil", "floor", "negative", "relu", "sqrt"):  # exactly rounded: bit-exact
        got = out.cpu().numpy()
        keep = ~np.isnan(expected)
        np.testing.assert_array_equal(got.view(np.uint32)[keep], expected.view(np.uint32)[keep])


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16", "int32", "int16"])
@pytest.mark.parametrize("cmp", kernels.COMPARE_OPS)
def test_where_vs_oracle(device, cmp, dtype):
    td = getattr(torch, dtype)
    make = _float_data if td.is_floating_point else _int_data
    x, y = make(td, 1), make(td, 2)
    y[-1000:] = x[-1000:]  # ties
    out = torch.empty(N, dtype=td, device=device)
    kernels.where_compare(x.to(device), y.to(device), out, cmp)
    torch.cuda.synchronize()
    _assert_same(out.cpu(), O.where_compare(_np(x, dtype), _np(y, dtype), cmp, dtype), dtype)
    s = torch.tensor(1 if not td.is_floating_point else 0.75, dtype=td)
    kernels.where_compare(x.to(device), s, out, cmp, true_value=0, false_value=1)
    torch.cuda.synchronize()
    _assert_same(out.cpu(), O.where_scalar(_np(x, dtype), s.item(), cmp, dtype, 0, 1), dtype)


def test_tile_op_argument_errors(device):
    x = torch.zeros(64, dtype=torch.int32, device=device)
    f = torch.zeros(64, device=device)
    with pytest.raises(TypeError):
        kernels.binary(x, x, x, "left_shift")  # shifts take a scalar amount
    with pytest.raises(ValueError, match="outside"):
        kernels.binary(x, 32, x, "left_shift")  # amount outside [0, 32), refused on the host
    with pytest.raises(TypeError):
        kernels.binary(f, x, f, "add")  # mixed tensor dtypes
    with pytest.raises(ValueError):
        kernels.unary_f32(f, f, "not_an_op")
    with pytest.raises(ValueError):
        kernels.binary(f, f, torch.zeros(8, device=device), "add")  # output too short


# --------------------------------------------- tile load / add / store (test_memory_ops.py)

@asc2.jit(always_compile=True)
def kernel_static(x_ptr, y_ptr, z_ptr, tensor_shape: asc.ConstExpr, tile_shape: asc.ConstExpr, tile_id: asc.ConstExpr,
                  offsets: asc.ConstExpr) -> None:
    ...  # declaration: binds the registered native kernel by signature


@asc2.jit(always_compile=True)
def kernel_dynamic_1D(x_ptr, y_ptr, z_ptr, ts0, tile_shape: asc.ConstExpr, tile_id: asc.ConstExpr,
                      offsets: asc.ConstExpr) -> None:
    ...  # declaration: binds the registered native kernel by signature


@asc2.jit(always_compile=True)
def kernel_dynamic_2D(x_ptr, y_ptr, z_ptr, ts0, ts1, tile_shape: asc.ConstExpr, tile_id: asc.ConstExpr,
                      offsets: asc.ConstExpr) -> None:
    ...  # declaration: binds the registered native kernel by signature


@asc2.jit(always_compile=True)
def kernel_scalar_load_store(x_ptr, y_ptr, z_ptr, tensor_shape: asc.ConstExpr, offsets: asc.ConstExpr) -> None:
    ...  # declaration: binds the registered native kernel by signature


MEMORY_TESTS = [  # test_memory_ops.py:8-48: dim, tensor_shape, tile_shape, tile_id, offsets, is_static
    (1, [64], [16], [0], None, True), (1, [64], [16], [3], None, True), (2, [128, 128], [32, 32], [0, 0], None, True),
    (2, [128, 128], [32, 32], [3, 3], None, True), (2, [1024, 512], [128, 64], [1, 2], None, True),
    (1, [37], [8], [3], None, True), (2, [123, 456], [13, 16], [2, 5], None, True),
    (1, [64], [16], None, [0], True), (1, [64], [16], None, [48], True), (2, [128, 128], [32, 32], None, [0, 0], True),
    (2, [128, 128], [32, 32], None, [96, 64], True), (2, [1024, 512], [128, 64], None, [256, 128], True),
    (1, [53], [16], None, [22], True), (2, [257, 511], [19, 24], None, [40, 64], True),
    (1, [32], [8], [1], None, False), (1, [32], [8], [3], None, False), (2, [16, 2048], [4, 512], [0, 3], None, False),
    (2, [16, 2048], [8, 256], [1, 7], None, False), (2, [512, 512], [64, 64], [4, 4], None, False),
    (1, [99], [16], [5], None, False), (2, [1000, 1000], [33, 40], [1, 1], None, False),
    (1, [32], [8], None, [16], False), (1, [32], [8], None, [24], False),
    (2, [16, 2048], [4, 512], None, [8, 1024], False), (2, [16, 2048], [12, 1024], None, [4, 0], False),
    (2, [512, 512], [64, 64], None, [128, 256], False), (1, [77], [24], None, [48], False),
    (2, [150, 300], [21, 40], None, [10, 20], False),
    (1, [32], None, None, [0], True), (2, [32, 32], None, None, [0, 0], True), (1, [1024], None, None, [0], True),
    (2, [512, 512], None, None, [0, 0], True),
]


@pytest.mark.parametrize("dim, tensor_shape, tile_shape, tile_id, offsets, is_static", MEMORY_TESTS, ids=str)
def test_memory_reference_cases(device, dim, tensor_shape, tile_shape, tile_id, offsets, is_static):
    # test_memory_ops.py:95-114
    x, y = [torch.randn(tensor_shape) for _ in range(2)]
    z = torch.zeros(tensor_shape, dtype=torch.float32)
    if is_static:
        if tile_shape is None:
            kernel_scalar_load_store[1](x, y, z, tensor_shape, offsets)
        else:
            kernel_static[1](x, y, z, tensor_shape, tile_shape, tile_id, offsets)
    elif dim == 1:
        kernel_dynamic_1D[1](x, y, z, tensor_shape[0], tile_shape, tile_id, offsets)
    else:
        kernel_dynamic_2D[1](x, y, z, tensor_shape[0], tensor_shape[1], tile_shape, tile_id, offsets)
    actual = [i * s for i, s in zip(tile_id, tile_shape)] if tile_id is not None else offsets
    slices = tuple(slice(o, o + s) for o, s in zip(actual, tile_shape)) if tile_shape is not None else tuple(actual)
    z_expected = torch.zeros_like(z)
    z_expected[slices] = x[slices] + y[slices]
    torch.testing.assert_close(z, z_expected, atol=1e-3, rtol=1e-3)


@asc2.jit(always_compile=True)
def store_1elem_kernel(x_ptr, y_ptr, tensor_shape: asc.ConstExpr, offsets: asc.ConstExpr):
    ...  # declaration: binds the registered native kernel by signature


store_1elem_kernel.fn_name = "kernel"  # defined as `kernel` inside the reference test (test_memory_ops.py:131)


@pytest.mark.parametrize("tensor_shape, offsets", [((16,), (0,)), ((16,), (7,)), ((16, 16), (0, 0)),
                                                   ((16, 16), (7, 7))], ids=str)
def test_store_1elem_reference_cases(device, tensor_shape, offsets):
    # test_memory_ops.py:117-143
    x = torch.randn(tensor_shape, dtype=torch.float32)
    y = torch.zeros_like(x)
    store_1elem_kernel[1](x, y, tensor_shape, offsets)
    y_ref = torch.zeros_like(x)
    y_ref[offsets] = x[offsets]
    torch.testing.assert_close(y, y_ref)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "int32", "float16"])
@pytest.mark.parametrize("shape, tile, offsets", [([4096, 4096], [1000, 3000], [3500, 2000]),
                                                  ([1, 3_000_001], [1, 2_000_000], [0, 1_500_000]),
                                                  ([777, 333], [64, 64], [0, 300])])
def test_tile_add_vs_oracle(device, dtype, shape, tile, offsets):
    # large tiles that run past the tensor edge: the store clips
    td = getattr(torch, dtype)
    make = _float_data if td.is_floating_point else _int_data
    n = shape[0] * shape[1]
    x, y = make(td, 1)[:n].repeat(1 + n // N)[:n], make(td, 2)[:n].repeat(1 + n // N)[:n]
    z = torch.zeros(n, dtype=td)
    zd = z.to(device)
    kernels.tile_binary(x.to(device), y.to(device), zd, "add", shape, tile, offsets)
    torch.cuda.synchronize()
    expected = O.tile_binary(_np(x, dtype).reshape(shape), _np(y, dtype).reshape(shape), _np(z, dtype).reshape(shape),
                             "add", tile, offsets, dtype)
    _assert_same(zd.cpu(), expected.reshape(-1), dtype)


# ---------------------------------------------------------------------- shape ops (test_shape_ops.py)

@asc2.jit(always_compile=True)
def shape_kernel(x_ptr, z_ptr, input_shape: asc.ConstExpr, output_shape: asc.ConstExpr, in_offsets: asc.ConstExpr,
                 out_offsets: asc.ConstExpr, op: asc.ConstExpr, op_param: asc.ConstExpr) -> None:
    ...  # declaration: binds the registered native kernel by signature


shape_kernel.fn_name = "kernel"  # defined as `kernel` inside the reference test (test_shape_ops.py:47)

SHAPE_OPS = [  # test_shape_ops.py:8-16
    (asc2.broadcast_to, torch.broadcast_to, [4, 32], [1, 32]), (asc2.broadcast_to, torch.broadcast_to, [50, 32], [1, 32]),
    (asc2.reshape, torch.reshape, [64], [2, 32]), (asc2.reshape, torch.reshape, [4, 16], [64]),
    (asc2.ravel, torch.ravel, [], [2, 32]), (asc2.expand_dims, torch.unsqueeze, [0], [32]),
    (asc2.squeeze, torch.squeeze, [0], [1, 32]),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.int32], ids=str)
@pytest.mark.parametrize("asc_op, torch_op, args, shape", SHAPE_OPS, ids=lambda v: getattr(v, "__name__", str(v)))
def test_shape_reference_cases(device, asc_op, torch_op, args, shape, dtype):
    # test_shape_ops.py:25-55
    def create_input(tensor_shape):
        if dtype.is_floating_point:
            return torch.randn(tensor_shape, dtype=dtype).clamp(1, 100)
        return torch.randint(1, 100, tensor_shape, dtype=dtype)

    x = create_input(shape)
    if asc_op in (asc2.expand_dims, asc2.squeeze):
        ref_z = torch_op(x, dim=args[0])
    elif not args:
        ref_z = torch_op(x)
    else:
        ref_z = torch_op(x, args)
    z = create_input(ref_z.shape)
    in_offsets = (0,) * len(x.shape)
    out_offsets = (0,) * len(ref_z.shape)
    shape_kernel[1](x, z, x.shape, ref_z.shape, in_offsets, out_offsets, asc_op, args)
    torch.testing.assert_close(z, ref_z, atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("elem", [torch.int8, torch.float16, torch.float32, torch.float64])
def test_broadcast_rows_vs_oracle(device, elem):
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(1, 4099, generator=g) * 50).to(elem)
    z = torch.zeros(2000, 4099, dtype=elem, device=device)
    kernels.broadcast_rows(x.reshape(-1).to(device), z.reshape(-1), 2000, 4099)
    torch.cuda.synchronize()
    assert torch.equal(z.cpu(), torch.from_numpy(O.broadcast_rows(x.numpy(), 2000, 4099)))


# ---------------------------------------------------------------------- atomic ops (test_atomic_ops.py)

@asc2.jit(always_compile=True)
def atomic_kernel(x_ptr: asc.GlobalAddress, z_ptr: asc.GlobalAddress, tensor_shape: asc.ConstExpr,
                  tile_length: asc.ConstExpr, op: asc.ConstExpr):
    ...  # declaration: binds the registered native kernel by signature


atomic_kernel.fn_name = "kernel"  # defined as `kernel` in the reference test (test_atomic_ops.py:33)

ATOMIC_OPS = [(asc2.atomic_add, torch.add), (asc2.atomic_max, torch.maximum), (asc2.atomic_min, torch.minimum)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.int32], ids=str)
@pytest.mark.parametrize("asc_op, torch_op", ATOMIC_OPS, ids=lambda v: getattr(v, "__name__", str(v)))
def test_atomic_reference_cases(device, asc_op, torch_op, dtype):
    # test_atomic_ops.py:45-68 (USE_CORE_NUM = 4 blocks over a 128-element tensor)
    def create_input(shape):
        if dtype == torch.float32:
            return torch.clamp(torch.randn(tuple(shape), dtype=dtype), 1, 100)
        return torch.randint(1, 100, tuple(shape), dtype=dtype)

    tile_length = 128 // 4
    x = create_input([128])
    z = create_input([tile_length])
    expected_z = z.clone()
    atomic_kernel[4](x, z, [128], tile_length, asc_op)
    for i in range(4):
        expected_z = torch_op(expected_z, x[i * tile_length:(i + 1) * tile_length] + 10)
    torch.testing.assert_close(z, expected_z, atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16", "int32", "int16"])
@pytest.mark.parametrize("op", ["add", "maximum", "minimum"])
@pytest.mark.parametrize("n_tiles, tile_len", [(64, (1 << 16) + 37), (1000, 257), (3, 1)])
def test_atomic_tiles_vs_oracle(device, op, dtype, n_tiles, tile_len):
    # max / min are order-independent (IEEE maximum / minimum, signed integers): random data
    # with edge values, bit-exact.  Integer add wraps, so any order gives the same bits.
    # Float add: tile values x + 3 in {0, 1}, so every partial sum, in any order, lies
    # between z and the column total, which stays below 256 (exact in bfloat16 too).
    td = getattr(torch, dtype)
    n = n_tiles * tile_len
    if td.is_floating_point and op == "add":
        g = torch.Generator().manual_seed(n_tiles)
        p = min(0.5, 100 / n_tiles)
        x = (torch.rand(n, generator=g) < p).to(torch.int32).sub(3).to(td)
        z0 = torch.randint(0, 9, (tile_len,), generator=g).to(td)
        totals = z0.to(torch.int64) + (x.to(torch.int64) + 3).reshape(n_tiles, tile_len).sum(0)
        assert int(totals.max()) < 256
    else:
        make = _float_data if td.is_floating_point else _int_data
        x = make(td, 1).repeat(1 + n // N)[:n]
        z0 = make(td, 2)[:tile_len]
    addend = 3 if td.is_floating_point and op == "add" else (-2 if op == "minimum" else 1)
    # z at an odd element offset: the 16-bit combines run on both halves of each word
    buf = torch.zeros(tile_len + 1, dtype=td, device=device)
    z = buf[1:]
    z.copy_(z0.to(device))
    kernels.atomic_tiles(x.to(device), z, op, n_tiles, tile_len, addend)
    torch.cuda.synchronize()
    expected = O.atomic_tiles(_np(x, dtype), _np(z0, dtype), op, n_tiles, tile_len, addend, dtype)
    _assert_same(z.cpu(), expected, dtype)
    assert _np(buf[:1].cpu(), dtype).view(np.uint8).sum() == 0  # the element before z is untouched


@asc2.jit(always_compile=True)
def broadcast_dup_kernel(out_ptr, shape: asc.ConstExpr, offsets: asc.ConstExpr):
    ...  # declaration: binds the registered native kernel by signature


broadcast_dup_kernel.fn_name = "kernel"  # defined as `kernel` inside the reference test (test_shape_ops.py:68)


@pytest.mark.parametrize("shape", ([32], [3, 32]), ids=str)
@pytest.mark.parametrize("dtype", (torch.float16, torch.float32, torch.int16, torch.int32), ids=str)
def test_broadcast_dup_reference_cases(device, shape, dtype):
    # test_shape_ops.py:62-78
    out = torch.zeros(shape, dtype=dtype)
    out_ref = torch.full_like(out, 777)
    size = tuple(out.size())
    broadcast_dup_kernel[1](out, size, [0] * len(size))
    torch.testing.assert_close(out, out_ref, atol=1e-6, rtol=1e-6)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16", "int32", "int16"])
@pytest.mark.parametrize("value", [777, -3.75, 1e30])
def test_fill_vs_oracle(device, dtype, value):
    td = getattr(torch, dtype)
    if not td.is_floating_point and value != 777:
        value = -123456 if dtype == "int32" else -1234
    z = torch.zeros((1 << 22) + 3, dtype=td, device=device)
    kernels.fill(z, value, z.numel() - 1)
    torch.cuda.synchronize()
    got = z.cpu()
    _assert_same(got[:-1], O.fill(z.numel() - 1, value, dtype), dtype)
    assert _np(got[-1:], dtype).view(np.uint8).sum() == 0


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("op", kernels.UNARY_OPS)
def test_unary_16bit_vs_oracle(device, op, dtype):
    # fp32 op on the widened element, one RNE rounding: within one ulp of the element type
    # (the fp32 libm error can move a value across a rounding boundary), exact ops bit for bit
    td = getattr(torch, dtype)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(N, generator=g) * 4
    if op in ("log", "log2", "rsqrt", "sqrt"):
        x = x.abs() + 1e-3
    if op in ("cosh", "sinh", "exp", "exp2"):
        x = x.clamp(-10, 10)
    x = x.to(td)
    out = torch.empty(N, dtype=td, device=device)
    unary_kernel[1](x.to(device), out, N, getattr(asc2, op))
    torch.cuda.synchronize()
    expected = O.unary(_np(x, dtype), op, dtype)
    got = _np(out.cpu(), dtype)
    as_f = (lambda a: O.bf16_bits_to_f32(a)) if dtype == "bfloat16" else (lambda a: a.astype(np.float32))
    if op in ("abs", "ceil", "floor", "negative", "relu", "sqrt"):
        np.testing.assert_array_equal(got, expected)
    else:
        ulp = 2.0 ** -10 if dtype == "float16" else 2.0 ** -7
        np.testing.assert_allclose(as_f(got), as_f(expected), rtol=ulp, atol=1e-6)
