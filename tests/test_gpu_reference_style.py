"""The reference's asc2 kernel tests, unchanged in form: kernels defined with
@asc2.jit and launched as kernel[grid](...) on numpy arrays / CPU torch tensors,
compared with the same golden expressions
(python/test/asc2/kernels/test_vadd.py, test_softmax.py, test_softmax_fused.py)."""
import numpy as np
import pytest
import torch

import asc
import asc2

pytestmark = pytest.mark.gpu


@asc2.jit(always_compile=True)
def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
    x_gm = asc2.tensor(x_ptr, [size])
    y_gm = asc2.tensor(y_ptr, [size])
    out_gm = asc2.tensor(out_ptr, [size])
    base_offset = asc2.block_idx() * tile_size * tile_per_block
    for i in range(tile_per_block):
        tile_offset = base_offset + i * tile_size
        x = asc2.load(x_gm, [tile_size], offsets=[tile_offset])
        y = asc2.load(y_gm, [tile_size], offsets=[tile_offset])
        asc2.store(x + y, out_gm, offsets=[tile_offset])


def vadd_launch(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    out = np.empty_like(x)
    size = out.size
    core_num = 16
    tile_size = 128
    num_tiles = asc.ceildiv(size, tile_size)
    vadd_kernel[core_num](x, y, out, size, tile_size, asc.ceildiv(num_tiles, core_num))
    return out


def test_vadd(device):
    rng = np.random.default_rng(seed=2026)
    size = 8192
    x = rng.random(size, dtype=np.float32) * 10
    y = rng.random(size, dtype=np.float32) * 10
    out = vadd_launch(x, y)
    np.testing.assert_array_equal(out, x + y)


def test_vadd_device_tensors_and_stream(device):
    x = torch.rand(8192, device=device)
    y = torch.rand(8192, device=device)
    out = torch.empty_like(x)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    vadd_kernel[16, s](x, y, out, 8192, 128, 4)
    s.synchronize()
    assert torch.equal(out.cpu(), x.cpu() + y.cpu())


def test_vadd_host_arrays_on_a_side_stream(device):
    # host inputs are copied in on torch's current stream; the launch on another stream
    # waits for them, and the outputs are copied back after it
    rng = np.random.default_rng(seed=7)
    x = rng.random(1 << 20, dtype=np.float32)
    y = rng.random(1 << 20, dtype=np.float32)
    out = np.zeros_like(x)
    s = torch.cuda.Stream()
    vadd_kernel[16, s](x, y, out, x.size, 128, (x.size // 128 + 15) // 16)
    np.testing.assert_array_equal(out, x + y)


@asc2.jit(always_compile=True, vf_fusion=True)
def softmax_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: int, num_cols: int,
                   tile_size: asc.ConstExpr[int]):
    x_gm = asc2.tensor(x_ptr, [num_rows, num_cols])
    out_gm = asc2.tensor(out_ptr, [num_rows, num_cols])
    for i in range(asc2.block_idx(), num_rows, asc2.block_num(), parallel=True):
        row = asc2.load(x_gm, [1, tile_size], offsets=[i, 0])
        row_minus_max = row - asc2.reduce_max(row)
        numerator = asc2.exp(row_minus_max)
        denominator = asc2.reduce_sum(numerator)
        asc2.store(numerator / denominator, out_gm, offsets=[i, 0])


def test_softmax(device):
    x = torch.rand((64, 1024), dtype=torch.float32)
    out = torch.empty_like(x)
    softmax_kernel[16](x, out, 64, 1024, tile_size=1024)
    torch.testing.assert_close(out, torch.softmax(x, dim=1))


def test_softmax_tile_wider_than_row(device):
    # softmax_kernel with tile_size > num_cols: the padded tile's zeros enter max and sum
    x = torch.rand((64, 1000), dtype=torch.float32)
    out = torch.zeros_like(x)
    softmax_kernel[16](x, out, 64, 1000, tile_size=1024)
    padded = torch.nn.functional.pad(x.double(), (0, 24))
    torch.testing.assert_close(out, torch.softmax(padded, dim=1)[:, :1000].float(), rtol=1e-6, atol=0)


def test_softmax_fused(device):
    @asc2.jit(always_compile=True)
    def softmax_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: int,
                       num_cols: asc.ConstExpr[int], block_size: asc.ConstExpr[int]):
        x_gm = asc2.tensor(x_ptr, [num_rows, num_cols])
        out_gm = asc2.tensor(out_ptr, [num_rows, num_cols])
        start_rows = asc2.block_idx() * block_size
        rows = asc2.load(x_gm, [block_size, num_cols], offsets=[start_rows, 0])
        asc2.store(asc2.softmax(rows), out_gm, offsets=[start_rows, 0])

    core_num = 16
    x = torch.rand((64, 1024), dtype=torch.float32)
    out = torch.empty_like(x)
    block_size = (64 + core_num - 1) // core_num
    softmax_kernel[core_num](x, out, 64, 1024, block_size)
    torch.testing.assert_close(out, torch.softmax(x, dim=1))


# ------------------------------------------------------------------------------------ matmul
# The reference's asc2 matmul tests, kernels with their bodies as written and launched as
# matmul_kernel[grid](...) on CPU tensors (the reference's host-tensor path: copied in,
# launched, copied back), each against its own golden and tolerance
# (python/test/asc2/kernels/test_matmul_{mnblock,tiled,fixpipe,l0c_to_l1}.py).

def _mnblock_kernel():
    @asc2.jit(always_compile=True)
    def matmul_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                      a_shape: asc.ConstExpr, b_shape: asc.ConstExpr, c_shape: asc.ConstExpr,
                      m_tile: asc.ConstExpr[int], m_tiles_per_block: asc.ConstExpr[int],
                      n_tile: asc.ConstExpr[int], n_tiles_per_block: asc.ConstExpr[int]):
        a_gm = asc2.tensor(a_ptr, a_shape)
        b_gm = asc2.tensor(b_ptr, b_shape)
        c_gm = asc2.tensor(c_ptr, c_shape)
        blockId = asc2.block_idx()
        m_elems_per_block = m_tile * m_tiles_per_block
        m_base_off = (m_elems_per_block * blockId) % a_shape[0]
        n_base_off = ((m_elems_per_block * blockId) // a_shape[0]) * (n_tile * n_tiles_per_block)
        for j in range(n_tiles_per_block):
            b_offset = n_base_off + j * n_tile
            b_j = asc2.load(b_gm, [b_shape[0], n_tile], offsets=[0, b_offset], location=asc2.TileLocation.L0B)
            for i in range(m_tiles_per_block):
                a_offset = m_base_off + i * m_tile
                a_i = asc2.load(a_gm, [m_tile, a_shape[1]], offsets=[a_offset, 0], location=asc2.TileLocation.L0A)
                c_ij = a_i @ b_j
                asc2.store(c_ij, c_gm, offsets=[a_offset, b_offset])

    return matmul_kernel


matmul_mnblock_kernel = _mnblock_kernel()


def _m_tiles_per_block(m, k, n, core_num, m_tile, n_tile, n_tiles_per_block):
    # eval_tiles of test_matmul_mnblock.py: the even split its asserts require
    tiles_per_core = (m // m_tile) * (n // n_tile) // core_num
    return tiles_per_core // n_tiles_per_block


@pytest.mark.parametrize("m, k, n, core_num, m_tile, n_tile, n_tiles_per_block", [
    (16, 16, 16, 1, 16, 16, 1),
    (16, 160, 16, 1, 16, 16, 1),
    (32, 16, 16, 2, 16, 16, 1),
    (16, 16, 32, 2, 16, 16, 1),
    (32, 16, 32, 2, 16, 16, 1),
    (32, 16, 32, 2, 16, 16, 2),
    (32, 16, 32, 4, 16, 16, 1),
    (480, 224, 1344, 30, 48, 32, 7),
])
def test_matmul_mnblock(device, m, k, n, core_num, m_tile, n_tile, n_tiles_per_block):
    torch.manual_seed(m * 7 + n)
    a = torch.rand((m, k), dtype=torch.float16)
    b = torch.rand((k, n), dtype=torch.float16)
    c = torch.zeros((m, n), dtype=torch.float32)
    mtpb = _m_tiles_per_block(m, k, n, core_num, m_tile, n_tile, n_tiles_per_block)
    matmul_mnblock_kernel[core_num](a, b, c, a.shape, b.shape, c.shape, m_tile, mtpb, n_tile, n_tiles_per_block)
    torch.testing.assert_close(c, a.to(torch.float32) @ b.to(torch.float32))


def _tiled_kernel():
    @asc2.jit(always_compile=True)
    def matmul_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                      a_shape: asc.ConstExpr, b_shape: asc.ConstExpr, c_shape: asc.ConstExpr,
                      k_tiles: asc.ConstExpr):
        a_gm = asc2.tensor(a_ptr, a_shape)
        b_gm = asc2.tensor(b_ptr, b_shape)
        c_gm = asc2.tensor(c_ptr, c_shape)
        acc = asc2.zeros_acc(c_shape, dtype=asc.float32)
        k_offset = a_shape[1] // k_tiles
        a_l1 = asc2.load(a_gm, a_shape, offsets=[0, 0], location=asc2.TileLocation.L1)
        b_l1 = asc2.load(b_gm, b_shape, offsets=[0, 0], location=asc2.TileLocation.L1)
        for i in range(k_tiles, unroll_factor=2, parallel=True):
            a_i = asc2.copy(a_l1, [a_shape[0], k_offset], offsets=[0, i * k_offset], location=asc2.TileLocation.L0A)
            b_i = asc2.copy(b_l1, [k_offset, b_shape[1]], offsets=[i * k_offset, 0], location=asc2.TileLocation.L0B)
            asc2.matmul_acc(a_i, b_i, acc)
        asc2.store(acc, c_gm, offsets=[0, 0])

    return matmul_kernel


matmul_tiled_kernel = _tiled_kernel()


@pytest.mark.parametrize("k_tiles", [2, 4, 8])
def test_matmul_tiled(device, k_tiles):
    torch.manual_seed(k_tiles)
    m, k, n = 64, 128, 256
    a = torch.rand((m, k), dtype=torch.float16)
    b = torch.rand((k, n), dtype=torch.float16)
    c = torch.zeros((m, n), dtype=torch.float32)
    matmul_tiled_kernel[1](a, b, c, a.shape, b.shape, c.shape, k_tiles)
    torch.testing.assert_close(c, a.to(torch.float32) @ b.to(torch.float32))


def _fixpipe_kernel():
    @asc2.jit(always_compile=True)
    def matmul_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                      a_shape: asc.ConstExpr, b_shape: asc.ConstExpr, c_shape: asc.ConstExpr):
        a_gm = asc2.tensor(a_ptr, a_shape)
        b_gm = asc2.tensor(b_ptr, b_shape)
        c_gm = asc2.tensor(c_ptr, c_shape)
        a = asc2.load(a_gm, a_shape, offsets=[0, 0], location=asc2.TileLocation.L0A)
        b = asc2.load(b_gm, b_shape, offsets=[0, 0], location=asc2.TileLocation.L0B)
        c = a @ b
        c = asc2.relu(c).to(asc.float16)
        asc2.store(c, c_gm, offsets=[0, 0])

    return matmul_kernel


matmul_fixpipe_kernel = _fixpipe_kernel()


@pytest.mark.parametrize("m, k, n, dtype", [
    (64, 128, 128, torch.float32),
    (64, 128, 256, torch.float16),
    (64, 128, 256, torch.bfloat16),
])
def test_matmul_fixpipe(device, m, k, n, dtype):
    torch.manual_seed(n)
    a = (torch.rand((m, k), dtype=dtype) - .5) * 10
    b = (torch.rand((k, n), dtype=dtype) - .5) * 10
    c = torch.zeros((m, n), dtype=torch.float16)
    matmul_fixpipe_kernel[1](a, b, c, a.shape, b.shape, c.shape)
    c_ref = (a.to(torch.float32) @ b.to(torch.float32)).relu().to(torch.float16)
    torch.testing.assert_close(c, c_ref, atol=1e-3, rtol=1e-3)


def _chained_kernel():
    @asc2.jit(always_compile=True)
    def matmul_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                      a_shape: asc.ConstExpr, b_shape: asc.ConstExpr, c_shape: asc.ConstExpr,
                      dtype: asc.ConstExpr):
        a_gm = asc2.tensor(a_ptr, a_shape)
        b_gm = asc2.tensor(b_ptr, b_shape)
        c_gm = asc2.tensor(c_ptr, c_shape)
        a = asc2.load(a_gm, a_shape, offsets=[0, 0], location=asc2.TileLocation.L0A)
        b = asc2.load(b_gm, b_shape, offsets=[0, 0], location=asc2.TileLocation.L0B)
        c = a @ b
        c = c.to(dtype)
        c_l1 = asc2.copy(c, c_shape, offsets=[0, 0], location=asc2.TileLocation.L1)
        c_l0a = asc2.copy(c_l1, c_shape, offsets=[0, 0], location=asc2.TileLocation.L0A)
        result = c_l0a @ b
        asc2.store(result, c_gm, offsets=[0, 0])

    return matmul_kernel


matmul_chained_kernel = _chained_kernel()


@pytest.mark.parametrize("m, k, n, torch_dtype, pyasc_dtype", [
    (32, 64, 64, torch.float16, asc.float16),
    (64, 64, 64, torch.bfloat16, asc.bfloat16),
])
def test_matmul_l0c_to_l1(device, m, k, n, torch_dtype, pyasc_dtype):
    torch.manual_seed(0)
    a = (torch.rand((m, k), dtype=torch_dtype) - .5) * 10
    b = (torch.rand((k, n), dtype=torch_dtype) - .5) * 10
    c = torch.zeros((m, n), dtype=torch.float32)
    matmul_chained_kernel[1](a, b, c, a.shape, b.shape, c.shape, pyasc_dtype)
    c_ref = (a.to(torch.float32) @ b.to(torch.float32)).to(torch_dtype)
    c_ref = c_ref.to(torch.float32) @ b.to(torch.float32)
    torch.testing.assert_close(c, c_ref, atol=1e-3, rtol=1e-3)


def test_matmul_l0c_to_l1_on_a_side_stream(device):
    # the chained kernel's intermediate lives on the launch stream until its matmuls ran:
    # allocations on torch's current stream meanwhile must not reuse it
    g = torch.Generator().manual_seed(5)
    a = ((torch.rand((256, 256), generator=g) - .5) * 4).to(torch.bfloat16).to(device)
    b = ((torch.rand((256, 256), generator=g) - .5) * 4).to(torch.bfloat16).to(device)
    expect = torch.zeros((256, 256), device=device)
    matmul_chained_kernel[1](a, b, expect, a.shape, b.shape, expect.shape, asc.bfloat16)
    torch.cuda.synchronize()
    c = torch.zeros((256, 256), device=device)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    matmul_chained_kernel[1, s](a, b, c, a.shape, b.shape, c.shape, asc.bfloat16)
    junk = [torch.full((256, 256), 7.0, dtype=torch.bfloat16, device=device) for _ in range(8)]
    torch.cuda.synchronize()
    assert torch.equal(c, expect)  # the same kernels on the same data: bit for bit
    assert all(bool((j == 7.0).all()) for j in junk)


def test_matmul_mnblock_device_tensors(device):
    # the same launch on device tensors: zero-copy, asynchronous on the current stream
    m, k, n, core_num, m_tile, n_tile, ntpb = 480, 224, 1344, 30, 48, 32, 7
    g = torch.Generator().manual_seed(5)
    a = torch.rand((m, k), generator=g).to(torch.float16)
    b = torch.rand((k, n), generator=g).to(torch.float16)
    c = torch.full((m, n), -1.0, device=device)
    mtpb = _m_tiles_per_block(m, k, n, core_num, m_tile, n_tile, ntpb)
    matmul_mnblock_kernel[core_num](a.to(device), b.to(device), c, a.shape, b.shape, c.shape, m_tile, mtpb, n_tile,
                                    ntpb)
    torch.testing.assert_close(c.cpu(), a.float() @ b.float())


def test_matmul_noncontiguous_device_output_is_refused(device):
    a = torch.rand((64, 128), device=device).to(torch.float16)
    b = torch.rand((128, 64), device=device).to(torch.float16)
    c = torch.zeros((64, 64), device=device).t()  # a transposed view
    with pytest.raises(ValueError, match="non-contiguous device tensor"):
        matmul_tiled_kernel[1](a, b, c, a.shape, b.shape, c.shape, 2)


# int8 kernels (build-defined asc2-style signatures), declared by signature, on the
# reference quant test's recipe (tests/golden/matmul_quant.npz: randint(-5, 5) int8,
# golden gen_golden of python/test/generalization/adv/test_matmul_quant.py:94-106)

@asc2.jit
def matmul_int8_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                       a_shape: asc.ConstExpr, b_shape: asc.ConstExpr, c_shape: asc.ConstExpr):
    """c (int32) = a (int8) @ b (int8), exact."""


@asc2.jit
def matmul_dequant_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                          quant_ptr: asc.GlobalAddress, a_shape: asc.ConstExpr, b_shape: asc.ConstExpr,
                          c_shape: asc.ConstExpr, trunc_scale: asc.ConstExpr):
    """c (fp16) = fp16(fp32(a @ b) * scale[n]); trunc_scale clears the scale's low 13 mantissa bits."""


@pytest.mark.parametrize("idx", [0, 1, 2])
def test_matmul_int8_and_dequant_on_quant_fixture(device, idx):
    import os
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "matmul_quant.npz"))
    a, b, scale = f[f"a{idx}"], f[f"b{idx}"], f[f"scale{idx}"]
    M, N = a.shape[0], b.shape[1]
    acc = np.zeros((M, N), np.int32)
    matmul_int8_kernel[16](a, b, acc, a.shape, b.shape, acc.shape)
    np.testing.assert_array_equal(acc, f[f"acc{idx}"])
    out = np.zeros((M, N), np.float16)
    matmul_dequant_kernel[16](a, b, out, scale, a.shape, b.shape, out.shape, True)
    np.testing.assert_array_equal(out.view(np.uint16), f[f"golden{idx}"].view(np.uint16))
