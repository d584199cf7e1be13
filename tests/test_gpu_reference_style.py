"""The reference's asc2 kernel tests in their launch form: kernels declared with @asc2.jit
by signature (declaration bodies bind the registered native kernel) and launched as
kernel[grid](...) on numpy arrays / CPU torch tensors, on each reference test's shapes,
seeds and golden expression (python/test/asc2/kernels/test_vadd.py, test_softmax.py,
test_softmax_fused.py, test_matmul_{mnblock,tiled,fixpipe,l0c_to_l1}.py).  The grid and
tile arguments are worked out here the way each reference test's launch helper does."""
import numpy as np
import pytest
import torch

import asc
import asc2

pytestmark = pytest.mark.gpu


@asc2.jit(always_compile=True)
def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
    """out = x + y on the tiles block b covers: tiles b*tile_per_block .. +tile_per_block,
    each tile_size elements, the store clipped to size."""


def _launch_vadd(x: np.ndarray, y: np.ndarray, grid: int = 16, tile: int = 128) -> np.ndarray:
    # test_vadd.py:31-38: 16 blocks of 128-element tiles, enough tiles per block to cover x
    out = np.empty_like(x)
    tiles = -(-x.size // tile)
    vadd_kernel[grid](x, y, out, x.size, tile, -(-tiles // grid))
    return out


def test_vadd(device):
    rng = np.random.default_rng(seed=2026)  # test_vadd.py:41-48
    x = rng.random(8192, dtype=np.float32) * 10
    y = rng.random(8192, dtype=np.float32) * 10
    np.testing.assert_array_equal(_launch_vadd(x, y), x + y)


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
    """Rows b, b+grid, ...: the first tile_size columns (zero-padded past num_cols) go
    through exp(x - max) / sum, both reductions over the whole tile."""


def test_softmax(device):
    x = torch.rand((64, 1024), dtype=torch.float32)  # test_softmax.py:38-43
    out = torch.empty_like(x)
    softmax_kernel[16](x, out, 64, 1024, tile_size=1024)
    torch.testing.assert_close(out, torch.softmax(x, dim=1))


def test_softmax_tile_wider_than_row(device):
    # tile_size > num_cols: the padded tile's zeros enter max and sum
    x = torch.rand((64, 1000), dtype=torch.float32)
    out = torch.zeros_like(x)
    softmax_kernel[16](x, out, 64, 1000, tile_size=1024)
    padded = torch.nn.functional.pad(x.double(), (0, 24))
    torch.testing.assert_close(out, torch.softmax(padded, dim=1)[:, :1000].float(), rtol=1e-6, atol=0)


def _softmax_fused_kernel():
    @asc2.jit(always_compile=True)
    def softmax_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: int,
                       num_cols: asc.ConstExpr[int], block_size: asc.ConstExpr[int]):
        """Block b: row softmax (asc2.softmax) of rows b*block_size .. +block_size."""

    return softmax_kernel


softmax_fused_kernel = _softmax_fused_kernel()


def test_softmax_fused(device):
    grid, rows = 16, 64  # test_softmax_fused.py:36-41
    x = torch.rand((rows, 1024), dtype=torch.float32)
    out = torch.empty_like(x)
    softmax_fused_kernel[grid](x, out, rows, 1024, -(-rows // grid))
    torch.testing.assert_close(out, torch.softmax(x, dim=1))


# ------------------------------------------------------------------------------------ matmul
# The reference's asc2 matmul tests, launched as matmul_kernel[grid](...) on CPU tensors (the
# reference's host-tensor path: copied in, launched, copied back), each against its own
# golden and tolerance (python/test/asc2/kernels/test_matmul_{mnblock,tiled,fixpipe,l0c_to_l1}.py).

def _mnblock_kernel():
    @asc2.jit(always_compile=True)
    def matmul_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                      a_shape: asc.ConstExpr, b_shape: asc.ConstExpr, c_shape: asc.ConstExpr,
                      m_tile: asc.ConstExpr[int], m_tiles_per_block: asc.ConstExpr[int],
                      n_tile: asc.ConstExpr[int], n_tiles_per_block: asc.ConstExpr[int]):
        """fp32 C tiles: block b owns m_tiles_per_block x n_tiles_per_block tiles of
        m_tile x n_tile, walking down M first, each the product over the whole K."""

    return matmul_kernel


matmul_mnblock_kernel = _mnblock_kernel()


def _m_tiles_per_block(m, k, n, core_num, m_tile, n_tile, n_tiles_per_block):
    # the even split test_matmul_mnblock.py's eval_tiles asserts
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
        """fp32 C = the sum over k_tiles K-slices of A_i @ B_i (one block)."""

    return matmul_kernel


def _fixpipe_kernel():
    @asc2.jit(always_compile=True)
    def matmul_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                      a_shape: asc.ConstExpr, b_shape: asc.ConstExpr, c_shape: asc.ConstExpr):
        """C = relu(A @ B), cast to fp16 on the store (one block)."""

    return matmul_kernel


def _chained_kernel():
    @asc2.jit(always_compile=True)
    def matmul_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                      a_shape: asc.ConstExpr, b_shape: asc.ConstExpr, c_shape: asc.ConstExpr,
                      dtype: asc.ConstExpr):
        """fp32 C = (A @ B rounded to dtype) @ B (one block)."""

    return matmul_kernel


matmul_tiled_kernel = _tiled_kernel()
matmul_fixpipe_kernel = _fixpipe_kernel()
matmul_chained_kernel = _chained_kernel()


@pytest.mark.parametrize("k_tiles", [2, 4, 8])
def test_matmul_tiled(device, k_tiles):
    torch.manual_seed(k_tiles)
    m, k, n = 64, 128, 256
    a = torch.rand((m, k), dtype=torch.float16)
    b = torch.rand((k, n), dtype=torch.float16)
    c = torch.zeros((m, n), dtype=torch.float32)
    matmul_tiled_kernel[1](a, b, c, a.shape, b.shape, c.shape, k_tiles)
    torch.testing.assert_close(c, a.to(torch.float32) @ b.to(torch.float32))


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
