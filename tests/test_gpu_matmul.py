"""fp16/bf16 (and fp32-input) matmul parity on the GPU through the C ABI.

Tolerances: the north-star bound for fp16/bf16 matmul is atol/rtol 1e-2 against
an fp32 torch CPU reference; the reference tests' own tolerances are used where
they are tighter (fixpipe / chained: 1e-3; mnblock / K-tiled fp32 output: the
default fp32 assert_close, relaxed to 2e-5 relative for fp32 accumulation order).
"""
import os

import numpy as np
import pytest
import torch

from oracle import asc2_oracle as O
from pyasc_amd import kernels

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
TOL = 1e-2  # north star: fp16/bf16 matmul within atol/rtol 1e-2 of fp32 CPU


def _gen(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def test_mnblock_fixture(device):
    f = np.load(os.path.join(GOLDEN, "matmul_mnblock_f16.npz"))
    for idx in range(len(f["cases"])):
        a = torch.from_numpy(f[f"a{idx}"]).to(device)
        b = torch.from_numpy(f[f"b{idx}"]).to(device)
        c = torch.zeros(a.shape[0], b.shape[1], device=device)
        kernels.matmul(a, b, c)
        torch.cuda.synchronize()
        torch.testing.assert_close(c.cpu(), torch.from_numpy(f[f"c{idx}"]), rtol=2e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (16, 16, 16), (17, 33, 65), (300, 257, 129), (256, 256, 64),
                                   (512, 768, 320), (64, 128, 256), (1000, 1000, 1000)])
def test_shapes_vs_oracle(device, dtype, out_dtype, M, N, K):
    a = _gen((M, K), dtype, M * 7 + K, 1 / np.sqrt(K))
    b = _gen((K, N), dtype, N * 11 + K)
    c = torch.full((M, N), 123.0, dtype=out_dtype, device=device)
    kernels.matmul(a.to(device), b.to(device), c)
    torch.cuda.synchronize()
    ref = torch.from_numpy(O.matmul(a.float().numpy(), b.float().numpy()))
    torch.testing.assert_close(c.cpu().float(), ref.to(out_dtype).float(), atol=TOL, rtol=TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_relu_cast_fixpipe(device, dtype):
    # python/test/asc2/kernels/test_matmul_fixpipe.py:36-48
    g = torch.Generator().manual_seed(5)
    a = (torch.rand((64, 128), generator=g, dtype=dtype) - .5) * 10
    b = (torch.rand((128, 256), generator=g, dtype=dtype) - .5) * 10
    c = torch.zeros((64, 256), dtype=torch.float16, device=device)
    kernels.matmul(a.to(device), b.to(device), c, relu=True)
    torch.cuda.synchronize()
    ref = (a.to(torch.float32) @ b.to(torch.float32)).relu().to(torch.float16)
    torch.testing.assert_close(c.cpu(), ref, atol=1e-3, rtol=1e-3)


def test_fp32_inputs(device):
    g = torch.Generator().manual_seed(6)
    a = (torch.rand((64, 128), generator=g) - .5) * 10
    b = (torch.rand((128, 128), generator=g) - .5) * 10
    c = torch.zeros((64, 128), dtype=torch.float16, device=device)
    kernels.matmul(a.to(device), b.to(device), c, relu=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(c.cpu(), (a @ b).relu().to(torch.float16), atol=1e-3, rtol=1e-3)


def test_strided_views(device):
    a = _gen((300, 200), torch.float16, 1, 0.1).to(device)
    b = _gen((200, 400), torch.float16, 2).to(device)
    c = torch.full((300, 400), -5.0, device=device)
    kernels.matmul(a[10:110, 8:136], b[8:136, 16:272], c[50:150, 100:356])
    torch.cuda.synchronize()
    ref = O.matmul(a[10:110, 8:136].float().cpu().numpy(), b[8:136, 16:272].float().cpu().numpy())
    got = c.cpu().numpy()
    np.testing.assert_allclose(got[50:150, 100:356], ref, atol=TOL, rtol=TOL)
    mask = np.ones_like(got, dtype=bool)
    mask[50:150, 100:356] = False
    assert (got[mask] == -5.0).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_config_8192_full(device, dtype):
    """BASELINE config: M=N=K=8192, randn/sqrt(K) inputs from seed 2; all of C is checked
    against the fp32 CPU product (python/test/asc2/kernels/test_matmul_tiled.py:49's golden)
    rounded to the output dtype."""
    n = 8192
    g = torch.Generator().manual_seed(2)
    a = (torch.randn(n, n, generator=g) / np.sqrt(n)).to(dtype)
    b = (torch.randn(n, n, generator=g) / np.sqrt(n)).to(dtype)
    c = torch.empty(n, n, dtype=dtype, device=device)
    kernels.matmul(a.to(device), b.to(device), c)
    torch.cuda.synchronize()
    ref = a.float() @ b.float()
    torch.testing.assert_close(c.cpu().float(), ref.to(dtype).float(), atol=TOL, rtol=TOL)


# fp32 inputs: the MFMA kernel up to 4096 output tiles of 32x32, the LDS FMA kernel beyond
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (17, 33, 5), (256, 256, 256), (100, 300, 1000), (31, 2, 17),
                                   (2048, 2048, 48), (2100, 2100, 40), (64, 64, 0)])
def test_f32_inputs_integer_valued_exact(device, M, N, K):
    # entries in [-4, 4]: every partial sum is an integer below 2^24, exact in any order
    g = torch.Generator().manual_seed(M + N + K)
    a = torch.randint(-4, 5, (M, K), generator=g).float()
    b = torch.randint(-4, 5, (K, N), generator=g).float()
    c = torch.full((M, N), float("nan"), device=device)
    kernels.matmul(a.to(device), b.to(device), c)
    torch.cuda.synchronize()
    assert torch.equal(c.cpu(), (a.double() @ b.double()).float())


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("act", ["none", "relu", "leaky"])
@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (77, 50, 33), (2100, 64, 2100)])
def test_f32_inputs_epilogues_vs_fp64(device, out_dtype, act, M, N, K):
    g = torch.Generator().manual_seed(7)
    a = torch.randn(M, K, generator=g) * 3
    b = torch.randn(K, N, generator=g) * 3
    bias = torch.randn(N, generator=g) * 10
    c = torch.empty(M, N, dtype=out_dtype, device=device)
    kw = {"bias": bias.to(device)}
    if act == "relu":
        kw["relu"] = True
    elif act == "leaky":
        kw["leaky_alpha"] = 0.01
    kernels.matmul(a.to(device), b.to(device), c, **kw)
    torch.cuda.synchronize()
    ref = a.double() @ b.double() + bias.double()
    if act == "relu":
        ref = ref.relu()
    elif act == "leaky":
        ref = torch.where(ref >= 0, ref, ref * 0.01)
    # fp32 accumulation: error below K * 2^-24 * sum|a b| per element, then the output rounding
    bound = K * 2.0 ** -24 * (a.double().abs() @ b.double().abs()) + ref.abs() * {
        torch.float32: 0.0, torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}[out_dtype] + 1e-6
    assert bool(((c.cpu().double() - ref).abs() <= bound).all())


def test_direct_path_repeat_runs_are_bit_identical(device):
    # the direct-to-LDS loop orders its DMA and operand reads with waits and barriers only;
    # repeated runs must agree bit for bit (a stage race would show here)
    g = torch.Generator().manual_seed(12)
    a = (torch.randn(4096, 4096, generator=g) / 64).to(torch.bfloat16).to(device)
    b = (torch.randn(4096, 4096, generator=g) / 64).to(torch.bfloat16).to(device)
    outs = []
    for _ in range(3):
        c = torch.empty(4096, 4096, dtype=torch.bfloat16, device=device)
        kernels.matmul(a, b, c)
        outs.append(c)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("dtype,out_dtype,M,N", [
    (torch.float16, torch.float32, 32, 64), (torch.bfloat16, torch.float32, 64, 64),  # test_matmul_l0c_to_l1.py
    (torch.float16, torch.float32, 256, 256), (torch.bfloat16, torch.float16, 512, 1024),  # tile-aligned
    (torch.bfloat16, torch.bfloat16, 100, 96)])  # ragged
def test_chained_entry_point(device, dtype, out_dtype, M, N):
    # asc_matmul_chained (one call, intermediate in a workspace) against the same two
    # matmuls launched one by one: identical kernels, so identical bits; and against the
    # reference test's fp32 recipe (test_matmul_l0c_to_l1.py:46-50)
    g = torch.Generator().manual_seed(M * 7 + N)
    a = ((torch.rand((M, N), generator=g) - .5) * 2).to(dtype).to(device)
    b = ((torch.rand((N, N), generator=g) - .5) * 2 / N ** .5).to(dtype).to(device)
    c = torch.full((M, N), 7.0, dtype=out_dtype, device=device)
    kernels.matmul_chained(a, b, c)
    t = torch.empty((M, N), dtype=dtype, device=device)
    c2 = torch.empty_like(c)
    kernels.matmul(a, b, t)
    kernels.matmul(t, b, c2)
    ws = torch.full((M * N + 64,), float("nan"), dtype=dtype, device=device)  # a larger workspace
    c3 = torch.empty_like(c)
    kernels.matmul_chained(a, b, c3, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(c.view(torch.int16) if out_dtype != torch.float32 else c.view(torch.int32),
                       c2.view(torch.int16) if out_dtype != torch.float32 else c2.view(torch.int32))
    assert torch.equal(c3, c)
    assert torch.equal(ws[:M * N].view(M, N), t)
    ref = (a.cpu().float() @ b.cpu().float()).to(dtype).float() @ b.cpu().float()
    tol = 1e-3 if out_dtype == torch.float32 else 1e-2
    torch.testing.assert_close(c.cpu().float(), ref, atol=tol, rtol=tol)


def test_chained_entry_point_on_a_side_stream(device):
    g = torch.Generator().manual_seed(5)
    a = ((torch.rand((256, 256), generator=g) - .5) * 2).half().to(device)
    b = ((torch.rand((256, 256), generator=g) - .5) / 8).half().to(device)
    c = torch.empty((256, 256), device=device)
    expected = torch.empty_like(c)
    kernels.matmul_chained(a, b, expected)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    for _ in range(3):  # the workspace of each call is taken from the allocator and recorded on s
        kernels.matmul_chained(a, b, c, stream=s)
    s.synchronize()
    assert torch.equal(c, expected)


def test_chained_entry_point_errors(device):
    a = torch.zeros((64, 32), dtype=torch.float16, device=device)
    b = torch.zeros((32, 64), dtype=torch.float16, device=device)
    with pytest.raises(ValueError, match="square"):
        kernels.matmul_chained(a, b, torch.empty((64, 64), device=device))
    sq = torch.zeros((32, 32), dtype=torch.float16, device=device)
    with pytest.raises(RuntimeError, match="workspace holds"):
        kernels.matmul_chained(a, sq, torch.empty((64, 32), device=device),
                               workspace=torch.empty(64 * 32 - 1, dtype=torch.float16, device=device))
    with pytest.raises(TypeError):
        kernels.matmul_chained(a.float(), sq.float(), torch.empty((64, 32), device=device))
