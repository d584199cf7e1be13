"""Matmul with a bias + activation epilogue on the GPU (the
05_matmul_leakyrelu tutorial, python/tutorials/05_matmul_leakyrelu/matmul_leakyrelu.py).

The tutorial's kernel is declared with its own signature and launched through the
asc.jit surface on CPU tensors; with its integer-valued inputs every product and sum
is exact in fp32, so the result must equal the tutorial's torch golden bit for bit
(its own bar is rtol/atol 1e-3).  The kernel API is then checked against the oracle
on tile-aligned (direct-to-LDS) and ragged shapes, again on integer-valued data."""
import numpy as np
import pytest
import torch

import asc
from oracle import asc2_oracle as O
from pyasc_amd import kernels

pytestmark = pytest.mark.gpu


@asc.jit(always_compile=True)
def matmul_leakyrelu_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress,
                            bias: asc.GlobalAddress, alpha: float, tiling: asc.adv.TCubeTiling,
                            workspace: asc.GlobalAddress):
    ...  # declaration: binds the registered native kernel by signature


def test_tutorial_recipe(device):
    m, k, n = 1024, 256, 640
    g = torch.Generator().manual_seed(7)
    a = torch.randint(-5, 5, (m, k), generator=g).to(torch.float16)
    b = torch.randint(-5, 5, (k, n), generator=g).to(torch.float16)
    bias = torch.randint(-5, 5, (1, n), generator=g).to(torch.float32)
    alpha = 0.001
    matmul = (torch.matmul(a.to(torch.float32), b.to(torch.float32)).to(torch.float32) + bias).to(torch.float32)
    c = torch.zeros((m, n), dtype=torch.float32)
    workspace = torch.zeros(16 * 1024 * 1024, dtype=torch.uint8)
    tiling = asc.adv.TCubeTiling(m=m, n=n, k=k, used_core_num=24)
    matmul_leakyrelu_kernel[tiling.used_core_num // 2](a, b, c, bias, alpha, tiling, workspace)
    golden = torch.where(matmul >= 0, matmul, matmul * alpha)
    assert torch.allclose(c, golden, rtol=1e-3, atol=1e-3)
    assert torch.equal(c, golden)


def _int_data(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-4, 5, shape, generator=g).to(dtype)


@pytest.mark.parametrize("in_dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("M,N,K", [(512, 512, 256), (300, 200, 100)])
def test_bias_leaky_relu_vs_oracle(device, in_dtype, out_dtype, M, N, K):
    a = _int_data((M, K), M + K, in_dtype)
    b = _int_data((K, N), N + K, in_dtype)
    bias = _int_data((N,), N, torch.float32) * 0.5
    c = torch.empty(M, N, dtype=out_dtype, device=device)
    kernels.matmul(a.to(device), b.to(device), c, bias=bias.to(device), leaky_alpha=0.125)
    torch.cuda.synchronize()
    expected = O.matmul_bias_leaky_relu(a.float().numpy(), b.float().numpy(), bias.numpy(), 0.125)
    if out_dtype == torch.float32:
        np.testing.assert_array_equal(c.cpu().numpy(), expected)
    elif out_dtype == torch.float16:
        np.testing.assert_array_equal(c.cpu().numpy(), expected.astype(np.float16))
    else:
        np.testing.assert_array_equal(c.cpu().view(torch.int16).numpy().view(np.uint16),
                                      O.f32_to_bf16_bits(expected))


@pytest.mark.parametrize("M,N,K", [(512, 512, 256), (77, 130, 64)])
def test_bias_with_relu_and_without_activation(device, M, N, K):
    a = _int_data((M, K), 3, torch.bfloat16)
    b = _int_data((K, N), 4, torch.bfloat16)
    bias = _int_data((N,), 5, torch.float32)
    exact = (a.double() @ b.double()).float() + bias
    for relu, expected in ((True, torch.relu(exact)), (False, exact)):
        c = torch.empty(M, N, dtype=torch.float32, device=device)
        kernels.matmul(a.to(device), b.to(device), c, relu=relu, bias=bias.to(device))
        torch.cuda.synchronize()
        assert torch.equal(c.cpu(), expected)


def test_leaky_without_bias_random_bf16(device):
    # random data at the north-star tolerance (atol/rtol 1e-2 vs fp32 CPU)
    g = torch.Generator().manual_seed(11)
    a = (torch.randn(1024, 768, generator=g) / 768 ** 0.5).bfloat16()
    b = (torch.randn(768, 512, generator=g) / 768 ** 0.5).bfloat16()
    c = torch.empty(1024, 512, dtype=torch.bfloat16, device=device)
    kernels.matmul(a.to(device), b.to(device), c, leaky_alpha=0.01)
    torch.cuda.synchronize()
    ref = a.float() @ b.float()
    ref = torch.where(ref >= 0, ref, ref * 0.01)
    torch.testing.assert_close(c.cpu().float(), ref, atol=1e-2, rtol=1e-2)


def test_epilogue_argument_errors(device):
    a = torch.zeros(64, 64, dtype=torch.float16, device=device)
    c = torch.empty(64, 64, dtype=torch.float32, device=device)
    with pytest.raises(ValueError):
        kernels.matmul(a, a, c, bias=torch.zeros(32, device=device))
    with pytest.raises(ValueError):
        kernels.matmul(a, a, c, relu=True, leaky_alpha=0.1)
