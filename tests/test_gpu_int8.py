"""int8 matmul parity on the GPU: int32 accumulators bit-exact, fp16 dequant
bit-exact against the oracle's fp16(fp32(acc) * scale) and, in trunc-19 mode,
against the reference test's golden (python/test/generalization/adv/test_matmul_quant.py:94-106)."""
import os

import numpy as np
import pytest
import torch

from oracle import asc2_oracle as O
from pyasc_amd import kernels

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _i8(shape, seed, lo=-127, hi=128):
    return torch.randint(lo, hi, shape, dtype=torch.int8, generator=torch.Generator().manual_seed(seed))


def _f16_bits(t):
    return t.cpu().numpy().view(np.uint16)


def test_reference_quant_fixture(device):
    f = np.load(os.path.join(GOLDEN, "matmul_quant.npz"))
    for idx in range(3):
        a, b = torch.from_numpy(f[f"a{idx}"]), torch.from_numpy(f[f"b{idx}"])
        scale = torch.from_numpy(f[f"scale{idx}"])
        M, K = a.shape
        N = b.shape[1]
        acc = torch.empty(M, N, dtype=torch.int32, device=device)
        kernels.matmul_i8(a.to(device), b.to(device), acc)
        out = torch.empty(M, N, dtype=torch.float16, device=device)
        kernels.matmul_i8(a.to(device), b.to(device), out, scale=scale.to(device), trunc19=True)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(acc.cpu().numpy(), f[f"acc{idx}"])
        np.testing.assert_array_equal(_f16_bits(out), f[f"golden{idx}"].view(np.uint16))


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (31, 45, 77), (256, 256, 128), (300, 520, 1000), (512, 11008 // 8, 4096),
                                   (257, 300, 129)])
def test_accumulators_and_dequant_vs_oracle(device, M, N, K):
    a, b = _i8((M, K), M + K), _i8((K, N), N + K)
    scale = torch.rand(N, generator=torch.Generator().manual_seed(N)) * 0.009 + 0.001
    acc = torch.empty(M, N, dtype=torch.int32, device=device)
    out = torch.empty(M, N, dtype=torch.float16, device=device)
    kernels.matmul_i8(a.to(device), b.to(device), acc)
    kernels.matmul_i8(a.to(device), b.to(device), out, scale=scale.to(device))
    torch.cuda.synchronize()
    exp_acc = O.matmul_i8_acc(a.numpy(), b.numpy())
    np.testing.assert_array_equal(acc.cpu().numpy(), exp_acc)
    np.testing.assert_array_equal(_f16_bits(out), O.dequant_f16(exp_acc, scale.numpy()).view(np.uint16))


def test_extremes(device):
    K = 4096
    a = torch.full((256, K), -128, dtype=torch.int8)
    b = torch.full((K, 256), -128, dtype=torch.int8)
    a[::2] = 127
    acc = torch.empty(256, 256, dtype=torch.int32, device=device)
    kernels.matmul_i8(a.to(device), b.to(device), acc)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), O.matmul_i8_acc(a.numpy(), b.numpy()))


def test_config_shape_full(device):
    """BASELINE config: M=4096, N=11008, K=4096, uniform[-127,127] int8 from seed 3,
    scale uniform[0.001, 0.01].  Every accumulator is checked exactly against the host's
    fp64 product (exact here: every partial sum is an integer below 4096 * 127^2 < 2^53),
    and every fp16 output against the dequant of those accumulators, bit for bit."""
    g = torch.Generator().manual_seed(3)
    a = torch.randint(-127, 128, (4096, 4096), dtype=torch.int8, generator=g)
    b = torch.randint(-127, 128, (4096, 11008), dtype=torch.int8, generator=g)
    scale = torch.rand(11008, generator=g) * 0.009 + 0.001
    ad, bd = a.to(device), b.to(device)
    acc = torch.empty(4096, 11008, dtype=torch.int32, device=device)
    out = torch.empty(4096, 11008, dtype=torch.float16, device=device)
    kernels.matmul_i8(ad, bd, acc)
    kernels.matmul_i8(ad, bd, out, scale=scale.to(device))
    torch.cuda.synchronize()
    acc_h = acc.cpu()
    bd64 = b.double()
    for r0 in range(0, 4096, 1024):  # the exact product in row blocks (bounded host memory)
        exact = (a[r0:r0 + 1024].double() @ bd64).to(torch.int32)
        assert torch.equal(acc_h[r0:r0 + 1024], exact), f"rows {r0}..{r0 + 1023}"
    del bd64
    np.testing.assert_array_equal(_f16_bits(out), O.dequant_f16(acc_h.numpy(), scale.numpy()).view(np.uint16))
    # whole-matrix checksums, exact in int64 (linearity): C 1 = A (B 1) and 1^T C = (1^T A) B,
    # so every accumulator of every tile enters an exact comparison
    a64, b64, acc64 = a.numpy().astype(np.int64), b.numpy().astype(np.int64), acc_h.numpy().astype(np.int64)
    np.testing.assert_array_equal(acc64.sum(axis=1), a64 @ b64.sum(axis=1))
    np.testing.assert_array_equal(acc64.sum(axis=0), a64.sum(axis=0) @ b64)
