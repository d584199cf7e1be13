"""asc_matmul_chained_noalloc (the allocation-free chained matmul, intermediate in the
library's per-GPU scratch buffer) against asc_matmul_chained (intermediate in a workspace
the caller passes), through the C ABI: bit-identical results on two calls in a row, the
first filling the whole 32 MiB buffer, the second smaller, with other dtypes; and the
optional overlap check (ASC_NOALLOC_CHECK=1) refusing a call on a second stream while the
first stream's call still uses the buffer."""
import pytest
import torch

from pyasc_amd import _native

pytestmark = pytest.mark.gpu

_CODES = {torch.float32: _native.DT_FLOAT32, torch.float16: _native.DT_FLOAT16, torch.bfloat16: _native.DT_BFLOAT16}


def _inputs(M, N, dtype, seed, device):
    g = torch.Generator().manual_seed(seed)
    a = ((torch.rand((M, N), generator=g) - .5) * 2).to(dtype).to(device)
    b = ((torch.rand((N, N), generator=g) - .5) * 2 / N ** .5).to(dtype).to(device)
    return a, b


def _run_both(a, b, out_dtype, device):
    M, N = a.shape
    stream = torch.cuda.current_stream().cuda_stream
    c_ws = torch.full((M, N), float("nan"), dtype=out_dtype, device=device)
    c_na = torch.full((M, N), float("nan"), dtype=out_dtype, device=device)
    ws = torch.empty(M * N, dtype=a.dtype, device=device)
    _native.call("asc_matmul_chained", _CODES[a.dtype], _CODES[out_dtype], a.data_ptr(), b.data_ptr(),
                 c_ws.data_ptr(), M, N, N, ws.data_ptr(), ws.numel() * ws.element_size(), stream)
    _native.call("asc_matmul_chained_noalloc", _CODES[a.dtype], _CODES[out_dtype], a.data_ptr(), b.data_ptr(),
                 c_na.data_ptr(), M, N, N, stream)
    torch.cuda.synchronize()
    return c_ws, c_na


def test_noalloc_matches_workspace_entry_point_on_consecutive_calls(device):
    # call 1 fills the whole scratch buffer (4096 x 4096 bf16 = 32 MiB); call 2 is smaller and
    # ragged, so it reads back only what it wrote over call 1's contents
    for (M, N, dtype, out_dtype, seed) in [(4096, 4096, torch.bfloat16, torch.float32, 1),
                                           (200, 192, torch.float16, torch.bfloat16, 2)]:
        print(f"chained noalloc vs workspace: M={M} N=K={N} {dtype} -> {out_dtype}", flush=True)
        a, b = _inputs(M, N, dtype, seed, device)
        c_ws, c_na = _run_both(a, b, out_dtype, device)
        bits = torch.int32 if out_dtype == torch.float32 else torch.int16
        assert not torch.isnan(c_ws).any()
        assert torch.equal(c_na.view(bits), c_ws.view(bits))
        # and the reference recipe (test_matmul_l0c_to_l1.py:48-50), on a slice of rows
        rows = slice(0, min(M, 256))
        ref = (a[rows].cpu().float() @ b.cpu().float()).to(dtype).float() @ b.cpu().float()
        torch.testing.assert_close(c_na[rows].cpu().float(), ref, atol=1e-2, rtol=1e-2)


def test_noalloc_rejects_an_intermediate_above_the_buffer(device):
    a = torch.zeros((4097, 4096), dtype=torch.float16, device=device)
    b = torch.zeros((4096, 4096), dtype=torch.float16, device=device)
    c = torch.zeros((4097, 4096), dtype=torch.float16, device=device)
    with pytest.raises(RuntimeError, match="scratch buffer"):
        _native.call("asc_matmul_chained_noalloc", _native.DT_FLOAT16, _native.DT_FLOAT16, a.data_ptr(),
                     b.data_ptr(), c.data_ptr(), 4097, 4096, 4096, torch.cuda.current_stream().cuda_stream)


def test_noalloc_check_refuses_an_overlapping_call_on_another_stream(device, monkeypatch):
    # ASC_NOALLOC_CHECK=1: a call on a second stream while the first stream's call still
    # holds the scratch buffer is refused before launching anything; once the first stream
    # has finished, the same call runs and matches the first bit for bit
    if not hasattr(torch.cuda, "_sleep"):
        pytest.skip("torch.cuda._sleep is not available")
    monkeypatch.setenv("ASC_NOALLOC_CHECK", "1")
    a, b = _inputs(256, 256, torch.bfloat16, 3, device)
    c1 = torch.full((256, 256), float("nan"), device=device)
    c2 = torch.full((256, 256), float("nan"), device=device)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())

    def call(c, s):
        _native.call("asc_matmul_chained_noalloc", _native.DT_BFLOAT16, _native.DT_FLOAT32, a.data_ptr(),
                     b.data_ptr(), c.data_ptr(), 256, 256, 256, s.cuda_stream)

    with torch.cuda.stream(s1):
        torch.cuda._sleep(50_000_000)  # a bounded spin that keeps s1 busy while the host goes on
    call(c1, s1)
    with pytest.raises(RuntimeError, match="has not finished"):
        call(c2, s2)
    s1.synchronize()
    call(c2, s2)
    s2.synchronize()
    assert not torch.isnan(c1).any()
    assert torch.equal(c1.view(torch.int32), c2.view(torch.int32))
    # one stream is never refused, busy or not
    with torch.cuda.stream(s1):
        torch.cuda._sleep(5_000_000)
    call(c1, s1)
    call(c1, s1)
    s1.synchronize()
    assert torch.equal(c1.view(torch.int32), c2.view(torch.int32))
