"""The asc2 launch path through prebuilt gfx950 code objects (pyasc_amd/asc/runtime/module.py):
vadd_kernel[grid](...) loads pyasc_amd/lib/co/asc2_vadd.hsaco with hipModuleLoad, keeps it per
specialisation in the memory cache and the file cache, and bypasses both under always_compile,
as the reference's launch path does with the binaries its compiler produces
(python/asc/runtime/jit.py:158-223, launcher.py:204-238).  Results are bit-identical to the
library path (asc_vadd), whose kernels share the device bodies."""
import os

import numpy as np
import pytest
import torch

import asc
import asc2
from pyasc_amd import kernels
from pyasc_amd.asc.runtime import module
from pyasc_amd.launchers import VADD_CODE_OBJECT

pytestmark = pytest.mark.gpu


def _vadd(**options):
    @asc2.jit(**options)
    def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                    tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
        """out = x + y over the tiles of block b (python/test/asc2/kernels/test_vadd.py's kernel)."""

    return vadd_kernel


@pytest.fixture
def cache_dir(tmp_path, monkeypatch):
    monkeypatch.setenv("PYASC_AMD_CACHE_DIR", str(tmp_path))
    return tmp_path


def _inputs(dtype, n, seed, device):
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.int32:
        x, y = (torch.randint(-2 ** 31, 2 ** 31 - 1, (n,), generator=g, dtype=torch.int32) for _ in range(2))
    else:
        x, y = ((torch.rand(n, generator=g) * 10).to(dtype) for _ in range(2))
    return x.to(device), y.to(device)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16, torch.int32])
@pytest.mark.parametrize("n,tile,tpb,grid,offset", [(8192, 128, 4, 16, 0), (100003, 128, 49, 16, 0),
                                                   (1000, 128, 2, 3, 0), (5000, 64, 5, 16, 1)])
def test_code_object_path_matches_library_path(device, cache_dir, dtype, n, tile, tpb, grid, offset):
    x, y = _inputs(dtype, n + offset, n + tile, device)
    x, y = x[offset:], y[offset:]  # offset 1: unaligned views take the element kernel only
    out_co = torch.full((n + offset,), 3, dtype=dtype, device=device)[offset:]
    out_lib = out_co.clone()
    _vadd()[grid](x, y, out_co, n, tile, tpb)
    kernels.vadd(x, y, out_lib, n, tile, tpb, grid)
    torch.cuda.synchronize()
    assert torch.equal(out_co, out_lib)
    covered = min(n, grid * tpb * tile)
    exp = (x.cpu().to(torch.int64) + y.cpu().to(torch.int64)).to(torch.int32) if dtype == torch.int32 else \
        x.cpu() + y.cpu()
    assert torch.equal(out_co.cpu()[:covered], exp[:covered])
    assert (out_co.cpu()[covered:] == 3).all()


def test_memory_and_file_cache_hits(device, cache_dir):
    x, y = _inputs(torch.float32, 8192, 1, device)
    out = torch.empty_like(x)
    k = _vadd()
    loads = module.stats["module_loads"]
    k[16](x, y, out, 8192, 128, 4)  # miss: the code object goes into the file cache and is loaded
    assert module.stats["module_loads"] == loads + 1
    files = list(cache_dir.rglob("vadd_kernel.hsaco"))
    assert len(files) == 1 and files[0].read_bytes() == VADD_CODE_OBJECT.path.read_bytes()
    mtime = files[0].stat().st_mtime_ns
    for _ in range(5):  # memory-cache hits: no load
        k[16](x, y, out, 8192, 128, 4)
    assert module.stats["module_loads"] == loads + 1
    torch.cuda.synchronize()
    assert torch.equal(out, x + y)
    # a new function object with the same source: memory miss, file-cache hit (the cached file is loaded)
    k2 = _vadd()
    k2[16](x, y, out, 8192, 128, 4)
    assert module.stats["module_loads"] == loads + 2
    assert list(cache_dir.rglob("vadd_kernel.hsaco")) == files and files[0].stat().st_mtime_ns == mtime
    # another specialisation (dtype) gets its own file-cache entry
    xh, yh = x.half(), y.half()
    outh = torch.empty_like(xh)
    k[16](xh, yh, outh, 8192, 128, 4)
    torch.cuda.synchronize()
    assert len(list(cache_dir.rglob("vadd_kernel.hsaco"))) == 2 and torch.equal(outh, xh + yh)


def test_always_compile_bypasses_both_caches(device, cache_dir):
    x, y = _inputs(torch.float32, 8192, 2, device)
    out = torch.empty_like(x)
    k = _vadd(always_compile=True)
    loads, unloads = module.stats["module_loads"], module.stats["module_unloads"]
    for _ in range(3):
        k[16](x, y, out, 8192, 128, 4)
    assert module.stats["module_loads"] == loads + 3 and module.stats["module_unloads"] == unloads + 3
    assert not list(cache_dir.rglob("*.hsaco")) and k.kernel_cache == {}
    torch.cuda.synchronize()
    assert torch.equal(out, x + y)


def test_reference_test_through_code_object(device, cache_dir):
    # python/test/asc2/kernels/test_vadd.py:41-48 on numpy inputs (host buffers copied in and back)
    rng = np.random.default_rng(seed=2026)
    x = rng.random(8192, dtype=np.float32) * 10
    y = rng.random(8192, dtype=np.float32) * 10
    out = np.empty_like(x)
    _vadd()[16](x, y, out, 8192, 128, asc.ceildiv(asc.ceildiv(8192, 128), 16))
    np.testing.assert_array_equal(out, x + y)
    assert os.path.isdir(cache_dir)


# --------------------------------------------------------------------------------------- softmax

def _softmax_rows(**options):
    @asc2.jit(**options)
    def softmax_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: int, num_cols: int,
                       tile_size: asc.ConstExpr[int]):
        """Grid-strided row softmax of the first tile_size columns
        (python/test/asc2/kernels/test_softmax.py's kernel)."""

    return softmax_kernel


def _softmax_fused(**options):
    @asc2.jit(**options)
    def softmax_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: int,
                       num_cols: asc.ConstExpr[int], block_size: asc.ConstExpr[int]):
        """asc2.softmax of block_size rows per block (python/test/asc2/kernels/test_softmax_fused.py's kernel)."""

    return softmax_kernel


def _softmax_inputs(dtype, rows, cols, seed, device, offset=0):
    g = torch.Generator().manual_seed(seed)
    base = (torch.randn(rows * cols + offset, generator=g) * 4).to(dtype).to(device)
    x = base[offset:].view(rows, cols)  # offset 1: rows no longer start 16-byte aligned
    out = torch.full((rows * cols + offset,), 7.0, dtype=dtype, device=device)[offset:].view(rows, cols)
    return x, out


@pytest.mark.parametrize("dtype,rows,cols,tile,offset", [
    # one case per planned kernel: wave_1x2, wave_2x2, block_2x128 / 2x256 / 2x512 / 8x256, long
    (torch.float32, 37, 100, 100, 0), (torch.float32, 64, 300, 300, 0), (torch.float32, 33, 1000, 1000, 0),
    (torch.float32, 16, 2000, 2000, 0), (torch.float32, 9, 4000, 4000, 0), (torch.float32, 5, 8000, 8000, 0),
    (torch.float32, 3, 9000, 9000, 0),
    (torch.float32, 64, 1024, 1000, 0),   # tile narrower than the row: the rest is untouched
    (torch.float32, 64, 1024, 1024, 1),   # unaligned rows
    (torch.float32, 30, 100, 128, 0),     # tile wider than the row: padded_f32
    (torch.float16, 64, 1024, 1024, 0), (torch.float16, 10, 100, 100, 1),  # f16
    (torch.float16, 30, 100, 128, 0),     # padded_f16
])
def test_softmax_code_object_matches_library(device, cache_dir, dtype, rows, cols, tile, offset):
    x, out_co = _softmax_inputs(dtype, rows, cols, rows * cols + tile, device, offset)
    out_lib = out_co.clone()
    plan = kernels.softmax_plan(x, out_co, rows, cols, tile, 16, False)
    _softmax_rows()[16](x, out_co, rows, cols, tile)
    kernels.softmax_rows(x, out_lib, rows, cols, tile, 16)
    torch.cuda.synchronize()
    assert torch.equal(out_co.view(torch.int16 if dtype == torch.float16 else torch.int32),
                       out_lib.view(torch.int16 if dtype == torch.float16 else torch.int32)), plan.kernel
    n = min(tile, cols)
    assert (out_co[:, n:] == 7.0).all()
    if tile <= cols:
        torch.testing.assert_close(out_co[:, :n].float(), torch.softmax(x[:, :n].float(), dim=1),
                                   rtol=1e-3 if dtype == torch.float16 else 1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype,rows,cols,block_size", [(torch.float32, 64, 1024, 4), (torch.float32, 100, 300, 3),
                                                        (torch.float16, 64, 1024, 4)])
def test_softmax_fused_code_object_matches_library(device, cache_dir, dtype, rows, cols, block_size):
    x, out_co = _softmax_inputs(dtype, rows, cols, rows + cols, device)
    out_lib = out_co.clone()
    _softmax_fused()[16](x, out_co, rows, cols, block_size)
    kernels.softmax_blocks(x, out_lib, rows, cols, block_size, 16)
    torch.cuda.synchronize()
    assert torch.equal(out_co, out_lib)
    covered = min(rows, 16 * block_size)
    assert (out_co[covered:] == 7.0).all()
    torch.testing.assert_close(out_co[:covered].float(), torch.softmax(x[:covered].float(), dim=1),
                               rtol=1e-3 if dtype == torch.float16 else 1e-5, atol=1e-6)


def test_softmax_code_object_cache(device, cache_dir):
    x, out = _softmax_inputs(torch.float32, 64, 1024, 3, device)
    k = _softmax_rows()
    loads = module.stats["module_loads"]
    launches = module.stats["launches"]
    for _ in range(4):  # one load, then memory-cache hits
        k[16](x, out, 64, 1024, 1024)
    assert module.stats["module_loads"] == loads + 1 and module.stats["launches"] == launches + 4
    assert len(list(cache_dir.rglob("softmax_kernel.hsaco"))) == 1
    always = _softmax_rows(always_compile=True)
    always[16](x, out, 64, 1024, 1024)
    always[16](x, out, 64, 1024, 1024)
    assert module.stats["module_loads"] == loads + 3
    torch.cuda.synchronize()
    torch.testing.assert_close(out, torch.softmax(x, dim=1), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------- leaky_relu / vmuladd / gelu

def _leaky_relu():
    @asc2.jit
    def leaky_relu_kernel(x_ptr: asc.GlobalAddress, alpha: float, out_ptr: asc.GlobalAddress, size: int,
                          tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
        """where(x >= 0, x, x * alpha) over the tiles of block b
        (python/test/asc2/kernels/test_leaky_relu.py's kernel)."""

    return leaky_relu_kernel


def _vmuladd():
    @asc2.jit(vf_fusion=True)
    def vmuladd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, z_ptr: asc.GlobalAddress,
                       out_ptr: asc.GlobalAddress, size: int, tile_size: asc.ConstExpr[int],
                       tile_per_block: asc.ConstExpr[int], buffer_factor: asc.ConstExpr[int]):
        """x * y + z, unfused, over the tiles of block b (python/test/asc2/kernels/test_vmuladd.py's kernel)."""

    return vmuladd_kernel


def _gelu():
    @asc2.jit
    def gelu_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: asc.ConstExpr,
                    num_columns: asc.ConstExpr, tile_size: asc.ConstExpr, approximate: asc.ConstExpr):
        """Grid-strided gelu rows, tanh or erf form (python/test/asc2/kernels/test_gelu.py's kernel)."""

    return gelu_kernel


def _bits_equal(a, b):
    view = torch.int16 if a.element_size() == 2 else torch.int32
    return torch.equal(a.view(view), b.view(view))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("size,tile,tpb,grid,offset", [(8192, 128, 4, 16, 0), (3001, 7, 5, 11, 0),
                                                      (1 << 20, 128, 512, 16, 0), (5000, 64, 5, 16, 1),
                                                      (1 << 21, 128, 1024, 16, 1)])
def test_leaky_relu_and_vmuladd_code_objects_match_library(device, cache_dir, dtype, size, tile, tpb, grid,
                                                           offset):
    # offset 1: unaligned views take the element kernel (past 2^20 elements: its grid-stride loop)
    g = torch.Generator().manual_seed(size + tile)
    x, y, z = ((torch.randn(size + offset, generator=g) * 3).to(dtype).to(device)[offset:] for _ in range(3))
    alpha = 0.1 if dtype == torch.float32 else float(torch.tensor(0.1, dtype=dtype).item())
    fill = torch.full((size + offset,), 5.0, dtype=dtype, device=device)[offset:]
    co, lib = fill.clone(), fill.clone()
    _leaky_relu()[grid](x, alpha, co, size, tile, tpb)
    kernels.leaky_relu(x, alpha, lib, size, tile, tpb, grid)
    torch.cuda.synchronize()
    assert _bits_equal(co, lib)
    co, lib = fill.clone(), fill.clone()
    _vmuladd()[grid](x, y, z, co, size, tile, tpb, 2)
    kernels.vmuladd(x, y, z, lib, size, tile, tpb, grid)
    torch.cuda.synchronize()
    assert _bits_equal(co, lib)
    covered = min(size, grid * tpb * tile)
    assert (co[covered:] == 5.0).all()
    if dtype != torch.float32:  # torch's own mul-then-add in that dtype, bit-exact
        assert _bits_equal(co[:covered], (x[:covered] * y[:covered] + z[:covered]))


@pytest.mark.parametrize("approximate", [True, False])
@pytest.mark.parametrize("rows,cols,tile,offset", [(30, 1024, 1024, 0), (37, 1000, 1000, 0), (64, 4096, 3000, 0),
                                                   (9, 100, 128, 0), (10000, 64, 64, 0), (33, 256, 256, 1)])
def test_gelu_code_object_matches_library(device, cache_dir, approximate, rows, cols, tile, offset):
    g = torch.Generator().manual_seed(rows * cols)
    x = (torch.randn(rows * cols + offset, generator=g) * 3).to(device)[offset:].view(rows, cols)
    fill = torch.full((rows * cols + offset,), 5.0, device=device)[offset:].view(rows, cols)
    co, lib = fill.clone(), fill.clone()
    _gelu()[16](x, co, rows, cols, tile, approximate)
    kernels.gelu_rows(x, lib, rows, cols, tile, approximate, 16)
    torch.cuda.synchronize()
    assert _bits_equal(co, lib)
    n = min(tile, cols)
    assert (co[:, n:] == 5.0).all()


def test_elementwise_code_object_loaded_once(device, cache_dir):
    x = torch.randn(8192, device=device)
    out = torch.empty_like(x)
    k = _leaky_relu()
    loads = module.stats["module_loads"]
    for _ in range(3):
        k[16](x, 0.2, out, 8192, 128, 4)
    assert module.stats["module_loads"] == loads + 1
    assert len(list(cache_dir.rglob("leaky_relu_kernel.hsaco"))) == 1
    torch.cuda.synchronize()
    assert torch.equal(out, torch.where(x >= 0, x, x * torch.tensor(0.2, dtype=torch.float32)))


# ------------------------------------------------------------- matmul / int8 / attention code objects

@pytest.fixture
def library_path(monkeypatch):
    """Calling it makes the registered kernels launch through the library's entry points
    instead of their code objects for the rest of the test (calls that resolve afresh:
    always_compile)."""
    import dataclasses
    from pyasc_amd import registry

    def force():
        for key, entry in list(registry._REGISTRY.items()):
            if entry.code_object is not None:
                monkeypatch.setitem(registry._REGISTRY, key, dataclasses.replace(entry, code_object=None))
    return force


def _both_paths(library_path, run):
    """run() through the code object, then through the library; returns both results."""
    launches = module.stats["launches"]
    first = run()
    torch.cuda.synchronize()
    assert module.stats["launches"] > launches  # the first call went through a code object
    library_path()
    launches = module.stats["launches"]
    second = run()
    torch.cuda.synchronize()
    assert module.stats["launches"] == launches  # the second did not
    return first, second


@pytest.mark.parametrize("form,dtype,m,k,n", [
    ("mnblock", torch.float16, 480, 224, 1344), ("mnblock", torch.bfloat16, 512, 256, 512),
    ("tiled", torch.float16, 64, 128, 256), ("fixpipe", torch.float32, 64, 128, 128),
    ("fixpipe", torch.float16, 64, 128, 256), ("fixpipe", torch.bfloat16, 1024, 512, 768),
    ("chained", torch.bfloat16, 64, 64, 64), ("chained", torch.float16, 256, 256, 256)])
def test_matmul_code_object_matches_library(device, cache_dir, library_path, form, dtype, m, k, n):
    import test_gpu_reference_style as ref
    g = torch.Generator().manual_seed(m + k + n)
    a = ((torch.rand((m, k), generator=g) - .5) * 4).to(dtype).to(device)
    b = ((torch.rand((k, n), generator=g) - .5) * 4).to(dtype).to(device)

    def run():
        if form == "mnblock":
            c = torch.zeros((m, n), device=device)
            cores, m_tile, n_tile, ntpb = (30, 48, 32, 7) if m == 480 else (4, 128, 64, 2)
            mtpb = ref._m_tiles_per_block(m, k, n, cores, m_tile, n_tile, ntpb)
            ref._mnblock_kernel()[cores](a, b, c, a.shape, b.shape, c.shape, m_tile, mtpb, n_tile, ntpb)
        elif form == "tiled":
            c = torch.zeros((m, n), device=device)
            ref._tiled_kernel()[1](a, b, c, a.shape, b.shape, c.shape, 4)
        elif form == "fixpipe":
            c = torch.zeros((m, n), dtype=torch.float16, device=device)
            ref._fixpipe_kernel()[1](a, b, c, a.shape, b.shape, c.shape)
        else:
            c = torch.zeros((m, n), device=device)
            ref._chained_kernel()[1](a, b, c, a.shape, b.shape, c.shape,
                                     asc.float16 if dtype == torch.float16 else asc.bfloat16)
        return c

    co, lib = _both_paths(library_path, run)
    assert _bits_equal(co, lib)
    expect = a.float() @ b.float()
    if form == "fixpipe":
        expect = expect.relu()
    if form != "chained":
        torch.testing.assert_close(co.float(), expect, atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("m,k,n", [(512, 256, 512), (100, 64, 300), (256, 4096, 256)])
def test_int8_code_object_matches_library(device, cache_dir, library_path, m, k, n):
    import test_gpu_reference_style as ref
    g = torch.Generator().manual_seed(m * n + k)
    a = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g).to(device)
    b = torch.randint(-127, 128, (k, n), dtype=torch.int8, generator=g).to(device)
    scale = (torch.rand(n, generator=g) * 0.009 + 0.001).to(device)

    def run():
        acc = torch.zeros((m, n), dtype=torch.int32, device=device)
        out = torch.zeros((m, n), dtype=torch.float16, device=device)
        ref.matmul_int8_kernel[16](a, b, acc, a.shape, b.shape, acc.shape, always_compile=True)
        ref.matmul_dequant_kernel[16](a, b, out, scale, a.shape, b.shape, out.shape, True, always_compile=True)
        return acc, out

    (acc_co, out_co), (acc_lib, out_lib) = _both_paths(library_path, run)
    assert torch.equal(acc_co, acc_lib) and _bits_equal(out_co, out_lib)
    assert torch.equal(acc_co.cpu(), (a.cpu().double() @ b.cpu().double()).to(torch.int32))


@pytest.mark.parametrize("B,H,S,D,causal", [(2, 4, 512, 128, False), (2, 4, 512, 128, True), (1, 3, 300, 64, True),
                                            (1, 8, 1024, 64, False)])
def test_attention_code_object_matches_library(device, cache_dir, library_path, B, H, S, D, causal):
    from test_gpu_attention import flash_attention_fwd_kernel
    g = torch.Generator().manual_seed(S + D)
    q, k, v = ((torch.randn(B, H, S, D, generator=g)).to(torch.bfloat16).to(device) for _ in range(3))

    def run():
        o = torch.empty_like(q)
        flash_attention_fwd_kernel[16](q, k, v, o, B, H, S, D, 1 / D ** 0.5, causal, 128, 64, always_compile=True)
        return o

    co, lib = _both_paths(library_path, run)
    assert _bits_equal(co, lib)
