"""Launch-surface behaviour (CPU only): decorator options, argument classification,
ConstExpr handling, signature dispatch and error paths of the asc/asc2 drop-in.
The native launch is replaced by a recorder, as the reference's unit tests patch
Launcher.run (python/test/unit/conftest.py:35-38)."""
import numpy as np
import pytest
import torch

import asc
import asc2
import asc.runtime.config as config
from pyasc_amd import registry
from pyasc_amd.asc.runtime import launcher as launcher_mod
from pyasc_amd.asc.runtime.jit import JITFunction
from pyasc_amd.launchers import mnblock_rectangles


@asc2.jit(always_compile=True)
def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
    """Declaration: binds the registered vadd kernel by its signature."""


@pytest.fixture
def recorded(monkeypatch):
    calls = []

    def fake_run(self, entry, function_name, runtime_args, constexprs, options=None, resolved=None):
        calls.append((entry, function_name, runtime_args, constexprs, self.options, options))

    monkeypatch.setattr(launcher_mod.Launcher, "run", fake_run)
    return calls


def test_dispatch_by_signature(recorded):
    x = np.zeros(8192, np.float32)
    vadd_kernel[16](x, x, x, 8192, 128, 4)
    entry, name, rt, ce, opts, _ = recorded[0]
    assert name == "vadd_kernel" and entry.params[-1] == "tile_per_block"
    assert entry.reference.startswith("python/test/asc2/kernels/test_vadd.py")
    assert list(rt) == ["x_ptr", "y_ptr", "out_ptr", "size"] and ce == {"tile_size": 128, "tile_per_block": 4}
    assert opts.core_num == 16 and opts.stream is None


def test_launch_tuple_with_stream(recorded):
    x = torch.zeros(16)
    vadd_kernel[4, 1234](x, x, x, 16, 4, 1)
    assert recorded[0][4].core_num == 4 and recorded[0][4].stream == 1234


def test_bad_launch_options():
    with pytest.raises(TypeError, match="Parse user launch options failed"):
        vadd_kernel[1, 2, 3]


def test_unknown_option_and_clash():
    with pytest.raises(RuntimeError, match="unknown"):
        asc2.jit(not_an_option=1)(lambda x: None)

    def k(x, always_compile):
        pass

    with pytest.raises(RuntimeError, match="conflict"):
        asc2.jit(k)


def test_reference_option_names_accepted():
    for opt in ("vf_fusion", "always_compile", "opt_level", "insert_sync", "static_alloc", "kernel_type"):
        asc2.jit(**{opt: None})(lambda x: None)


def test_constexpr_type_check(recorded):
    with pytest.raises(RuntimeError, match=r"ConstExpr\[int\] is required for 'tile_size'"):
        vadd_kernel[1](np.zeros(4, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32), 4, 1.5, 1)


def test_arg_type_classification():
    gat = JITFunction.get_arg_type
    assert gat(True).kind == "plain" and str(gat(True).dtype) == "int8"
    assert str(gat(3).dtype) == "int32" and str(gat(3.0).dtype) == "float32"
    assert gat(np.zeros(3, np.float16)).kind == "pointer"
    assert gat(np.float32(1)).kind == "plain"
    assert gat(torch.zeros(2, dtype=torch.bfloat16)).kind == "pointer"
    t0 = gat(torch.tensor(1.0, dtype=torch.bfloat16))
    assert t0.kind == "plain" and str(t0.dtype) == "bfloat16"
    with pytest.raises(TypeError, match="not supported: str"):
        gat("x")


def test_unsupported_runtime_arg_raises(recorded):
    with pytest.raises(TypeError):
        vadd_kernel[1]("a", "b", "c", 4, 1, 1)


def test_unknown_kernel_raises():

    @asc2.jit
    def my_kernel(a_ptr: asc.GlobalAddress, n: int):
        pass

    with pytest.raises(NotImplementedError, match="my_kernel"):
        my_kernel[1](np.zeros(4, np.float32), 4)


def test_core_num_and_dry_run(monkeypatch):
    monkeypatch.delenv("DRY_RUN", raising=False)
    with pytest.raises(ValueError, match="Core number"):
        vadd_kernel[0](np.zeros(4, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32), 4, 4, 1)
    monkeypatch.setenv("DRY_RUN", "1")
    vadd_kernel[1](np.zeros(4, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32), 4, 4, 1)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device error")
def test_no_device_fails_loudly(monkeypatch):
    monkeypatch.delenv("DRY_RUN", raising=False)
    with pytest.raises(RuntimeError, match="No HIP device"):
        vadd_kernel[1](np.zeros(4, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32), 4, 4, 1)


def test_missing_library_or_code_object_fails_loudly(tmp_path):
    # no CPU fallback: an unbuilt library or code object is an error naming the build step
    from pyasc_amd import _native
    from pyasc_amd.asc.runtime import module
    with pytest.raises(RuntimeError, match="not built"):
        _native.load_library(tmp_path / "libasc_hip.so")
    missing = module.CodeObject("absent", ("k",), lambda call, functions: None, "pyasc_amd/csrc/co/absent.hip")
    with pytest.raises(RuntimeError, match="not built"):
        module.compiled_path(missing, None, "k")


def test_tile_ops_are_not_callable_outside_kernels():
    with pytest.raises(RuntimeError, match="only appear inside"):
        asc2.load(None, [1], offsets=[0])
    with pytest.raises(ValueError):
        asc2.range(4, unroll_factor=0)


def test_kernel_called_without_grid():
    with pytest.raises(TypeError, match="launch it as"):
        vadd_kernel(1, 2, 3, 4, 5, 6)


def test_registry_contents():
    names = {(n, p[-1]) for n, p in registry.entries()}
    assert ("softmax_kernel", "tile_size") in names and ("softmax_kernel", "block_size") in names
    # four asc2 matmul tests, two asc1 ones (python/test/kernels/test_matmul.py, test_matmul_torch.py),
    # tutorials 03 and 04
    assert sum(1 for n, _ in registry.entries() if n == "matmul_kernel") == 8
    vadds = {p for n, p in registry.entries() if n == "vadd_kernel"}
    assert ("x", "y", "z", "BLOCK_LENGTH", "BUFFER_NUM", "TILE_LENGTH", "TILE_NUM") in vadds  # asc1 test_vadd.py
    assert ("x", "y", "z", "block_length") in vadds and ("x", "y", "z", "block_length", "tile_length") in vadds
    assert ("flash_attention_fwd_kernel", "block_n") in names
    assert ("matmul_dequant_kernel", "c_shape") in names
    assert ("leaky_relu_kernel", "tile_per_block") in names and ("vmuladd_kernel", "buffer_factor") in names
    assert ("gelu_kernel", "approximate") in names


@asc2.jit(always_compile=True)
def leaky_relu_kernel(x_ptr: asc.GlobalAddress, alpha: float, out_ptr: asc.GlobalAddress, size: int,
                      tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
    pass


@asc2.jit(always_compile=True)
def gelu_kernel(x_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, num_rows: asc.ConstExpr,
                num_columns: asc.ConstExpr, tile_size: asc.ConstExpr, approximate: asc.ConstExpr):
    pass


def test_scalar_and_bare_constexpr_arguments(recorded):
    # test_leaky_relu.py passes alpha as a 0-dim bf16 tensor to an `alpha: float` parameter (by value);
    # test_gelu.py annotates with bare asc.ConstExpr
    x = torch.zeros(256, dtype=torch.bfloat16)
    alpha = torch.tensor(0.1, dtype=torch.bfloat16)
    leaky_relu_kernel[16](x, alpha, x, 256, 128, 1)
    entry, name, rt, ce, _, _ = recorded[0]
    assert entry.params[1] == "alpha" and rt["alpha"] is alpha and ce == {"tile_size": 128, "tile_per_block": 1}
    assert launcher_mod.Launcher.scalar_value(rt["alpha"]) == float(alpha.item())
    gelu_kernel[16](torch.zeros(2, 8), torch.zeros(2, 8), 2, 8, 8, True)
    assert recorded[1][3] == {"num_rows": 2, "num_columns": 8, "tile_size": 8, "approximate": True}


def test_set_platform_surface():
    with pytest.raises(ValueError):
        config.set_platform("Bogus")
    config.set_platform(config.Backend.Model, config.Platform.Ascend950PR_9599, 0, check=False)
    assert config.platform_to_arch(config.Platform.Ascend950PR_9599) == config.CompilationArch.C310
    assert config.platform_to_arch(config.Platform.MI355X) == config.CompilationArch.GFX950


def test_launcher_mnblock_rectangles_merge():
    # all 8 parametrisations of test_matmul_mnblock.py cover C exactly
    rects = mnblock_rectangles(480, 1344, 30, 48, 2, 32, 7)  # 420 tiles, 14 per block
    area = sum((m1 - m0) * (n1 - n0) for m0, m1, n0, n1 in rects)
    assert area == 480 * 1344


def test_ceildiv_and_dtypes():
    assert asc.ceildiv(8192, 128) == 64 and asc.ceildiv(1, 16) == 1
    assert asc.float16.to_torch() == torch.float16 and asc.bfloat16.is_float() and asc.int8.is_int()


# ---------------------------------------------------------------------------------- kernel cache
# The reference caches what a call compiles to under its cache factors and skips the
# cache with always_compile (python/asc/runtime/jit.py:139-186); here the cached
# value is the resolved native kernel.

def _cached_vadd(**options):
    @asc2.jit(**options)
    def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                    tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
        pass

    return vadd_kernel


@pytest.fixture
def lookups(monkeypatch):
    seen = []
    real = registry.lookup

    def counting(name, params, body_fingerprint=None):
        seen.append(name)
        return real(name, params, body_fingerprint)

    monkeypatch.setattr(registry, "lookup", counting)
    return seen


def test_cache_hit_skips_resolution(recorded, lookups):
    k = _cached_vadd()
    x = torch.zeros(64)
    for _ in range(3):
        k[2](x, x, x, 64, 8, 4)
    assert len(lookups) == 1 and len(k.kernel_cache) == 1
    assert [r[3] for r in recorded] == [{"tile_size": 8, "tile_per_block": 4}] * 3
    assert all(r[0] is recorded[0][0] for r in recorded)
    # new specialisations: a ConstExpr value, an argument dtype, a by-value type, an option
    k[2](x, x, x, 64, 16, 4)
    k[2](x.double(), x, x, 64, 8, 4)
    k[2](x, x, x, torch.tensor(64), 8, 4)
    k[2](x, x, x, 64, 8, 4, debug=True)
    assert len(k.kernel_cache) == 5 and len(lookups) == 5
    # the launch options are not part of the key (LaunchOptions are not cache factors)
    k[7](x, x, x, 64, 8, 4)
    assert len(k.kernel_cache) == 5 and recorded[-1][4].core_num == 7


def test_always_compile_bypasses_cache(recorded, lookups):
    k = _cached_vadd(always_compile=True)
    x = torch.zeros(64)
    k[2](x, x, x, 64, 8, 4)
    k[2](x, x, x, 64, 8, 4)
    assert len(lookups) == 2 and k.kernel_cache == {}
    k2 = _cached_vadd()
    k2[2](x, x, x, 64, 8, 4)
    k2[2](x, x, x, 64, 8, 4, always_compile=True)  # per-call option: resolved afresh, nothing stored
    assert len(lookups) == 4 and len(k2.kernel_cache) == 1


def test_cache_miss_still_validates(recorded):
    k = _cached_vadd()
    x = torch.zeros(64)
    k[2](x, x, x, 64, 8, 4)
    with pytest.raises(RuntimeError, match="ConstExpr"):
        k[2](x, x, x, 64, 8.0, 4)  # ConstExpr[int] given a float: a new key, validated
    with pytest.raises(TypeError):
        k[2](x, x, x, "64", 8, 4)  # unsupported runtime argument type
    assert len(k.kernel_cache) == 1


def test_cache_key_components():
    from pyasc_amd.asc.runtime import cache
    k = _cached_vadd()
    factors = k._gen_cache_factors({"x_ptr": "pointer:float32", "size": "plain:int32"}, {"tile_size": 8},
                                   {"debug": True, "core_num": 3})
    assert factors == "debug=True__tile_size=8__x_ptr=pointer:float32;size=plain:int32__fn_name=vadd_kernel"
    assert cache.get_mem_cache_key(factors) == cache.hexdigest(f"{cache.library_key()}__{factors}".encode())
    assert k.cache_key == _cached_vadd().cache_key != vadd_kernel.cache_key
    assert JITFunction.arg_kind(torch.zeros(3, dtype=torch.bfloat16)) == "pointer:bfloat16"
    assert JITFunction.arg_kind(torch.tensor(1.5)) == "plain:float32"
    assert JITFunction.arg_kind(np.zeros(3, np.int8)) == "pointer:int8"
    assert JITFunction.arg_kind(np.float16(1)) == "plain:float16"
    assert JITFunction.arg_kind(True) == "plain:int8"


def test_string_annotations_with_local_import(recorded, tmp_path):
    # `from __future__ import annotations` with asc imported inside a function: the
    # annotation strings cannot be evaluated in the module globals, ConstExpr is
    # still recognised by its text
    import importlib.util
    src = (
        "from __future__ import annotations\n"
        "def make():\n"
        "    import asc, asc2\n"
        "    @asc2.jit\n"
        "    def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress,\n"
        "                    size: int, tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):\n"
        "        pass\n"
        "    return vadd_kernel\n")
    path = tmp_path / "local_import_kernels.py"
    path.write_text(src)  # a real file, so the body's source can be read for its fingerprint
    spec = importlib.util.spec_from_file_location("local_import_kernels", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    k = mod.make()
    x = torch.zeros(64)
    k[2](x, x, x, 64, 8, 4)
    k[2](x, x, x, 64, 8, 4, always_compile=True)
    assert [r[3] for r in recorded] == [{"tile_size": 8, "tile_per_block": 4}] * 2
    assert list(recorded[0][2]) == ["x_ptr", "y_ptr", "out_ptr", "size"]


def test_asc1_signatures_evaluate_and_runtime_checks():
    # asc1 helper signatures annotate with asc.TQue / asc.GlobalTensor
    # (python/test/kernels/test_vadd.py:38-64); the names exist, constructing them raises
    import asc.lib.runtime as rt

    @asc.jit
    def copy_out(i: int, z_gm: asc.GlobalTensor, out_queue_z: asc.TQue, TILE_LENGTH: asc.ConstExpr[int]):
        pass

    assert copy_out.fn_name == "copy_out"
    with pytest.raises(RuntimeError, match="only appear inside"):
        asc.TQue()
    assert rt.default_device() == 0
    rt.check_device_handle(3)
    for bad in (-1, "0", 1.0, True):
        with pytest.raises(RuntimeError, match="int >= 0"):
            rt.check_device_handle(bad)
    with pytest.raises(ValueError, match="priority 0"):
        rt.create_stream(priority=-1)


@pytest.mark.parametrize("m, n, k, dim", [(512, 1024, 512, 48), (128, 30720, 64, 24), (1, 1, 1, 1), (7, 5, 3, 2),
                                          (4096, 4096, 64, 512), (300, 17, 9, 7)])
def test_host_tiling_covers_the_output(m, n, k, dim):
    # the split is build-defined; what a launch needs is that used_core_num instances of
    # single_core_m x single_core_n tiles cover m x n, with at most dim instances
    import asc.lib.host as host
    t = host.MultiCoreMatmulTiling(host.get_ascendc_platform())
    assert t.set_a_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT16, False) == 0
    assert t.set_c_type(host.TPosition.GM, host.CubeFormat.ND, host.DataType.DT_FLOAT) == 0
    assert t.set_dim(dim) == 0 and t.set_org_shape(m, n, k) == 0 and t.set_shape(m, n, k) == 0
    assert t.enable_bias(True) == 0 and t.set_buffer_space(-1, -1, -1) == 0
    tiling = asc.adv.TCubeTiling()
    assert t.get_tiling(tiling) == 0
    tiles = -(-m // tiling.single_core_m) * -(-n // tiling.single_core_n)
    assert tiles == tiling.used_core_num <= dim
    assert (tiling.m, tiling.n, tiling.k_a, tiling.k_b, tiling.is_bias) == (m, n, k, k, 1)
    assert tiling.single_core_m % 16 == 0 and tiling.single_core_n % 16 == 0
    assert host.DataType.DT_BFLOAT16 is host.DataType.DT_BF16


def test_compile_options_reach_the_launch(recorded):
    # matmul_cube_only decides how many instances an asc1 Matmul launch runs
    # (python/asc/runtime/compiler.py:291-299); it travels with the call
    @asc.jit(matmul_cube_only=True)
    def matmul_kernel(a: asc.GlobalAddress, b: asc.GlobalAddress, c: asc.GlobalAddress, bias: asc.GlobalAddress,
                      tiling: asc.adv.TCubeTiling, workspace: asc.GlobalAddress):
        pass

    a = np.zeros((4, 4), np.float16)
    matmul_kernel[3](a, a, np.zeros((4, 4), np.float32), np.zeros(4, np.float32), asc.adv.TCubeTiling(), a)
    assert recorded[-1][-1]["matmul_cube_only"] is True


@pytest.mark.parametrize("n, grid, stride, cover", [(8192, 16, 512, 512), (8191, 16, 512, 1024), (100, 3, 40, 7),
                                                    (10, 5, 4, 3), (5, 16, 1, 8), (0, 4, 4, 4), (50, 0, 4, 4)])
def test_block_ranges_match_oracle_coverage(n, grid, stride, cover):
    # the launchers' asc1 block ranges write exactly the elements the oracle's block_add writes
    from oracle import asc2_oracle as O
    from pyasc_amd.launchers_asc1 import _block_ranges
    mask = np.zeros(n, bool)
    for s, e in _block_ranges(n, grid, stride, cover):
        assert 0 <= s < e <= n
        mask[s:e] = True
    written = O.block_add(np.ones(n, np.float32), np.ones(n, np.float32), np.zeros(n, np.float32), grid, stride,
                          cover) != 0
    np.testing.assert_array_equal(mask, written)


def test_matmul_instances_per_kernel_type():
    # MIX_AIC_1_2 (the default for mixed Matmul kernels) runs two instances per block,
    # AIC_ONLY / matmul_cube_only and the other types one (python/asc/runtime/compiler.py:291-299)
    from pyasc_amd.launchers_asc1 import _matmul_instances
    from pyasc_amd.registry import KernelCall
    import asc.runtime.config as config

    def call(**options):
        return KernelCall("matmul_kernel", {}, {}, 12, 0, {"options": options})
    assert _matmul_instances(call()) == 24
    assert _matmul_instances(call(matmul_cube_only=True)) == 12
    assert _matmul_instances(call(kernel_type=config.KernelType.MIX_AIC_1_2)) == 24
    assert _matmul_instances(call(kernel_type=config.KernelType.AIC_ONLY)) == 12
    assert _matmul_instances(call(kernel_type=config.KernelType.MIX_AIC_1_1)) == 12


def test_quick_key_keeps_cache_factors_apart(recorded):
    # 1, True and 1.0 are equal in Python but distinct cache factors (their reprs differ);
    # the quick key tags values with their types, so each gets its own specialisation
    @asc2.jit
    def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                    tile_size: asc.ConstExpr, tile_per_block: asc.ConstExpr):
        pass

    import torch
    for x in (np.zeros(8, np.float32), torch.zeros(8)):  # numpy takes the full path, torch the quick key
        keys = set()
        for tpb in (1, True, 1.0, 1, True):
            resolved, _, consts = vadd_kernel.resolve(x, x, x, 8, 8, tpb)
            keys.add(resolved.cache_key)
            assert consts["tile_per_block"] == tpb and type(consts["tile_per_block"]) is type(tpb)
        assert len(keys) == 3
    t = torch.zeros(8)
    assert vadd_kernel.resolve(t, t, t, 8, 8, 1)[0].cache_key != \
        vadd_kernel.resolve(t.half(), t, t, 8, 8, 1)[0].cache_key
    assert vadd_kernel.resolve(t, t, t, 8, 8, 1)[0].cache_key != \
        vadd_kernel.resolve(t, t, t, torch.tensor(8), 8, 1)[0].cache_key


def test_invalid_compile_option(recorded):
    # python/test/unit/runtime/test_compiler.py:89-92: opt_level 0 is rejected when the kernel
    # is compiled; here, when the call is resolved without a cached specialisation
    for bad in ({"opt_level": 0}, {"kernel_type": 3}):
        @asc.jit(**bad)
        def copy_kernel(x: asc.GlobalAddress, z: asc.GlobalAddress, data_size: asc.ConstExpr[int]):
            pass

        x = np.zeros(8, np.float32)
        with pytest.raises(RuntimeError, match="Please check input compile option"):
            copy_kernel[1](x, x, 8)
    import asc.runtime.config as config

    @asc.jit(opt_level=2, kernel_type=config.KernelType.AIV_ONLY)
    def copy_kernel(x: asc.GlobalAddress, z: asc.GlobalAddress, data_size: asc.ConstExpr[int]):
        pass

    copy_kernel[1](np.zeros(8, np.float32), np.zeros(8, np.float32), 8)
    assert recorded[-1][-1]["opt_level"] == 2


# ------------------------------------------------------------------------------ body fingerprints
# Dispatch is by (name, parameter names); the body must also be one the native kernel
# implements (a reference body of that signature) or a declaration.

REFERENCE_ROOT = "/root/reference"
_HAVE_REFERENCE = __import__("os").path.isdir(REFERENCE_ROOT + "/python/test")


def _reference_kernel_node(relpath: str, name: str):
    """The reference kernel's definition, parsed from its file as text (never imported)."""
    import ast
    import os
    with open(os.path.join(REFERENCE_ROOT, relpath), encoding="utf-8") as f:
        tree = ast.parse(f.read())
    return next(n for n in ast.walk(tree) if isinstance(n, ast.FunctionDef) and n.name == name)


class _Rename(__import__("ast").NodeTransformer):
    """Gives every local a new name and adds loop hints to range calls."""

    def __init__(self, params):
        self.params, self.names = set(params), {}

    def visit_Name(self, node):
        if node.id not in self.params and node.id not in ("asc", "asc2", "range"):
            node.id = self.names.setdefault(node.id, f"renamed_{len(self.names)}")
        return node

    def visit_Call(self, node):
        import ast
        self.generic_visit(node)
        if isinstance(node.func, ast.Name) and node.func.id == "range":
            node.keywords.append(ast.keyword(arg="unroll_factor", value=ast.Constant(2)))
        return node


@pytest.mark.skipif(not _HAVE_REFERENCE, reason="the reference tree is present only in the build container")
def test_reference_body_binds_and_renaming_keeps_its_fingerprint():
    # the reference's asc2 vadd kernel (python/test/asc2/kernels/test_vadd.py:16-28), read as
    # text: its fingerprint is in the table and binds; renaming its locals and adding loop
    # hints (a different text of the same computation) keeps the fingerprint
    import ast
    import copy
    from pyasc_amd import fingerprint
    node = _reference_kernel_node("python/test/asc2/kernels/test_vadd.py", "vadd_kernel")
    params = tuple(a.arg for a in node.args.args)
    fp = fingerprint.body_fingerprint(node)
    assert fp in fingerprint.known_fingerprints()[fingerprint.signature_key("vadd_kernel", params)]
    assert registry.lookup("vadd_kernel", params, fp).name == "vadd_kernel"
    renamed = _Rename(params).visit(copy.deepcopy(node))
    assert ast.unparse(renamed) != ast.unparse(node)
    assert fingerprint.body_fingerprint(renamed) == fp


def test_fingerprint_normalisation():
    # locals renamed, a single-use temporary inlined, loop hints and a docstring dropped:
    # the same fingerprint; another operator: a different one
    import ast
    from pyasc_amd import fingerprint

    def fp(text):
        return fingerprint.body_fingerprint(ast.parse(text).body[0])

    a = ("def k(p, n):\n    t = asc2.tensor(p, [n])\n    for i in range(n):\n"
         "        v = asc2.load(t, [1], offsets=[i])\n        w = v * 2\n        asc2.store(w, t, offsets=[i])\n")
    b = ("def k(p, n):\n    'Doubles p in place.'\n    g = asc2.tensor(p, [n])\n"
         "    for j in range(n, unroll_factor=4, parallel=True):\n"
         "        u = asc2.load(g, [1], offsets=[j])\n        asc2.store(u * 2, g, offsets=[j])\n")
    c = a.replace("v * 2", "v + 2")
    assert fp(a) == fp(b) != fp(c)
    assert fp("def k(p, n):\n    'Declared.'\n    ...\n") == fingerprint.DECLARATION
    assert fp("def k(p, n):\n    pass\n") == fingerprint.DECLARATION


def _declared_vadd():
    @asc2.jit
    def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                    tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
        """Declaration: binds the registered vadd kernel by its signature."""

    return vadd_kernel


def _different_vadd_body():
    # the vadd signature with a body that computes something else (out = 2 x over one tile)
    @asc2.jit
    def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress, size: int,
                    tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
        src = asc2.load(asc2.tensor(x_ptr, [size]), [tile_size], offsets=[0])
        asc2.store(src * 2, asc2.tensor(out_ptr, [size]), offsets=[0])

    return vadd_kernel


def test_declaration_dispatch(recorded):
    x = np.zeros(64, np.float32)
    for k in (_declared_vadd(), _cached_vadd()):
        k[2](x, x, x, 64, 8, 4)
    assert len(recorded) == 2 and all(r[0].name == "vadd_kernel" for r in recorded)
    assert _declared_vadd().body_fingerprint == _cached_vadd().body_fingerprint == "declaration"


def test_different_body_is_refused(recorded, monkeypatch):
    monkeypatch.delenv(registry.ALLOW_BODY_MISMATCH_ENV, raising=False)
    x = np.zeros(64, np.float32)
    for options in ({}, {"always_compile": True}):
        k = _different_vadd_body()
        with pytest.raises(registry.KernelBodyMismatch, match="differs from every body"):
            k[2](x, x, x, 64, 8, 4, **options)
    assert not recorded
    # the explicit opt-out runs the registered kernel with a warning
    monkeypatch.setenv(registry.ALLOW_BODY_MISMATCH_ENV, "1")
    with pytest.warns(RuntimeWarning, match="differs from every body"):
        _different_vadd_body()[2](x, x, x, 64, 8, 4)
    assert len(recorded) == 1


def test_build_defined_kernels_accept_declarations_only(recorded, monkeypatch):
    monkeypatch.delenv(registry.ALLOW_BODY_MISMATCH_ENV, raising=False)

    @asc2.jit
    def matmul_int8_kernel(a_ptr: asc.GlobalAddress, b_ptr: asc.GlobalAddress, c_ptr: asc.GlobalAddress,
                           a_shape: asc.ConstExpr, b_shape: asc.ConstExpr, c_shape: asc.ConstExpr):
        c = asc2.matmul(asc2.load(a_ptr, a_shape, offsets=[0, 0]), asc2.load(b_ptr, b_shape, offsets=[0, 0]))
        asc2.store(c, c_ptr, offsets=[0, 0])

    a = np.zeros((4, 4), np.int8)
    with pytest.raises(registry.KernelBodyMismatch):
        matmul_int8_kernel[1](a, a, np.zeros((4, 4), np.int32), [4, 4], [4, 4], [4, 4])


def test_source_unavailable_is_refused(monkeypatch):
    monkeypatch.delenv(registry.ALLOW_BODY_MISMATCH_ENV, raising=False)
    ns = {"asc": asc, "asc2": asc2}
    exec("def vadd_kernel(x_ptr, y_ptr, out_ptr, size, tile_size, tile_per_block):\n    pass\n", ns)
    k = asc2.jit(ns["vadd_kernel"])
    assert k.body_fingerprint is None
    with pytest.raises(registry.KernelBodyMismatch, match="source is not available"):
        k.resolve(np.zeros(4, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32), 4, 4, 1)


def test_fingerprint_table_covers_the_registry():
    from pyasc_amd import fingerprint
    table = fingerprint.known_fingerprints()
    keys = {fingerprint.signature_key(n, p) for n, p in registry.entries()}
    assert keys == set(table)
    build_defined = {k for k, v in table.items() if not v}
    assert {k.split("(")[0] for k in build_defined} == {
        "flash_attention_fwd_kernel", "matmul_int8_kernel", "matmul_dequant_kernel", "rms_norm_kernel"}


@pytest.mark.skipif(not __import__("os").path.isdir("/root/reference/python/test"),
                    reason="the reference tree is present only where the table is generated")
def test_fingerprint_table_matches_the_reference(tmp_path, monkeypatch):
    # regenerate from the reference's sources (parsed as text) and compare with the committed table
    import json
    from pyasc_amd import fingerprint, make_fingerprints
    out = tmp_path / "fp.json"
    monkeypatch.setattr(make_fingerprints, "FINGERPRINTS_FILE", str(out))
    make_fingerprints.main(["x", "/root/reference"])
    with open(fingerprint.FINGERPRINTS_FILE) as f:
        committed = json.load(f)["kernels"]
    assert json.loads(out.read_text())["kernels"] == committed


# ------------------------------------------------------------------- host-side layout checks
# Refused on the host, before the C ABI is reached (no GPU needed).

@pytest.fixture
def no_native(monkeypatch):
    """kernels.* with CPU tensors standing in for device tensors; records C-ABI calls."""
    from pyasc_amd import kernels
    calls = []
    monkeypatch.setattr(kernels, "_device_tensor", lambda t, name: t)
    monkeypatch.setattr(kernels._native, "call", lambda *a: calls.append(a))
    monkeypatch.setattr(kernels, "_stream", lambda s: 0)
    return calls


@pytest.mark.parametrize("which", ["a", "b", "c"])
def test_matmul_refuses_overlapping_rows(no_native, which):
    from pyasc_amd import kernels
    ops = {"a": torch.zeros(64, 32, dtype=torch.bfloat16), "b": torch.zeros(32, 48, dtype=torch.bfloat16),
           "c": torch.zeros(64, 48, dtype=torch.bfloat16)}
    shape = ops[which].shape
    ops[which] = torch.zeros(1, shape[1], dtype=torch.bfloat16).expand(shape[0], shape[1])  # row stride 0
    with pytest.raises(ValueError, match="row stride 0 below its row length"):
        kernels.matmul(ops["a"], ops["b"], ops["c"])
    assert not no_native
    # a strided row-major view with room between rows is accepted and passes its leading dimension
    big = torch.zeros(64, 100, dtype=torch.bfloat16)
    kernels.matmul(big[:, :32], torch.zeros(32, 48, dtype=torch.bfloat16), torch.zeros(64, 48, dtype=torch.bfloat16))
    assert no_native[-1][0] == "asc_matmul" and no_native[-1][9] == 100  # lda


def test_launcher_refuses_noncontiguous_device_tensors():
    c = torch.zeros(8, 4).t()  # transposed view: writes through reshape(-1) would land in a copy
    with pytest.raises(ValueError, match="non-contiguous device tensor"):
        launcher_mod.require_contiguous("c_ptr", c)
    t = torch.zeros(4, 8)
    assert launcher_mod.require_contiguous("c_ptr", t) is t


def test_reduce_all_refuses_shapes_beyond_the_tensors(no_native):
    # kernel_all's input_shape / output_shape must fit the tensors; a shape larger than the
    # tensor is an error, not a reduction over the elements that happen to exist
    import asc2
    from pyasc_amd import launchers
    from pyasc_amd.registry import KernelCall

    def call(x, out, in_shape, out_shape):
        consts = {"input_shape": in_shape, "input_offsets": [0] * len(in_shape), "output_shape": out_shape,
                  "output_offsets": [0] * len(out_shape), "op": asc2.reduce_sum}
        return KernelCall("kernel_all", {"input_ptr": x, "output_ptr": out}, consts, 1, 0, {})
    with pytest.raises(ValueError, match="'input_ptr' holds 60 elements, its shape needs 64"):
        launchers._reduce_all(call(torch.zeros(60), torch.zeros(8), [8, 8], [8]))
    with pytest.raises(ValueError, match="'output_ptr' holds 4 elements, its shape needs 8"):
        launchers._reduce_all(call(torch.zeros(64), torch.zeros(4), [8, 8], [8]))
    assert not no_native
    launchers._reduce_all(call(torch.zeros(64), torch.zeros(8), [8, 8], [8]))
    assert no_native[-1][0] == "asc_reduce_f32" and no_native[-1][4:8] == (1, 64, -1, 8)


@pytest.mark.parametrize("dtype,bad", [(torch.int32, 32), (torch.int32, -1), (torch.int16, 16)])
def test_shift_amount_range(no_native, dtype, bad):
    from pyasc_amd import kernels
    x = torch.zeros(16, dtype=dtype)
    with pytest.raises(ValueError, match="outside"):
        kernels.binary(x, bad, torch.empty_like(x), "left_shift")
    kernels.binary(x, torch.iinfo(dtype).bits - 1, torch.empty_like(x), "right_shift")
    assert len(no_native) == 1


# ------------------------------------------------------------------- code objects and the file cache
# The asc2 vadd_kernel launches through a prebuilt gfx950 code object kept per specialisation in
# the file cache (pyasc_amd/asc/runtime/{cache,module}.py); these parts need no GPU.

def test_file_cache_manager(tmp_path, monkeypatch):
    from pyasc_amd.asc.runtime import cache
    monkeypatch.setenv("PYASC_AMD_CACHE_DIR", str(tmp_path))
    key = cache.hexdigest(b"factors")
    m = cache.get_cache_manager(key)
    assert m.cache_dir.startswith(str(tmp_path)) and not m.has_file("k.hsaco") and m.get_file("k.hsaco") is None
    path = m.put(b"\x7fELF-bytes", "k.hsaco")
    assert m.get_file("k.hsaco") == path and open(path, "rb").read() == b"\x7fELF-bytes"
    assert sorted(p.name for p in tmp_path.rglob("*")) == [m.key, "k.hsaco"]  # no temporary left behind
    # the file key separates functions and factors and follows the prebuilt binaries' identity
    k1 = cache.get_file_cache_key("fnA", "f=1")
    assert k1 != cache.get_file_cache_key("fnB", "f=1") and k1 != cache.get_file_cache_key("fnA", "f=2")


def test_code_object_compiled_path(tmp_path, monkeypatch):
    from pyasc_amd.asc.runtime import cache, module
    from pyasc_amd.launchers import VADD_CODE_OBJECT
    monkeypatch.setenv("PYASC_AMD_CACHE_DIR", str(tmp_path))
    assert VADD_CODE_OBJECT.path.exists(), "build() produces pyasc_amd/lib/co/asc2_vadd.hsaco"
    key = cache.get_file_cache_key("fn", "factors")
    p1 = module.compiled_path(VADD_CODE_OBJECT, key, "vadd_kernel")
    assert p1.startswith(str(tmp_path)) and open(p1, "rb").read() == VADD_CODE_OBJECT.path.read_bytes()
    assert module.compiled_path(VADD_CODE_OBJECT, key, "vadd_kernel") == p1  # a file-cache hit
    assert module.compiled_path(VADD_CODE_OBJECT, None, "vadd_kernel") == str(VADD_CODE_OBJECT.path)  # bypassed
    # the code object is a gfx950 ELF holding every kernel the launcher names
    data = VADD_CODE_OBJECT.path.read_bytes()
    assert data[:4] == b"\x7fELF"
    for name in VADD_CODE_OBJECT.functions:
        assert name.encode() + b".kd" in data


def test_every_code_object_holds_its_kernels():
    # each registered code object is built and is a gfx950 ELF with every kernel its launcher names
    from pyasc_amd import launchers  # noqa: F401  (registers the kernels)
    from pyasc_amd.registry import entries
    with_co = {(name, params): e.code_object for (name, params), e in entries().items() if e.code_object}
    assert {name for name, _ in with_co} == {"vadd_kernel", "softmax_kernel", "leaky_relu_kernel", "vmuladd_kernel",
                                             "gelu_kernel", "matmul_kernel", "matmul_int8_kernel",
                                             "matmul_dequant_kernel", "flash_attention_fwd_kernel"}
    # every asc2 matmul form (mnblock, K-tiled, fixpipe, chained) goes through the code object
    assert sum(name == "matmul_kernel" for name, _ in with_co) == 4
    for co in set(with_co.values()):
        data = co.path.read_bytes()
        assert data[:4] == b"\x7fELF" and b"gfx950" in data, co.name
        for name in co.functions:
            assert name.encode() + b".kd" in data, (co.name, name)


def test_launch_refuses_grids_beyond_one_launch():
    # checked before any HIP call: 2^24 workgroups of 256 threads is 2^32 threads
    from pyasc_amd.asc.runtime import module
    for grid, block in ((0, 256), (1 << 24, 256), (1 << 32, 1)):
        with pytest.raises(ValueError, match="launch range"):
            module.launch_blob(1, grid, block, b"", 0)


def test_pack_args_layout():
    from pyasc_amd.asc.runtime import module
    blob = module.pack_args([("ptr", 0x1000), ("i32", 7), ("i64", -2), ("f32", 1.5), ("ptr", 0x2000)])
    import struct
    # natural alignment: ptr @0, i32 @8, (pad) i64 @16, f32 @24, (pad) ptr @32
    assert len(blob) == 40
    assert struct.unpack_from("<Q", blob, 0)[0] == 0x1000 and struct.unpack_from("<i", blob, 8)[0] == 7
    assert struct.unpack_from("<q", blob, 16)[0] == -2 and struct.unpack_from("<f", blob, 24)[0] == 1.5
    assert struct.unpack_from("<Q", blob, 32)[0] == 0x2000 and blob[12:16] == b"\0" * 4


def test_vadd_entry_has_code_object_and_resolution_records_file_key(tmp_path, monkeypatch):
    monkeypatch.setenv("PYASC_AMD_CACHE_DIR", str(tmp_path))
    k = _cached_vadd()
    x = np.zeros(64, np.float32)
    resolved, _, _ = k.resolve(x, x, x, 64, 8, 4)
    assert resolved.entry.code_object is not None and resolved.entry.code_object.name == "asc2_vadd"
    assert len(resolved.file_cache_key) == 32 and resolved.launched is None
    fresh, _, _ = _cached_vadd(always_compile=True).resolve(x, x, x, 64, 8, 4)
    assert fresh.cache_key == "" and fresh.file_cache_key == ""
