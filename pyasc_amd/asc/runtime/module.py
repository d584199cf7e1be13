"""Code objects: loading, per-specialisation caching and launching of prebuilt gfx950 kernels.

The reference's launch path registers the binary its compiler produced, looks up
the kernel function, launches it with a packed argument blob, and either keeps
the function handle for the next call (a ``LaunchedKernel`` in the memory cache)
or, with ``always_compile``, unregisters the binary again
(python/asc/runtime/launcher.py:204-238; python/asc/runtime/jit.py:158-223).

Here the binaries are standalone gfx950 code objects built ahead of time
(pyasc_amd/lib/co/<name>.hsaco, from pyasc_amd/csrc/co/<name>.hip):
  - ``compiled_path`` is the per-specialisation binary: the code object copied
    into the file cache under the call's file cache key (``FileCacheManager.put``
    on first use, ``get_file`` afterwards), or the prebuilt file itself when the
    caches are bypassed;
  - ``load`` runs hipModuleLoad on it and hipModuleGetFunction for each of the
    code object's kernels (asc_module_load / asc_module_get_function of the C ABI);
  - ``launch`` packs the arguments into one blob, laid out as the kernel declares
    them (natural alignment, 8-byte pointers), and calls asc_module_launch
    (hipModuleLaunchKernel with the blob as its argument buffer).
Loaded modules belong to the process and the current device; a cached
``LaunchedKernel`` is reused by every later call of its specialisation.
"""
from __future__ import annotations

import ctypes
import functools
import struct
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable, Dict, Optional, Sequence, Tuple

from ... import _native

CODE_OBJECT_DIR = Path(__file__).resolve().parents[2] / "lib" / "co"

# counts hipModuleLoad calls (tests check that a cache hit loads nothing)
stats: Dict[str, int] = {"module_loads": 0, "module_unloads": 0, "launches": 0}


@dataclass(frozen=True)
class CodeObject:
    """A prebuilt code object and how a registered kernel launches through it."""
    name: str                      # lib/co/<name>.hsaco
    functions: Tuple[str, ...]     # kernel symbols to look up
    launch: Callable               # launch(call, functions: Dict[str, int]) -> None
    source: str                    # the csrc/co file it is built from

    @property
    def path(self) -> Path:
        return CODE_OBJECT_DIR / f"{self.name}.hsaco"


@dataclass
class LaunchedKernel:
    """A loaded code object: the module and its kernels' function handles."""
    code_object: CodeObject
    path: str
    module: int
    functions: Dict[str, int] = field(default_factory=dict)


def compiled_path(co: CodeObject, file_cache_key: Optional[str], fn_name: str) -> str:
    """The binary of one specialisation: from the file cache under ``file_cache_key``
    (stored there on first use), or the prebuilt code object when the key is None
    (the caches are bypassed)."""
    if not co.path.exists():
        raise RuntimeError(f"{co.path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    if file_cache_key is None:
        return str(co.path)
    from .cache import get_cache_manager
    manager = get_cache_manager(file_cache_key)
    filename = f"{fn_name}.hsaco"
    path = manager.get_file(filename)
    if path is None:
        path = manager.put(co.path.read_bytes(), filename)
    return path


def load(co: CodeObject, path: str) -> LaunchedKernel:
    """hipModuleLoad of ``path`` and the handles of the code object's kernels."""
    module = ctypes.c_void_p()
    _native.call("asc_module_load", path.encode(), ctypes.byref(module))
    stats["module_loads"] += 1
    lk = LaunchedKernel(co, path, int(module.value))
    try:
        for name in co.functions:
            fn = ctypes.c_void_p()
            _native.call("asc_module_get_function", ctypes.c_void_p(lk.module), name.encode(), ctypes.byref(fn))
            lk.functions[name] = int(fn.value)
    except Exception:
        unload(lk)
        raise
    return lk


def unload(lk: LaunchedKernel) -> None:
    _native.call("asc_module_unload", ctypes.c_void_p(lk.module))
    stats["module_unloads"] += 1


_FIELD_CODES = {"ptr": "Q", "i64": "q", "i32": "i", "f32": "f"}


@functools.lru_cache(maxsize=256)
def _layout(kinds: Tuple[str, ...]) -> struct.Struct:
    """struct layout of one argument list: each field at its natural alignment, the
    padding spelled out as pad bytes."""
    fmt, offset = "<", 0
    for kind in kinds:
        code = _FIELD_CODES[kind]
        size = struct.calcsize(code)
        pad = -offset % size
        fmt += "x" * pad + code
        offset += pad + size
    return struct.Struct(fmt)


def pack_args(fields: Sequence[Tuple[str, object]]) -> bytes:
    """Kernel arguments as one blob: each field ("ptr" / "i64" / "i32" / "f32", value)
    at its natural alignment, the way the kernel's argument list lays them out."""
    return _layout(tuple(kind for kind, _ in fields)).pack(*(value for _, value in fields))


def launch(function: int, grid: int, block: int, fields: Sequence[Tuple[str, object]], stream: int) -> None:
    """One launch of a loaded kernel on ``stream`` (asc_module_launch), its arguments
    packed from ``fields``."""
    launch_blob(function, grid, block, pack_args(fields), stream)


def launch_blob(function: int, grid: int, block: int, blob: bytes, stream: int) -> None:
    """One launch of a loaded kernel on ``stream`` with an argument blob laid out as the
    kernel declares its arguments."""
    if grid <= 0 or block <= 0 or grid * block >= 1 << 32:
        raise ValueError(f"{grid} workgroups of {block} threads: outside the launch range (under 2^32 threads)")
    buf = ctypes.create_string_buffer(blob, len(blob))
    _native.call("asc_module_launch", ctypes.c_void_p(function), grid, block, buf, len(blob), ctypes.c_void_p(stream))
    stats["launches"] += 1


def launch_plan(functions: Dict[str, int], plan, stream: int) -> None:
    """Launches an asc_launch_plan_t (``_native.LaunchPlan``) filled by one of the
    library's plan functions; nothing when its grid is 0."""
    if plan.grid:
        launch_blob(functions[plan.kernel.decode()], plan.grid, plan.block, plan.blob(), stream)
