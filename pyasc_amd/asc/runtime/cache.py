"""Kernel cache keys: the reference's two-level cache, re-expressed for prebuilt code.

The reference compiles a decorated function per specialisation and caches the
result twice (python/asc/runtime/jit.py:158-186, python/asc/runtime/cache.py):
  - in memory, per JITFunction, under ``get_mem_cache_key(cache_factors)``
    (cache.py:162-164), where the cache factors are the codegen options, the
    compile options, the ConstExpr values, the runtime argument kinds/dtypes and
    the function name (jit.py:139-156);
  - on disk, under ``get_file_cache_key(fn.cache_key, cache_factors)``
    (cache.py:156-159), whose first component identifies the compiler itself
    (``pyasc_key``: a hash of the package sources and libpyasc).
``always_compile=True`` skips both lookups and stores nothing.

Here every kernel is already compiled for gfx950 into libasc_hip.so, so a cache
entry holds what resolving a call produces instead of a binary: the registered
native kernel, with the ConstExpr values validated and the argument kinds
classified (``ResolvedKernel`` in jit.py).  The library's own identity takes the
place of ``pyasc_key`` (``library_key``): a rebuilt library changes every key.
There is no file level -- nothing is compiled at run time, so there is nothing to
persist between processes.
"""
from __future__ import annotations

import functools
import hashlib
from pathlib import Path


def hexdigest(data: bytes) -> str:
    """Same hash as the reference's default driver (blake2b, 16-byte digest; cache.py:31-41)."""
    h = hashlib.blake2b(digest_size=16)
    h.update(data)
    return h.hexdigest()


@functools.lru_cache()
def library_key() -> str:
    """Identity of the prebuilt kernels: hash of libasc_hip.so (the counterpart of pyasc_key)."""
    from ... import _native
    path = Path(_native.LIB_PATH)
    h = hashlib.blake2b(digest_size=16)
    try:
        with open(path, "rb") as f:
            for chunk in iter(lambda: f.read(1 << 20), b""):
                h.update(chunk)
    except FileNotFoundError:
        h.update(b"unbuilt")
    return h.hexdigest()


@functools.lru_cache(maxsize=4096)
def get_mem_cache_key(cache_factors: str) -> str:
    """In-memory cache key of one specialisation (cache.py:162-164), tied to the library build."""
    return hexdigest(f"{library_key()}__{cache_factors}".encode("utf-8"))
