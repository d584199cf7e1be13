"""Kernel cache: the reference's two-level cache, re-expressed for prebuilt gfx950 code.

The reference compiles a decorated function per specialisation and caches the
result twice (python/asc/runtime/jit.py:158-186, python/asc/runtime/cache.py):
  - in memory, per JITFunction, under ``get_mem_cache_key(cache_factors)``
    (cache.py:162-164), where the cache factors are the codegen options, the
    compile options, the ConstExpr values, the runtime argument kinds/dtypes and
    the function name (jit.py:139-156);
  - on disk, under ``get_file_cache_key(fn.cache_key, cache_factors)``
    (cache.py:156-159), whose first component identifies the compiler itself
    (``pyasc_key``: a hash of the package sources and libpyasc), as files kept by
    ``FileCacheManager`` (cache.py:56-125) in ``$PYASC_CACHE_DIR`` (default
    ``~/.pyasc/cache``).
``always_compile=True`` skips both lookups and stores nothing.

Here the kernels are compiled for gfx950 ahead of time: into libasc_hip.so (the
C-ABI entry points) and, for the kernels the asc2 launch path loads itself, into
standalone code objects (pyasc_amd/lib/co/*.hsaco, see module.py).  The memory
level holds what resolving a call produces (``ResolvedKernel`` in jit.py) and,
after the first launch, the loaded code object's function handles; the file level
keeps each specialisation's code object under its file cache key in
``$PYASC_AMD_CACHE_DIR`` (default ``~/.pyasc_amd/cache``), one directory per key,
where the next process loads it from.  The prebuilt binaries' identity takes the place of ``pyasc_key``
(``library_key``): a rebuilt library or code object changes every key.
"""
from __future__ import annotations

import contextlib
import functools
import hashlib
import os
import tempfile
from pathlib import Path
from typing import Optional


def hexdigest(data: bytes) -> str:
    """Same hash as the reference's default driver (blake2b, 16-byte digest; cache.py:31-41)."""
    h = hashlib.blake2b(digest_size=16)
    h.update(data)
    return h.hexdigest()


@functools.lru_cache()
def library_key() -> str:
    """Identity of the prebuilt kernels: hash of libasc_hip.so and of every code object
    under lib/co (the counterpart of pyasc_key)."""
    from ... import _native
    lib = Path(_native.LIB_PATH)
    h = hashlib.blake2b(digest_size=16)
    for path in [lib, *sorted((lib.parent / "co").glob("*.hsaco"))]:
        h.update(path.name.encode() + b"\0")
        try:
            with open(path, "rb") as f:
                for chunk in iter(lambda: f.read(1 << 20), b""):
                    h.update(chunk)
        except FileNotFoundError:
            h.update(b"unbuilt")
    return h.hexdigest()


def cache_dir() -> str:
    """Root of the file cache: $PYASC_AMD_CACHE_DIR, else ~/.pyasc_amd/cache (the reference's
    PYASC_CACHE_DIR / ~/.pyasc/cache, cache.py:30-34)."""
    home = os.getenv("PYASC_AMD_HOME", os.path.expanduser("~/"))
    return os.getenv("PYASC_AMD_CACHE_DIR", os.path.join(home, ".pyasc_amd", "cache"))


class FileCacheManager:
    """The files of one cache key, in a directory named by the key.  A file is
    published by writing it to a temporary file in that directory and renaming it
    over its name: a reader finds either no file or the whole file, and writers of
    the same key in several processes leave one complete copy."""

    def __init__(self, key: str):
        root = cache_dir()
        if not root:
            raise RuntimeError("Could not create or locate cache dir")
        self.key = key
        self.cache_dir = os.path.join(root, key)
        os.makedirs(self.cache_dir, exist_ok=True)

    def get_file(self, filename: str) -> Optional[str]:
        path = os.path.join(self.cache_dir, filename)
        return path if os.path.isfile(path) else None

    def has_file(self, filename: str) -> bool:
        return self.get_file(filename) is not None

    def put(self, data, filename: str) -> str:
        payload = data if isinstance(data, bytes) else str(data).encode("utf-8")
        path = os.path.join(self.cache_dir, filename)
        fd, tmp = tempfile.mkstemp(prefix=f".{filename}.", dir=self.cache_dir)
        try:
            with os.fdopen(fd, "wb") as f:
                f.write(payload)
            os.replace(tmp, path)
        except BaseException:
            with contextlib.suppress(FileNotFoundError):
                os.unlink(tmp)
            raise
        return path


def get_cache_manager(key: str) -> FileCacheManager:
    """The file cache of a hex key (the reference's get_cache_manager, cache.py:128-134)."""
    return FileCacheManager(key)


@functools.lru_cache(maxsize=4096)
def get_file_cache_key(fn_cache_key: str, cache_factors: str) -> str:
    """File cache key of one specialisation (cache.py:156-159): the prebuilt binaries'
    identity, the function's source identity and the cache factors."""
    return hexdigest(f"{library_key()}__{fn_cache_key}__{cache_factors}".encode("utf-8"))


@functools.lru_cache(maxsize=4096)
def get_mem_cache_key(cache_factors: str) -> str:
    """In-memory cache key of one specialisation (cache.py:162-164), tied to the library build."""
    return hexdigest(f"{library_key()}__{cache_factors}".encode("utf-8"))
