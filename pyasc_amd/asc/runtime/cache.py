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
    ``~/.pyasc/cache``), one directory per key.
``always_compile=True`` skips both lookups and stores nothing.

Here the kernels are compiled for gfx950 ahead of time: into libasc_hip.so (the
C-ABI entry points) and, for the kernels the asc2 launch path loads itself, into
standalone code objects (pyasc_amd/lib/co/*.hsaco, see module.py).  The memory
level holds what resolving a call produces (``ResolvedKernel`` in jit.py) and,
after the first launch, the loaded code object's function handles; the file level
keeps each specialisation's code object under its file cache key in
``$PYASC_AMD_CACHE_DIR`` (default ``~/.pyasc_amd/cache``), where the next process
loads it from.  The prebuilt binaries' identity takes the place of ``pyasc_key``
(``library_key``): a rebuilt library or code object changes every key.
"""
from __future__ import annotations

import base64
import functools
import hashlib
import os
import uuid
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
    """Files of one cache key, in their own directory (cache.py:56-125): ``get_file``
    returns a file's path if present, ``put`` writes it atomically (a temporary
    directory named by pid and a random id, then os.replace)."""

    def __init__(self, key: str):
        self.key = key
        root = cache_dir()
        if not root:
            raise RuntimeError("Could not create or locate cache dir")
        self.cache_dir = os.path.join(root, key)
        os.makedirs(self.cache_dir, exist_ok=True)

    def _make_path(self, filename: str) -> str:
        return os.path.join(self.cache_dir, filename)

    def has_file(self, filename: str) -> bool:
        return os.path.exists(self._make_path(filename))

    def get_file(self, filename: str) -> Optional[str]:
        return self._make_path(filename) if self.has_file(filename) else None

    def put(self, data, filename: str) -> str:
        binary = isinstance(data, bytes)
        if not binary:
            data = str(data)
        path = self._make_path(filename)
        temp_dir = os.path.join(self.cache_dir, f"tmp.pid_{os.getpid()}_{uuid.uuid4()}")
        os.makedirs(temp_dir, exist_ok=True)
        temp_path = os.path.join(temp_dir, filename)
        with open(temp_path, "wb" if binary else "w") as f:
            f.write(data)
        os.replace(temp_path, path)  # atomic on POSIX: readers never see a partial file
        os.removedirs(temp_dir)
        return path


def _base32(key: str) -> str:
    return base64.b32encode(bytes.fromhex(key)).decode("utf-8").rstrip("=")


def get_cache_manager(key: str) -> FileCacheManager:
    """The file cache of a hex key, in a directory named by its base32 form (cache.py:128-134)."""
    return FileCacheManager(_base32(key))


@functools.lru_cache(maxsize=4096)
def get_file_cache_key(fn_cache_key: str, cache_factors: str) -> str:
    """File cache key of one specialisation (cache.py:156-159): the prebuilt binaries'
    identity, the function's source identity and the cache factors."""
    return hexdigest(f"{library_key()}__{fn_cache_key}__{cache_factors}".encode("utf-8"))


@functools.lru_cache(maxsize=4096)
def get_mem_cache_key(cache_factors: str) -> str:
    """In-memory cache key of one specialisation (cache.py:162-164), tied to the library build."""
    return hexdigest(f"{library_key()}__{cache_factors}".encode("utf-8"))
