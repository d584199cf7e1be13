"""Builds libasc_hip.so (all HIP kernels + the C ABI of include/asc_hip.h) for gfx950.

Each ``csrc/*.hip`` file is compiled separately with hipcc (in parallel), then
linked into ``pyasc_amd/lib/libasc_hip.so``.  Each ``csrc/co/*.hip`` file becomes a
standalone gfx950 code object ``pyasc_amd/lib/co/<name>.hsaco`` (an unbundled ELF
for hipModuleLoad), the binaries the asc2 launch path loads and caches.  The
results stay in-tree so they travel with the source tree to the GPU machine.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC_DIR = PKG_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
LIB_DIR = PKG_DIR / "lib"
LIB_PATH = LIB_DIR / "libasc_hip.so"
CO_SRC_DIR = CSRC_DIR / "co"
CO_DIR = LIB_DIR / "co"
BUILD_DIR = PKG_DIR / "_build"

ARCH = "gfx950"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU forms are disabled for every device pass.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
    f"-I{CSRC_DIR}",
]

# Files whose results are compared bit-exactly (or to 1e-6) keep IEEE op-by-op
# rounding: no FMA contraction.
PER_FILE_FLAGS = {
    "vadd.hip": ["-ffp-contract=off"],
    "asc2_vadd.hip": ["-ffp-contract=off"],
    "softmax.hip": ["-ffp-contract=off"],
    "asc2_softmax.hip": ["-ffp-contract=off"],
    "matmul_i8.hip": ["-ffp-contract=off"],
    "asc2_matmul_i8.hip": ["-ffp-contract=off"],
    "elementwise.hip": ["-ffp-contract=off"],
    "asc2_elementwise.hip": ["-ffp-contract=off"],
    "tile_ops.hip": ["-ffp-contract=off"],
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build libasc_hip.so)")
    return path


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected.
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    msg = "\n".join(line for line in (res.stdout + res.stderr).splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msg}")
    if msg.strip() and verbose:
        print(msg, flush=True)
    return obj


def _compile_code_object(src: Path, verbose: bool) -> Path:
    """One standalone gfx950 code object (unbundled ELF) from csrc/co/<name>.hip."""
    out = CO_DIR / (src.stem + ".hsaco")
    tmp = out.with_suffix(".hsaco.tmp")
    cmd = [hipcc(), "--genco", "--no-gpu-bundle-output", *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), str(src),
           "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    msg = "\n".join(line for line in (res.stdout + res.stderr).splitlines() if noise not in line)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc --genco failed for {src.name}:\n{msg}")
    os.replace(tmp, out)
    return out


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compiles every csrc/*.hip and links libasc_hip.so, and builds every csrc/co/*.hip
    code object; returns the library's path."""
    BUILD_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    CO_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC_DIR.glob("*.hip"))
    co_sources = sorted(CO_SRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    jobs = jobs or min(len(sources) + len(co_sources), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        co_jobs = [pool.submit(_compile_code_object, s, verbose) for s in co_sources]
        objs = list(pool.map(lambda s: _compile(s, verbose), sources))
        for job in co_jobs:
            job.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of libasc_hip.so failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
