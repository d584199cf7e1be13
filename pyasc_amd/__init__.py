"""pyasc_amd -- MI355X (gfx950) implementation of the kernels PyAsc's asc2 tile API
tutorials and tests compile and run: vadd, row softmax, fp16/bf16 matmul, int8
matmul with per-channel dequant, and flash-attention forward.

The kernels live in libasc_hip.so (HIP C++, C ABI in include/asc_hip.h).  User
code keeps the reference's launch surface:

    from pyasc_amd import asc, asc2          # or pyasc_amd.install_aliases(); import asc, asc2

    @asc2.jit
    def vadd_kernel(x_ptr: asc.GlobalAddress, y_ptr: asc.GlobalAddress, out_ptr: asc.GlobalAddress,
                    size: int, tile_size: asc.ConstExpr[int], tile_per_block: asc.ConstExpr[int]):
        ...

    vadd_kernel[16](x, y, out, 8192, 128, 4)
"""
from __future__ import annotations

import sys

from . import asc, asc2  # noqa: F401

__version__ = "0.1.0"


def install_aliases() -> None:
    """Makes ``import asc``, ``import asc2``, ``import asc.runtime.config`` and
    ``import asc.lib.runtime`` / ``asc.lib.host`` resolve to this package, so code written against the
    reference imports unchanged."""
    from .asc import runtime
    from .asc.runtime import config, jit, launcher
    sys.modules.setdefault("asc", asc)
    sys.modules.setdefault("asc.runtime", runtime)
    sys.modules.setdefault("asc.runtime.config", config)
    sys.modules.setdefault("asc.runtime.jit", jit)
    sys.modules.setdefault("asc.runtime.launcher", launcher)
    from .asc import lib
    from .asc.lib import host as lib_host, runtime as lib_runtime
    sys.modules.setdefault("asc.lib", lib)
    sys.modules.setdefault("asc.lib.runtime", lib_runtime)
    sys.modules.setdefault("asc.lib.host", lib_host)
    sys.modules.setdefault("asc2", asc2)
