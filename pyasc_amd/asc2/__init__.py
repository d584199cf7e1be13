"""MI355X drop-in for the reference's ``asc2`` tile API surface (python/asc2/__init__.py:9-177).

``asc2.jit`` returns a JITFunction whose launches run hand-written gfx950 HIP
kernels, selected by the decorated function's name and parameter names.  The
tile operations (``asc2.load``, ``asc2.reduce_max`` ...) keep their names so that
kernel bodies written for the reference still import and parse, but the bodies
are never executed: calling one of these functions outside a kernel raises.
"""
from __future__ import annotations

from enum import Enum
from typing import Callable, Optional

from ..asc.runtime.jit import JITFunction


class TileLocation(Enum):
    """Tile placement names of the reference (UB / L1 / L0A / L0B / L0C)."""
    UB = "UB"
    L1 = "L1"
    L0A = "L0A"
    L0B = "L0B"
    L0C = "L0C"


class range:  # noqa: A001  (same name as the reference's asc2.range)
    """``asc2.range(start, stop, step, unroll_factor=1, parallel=False)``
    (python/asc/language/tile/range.py:16-36): argument checks only; the loop
    itself lives in the native kernel."""

    def __init__(self, *args, unroll_factor: int = 1, parallel: bool = False):
        if not isinstance(unroll_factor, int):
            raise TypeError("'unroll_factor' must be int")
        if not isinstance(parallel, bool):
            raise TypeError("'parallel' must be bool")
        if unroll_factor < 1:
            raise ValueError(f"Loop unroll factor must be 1 or greater, got {unroll_factor}")
        if not 1 <= len(args) <= 3:
            raise TypeError("range expects 1 to 3 positional arguments")
        self.args = args
        self.unroll_factor = unroll_factor
        self.parallel = parallel


def jit(fn: Optional[Callable] = None, **options):
    """``@asc2.jit`` / ``@asc2.jit(**options)`` with the asc2 defaults of python/asc2/jit.py:44-46."""
    options.setdefault("custom_builtins", {"range": range})
    options.setdefault("insert_sync", True)
    options.setdefault("run_asc2_passes", True)

    def decorator(f: Callable) -> JITFunction:
        return JITFunction(f, **options)

    if fn is None:
        return decorator
    return decorator(fn)


_TILE_OPS = (
    "tensor", "atomic_add", "atomic_max", "atomic_min", "add", "div", "equal", "greater", "greater_equal",
    "left_shift", "less", "less_equal", "matmul", "matmul_acc", "maximum", "minimum", "mul", "not_equal",
    "right_shift", "sub", "concat", "full", "full_like", "zeros", "zeros_acc", "zeros_like", "copy", "load",
    "store", "block_idx", "block_num", "num_tiles", "broadcast_to", "expand_dims", "ravel", "reshape", "squeeze",
    "abs", "ceil", "cos", "cosh", "erf", "exp", "exp2", "floor", "log", "log2", "negative", "relu", "rms_norm",
    "rsqrt", "sin", "sinh", "softmax", "sqrt", "tan", "tanh", "mask", "where", "reduce_sum", "reduce_max",
    "reduce_min", "reduce_prod")


def _make_tile_op(name: str) -> Callable:

    def op(*args, **kwargs):
        raise RuntimeError(f"asc2.{name} can only appear inside an @asc2.jit kernel body; bodies are not executed "
                           "here, each registered kernel signature runs a native gfx950 kernel")

    op.__name__ = name
    op.__qualname__ = name
    return op


for _name in _TILE_OPS:
    globals()[_name] = _make_tile_op(_name)
del _name

__all__ = ["TileLocation", "range", "jit", *_TILE_OPS]
