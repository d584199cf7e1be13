"""Signature registry: which native kernel a decorated asc2 function launches.

The reference compiles the decorated Python body (python/asc/runtime/jit.py:158-198).
Here every kernel of the hot path is a hand-written HIP kernel, so a decorated
function is matched by its name and parameter-name tuple.  Names collide across
the reference's tests (``softmax_kernel`` has two signatures, ``matmul_kernel``
four), which is why the parameter names are part of the key.  An unknown
signature raises NotImplementedError instead of silently doing something else.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable, Dict, Optional, Tuple


@dataclass
class KernelCall:
    """Everything a native launcher needs for one ``kernel[grid](...)`` call."""
    name: str
    args: Dict[str, Any]      # runtime args: device tensors / python scalars
    consts: Dict[str, Any]    # ConstExpr args, unwrapped
    grid: int                 # logical block count (kernel[grid])
    stream: int               # hipStream_t handle
    extra: Dict[str, Any] = field(default_factory=dict)

    def get(self, key: str) -> Any:
        if key in self.args:
            return self.args[key]
        return self.consts[key]


@dataclass(frozen=True)
class KernelEntry:
    name: str
    params: Tuple[str, ...]
    launch: Callable[[KernelCall], None]
    reference: str  # file:line of the reference kernel this entry stands for


_REGISTRY: Dict[Tuple[str, Tuple[str, ...]], KernelEntry] = {}


def register(name: str, params: Tuple[str, ...], reference: str):
    """Decorator registering ``launch`` for kernels named ``name`` with ``params``."""

    def deco(launch: Callable[[KernelCall], None]) -> Callable[[KernelCall], None]:
        key = (name, tuple(params))
        if key in _REGISTRY:
            raise RuntimeError(f"kernel signature registered twice: {name}{tuple(params)}")
        _REGISTRY[key] = KernelEntry(name, tuple(params), launch, reference)
        return launch

    return deco


def lookup(name: str, params: Tuple[str, ...]) -> KernelEntry:
    _ensure_loaded()
    entry = _REGISTRY.get((name, tuple(params)))
    if entry is None:
        known = sorted(f"{n}({', '.join(p)})" for n, p in _REGISTRY)
        raise NotImplementedError(f"No native MI355X kernel is registered for {name}({', '.join(params)}). "
                                  "Registered kernels: " + "; ".join(known))
    return entry


def entries() -> Dict[Tuple[str, Tuple[str, ...]], KernelEntry]:
    _ensure_loaded()
    return dict(_REGISTRY)


_loaded: Optional[bool] = None


def _ensure_loaded() -> None:
    global _loaded
    if not _loaded:
        from . import launchers, launchers_asc1  # noqa: F401  (register the entries)
        _loaded = True
