"""Signature registry: which native kernel a decorated asc2 function launches.

The reference compiles the decorated Python body (python/asc/runtime/jit.py:158-198).
Here every kernel of the hot path is a hand-written HIP kernel, so a decorated
function is matched by its name and parameter-name tuple.  Names collide across
the reference's tests (``softmax_kernel`` has two signatures, ``matmul_kernel``
four), which is why the parameter names are part of the key.  An unknown
signature raises NotImplementedError instead of silently doing something else,
and so does a registered signature whose body is not one of the bodies the
native kernel implements (compared by fingerprint, pyasc_amd.fingerprint).
"""
from __future__ import annotations

import os
import warnings
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
    # the prebuilt code object the asc2 launch path loads for this kernel (module.py);
    # None: the kernel launches through the library's C ABI
    code_object: Any = None


_REGISTRY: Dict[Tuple[str, Tuple[str, ...]], KernelEntry] = {}


def register(name: str, params: Tuple[str, ...], reference: str, code_object: Any = None):
    """Decorator registering ``launch`` for kernels named ``name`` with ``params``;
    ``code_object`` (a module.CodeObject) makes the asc2 launch path load and launch
    that prebuilt code object instead of calling ``launch``."""

    def deco(launch: Callable[[KernelCall], None]) -> Callable[[KernelCall], None]:
        key = (name, tuple(params))
        if key in _REGISTRY:
            raise RuntimeError(f"kernel signature registered twice: {name}{tuple(params)}")
        _REGISTRY[key] = KernelEntry(name, tuple(params), launch, reference, code_object)
        return launch

    return deco


# Set to 1 to let a kernel whose body differs from every registered body of its
# signature run the registered native kernel anyway (a warning is issued instead of
# the error).  Off by default: the native kernel computes what the registered bodies
# compute, not what a different body would.
ALLOW_BODY_MISMATCH_ENV = "PYASC_AMD_ALLOW_BODY_MISMATCH"


class KernelBodyMismatch(NotImplementedError):
    """A kernel's signature is registered but its body is not one the native kernel implements."""


def lookup(name: str, params: Tuple[str, ...], body_fingerprint: Optional[str] = None) -> KernelEntry:
    """The native kernel for ``name(params)`` whose registered bodies include
    ``body_fingerprint`` (pyasc_amd.fingerprint).  A declaration body (docstring,
    ``pass``, ``...``) binds by signature alone; None means the source was not
    available and is refused like a differing body."""
    _ensure_loaded()
    entry = _REGISTRY.get((name, tuple(params)))
    if entry is None:
        known = sorted(f"{n}({', '.join(p)})" for n, p in _REGISTRY)
        raise NotImplementedError(f"No native MI355X kernel is registered for {name}({', '.join(params)}). "
                                  "Registered kernels: " + "; ".join(known))
    _check_body(entry, body_fingerprint)
    return entry


def _check_body(entry: KernelEntry, body_fingerprint: Optional[str]) -> None:
    from . import fingerprint
    if body_fingerprint == fingerprint.DECLARATION:
        return
    key = fingerprint.signature_key(entry.name, entry.params)
    if body_fingerprint is not None and body_fingerprint in fingerprint.known_fingerprints().get(key, ()):
        return
    what = ("its source is not available to compare" if body_fingerprint is None else
            f"its body (fingerprint {body_fingerprint}) differs from every body this native kernel implements "
            f"({entry.reference})")
    msg = (f"{key}: the signature is registered, but {what}. Declare the kernel with an empty body "
           f"(a docstring, pass or ...) to bind it by signature, or set {ALLOW_BODY_MISMATCH_ENV}=1 to run "
           "the registered kernel anyway.")
    if os.environ.get(ALLOW_BODY_MISMATCH_ENV, "") not in ("", "0"):
        warnings.warn(msg, RuntimeWarning, stacklevel=4)
        return
    raise KernelBodyMismatch(msg)


def entries() -> Dict[Tuple[str, Tuple[str, ...]], KernelEntry]:
    _ensure_loaded()
    return dict(_REGISTRY)


_loaded: Optional[bool] = None


def _ensure_loaded() -> None:
    global _loaded
    if not _loaded:
        from . import launchers, launchers_asc1  # noqa: F401  (register the entries)
        _loaded = True
