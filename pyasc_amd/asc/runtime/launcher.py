"""Kernel launch: argument handling, host<->device copies, stream choice.

Mirrors python/asc/runtime/launcher.py:
  - ``LaunchOptions(core_num, stream)`` (launcher.py:79-102): ``kernel[n]`` or
    ``kernel[n, stream]``; ``core_num`` is the logical block count the kernel body
    is written for.
  - ``Launcher.run`` (launcher.py:204-238): DRY_RUN skips the launch; a block count
    <= 0 raises ValueError.
  - Host buffers (CPU torch tensors, numpy arrays) are copied to the device, the
    kernel runs, the stream is synchronised and every pointer argument is copied
    back (launcher.py:176-195).  ROCm torch tensors are passed zero-copy and the
    launch stays asynchronous on the chosen stream; they must be contiguous
    (a strided device view raises ValueError instead of being written through
    a temporary copy).
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple

import numpy as np

from ... import _native
from ...registry import KernelCall, KernelEntry


@dataclass(frozen=True)
class LaunchOptions:
    core_num: int = 0
    stream: Optional[Any] = None


def stream_handle(stream: Any) -> int:
    """hipStream_t of ``stream`` (None -> torch's current stream)."""
    if stream is None:
        return _native.current_stream_handle()
    if isinstance(stream, int):
        return stream
    handle = getattr(stream, "cuda_stream", None)
    if handle is None:
        raise TypeError(f"Unsupported stream object: {stream!r}")
    return int(handle)


def is_pointer_arg(value: Any) -> bool:
    if isinstance(value, np.ndarray):
        return True
    try:
        import torch
        return isinstance(value, torch.Tensor) and value.dim() > 0
    except ModuleNotFoundError:
        return False


_device_seen = False


def require_device() -> None:
    """Raises unless a HIP device is visible (checked until one is, then remembered)."""
    global _device_seen
    if _device_seen:
        return
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("No HIP device is available: asc2 kernels run only on the MI355X (gfx950) device "
                           "through libasc_hip.so; there is no CPU fallback.")
    _device_seen = True


def require_contiguous(name: str, value: Any) -> Any:
    """A device tensor is passed by its address (zero-copy): the kernel sees contiguous
    memory from data_ptr(), so any other layout is refused rather than written through
    a temporary copy the caller never sees."""
    if not value.is_contiguous():
        raise ValueError(f"argument '{name}' is a non-contiguous device tensor (shape {tuple(value.shape)}, "
                         f"stride {tuple(value.stride())}); pass a contiguous tensor")
    return value


class Launcher:

    def __init__(self, options: LaunchOptions):
        self.options = options

    @staticmethod
    def scalar_value(value: Any) -> Any:
        """Python value of a by-value argument (0-dim tensor, numpy scalar, int, float, bool)."""
        if isinstance(value, np.generic):
            return value.item()
        try:
            import torch
            if isinstance(value, torch.Tensor) and value.dim() == 0:
                return value.item()
        except ModuleNotFoundError:
            pass
        return value

    def prepare(self, runtime_args: Dict[str, Any]) -> Tuple[Dict[str, Any], List[Tuple[Any, Any]]]:
        """Device-side view of every runtime arg, plus (host, device) pairs to copy back."""
        import torch
        device_args: Dict[str, Any] = {}
        copy_back: List[Tuple[Any, Any]] = []
        for name, value in runtime_args.items():
            if isinstance(value, np.ndarray):
                dev = torch.from_numpy(np.ascontiguousarray(value)).to("cuda")
                device_args[name] = dev
                copy_back.append((value, dev))
            elif isinstance(value, torch.Tensor) and value.dim() > 0:
                if value.device.type == "cuda":
                    device_args[name] = require_contiguous(name, value)
                else:
                    dev = value.contiguous().to("cuda")
                    device_args[name] = dev
                    copy_back.append((value, dev))
            else:
                device_args[name] = self.scalar_value(value)
        return device_args, copy_back

    def run(self, entry: KernelEntry, function_name: str, runtime_args: Dict[str, Any],
            constexprs: Dict[str, Any], options: Optional[Dict[str, Any]] = None, resolved: Any = None) -> None:
        """Launches one call.  For an entry with a code object (module.py), ``resolved``
        (the JIT's cached specialisation) holds the loaded code object after the first
        launch; without it, or with ``always_compile``, the code object is loaded for
        this launch and unloaded after it (launcher.py:226-238)."""
        if os.environ.get("DRY_RUN"):
            return
        if self.options.core_num <= 0:
            raise ValueError("Core number should be large than 0")
        require_device()
        device_args, copy_back = self.prepare(runtime_args)
        stream = stream_handle(self.options.stream)
        if copy_back and self.options.stream is not None:
            # host buffers were copied in on torch's current stream; a launch on another
            # stream must not start before those copies are done
            import torch
            if stream != _native.current_stream_handle():
                torch.cuda.current_stream().synchronize()
        call = KernelCall(function_name, device_args, constexprs, int(self.options.core_num), stream,
                          {"options": dict(options or {})})
        if entry.code_object is None:
            entry.launch(call)
        else:
            self._launch_code_object(entry, call, resolved)
        if copy_back:
            _native.call("asc_stream_synchronize", stream)
            for host, dev in copy_back:
                if isinstance(host, np.ndarray):
                    np.copyto(host, dev.cpu().numpy())
                else:
                    host.copy_(dev.cpu())

    @staticmethod
    def _launch_code_object(entry: KernelEntry, call: KernelCall, resolved: Any) -> None:
        from . import module
        co = entry.code_object
        cached = resolved is not None and getattr(resolved, "file_cache_key", None)
        if cached and resolved.launched is not None:
            co.launch(call, resolved.launched.functions)  # memory-cache hit: nothing to load
            return
        path = module.compiled_path(co, resolved.file_cache_key if cached else None, call.name)
        launched = module.load(co, path)
        if cached:
            resolved.launched = launched
            co.launch(call, launched.functions)
            return
        try:  # caches bypassed: the module lives for this launch only
            co.launch(call, launched.functions)
            _native.call("asc_stream_synchronize", call.stream)
        finally:
            module.unload(launched)
