"""``asc.lib.runtime`` on HIP: devices, streams and synchronisation.

Mirrors the user-facing functions of the reference's runtime module
(python/asc/lib/runtime/interface.py, exported by python/asc/lib/runtime/__init__.py),
which kernels launched as ``kernel[grid, rt.current_stream()](...)`` use
(python/test/kernels/test_vadd.py:79, python/tutorials/01_add/add.py:79).

Streams are torch's HIP streams: ``current_stream`` returns torch's current stream
of the device, and a launch on it runs in order with the caller's torch work.  New
streams run at the default priority only.  Kernel binaries, raw device memory and
argument blobs (register_device_binary_kernel, malloc, launch_kernel ...) belong to
the reference's NPU launch path; here kernels are prebuilt into libasc_hip.so and
memory is owned by torch, so those functions are not provided.
"""
from __future__ import annotations

import time
from typing import Any, Optional

import torch


def check_device_handle(device_id: Any) -> None:
    """A device id is an int >= 0 (interface.py:110-113)."""
    if isinstance(device_id, int) and not isinstance(device_id, bool) and device_id >= 0:
        return
    raise RuntimeError(f"Device handle should be int >= 0, but '{device_id}' with {type(device_id)} type was given")


def is_available() -> bool:
    return torch.cuda.is_available()


def default_device() -> int:
    return 0


def current_device() -> int:
    return torch.cuda.current_device()


def device_count() -> int:
    return torch.cuda.device_count()


def _device(device_id: Optional[int]) -> int:
    if device_id is None:
        return current_device()
    check_device_handle(device_id)
    return device_id


def set_device(device_id: int) -> None:
    check_device_handle(device_id)
    torch.cuda.set_device(device_id)


def current_platform() -> str:
    """The device's architecture name (the reference returns the SoC version string)."""
    return torch.cuda.get_device_properties(current_device()).gcnArchName.split(":")[0]


def current_stream(device_id: Optional[int] = None) -> torch.cuda.Stream:
    """The stream launches go to (interface.py:125-127): torch's current stream."""
    return torch.cuda.current_stream(_device(device_id))


def create_stream(priority: int = 0) -> torch.cuda.Stream:
    """A new stream on the current device (interface.py:204-212).  Only the default
    priority is provided."""
    if priority != 0:
        raise ValueError(f"only priority 0 streams are provided, got {priority}")
    return torch.cuda.Stream()


def destroy_stream(stream_handle: torch.cuda.Stream) -> None:
    """Waits for the stream's work; the stream is released with its last reference."""
    synchronize(stream_handle)


def synchronize(stream_handle: Optional[torch.cuda.Stream] = None, timeout: int = 0) -> None:
    """Waits for the stream's work (interface.py:342-356).  With ``timeout`` > 0 (ms), raises
    RuntimeError when the work has not finished in time; the work itself keeps running."""
    stream = current_stream() if stream_handle is None else stream_handle
    if timeout <= 0:
        stream.synchronize()
        return
    deadline = time.monotonic() + timeout / 1000.0
    while not stream.query():
        if time.monotonic() > deadline:
            raise RuntimeError(f"stream synchronization timed out after {timeout} ms")
        time.sleep(50e-6)


def synchronize_device() -> None:
    torch.cuda.synchronize()
