"""Platform selection, kept call-compatible with python/asc/runtime/config.py:15-101.

On MI355X there is one backend: the HIP device.  ``set_platform`` accepts the
reference's backend and SoC values so unchanged launch code runs; the Ascend SoC
names only select nothing.  ``device_id`` selects the HIP device.
"""
from __future__ import annotations

from enum import Enum
from typing import Optional, Union


class Backend(Enum):
    Model = "Model"  # the reference's cycle simulator; runs on the HIP device here
    NPU = "NPU"      # the reference's hardware backend; runs on the HIP device here
    HIP = "HIP"


class Platform(Enum):
    """SoC names accepted by set_platform (python/asc/runtime/config.py:20-43) plus MI355X."""
    MI355X = "MI355X"
    Ascend910B1 = "Ascend910B1"
    Ascend910B2 = "Ascend910B2"
    Ascend910B2C = "Ascend910B2C"
    Ascend910B3 = "Ascend910B3"
    Ascend910B4 = "Ascend910B4"
    Ascend910B4_1 = "Ascend910B4-1"
    Ascend910_9362 = "Ascend910_9362"
    Ascend910_9372 = "Ascend910_9372"
    Ascend910_9381 = "Ascend910_9381"
    Ascend910_9382 = "Ascend910_9382"
    Ascend910_9391 = "Ascend910_9391"
    Ascend910_9392 = "Ascend910_9392"
    Ascend910_9579 = "Ascend910_9579"
    Ascend910_9589 = "Ascend910_9589"
    Ascend910_9599 = "Ascend910_9599"
    Ascend950PR_950z = "Ascend950PR_950z"
    Ascend950PR_9579 = "Ascend950PR_9579"
    Ascend950PR_957b = "Ascend950PR_957b"
    Ascend950PR_957c = "Ascend950PR_957c"
    Ascend950PR_957d = "Ascend950PR_957d"
    Ascend950PR_9589 = "Ascend950PR_9589"
    Ascend950PR_958b = "Ascend950PR_958b"
    Ascend950PR_9599 = "Ascend950PR_9599"


class CompilationArch(Enum):
    C220 = "c220"
    C310 = "c310"
    GFX950 = "gfx950"

    def __str__(self) -> str:
        return self.value


class KernelType(Enum):
    """Core mix a kernel runs on (python/asc/runtime/config.py:54-62), accepted as the
    ``kernel_type`` jit option.  On MI355X every kernel runs on the same compute units; the
    value matters only where it fixes how many instances a launch runs: an asc1 Matmul
    kernel as MIX_AIC_1_2 runs two per block (one cube core, two vector cores), any other
    type one."""
    AIV_ONLY = 0
    AIC_ONLY = 1
    MIX_AIV_HARD_SYNC = 2
    MIX_AIC_HARD_SYNC = 3
    MIX_AIV_1_0 = 4
    MIX_AIC_1_0 = 5
    MIX_AIC_1_1 = 6
    MIX_AIC_1_2 = 7


_state = {"backend": Backend.HIP, "platform": Platform.MI355X, "device_id": 0}


def set_platform(backend: Union[Backend, str], soc_version: Optional[Union[Platform, str]] = None,
                 device_id: Optional[int] = None, check: bool = True) -> None:
    """Selects the device; unknown backend values raise ValueError as in the reference."""
    backend = Backend(backend)
    platform = Platform(soc_version) if soc_version is not None else Platform.MI355X
    _state.update(backend=backend, platform=platform)
    if device_id is not None:
        _state["device_id"] = int(device_id)
    if check:
        import torch
        if not torch.cuda.is_available():
            raise RuntimeError("Runtime library is not available! No HIP device is visible to PyTorch-ROCm.")
        if device_id is not None:
            torch.cuda.set_device(int(device_id))


def current_device() -> int:
    return _state["device_id"]


def platform_to_arch(platform: Union[Platform, str]) -> CompilationArch:
    """Every platform runs the gfx950 kernels; Ascend names keep their reference mapping."""
    name = Platform(platform).value
    if name.startswith("Ascend910B") or name.startswith("Ascend910_93"):
        return CompilationArch.C220
    if name.startswith("Ascend910_95") or name.startswith("Ascend950PR_95"):
        return CompilationArch.C310
    return CompilationArch.GFX950
