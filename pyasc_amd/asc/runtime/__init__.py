"""Runtime part of the ``asc`` drop-in: JIT object, launcher, platform config."""
from . import config
from .jit import JITFunction, jit
from .launcher import LaunchOptions, Launcher

__all__ = ["config", "JITFunction", "jit", "LaunchOptions", "Launcher"]
