"""``JITFunction``: the object ``@asc2.jit`` returns.

Follows python/asc/runtime/jit.py:33-223 in its user-visible behaviour:
  - option names are validated at decoration (unknown -> RuntimeError, names that
    clash with kernel parameters -> RuntimeError; jit.py:38-49);
  - ``kernel[grid]`` / ``kernel[grid, stream]`` set the launch options and return
    the runner (jit.py:51-60);
  - a call merges decorator and call options, binds arguments with
    ``inspect.signature`` and splits ConstExpr arguments by annotation
    (jit.py:215-223; python/asc/codegen/function.py:119-132);
  - runtime argument types are classified as in jit.py:69-96 (TypeError for
    unsupported ones).
Instead of compiling the body, the (name, parameter names) pair selects a
registered native kernel (pyasc_amd.registry).
"""
from __future__ import annotations

import inspect
from typing import Any, Callable, Dict, List, Tuple, Union, get_args, get_origin

import numpy as np

from ... import registry
from ..core import ConstExpr, DataType, require_constexpr
from .launcher import LaunchOptions, Launcher

CODEGEN_OPTIONS = ("capture_exceptions", "ir_multithreading", "custom_builtins")
COMPILE_OPTIONS = ("debug", "strip_loc", "verify_sync", "print_ir_before_all", "run_passes", "kernel_type",
                   "auto_sync", "auto_sync_log", "matmul_cube_only", "always_compile", "bisheng_options",
                   "opt_level", "run_asc2_passes", "densify_load_store", "insert_sync", "reuse_ub",
                   "reuse_ub_in_out", "static_alloc", "vf_fusion")
LAUNCH_OPTIONS = ("core_num", "stream")


class ArgType:
    """Classification of one runtime argument: pointer or by-value, with its dtype name."""

    def __init__(self, kind: str, dtype: DataType):
        self.kind = kind  # "pointer" | "plain" | "struct"
        self.dtype = dtype

    def __repr__(self) -> str:
        return f"{self.kind}:{self.dtype}"


def _annotations(fn: Callable) -> Dict[str, Any]:
    try:
        return inspect.get_annotations(fn, eval_str=True)
    except Exception:  # unresolvable string annotations: fall back to the raw ones
        return dict(getattr(fn, "__annotations__", {}))


class JITFunction:

    def __init__(self, fn: Callable, **options):
        self.fn = fn
        self.fn_name = fn.__name__
        self.signature = inspect.signature(fn)
        self.params: Tuple[str, ...] = tuple(self.signature.parameters)
        clashed = self.get_clashed_args(fn)
        if clashed:
            raise RuntimeError("The following argument names conflict with JIT configuration options: " +
                               ", ".join(clashed))
        unknown = set(options).difference(self.get_config_keywords())
        if unknown:
            raise RuntimeError("The following option names are unknown: " + ", ".join(sorted(unknown)))
        self.default_options: Dict[str, Any] = options
        self.launch_options = LaunchOptions()
        self.__doc__ = fn.__doc__
        self.__name__ = fn.__name__

    def __repr__(self) -> str:
        return f"JITFunction({self.fn.__module__}.{self.fn.__qualname__})"

    def __getitem__(self, user_launch_options: Union[int, tuple]) -> Callable:
        try:
            if isinstance(user_launch_options, int):
                self.launch_options = LaunchOptions(core_num=user_launch_options)
            else:
                self.launch_options = LaunchOptions(*user_launch_options)
        except Exception as e:
            raise TypeError("Parse user launch options failed") from e
        return self._run

    def __call__(self, *args, **kwargs):
        raise TypeError(f"{self.fn_name} is a kernel: launch it as {self.fn_name}[grid](...)")

    @staticmethod
    def get_config_keywords() -> List[str]:
        return [*CODEGEN_OPTIONS, *COMPILE_OPTIONS, *LAUNCH_OPTIONS]

    @classmethod
    def get_clashed_args(cls, fn: Callable) -> List[str]:
        return [p for p in inspect.signature(fn).parameters if p in cls.get_config_keywords()]

    @staticmethod
    def get_arg_type(value: Any) -> ArgType:
        if isinstance(value, bool):
            return ArgType("plain", DataType("int8"))
        if isinstance(value, int):
            return ArgType("plain", DataType("int32"))
        if isinstance(value, float):
            return ArgType("plain", DataType("float32"))
        if isinstance(value, np.ndarray):
            return ArgType("pointer", DataType(str(np.dtype(value.dtype))))
        if isinstance(value, np.generic):
            return ArgType("plain", DataType(str(value.dtype)))
        from ..adv import TCubeTiling
        if isinstance(value, TCubeTiling):
            # passed by value as a struct on the reference (python/asc/runtime/launcher.py:156-184)
            return ArgType("struct", DataType("void"))
        try:
            import torch
            if isinstance(value, torch.Tensor):
                name = str(value.dtype)
                name = name[6:] if name.startswith("torch.") else name
                return ArgType("plain" if value.dim() == 0 else "pointer", DataType(name))
        except ModuleNotFoundError:
            pass
        raise TypeError(f"Argument type in JIT function is not supported: {value.__class__.__name__}")

    @staticmethod
    def split_args(args: Dict[str, Any], annotations: Dict[str, Any]) -> Tuple[Dict[str, Any], Dict[str, Any]]:
        runtime_args: Dict[str, Any] = {}
        constexprs: Dict[str, Any] = {}
        for name, value in args.items():
            ann_type = annotations.get(name, object)
            origin = get_origin(ann_type) or ann_type
            if inspect.isclass(origin) and issubclass(origin, ConstExpr):
                ann_args = get_args(ann_type)
                if len(ann_args) != 0:
                    require_constexpr(value, *ann_args, arg_name=name)
                constexprs[name] = ConstExpr.unwrap(value)
            else:
                runtime_args[name] = value
        return runtime_args, constexprs

    def bind(self, *args, **kwargs) -> Tuple[Dict[str, Any], Dict[str, Any], Dict[str, Any]]:
        """(runtime args, constexprs, options) of one call, without launching."""
        kwargs = {**self.default_options, **kwargs}
        options = {k: kwargs.pop(k) for k in list(kwargs) if k in self.get_config_keywords()}
        call_args = self.signature.bind(*args, **kwargs)
        call_args.apply_defaults()
        runtime_args, constexprs = self.split_args(dict(call_args.arguments), _annotations(self.fn))
        for value in runtime_args.values():
            self.get_arg_type(value)
        return runtime_args, constexprs, options

    def _run(self, *args, **kwargs) -> None:
        runtime_args, constexprs, _ = self.bind(*args, **kwargs)
        entry = registry.lookup(self.fn_name, self.params)
        Launcher(self.launch_options).run(entry, self.fn_name, runtime_args, constexprs)


def jit(fn: Callable = None, **options):
    """``@asc.jit`` / ``@asc.jit(**options)`` (python/asc/runtime/jit.py:226-250)."""

    def decorator(f: Callable) -> JITFunction:
        return JITFunction(f, **options)

    if fn is None:
        return decorator
    return decorator(fn)
