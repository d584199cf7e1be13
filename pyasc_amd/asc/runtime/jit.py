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
registered native kernel (pyasc_amd.registry), provided the body is one that
kernel implements (its fingerprint, pyasc_amd.fingerprint) or a declaration.
What a call resolves to is cached per JITFunction under the reference's cache
factors (jit.py:139-186; see cache.py): a hit skips annotation evaluation, ConstExpr validation, argument
classification and the registry lookup.  ``always_compile=True`` bypasses the
cache, as it bypasses the reference's.
"""
from __future__ import annotations

import hashlib
import inspect
import re
from dataclasses import dataclass
from typing import Any, Callable, Dict, FrozenSet, List, Optional, Tuple, Union, get_args, get_origin

import numpy as np

from ... import fingerprint, registry
from ..core import ConstExpr, DataType, require_constexpr
from .cache import get_file_cache_key, get_mem_cache_key
from .launcher import LaunchOptions, Launcher

CODEGEN_OPTIONS = ("capture_exceptions", "ir_multithreading", "custom_builtins")
COMPILE_OPTIONS = ("debug", "strip_loc", "verify_sync", "print_ir_before_all", "run_passes", "kernel_type",
                   "auto_sync", "auto_sync_log", "matmul_cube_only", "always_compile", "bisheng_options",
                   "opt_level", "run_asc2_passes", "densify_load_store", "insert_sync", "reuse_ub",
                   "reuse_ub_in_out", "static_alloc", "vf_fusion")
LAUNCH_OPTIONS = ("core_num", "stream")
_CONFIG_KEYWORDS = frozenset(CODEGEN_OPTIONS + COMPILE_OPTIONS + LAUNCH_OPTIONS)


_UNSET = object()


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


# a string annotation that could not be evaluated (e.g. `from __future__ import
# annotations` with `asc` imported inside a function) is recognised by its text
_CONSTEXPR_TEXT = re.compile(r"^\s*(?:[A-Za-z_][\w.]*\.)?ConstExpr\b")


def _is_constexpr_annotation(ann_type: Any) -> bool:
    if isinstance(ann_type, str):
        return _CONSTEXPR_TEXT.match(ann_type) is not None
    origin = get_origin(ann_type) or ann_type
    return inspect.isclass(origin) and issubclass(origin, ConstExpr)


@dataclass
class ResolvedKernel:
    """One cached specialisation: the native kernel a call resolves to (the
    counterpart of the reference's CompiledKernel / LaunchedKernel cache entry).
    For a kernel with a code object, ``file_cache_key`` names its binary in the file
    cache and ``launched`` holds the loaded module after the first launch."""
    entry: registry.KernelEntry
    cache_key: str
    file_cache_key: str = ""
    launched: Any = None


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
        self.kernel_cache: Dict[str, ResolvedKernel] = {}
        # first level in front of kernel_cache: a tuple of cheap per-call facts that determine
        # the same cache factors (see _quick_key); it maps to the entry of kernel_cache
        self._quick_cache: Dict[tuple, ResolvedKernel] = {}
        self._const_names: Optional[FrozenSet[str]] = None  # ConstExpr parameters, from the annotations
        self._hash: Optional[str] = None
        self._fingerprint: Any = _UNSET
        # plain positional calls can skip inspect.Signature.bind
        self._positional_only_call = all(
            p.kind in (inspect.Parameter.POSITIONAL_ONLY, inspect.Parameter.POSITIONAL_OR_KEYWORD)
            for p in self.signature.parameters.values())
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
            if _is_constexpr_annotation(ann_type):
                ann_args = () if isinstance(ann_type, str) else get_args(ann_type)
                if len(ann_args) != 0:
                    require_constexpr(value, *ann_args, arg_name=name)
                constexprs[name] = ConstExpr.unwrap(value)
            else:
                runtime_args[name] = value
        return runtime_args, constexprs

    def bind(self, *args, **kwargs) -> Tuple[Dict[str, Any], Dict[str, Any], Dict[str, Any]]:
        """(runtime args, constexprs, options) of one call, validated, without launching."""
        kwargs = {**self.default_options, **kwargs}
        options = {k: kwargs.pop(k) for k in list(kwargs) if k in self.get_config_keywords()}
        call_args = self.signature.bind(*args, **kwargs)
        call_args.apply_defaults()
        runtime_args, constexprs = self.split_args(dict(call_args.arguments), _annotations(self.fn))
        for value in runtime_args.values():
            self.get_arg_type(value)
        _check_compile_options(options)
        return runtime_args, constexprs, options

    # ------------------------------------------------------------------------------------ cache

    @property
    def cache_key(self) -> str:
        """Identity of the decorated function (source text and qualified name), as the
        reference's Function.cache_key (python/asc/codegen/function.py:63-87)."""
        if self._hash is None:
            try:
                src = inspect.getsource(self.fn)
            except (OSError, TypeError):
                src = ""
            self._hash = hashlib.sha256(f"{self.fn.__module__}.{self.fn.__qualname__}\n{src}".encode()).hexdigest()
        return self._hash

    @property
    def body_fingerprint(self) -> Optional[str]:
        """Fingerprint of the decorated body (pyasc_amd.fingerprint): the registry runs
        the native kernel only for a body it implements, or for a declaration body."""
        if self._fingerprint is _UNSET:
            self._fingerprint = fingerprint.fingerprint_of(self.fn)
        return self._fingerprint

    @staticmethod
    def arg_kind(value: Any) -> str:
        """``kind:dtype`` of a runtime argument, the reference's per-argument cache factor
        (jit.py:151-152); raises TypeError like get_arg_type for unsupported types."""
        cls = value.__class__
        if cls is bool:
            return "plain:int8"
        if cls is int:
            return "plain:int32"
        if cls is float:
            return "plain:float32"
        dtype = getattr(value, "dtype", None)
        dim = getattr(value, "dim", None)
        if dtype is not None and callable(dim) and cls.__module__.startswith("torch"):
            name = str(dtype)
            return ("plain:" if dim() == 0 else "pointer:") + (name[6:] if name.startswith("torch.") else name)
        t = JITFunction.get_arg_type(value)
        return f"{t.kind}:{t.dtype}"

    def _gen_cache_factors(self, arg_kinds: Dict[str, str], constexprs: Dict[str, Any],
                           options: Dict[str, Any]) -> str:
        """Cache factors in the reference's order (jit.py:139-156): options, ConstExpr
        values, argument kinds/dtypes, function name."""
        factors = [
            ";".join(f"{k}={options[k]!r}" for k in sorted(options) if k not in LAUNCH_OPTIONS),
            ";".join(f"{name}={val!r}" for name, val in constexprs.items()),
            ";".join(f"{name}={kind}" for name, kind in arg_kinds.items()),
            f"fn_name={self.fn_name}",
        ]
        return "__".join(factors)

    def _constexpr_names(self) -> FrozenSet[str]:
        if self._const_names is None:
            ann = _annotations(self.fn)
            self._const_names = frozenset(n for n in self.params if _is_constexpr_annotation(ann.get(n, object)))
        return self._const_names

    def _fast_bind(self, args: tuple, kwargs: Dict[str, Any]) -> Tuple[Dict[str, Any], Dict[str, Any], Dict[str, Any]]:
        """Binding and ConstExpr split without validation (validation runs on a cache miss)."""
        options = dict(self.default_options)
        if kwargs:
            for k in [k for k in kwargs if k in _CONFIG_KEYWORDS]:
                options[k] = kwargs.pop(k)
        if not kwargs and self._positional_only_call and len(args) == len(self.params):
            bound = dict(zip(self.params, args))
        else:
            call_args = self.signature.bind(*args, **kwargs)
            call_args.apply_defaults()
            bound = dict(call_args.arguments)
        const_names = self._constexpr_names()
        runtime_args: Dict[str, Any] = {}
        constexprs: Dict[str, Any] = {}
        for name, value in bound.items():
            if name in const_names:
                constexprs[name] = ConstExpr.unwrap(value)
            else:
                runtime_args[name] = value
        return runtime_args, constexprs, options

    @staticmethod
    def _quick_key(runtime_args: Dict[str, Any], constexprs: Dict[str, Any], call_options: Dict[str, Any]):
        """A hashable tuple that determines the same cache factors as _gen_cache_factors, built
        without string formatting: per runtime argument its class, and for tensors the dtype
        and whether it is 0-dim (the pointer / by-value split); ConstExpr values and the options
        given at the call tagged with their types (so 1, True and 1.0 stay distinct, as their
        reprs are).  The decorator's options are the same for every call of this function and
        the quick cache is per function, so they need no place in the key.  None when an
        argument or value has no cheap form; the caller then takes the full path."""
        parts = []
        for value in runtime_args.values():
            cls = value.__class__
            if cls is int or cls is float or cls is bool:
                parts.append(cls)
            elif cls.__module__ == "torch" and cls.__name__ in ("Tensor", "Parameter"):
                parts.append((value.dtype, value.dim() == 0))
            else:
                return None
        try:
            consts = tuple(_tagged(v) for v in constexprs.values())
            opts = tuple(sorted((k, _tagged(v)) for k, v in call_options.items() if k not in LAUNCH_OPTIONS)) \
                if call_options else ()
            key = (tuple(parts), consts, opts)
            hash(key)
        except TypeError:
            return None
        return key

    def resolve(self, *args, **kwargs) -> Tuple[ResolvedKernel, Dict[str, Any], Dict[str, Any]]:
        """(cached specialisation, runtime args, constexprs) of one call, without launching."""
        if kwargs.get("always_compile", self.default_options.get("always_compile", False)):
            # no lookup and no store (jit.py:164-186): resolve from scratch
            runtime_args, constexprs, _ = self.bind(*args, **kwargs)
            return ResolvedKernel(registry.lookup(self.fn_name, self.params, self.body_fingerprint), ""), \
                runtime_args, constexprs
        runtime_args, constexprs, options = self._fast_bind(args, dict(kwargs))
        quick = self._quick_key(runtime_args, constexprs,
                                {k: v for k, v in kwargs.items() if k in options} if kwargs else {})
        if quick is not None:
            hit = self._quick_cache.get(quick)
            if hit is not None:
                return hit, runtime_args, constexprs
        arg_kinds = {name: self.arg_kind(value) for name, value in runtime_args.items()}
        factors = self._gen_cache_factors(arg_kinds, constexprs, options)
        key = get_mem_cache_key(factors)
        hit = self.kernel_cache.get(key)
        if hit is not None:
            if quick is not None:
                self._quick_cache[quick] = hit
            return hit, runtime_args, constexprs
        # miss: full validation (ConstExpr types, argument types), then the registry
        runtime_args, constexprs, _ = self.bind(*args, **kwargs)
        entry = registry.lookup(self.fn_name, self.params, self.body_fingerprint)
        file_key = get_file_cache_key(self.cache_key, factors) if entry.code_object is not None else ""
        resolved = ResolvedKernel(entry, key, file_key)
        self.kernel_cache[key] = resolved
        if quick is not None:
            self._quick_cache[quick] = resolved
        return resolved, runtime_args, constexprs

    def _run(self, *args, **kwargs) -> None:
        resolved, runtime_args, constexprs = self.resolve(*args, **kwargs)
        options = {**self.default_options, **{k: v for k, v in kwargs.items() if k in COMPILE_OPTIONS}}
        Launcher(self.launch_options).run(resolved.entry, self.fn_name, runtime_args, constexprs, options,
                                          resolved=resolved if resolved.cache_key else None)


def _check_compile_options(options: Dict[str, Any]) -> None:
    """The compiler's option check, run where the reference builds its Compiler (a cache miss
    or always_compile; python/asc/runtime/compiler.py:137-141, 322-329): opt_level must be
    1, 2 or 3 and kernel_type None or a config.KernelType.  The SoC-version part of that
    check is about Ascend targets and has no counterpart here."""
    from .config import KernelType
    kernel_type = options.get("kernel_type")
    if options.get("opt_level", 3) not in (1, 2, 3) or not (kernel_type is None or
                                                         isinstance(kernel_type, KernelType)):
        raise RuntimeError("Please check input compile option")


def _tagged(value: Any):
    """Hashable, type-tagged form of a ConstExpr value or option (lists and tuples element-wise)."""
    cls = value.__class__
    if cls is list or cls is tuple:
        return (cls, tuple(_tagged(v) for v in value))
    return (cls, value)


def jit(fn: Callable = None, **options):
    """``@asc.jit`` / ``@asc.jit(**options)`` (python/asc/runtime/jit.py:226-250)."""

    def decorator(f: Callable) -> JITFunction:
        return JITFunction(f, **options)

    if fn is None:
        return decorator
    return decorator(fn)
