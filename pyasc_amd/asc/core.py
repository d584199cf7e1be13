"""Launch-surface types of the reference's ``asc`` package.

Only the names a kernel signature or launch helper uses are provided:
``ConstExpr`` / ``require_constexpr`` (python/asc/language/core/constexpr.py:21-72),
``GlobalAddress`` (python/asc/language/core/ir_value.py:36-60), ``DataType`` and the
predefined dtypes (python/asc/language/core/dtype.py:18-153) and ``ceildiv``
(python/asc/language/core/utils.py:173-174).  They carry the same meaning; there is
no IR behind them because kernel bodies are not compiled here.
"""
from __future__ import annotations

import re
from enum import Enum
from typing import Any, Generic, Optional, Type, TypeVar, Union, get_args

T_co = TypeVar("T_co", covariant=True)


class ConstExpr(Generic[T_co]):
    """A compile-time kernel argument (``tile_size: asc.ConstExpr[int]``)."""

    def __init__(self, value):
        self.value = self.unwrap(value)

    def __str__(self) -> str:
        return str(self.value)

    def __repr__(self) -> str:
        return f"ConstExpr[{self.value.__class__.__name__}]({self.value!r})"

    def __format__(self, format_spec: str) -> str:
        return format(self.value, format_spec)

    def __eq__(self, other) -> bool:
        return self.value == self.unwrap(other)

    def __hash__(self) -> int:
        return hash(self.value)

    @staticmethod
    def unwrap(obj):
        return obj.value if isinstance(obj, ConstExpr) else obj


def require_constexpr(obj: Any, *constraints: Type, arg_name: Optional[str] = None) -> None:
    """Raises RuntimeError unless ``obj`` (or the value it wraps) is one of ``constraints``."""
    if len(constraints) == 0:
        raise RuntimeError("Constraints must be provided for ConstExpr requirement")
    if isinstance(obj, constraints):
        return
    if isinstance(obj, ConstExpr):
        require_constexpr(obj.value, *constraints, arg_name=arg_name)
        return
    names = " | ".join(getattr(t, "__name__", str(t)) for t in constraints)
    note = "" if arg_name is None else f" for '{arg_name}' argument"
    raise RuntimeError(f"ConstExpr[{names}] is required{note}, {obj.__class__.__name__} was provided: {obj}")


class GlobalAddress:
    """Annotation marker for a global-memory (HBM) pointer argument."""

    def __init__(self, handle: Any = None, dtype: Optional["DataType"] = None):
        self.handle = handle
        self.dtype = dtype

    def __repr__(self) -> str:
        return f"GlobalAddress(dtype={self.dtype}, handle=...)"


class _BodyOnlyName:
    """A name of asc1's on-chip API (python/asc/language/core/tensor.py, fwk/tpipe.py) that
    kernel signatures use as an annotation (``z_gm: asc.GlobalTensor``, ``in_queue: asc.TQue``).
    The annotation evaluates; constructing one raises, since kernel bodies are not executed
    here: each registered kernel signature runs a native gfx950 kernel."""

    def __init__(self, *args, **kwargs):
        raise RuntimeError(f"asc.{type(self).__name__} can only appear inside an @asc.jit kernel body; bodies are "
                           "not executed here, each registered kernel signature runs a native gfx950 kernel")


class GlobalTensor(_BodyOnlyName):
    """Global-memory tensor view of asc1 (python/asc/language/core/tensor.py)."""


class LocalTensor(_BodyOnlyName):
    """On-chip tensor of asc1 (python/asc/language/core/tensor.py)."""


class TQue(_BodyOnlyName):
    """Pipeline queue of asc1 (python/asc/language/fwk/tpipe.py)."""


class TBuf(_BodyOnlyName):
    """Scratch buffer of asc1 (python/asc/language/fwk/tpipe.py)."""


class TPipe(_BodyOnlyName):
    """Buffer manager of asc1 (python/asc/language/fwk/tpipe.py)."""


class DataType:
    """Element type named like numpy/torch (``float16``, ``bfloat16``, ``int8`` ...)."""

    _re_matcher = re.compile("^(u?int|b?float)([0-9]+)$")

    class Kind(Enum):
        Any = ""
        Int = "int"
        Float = "float"
        UInt = "uint"

    def __init__(self, name: str):
        self.name = name
        self.kind = self.Kind.Any
        self.bitwidth: Optional[int] = None
        match = self._re_matcher.match(name)
        if match:
            self.kind = {"bfloat": self.Kind.Float, "float": self.Kind.Float, "int": self.Kind.Int,
                         "uint": self.Kind.UInt}.get(match[1], self.Kind.Any)
            self.bitwidth = int(match[2])

    def __eq__(self, other) -> bool:
        return isinstance(other, DataType) and self.name == other.name

    def __hash__(self) -> int:
        return hash(self.name)

    def __str__(self) -> str:
        return self.name

    def __repr__(self) -> str:
        return f"DataType({self.name!r})"

    def is_int(self) -> bool:
        return self.kind in (self.Kind.Int, self.Kind.UInt)

    def is_float(self) -> bool:
        return self.kind == self.Kind.Float

    def to_torch(self):
        import torch
        mapping = {"int1": torch.bool, "int8": torch.int8, "int16": torch.int16, "int32": torch.int32,
                   "int64": torch.int64, "float16": torch.float16, "bfloat16": torch.bfloat16,
                   "float32": torch.float32, "float64": torch.float64, "uint8": torch.uint8}
        if self.name not in mapping:
            raise TypeError(f"no torch dtype for {self.name}")
        return mapping[self.name]


void = DataType("void")
int1 = DataType("int1")
int8 = DataType("int8")
int16 = DataType("int16")
int32 = DataType("int32")
int64 = DataType("int64")
float16 = DataType("float16")
bfloat16 = DataType("bfloat16")
float32 = DataType("float32")
float64 = DataType("float64")
uint8 = DataType("uint8")
uint16 = DataType("uint16")
uint32 = DataType("uint32")
uint64 = DataType("uint64")
bit = int1
bool_ = int8
int_ = int32
half = float16
float_ = float32
double = float64


def ceildiv(x: int, y: int) -> int:
    return (x + y - 1) // y


def as_torch_dtype(dtype: Union[DataType, Any]):
    """Maps an ``asc`` DataType (or a torch dtype) to the torch dtype."""
    import torch
    if isinstance(dtype, ConstExpr):
        dtype = dtype.value
    if isinstance(dtype, torch.dtype):
        return dtype
    if isinstance(dtype, DataType):
        return dtype.to_torch()
    raise TypeError(f"expected an asc DataType, got {dtype!r}")


__all__ = [
    "ConstExpr", "require_constexpr", "GlobalAddress", "GlobalTensor", "LocalTensor", "TQue", "TBuf", "TPipe",
    "DataType", "ceildiv", "as_torch_dtype", "void", "int1",
    "int8", "int16", "int32", "int64", "float16", "bfloat16", "float32", "float64", "uint8", "uint16", "uint32",
    "uint64", "bit", "bool_", "int_", "half", "float_", "double"
]
