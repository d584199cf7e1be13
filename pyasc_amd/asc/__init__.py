"""MI355X drop-in for the names user code takes from the reference's ``asc`` package.

Kernel signatures and launch helpers use ``asc.GlobalAddress``, ``asc.ConstExpr``,
``asc.ceildiv``, dtypes such as ``asc.float16`` and ``asc.runtime.config``; those are
provided with the reference's meaning.  asc1's intrinsic API (python/asc/language/
basic, adv, fwk) is not: it addresses Ascend hardware units that MI355X does not have.
The asc1 names that kernel signatures use as annotations (GlobalTensor, LocalTensor,
TQue, TBuf, TPipe) exist so those signatures evaluate; they raise when constructed.
"""
from . import adv, runtime
from .core import (ConstExpr, DataType, GlobalAddress, GlobalTensor, LocalTensor, TBuf, TPipe, TQue, as_torch_dtype,
                   bfloat16, bit, bool_, ceildiv, double, float16, float32, float64, float_, half, int1, int8, int16,
                   int32, int64, int_, require_constexpr, uint8, uint16, uint32, uint64, void)
from .runtime import JITFunction, LaunchOptions, jit

__all__ = [
    "adv", "runtime", "ConstExpr", "DataType", "GlobalAddress", "GlobalTensor", "LocalTensor", "TQue", "TBuf",
    "TPipe", "as_torch_dtype", "ceildiv", "require_constexpr", "jit",
    "JITFunction", "LaunchOptions", "void", "int1", "int8", "int16", "int32", "int64", "float16", "bfloat16",
    "float32", "float64", "uint8", "uint16", "uint32", "uint64", "bit", "bool_", "int_", "half", "float_", "double"
]
