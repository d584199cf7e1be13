"""ctypes binding of libasc_hip.so (the C ABI declared in include/asc_hip.h).

This replaces the reference's runtime shim: rt_wrapper.cpp compiled at first
use and loaded with ctypes (python/asc/lib/runtime/state.py:25-50,140-144;
python/asc/lib/runtime/interface.py:25-39).  Error handling keeps the
reference's contract: a nonzero return becomes
``RuntimeError("Function <name> returned <code>")``
(python/asc/lib/runtime/state.py:63-75), extended with the library's message.

There is no fallback: if the library is missing, or no HIP device is present
when a kernel is launched, the call raises.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path
from typing import Optional

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libasc_hip.so"

# dtype codes of include/asc_hip.h
DT_FLOAT32 = 0
DT_FLOAT16 = 1
DT_BFLOAT16 = 2
DT_INT32 = 3
DT_INT8 = 4
DT_INT16 = 5

ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_ALIGNMENT = -3
ERR_BUSY = -4

_c_i32, _c_i64, _c_p, _c_f32, _c_f64 = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float, ctypes.c_double



class SoftmaxPlan(ctypes.Structure):
    """asc_softmax_plan_t: a softmax launch as kernel name, grid, block and arguments."""
    _fields_ = [("kernel", ctypes.c_char * 32), ("grid", ctypes.c_uint32), ("block", ctypes.c_uint32),
                ("rows", _c_i64), ("stride", _c_i64), ("len", _c_i32), ("flag", _c_i32)]


class LaunchPlan(ctypes.Structure):
    """asc_launch_plan_t: a code-object kernel's name, grid, block and argument blob."""
    _fields_ = [("kernel", ctypes.c_char * 64), ("grid", ctypes.c_uint32), ("block", ctypes.c_uint32),
                ("args_size", ctypes.c_uint64), ("args", ctypes.c_uint64 * 16)]

    def blob(self) -> bytes:
        return ctypes.string_at(ctypes.addressof(self.args), self.args_size)


# name -> argtypes; every entry point returns int32_t.
SIGNATURES = {
    "asc_device_info": [_c_i32, ctypes.POINTER(_c_i32), ctypes.POINTER(_c_i32), ctypes.POINTER(_c_i32),
                        ctypes.c_char_p],
    "asc_stream_synchronize": [_c_p],
    "asc_module_load": [ctypes.c_char_p, ctypes.POINTER(_c_p)],
    "asc_module_unload": [_c_p],
    "asc_module_get_function": [_c_p, ctypes.c_char_p, ctypes.POINTER(_c_p)],
    "asc_module_launch": [_c_p, ctypes.c_uint32, ctypes.c_uint32, _c_p, ctypes.c_uint64, _c_p],
    "asc_vadd": [_c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_p],
    "asc_copy_bytes": [_c_p, _c_p, _c_i64, _c_p],
    "asc_leaky_relu": [_c_i32, _c_p, _c_f32, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_p],
    "asc_vmuladd": [_c_i32, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_p],
    "asc_gelu_rows_f32": [_c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_p],
    "asc_softmax_rows_f32": [_c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p],
    "asc_reduce_f32": [_c_i32, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i64, _c_p],
    "asc_rms_norm": [_c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_f32, _c_p],
    "asc_softmax_blocks_f32": [_c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p],
    "asc_softmax_rows_f16": [_c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p],
    "asc_softmax_blocks_f16": [_c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p],
    "asc_softmax_plan": [_c_i32, _c_i32, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, ctypes.POINTER(SoftmaxPlan)],
    "asc_matmul": [_c_i32, _c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_p],
    "asc_matmul_bias_act": [_c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                            _c_i32, _c_f32, _c_p],
    "asc_matmul_chained": [_c_i32, _c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p],
    "asc_matmul_chained_noalloc": [_c_i32, _c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p],
    "asc_matmul_i8_i32": [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p],
    "asc_matmul_i8_dequant_f16": [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p],
    "asc_flash_attention_fwd_bf16": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_f32, _c_i32,
                                     _c_p],
    "asc_flash_attention_plan": [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_f32, _c_i32,
                                 ctypes.POINTER(LaunchPlan)],
    "asc_matmul_plan": [_c_i32, _c_i32, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32,
                        _c_f32, ctypes.POINTER(LaunchPlan)],
    "asc_matmul_i8_plan": [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, ctypes.POINTER(LaunchPlan)],
    "asc_unary_f32": [_c_i32, _c_p, _c_p, _c_i64, _c_p],
    "asc_binary": [_c_i32, _c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_f64, _c_i64, _c_p],
    "asc_where_cmp": [_c_i32, _c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_f64, _c_i64, _c_f64, _c_f64, _c_p],
    "asc_rect_binary": [_c_i32, _c_i32, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p],
    "asc_broadcast_rows": [_c_i32, _c_p, _c_p, _c_i64, _c_i64, _c_p],
    "asc_atomic_tiles": [_c_i32, _c_i32, _c_p, _c_p, _c_i64, _c_i64, _c_f64, _c_i64, _c_p],
    "asc_fill": [_c_i32, _c_p, _c_i64, _c_f64, _c_i64, _c_p],
    "asc_unary": [_c_i32, _c_i32, _c_p, _c_p, _c_i64, _c_p],
    "asc_axpy": [_c_i32, _c_p, _c_p, _c_f64, _c_i64, _c_p],
    "asc_transpose_batched": [_c_i32, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p],
    "asc_quant_i8": [_c_i32, _c_p, _c_p, _c_f64, _c_f64, _c_i64, _c_p],
}
# entry points returning a C string
STRING_FUNCS = ("asc_last_error", "asc_version")

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def load_library(path: Optional[Path] = None) -> ctypes.CDLL:
    """Loads libasc_hip.so once and declares every entry point's prototype."""
    global _lib
    lib = _lib
    if lib is not None and path is None:  # loaded: no lock on the per-launch path
        return lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        lib_path = Path(path) if path is not None else LIB_PATH
        if not lib_path.exists():
            raise RuntimeError(f"{lib_path} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
                               "or `python pyasc_amd/build.py`")
        # torch's bundled HIP runtime has the same soname as ROCm's; importing
        # torch first makes the library bind to that already-loaded runtime, so
        # torch tensors and streams are valid in both.
        import torch  # noqa: F401
        lib = ctypes.CDLL(str(lib_path), mode=ctypes.RTLD_GLOBAL)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int32
        for name in STRING_FUNCS:
            fn = getattr(lib, name)
            fn.argtypes = []
            fn.restype = ctypes.c_char_p
        if path is None:
            _lib = lib
        return lib


def current_stream_handle() -> int:
    """hipStream_t of torch's current stream on the current device, read without building
    a torch Stream object (the launch paths ask for it on every call)."""
    import torch
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is None:
        return int(torch.cuda.current_stream().cuda_stream)
    return int(raw(torch.cuda.current_device()))


def last_error() -> str:
    msg = load_library().asc_last_error()
    return msg.decode() if msg else ""


def check(code: int, fn_name: str) -> None:
    """Raises the reference's RuntimeError form for a nonzero return code."""
    if code != 0:
        detail = last_error()
        raise RuntimeError(f"Function {fn_name} returned {code}" + (f": {detail}" if detail else ""))


def call(fn_name: str, *args) -> None:
    fn = getattr(load_library(), fn_name)
    check(fn(*args), fn_name)


def version() -> str:
    return load_library().asc_version().decode()


def device_info(device: int = 0) -> dict:
    cu, lds, wave = _c_i32(), _c_i32(), _c_i32()
    arch = ctypes.create_string_buffer(64)
    call("asc_device_info", device, ctypes.byref(cu), ctypes.byref(lds), ctypes.byref(wave), arch)
    return {"cu_count": cu.value, "lds_bytes": lds.value, "wave_size": wave.value, "arch": arch.value.decode()}
