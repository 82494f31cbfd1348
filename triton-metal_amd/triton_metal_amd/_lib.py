"""ctypes binding of libtm_hip.so (the C ABI declared in include/tm_hip.h).

The library is loaded lazily on first use.  PyTorch is imported first so that
its HIP runtime is the one the library binds to (the library resolves HIP
entry points from the runtime already present in the process).
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

from .errors import HipLaunchError, KernelLoadError, NativeLibraryMissing, NoDeviceError

LIB_PATH = Path(__file__).resolve().parent / "libtm_hip.so"

TM_DT_NONE, TM_DT_F32, TM_DT_F16, TM_DT_BF16, TM_DT_U8 = -1, 0, 1, 2, 3
TM_DT_FP8_E4M3, TM_DT_FP8_E5M2, TM_DT_FP8_E4M3B15, TM_DT_FP8_E4M3B8, TM_DT_FP8_E5M2B16 = (
    4, 5, 6, 7, 8)
TM_EPI_NONE, TM_EPI_ADD_MATRIX, TM_EPI_ADD_ROWS, TM_EPI_ADD_COLS, TM_EPI_SOFTMAX, \
    TM_EPI_CHAIN_DOT = range(6)
TM_ERR_INVALID_ARG, TM_ERR_UNSUPPORTED, TM_ERR_NO_RUNTIME, TM_ERR_NOT_FOUND, TM_ERR_LOAD = (
    -1, -2, -3, -4, -5)
TM_WQ_ALIGN_XW16, TM_WQ_ALIGN_S16, TM_WQ_ALIGN_Z16, TM_WQ_ALIGN_SZ4 = 1, 2, 4, 8
TM_WQ_ALIGN_ALL = 15
TM_GEMM_ALIGN_AB16, TM_GEMM_ALIGN_C16, TM_GEMM_ALIGN_ALL = 1, 2, 3

vp, i32, u32, sz = C.c_void_p, C.c_int, C.c_uint, C.c_size_t

# name -> argtypes (restype is int for every entry unless listed in _RESTYPES)
SIGNATURES = {
    "tm_init": [],
    "tm_last_error": [],
    "tm_version": [],
    "tm_device_info": [i32, C.c_char_p, sz, C.POINTER(i32), C.POINTER(i32), C.POINTER(i32)],
    "tm_num_builtin_modules": [],
    "tm_builtin_module_name": [i32],
    "tm_module_load": [vp, sz, C.POINTER(vp)],
    "tm_module_unload": [vp],
    "tm_module_get_function": [vp, C.c_char_p, C.POINTER(vp), C.POINTER(i32), C.POINTER(i32),
                               C.POINTER(i32), C.POINTER(i32)],
    "tm_builtin_get_function": [C.c_char_p, C.POINTER(vp)],
    "tm_launch": [vp, u32, u32, u32, u32, u32, u32, u32, vp, C.POINTER(vp)],
    "tm_synchronize": [vp],
    "tm_int8_matmul": [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp],
    "tm_int4_matmul": [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp],
    "tm_int8_linear": [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp],
    "tm_int4_linear": [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp],
    "tm_wq_dequant": [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp],
    "tm_wq_matmul_ws": [i32, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, sz,
                        vp],
    "tm_wq_workspace_bytes": [i32, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32],
    "tm_wq_plan": [i32, i32, i32, i32, i32, i32, i32, i32, u32, i32, sz, i32, C.c_char_p, sz,
                   C.POINTER(u32), C.POINTER(u32), C.POINTER(u32), C.POINTER(u32),
                   C.POINTER(sz)],
    "tm_wq_repack_gptq": [vp, vp, vp, i32, i32, i32, i32, vp, vp, vp, vp],
    "tm_wq_repack_awq": [vp, vp, vp, i32, i32, i32, vp, vp, vp, vp],
    "tm_matmul": [vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, i32, vp],
    "tm_linear": [vp, vp, vp, vp, i32, i32, i32, i32, i32, vp],
    "tm_gemm_plan": [i32, i32, i32, i32, i32, i32, i32, i32, i32, i32, u32, C.c_char_p, sz,
                     C.POINTER(u32), C.POINTER(u32)],
    "tm_matmul_2d": [vp, vp, vp, vp, vp, vp, i32, i32, sz, sz, sz, i32, i32, vp],
    "tm_matmul_swizzled": [vp, vp, vp, vp, vp, vp, i32, i32, sz, sz, sz, i32, i32, i32, vp],
    "tm_dot": [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, C.POINTER(C.c_longlong), i32, i32,
               i32, i32, i32, vp],
    "tm_flash_attention": [vp, vp, vp, vp, vp, i32, i32, i32, i32, C.POINTER(C.c_longlong),
                           C.c_float, i32, i32, vp],
    "tm_kda_workspace_size": [i32, i32, i32, i32, i32, i32],
    "tm_decode_attention_workspace_size": [i32, i32, i32, i32, i32, i32],
    "tm_decode_attention": [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i32,
                            C.POINTER(C.c_longlong), vp, i32, i32, C.c_float, i32, i32, i32, vp,
                            sz, vp],
    "tm_decode_attention_noalloc": [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp, i32,
                                    C.POINTER(C.c_longlong), vp, i32, i32, C.c_float, i32, i32,
                                    i32, vp],
    "tm_kda_chunk_fwd": [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, C.c_float,
                         i32, vp, sz, vp],
    "tm_kda_recurrent_fwd": [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, C.c_float,
                             i32, vp],
}
_RESTYPES = {
    "tm_last_error": C.c_char_p,
    "tm_version": C.c_char_p,
    "tm_builtin_module_name": C.c_char_p,
    "tm_kda_workspace_size": sz,
    "tm_decode_attention_workspace_size": sz,
    "tm_wq_workspace_bytes": sz,
}

_lock = threading.Lock()
_lib = None


def lib():
    """Load (once) and return the ctypes handle of libtm_hip.so."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NativeLibraryMissing(
                f"{LIB_PATH} is missing; build it with triton_metal_amd.build.build()")
        try:
            import torch  # noqa: F401  (bind to torch's HIP runtime)
        except ImportError:
            pass
        h = C.CDLL(str(LIB_PATH))
        for name, args in SIGNATURES.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = _RESTYPES.get(name, i32)
        _lib = h
        return _lib


def last_error() -> str:
    msg = lib().tm_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str, kernel_name=None, grid=None):
    """Raise the error class matching a non-zero return code."""
    if rc == 0:
        return
    msg = last_error()
    if rc == TM_ERR_NO_RUNTIME:
        raise NoDeviceError(f"{what}: {msg}")
    if rc in (TM_ERR_LOAD, TM_ERR_NOT_FOUND):
        raise KernelLoadError(f"{what}: {msg}", code=rc)
    raise HipLaunchError(f"{what} failed (code {rc})", kernel_name=kernel_name, grid=grid,
                         reason=msg, code=rc)
