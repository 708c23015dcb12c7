"""Loads libiris_hip.so (built in-tree by iris_amd.build) through ctypes.

There is no CPU fallback anywhere in this package: if the library is missing
or the device cannot be used, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libiris_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "iris_hip.h")

_lib = None


class IrisError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"{what} failed: {error_text(code)} (code {code})")


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m iris_amd.build` "
                               "(there is no CPU fallback)")
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def error_text(code: int) -> str:
    return lib().q8gpu_error(code).decode()


def check(code: int, what: str):
    if code != 0:
        raise IrisError(code, what)


i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")


def _declare(L):
    vp, u32, i32, u64 = C.c_void_p, C.c_uint32, C.c_int32, C.c_uint64
    pp = C.POINTER(C.c_void_p)
    sig = {
        "q8gpu_error": (C.c_char_p, [C.c_int]),
        "q8gpu_init": (C.c_int, []),
        "q8gpu_upload": (C.c_int, [i8p, i64p, u32, u32, pp]),
        "q8gpu_free": (None, [vp]),
        "q8gpu_product": (C.c_int, [vp, i32p, u32, i32p]),
        "q8gpu_upload_q8_0": (C.c_int, [u8p, u32, u32, pp]),
        "q8gpu_product_device": (C.c_int, [vp, vp, u32, vp, vp]),
        "q8gpu_workspace_bytes": (u64, [vp, u32]),
        "q8gpu_product_device_ws": (C.c_int, [vp, vp, u32, vp, vp, u64, vp]),
        "q8gpu_product_device_noalloc": (C.c_int, [vp, vp, u32, vp, vp]),
        "q8gpu_prepare_matrix_cores": (C.c_int, [vp, vp]),
        "q8gpu_matrix_info": (C.c_int, [vp, C.POINTER(u32), C.POINTER(u32), C.POINTER(C.c_int), C.POINTER(u64)]),
        "q8gpu_synchronize": (C.c_int, []),
        "iris_device_malloc": (C.c_int, [u64, pp]),
        "iris_device_free": (C.c_int, [vp]),
        "iris_memcpy_h2d": (C.c_int, [vp, vp, u64]),
        "iris_memcpy_d2h": (C.c_int, [vp, vp, u64]),
        "iris_memcpy_d2d": (C.c_int, [vp, vp, u64]),
        "iris_time_product": (C.c_int, [vp, u32, vp, u32, vp, u32, C.POINTER(C.c_double)]),
        "iris_time_bcast_product": (C.c_int, [vp, u32, vp, vp, u32, C.POINTER(C.c_double)]),
        "iris_attention_numerics": (C.c_int, [vp, vp, vp, vp, u32, u32, vp, vp, vp]),
        "iris_silu_device": (C.c_int, [vp, u32, vp]),
        "iris_silu_table_device": (C.c_int, [vp, u32, vp]),
        "iris_time_product_ws": (C.c_int, [vp, vp, u32, vp, vp, u64, u32, C.POINTER(C.c_double)]),
        "iris_kernel_tracer_loaded": (C.c_int, []),
        "iris_probe_hbm_read": (C.c_int, [vp, u64, u32, C.POINTER(C.c_double)]),
        "iris_probe_mfma_i8": (C.c_int, [u32, u32, C.POINTER(C.c_double)]),
        "iris_probe_handoff": (C.c_int, [u32, C.POINTER(C.c_double), C.POINTER(C.c_double), C.POINTER(C.c_double)]),
        "iris_probe_row_latency": (C.c_int, [u32, C.POINTER(C.c_double), C.POINTER(C.c_double)]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def kernel_tracer_loaded() -> bool:
    """True when a kernel tracer (rocprofv3's profiler SDK) is loaded in this
    process: the library then refuses graph replays of the decode pass."""
    return bool(lib().iris_kernel_tracer_loaded())


def header_functions() -> list:
    """Names of the functions include/iris_hip.h declares."""
    import re
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b([a-z][a-z0-9_]*)\s*\([^;{]*\)\s*;", text)))


class DeviceBuffer:
    """A device allocation (plumbing for tests and benchmarks)."""

    def __init__(self, nbytes: int):
        self.nbytes = nbytes
        self.ptr = C.c_void_p()
        check(lib().iris_device_malloc(nbytes, C.byref(self.ptr)), "device malloc")

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        check(lib().iris_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes), "copy to device")
        return b

    def to_array(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        check(lib().iris_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes), "copy to host")
        return out

    def free(self):
        if self.ptr:
            lib().iris_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
