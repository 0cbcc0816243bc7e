"""ctypes binding of lib/libkq_adapter.so's test surface (the C++ PACKED_LINEAR adapter, kidi_amd/adapter)."""

import ctypes
import os

from kidi_amd import _native as N

PATH = os.path.join(os.path.dirname(N.LIB_PATH), "libkq_adapter.so")
EXPORTS = ["kqa_last_error", "kqa_operation_name", "kqa_prepare", "kqa_prepare_other", "kqa_run", "kqa_run_into",
           "kqa_run_", "kqa_synchronize", "kqa_allocations", "kqa_supports_replay", "kqa_release", "kqa_free"]
_lib = None


def load():
    global _lib
    if _lib is None:
        N.load()  # libkq_hip.so first (the adapter links against it)
        L = ctypes.CDLL(PATH)
        vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
        L.kqa_last_error.restype = ctypes.c_char_p
        L.kqa_operation_name.argtypes = [ctypes.c_int]
        L.kqa_operation_name.restype = ctypes.c_char_p
        L.kqa_prepare.argtypes = [ctypes.POINTER(N.PackDesc), f32, f32, ctypes.c_int, vp, ctypes.POINTER(vp)]
        L.kqa_prepare_other.argtypes = [ctypes.c_int, ctypes.c_int]
        L.kqa_run.argtypes = [vp, vp, ctypes.c_int, i64, i64, ctypes.c_int, ctypes.c_int, ctypes.POINTER(vp)]
        L.kqa_run_into.argtypes = [vp, vp, ctypes.c_int, i64, i64, vp, i64, i64, ctypes.c_int]
        L.kqa_run_.argtypes = [vp, vp, ctypes.c_int, i64, i64, vp, i64, ctypes.c_int]
        L.kqa_synchronize.argtypes = [vp]
        L.kqa_allocations.argtypes = [vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]
        L.kqa_allocations.restype = None
        L.kqa_supports_replay.argtypes = [vp]
        L.kqa_release.argtypes = [vp]
        L.kqa_release.restype = None
        L.kqa_free.argtypes = [vp]
        L.kqa_free.restype = None
        _lib = L
    return _lib


def error():
    return load().kqa_last_error().decode()
