"""ctypes binding of the C ABI in include/kq.h (kidi_amd/lib/libkq_hip.so).

Importing this module fails loudly (ImportError) when the HIP library has not been built: there is no fallback.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libkq_hip.so")

# kq_status (kidi::core::ErrorCode + 1)
KQ_OK, KQ_INVALID_ARGUMENT, KQ_IO, KQ_INVALID_MANIFEST, KQ_UNSUPPORTED, KQ_RUNTIME = range(6)
STATUS_NAMES = {1: "INVALID_ARGUMENT", 2: "IO", 3: "INVALID_MANIFEST", 4: "UNSUPPORTED", 5: "RUNTIME"}
# kq_dtype
KQ_NONE, KQ_F32, KQ_F16, KQ_BF16, KQ_U8, KQ_I8, KQ_ZP_U8 = -1, 0, 1, 2, 3, 4, 5
KQ_HOST, KQ_DEVICE = 0, 1
PATH_BLOCKWISE, PATH_SYMMETRIC, PATH_PORTABLE = 0, 1, 2

# Every symbol include/kq.h declares.
EXPORTS = (
    "kq_last_error", "kq_version", "kq_arch", "kq_weight_pack", "kq_weight_free", "kq_weight_info",
    "kq_select_path", "kq_linear_workspace_size", "kq_packed_linear", "kq_weight_pack_concat",
    "kq_packed_linear_gelu_gate", "kq_debug_quantize", "kq_debug_partials", "kq_layout_bytes",
    "kq_layout_encode_host", "kq_layout_decode_host", "kq_ffn_workspace_size", "kq_gated_feed_forward",
    "kq_greedy_workspace_size", "kq_greedy_token", "kq_greedy_linear_workspace_size", "kq_packed_linear_greedy",
    "kq_weight_export_size", "kq_weight_export", "kq_weight_import", "kq_rms_norm", "kq_rms_linear_workspace_size",
    "kq_packed_linear_rms", "kq_quantize_weight", "kq_debug_read_floor", "kq_debug_read_floor_shape",
    "kq_debug_mfma_ceiling_workgroups", "kq_debug_mfma_ceiling",
    "kq_debug_route", "kq_debug_route_shape",
    "kq_lowbit_parity_linear", "kq_packed_linear_noalloc", "kq_gelu_multiply", "kq_silu_multiply",
)

# kq_debug_route values: the kernel sequence a projection call runs
ROUTE_NONE, ROUTE_DECODE, ROUTE_SKINNY, ROUTE_GEMM_I4, ROUTE_GEMM_I4G, ROUTE_GEMV, ROUTE_GEMM, ROUTE_ROWMAJOR, \
    ROUTE_PORTABLE, ROUTE_GEMM8, ROUTE_GEMM8W = range(11)
ROUTE_NAMES = ("none", "decode_kernel", "skinny_kernel", "gemm_i4_kernel", "gemm_i4g_kernel", "gemv_kernel",
               "gemm_kernel", "rowmajor_kernel", "portable_kernel", "gemm8_kernel", "gemm8w_kernel")


class PackDesc(ctypes.Structure):
    _fields_ = [
        ("bits", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("values", ctypes.c_void_p),
        ("values_dtype", ctypes.c_int),
        ("scales", ctypes.c_void_p),
        ("scales_dtype", ctypes.c_int),
        ("zeros", ctypes.c_void_p),
        ("zeros_dtype", ctypes.c_int),
        ("memory", ctypes.c_int),
    ]


class FfnArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int),
        ("m", ctypes.c_int64),
        ("gate_up_input_scale", ctypes.c_float),
        ("gate_up_output_scale", ctypes.c_float),
        ("down_input_scale", ctypes.c_float),
        ("down_output_scale", ctypes.c_float),
        ("silu", ctypes.c_int32),
        ("y", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class LinearArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int),
        ("m", ctypes.c_int64),
        ("input_scale", ctypes.c_float),
        ("output_scale", ctypes.c_float),
        ("y", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class RmsArgs(ctypes.Structure):
    _fields_ = [
        ("x", ctypes.c_void_p),
        ("x_dtype", ctypes.c_int),
        ("rows", ctypes.c_int64),
        ("width", ctypes.c_int64),
        ("weight", ctypes.c_void_p),
        ("residual", ctypes.c_void_p),
        ("output_scale", ctypes.c_void_p),
        ("epsilon", ctypes.c_float),
        ("y", ctypes.c_void_p),
    ]


class NormDesc(ctypes.Structure):
    _fields_ = [
        ("weight", ctypes.c_void_p),
        ("epsilon", ctypes.c_float),
        ("residual", ctypes.c_void_p),
        ("residual_weight", ctypes.c_void_p),
        ("residual_scale", ctypes.c_void_p),
        ("residual_epsilon", ctypes.c_float),
        ("hidden", ctypes.c_void_p),
    ]


class KqError(RuntimeError):
    """A non-OK kq_status; ``code`` is the kidi::core::ErrorCode name."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.code = STATUS_NAMES.get(status, str(status))
        super().__init__(f"{self.code}: {message}")


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"kidi_amd HIP library not built: {LIB_PATH} is missing (run __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, i64, f32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t
    L.kq_last_error.restype = ctypes.c_char_p
    L.kq_version.restype = i32
    L.kq_arch.restype = ctypes.c_char_p
    L.kq_weight_pack.argtypes = [ctypes.POINTER(PackDesc), vp, ctypes.POINTER(vp)]
    L.kq_weight_pack.restype = ctypes.c_int
    L.kq_weight_pack_concat.argtypes = [ctypes.POINTER(PackDesc), i32, vp, ctypes.POINTER(vp)]
    L.kq_weight_pack_concat.restype = ctypes.c_int
    L.kq_weight_free.argtypes = [vp]
    L.kq_weight_free.restype = None
    L.kq_weight_info.argtypes = [vp, ctypes.POINTER(i32), ctypes.POINTER(i32), ctypes.POINTER(i64),
                                 ctypes.POINTER(i64), ctypes.POINTER(i32), ctypes.POINTER(sz)]
    L.kq_weight_info.restype = ctypes.c_int
    L.kq_select_path.argtypes = [i32, i64, i64, i64, i32, f32]
    L.kq_select_path.restype = i32
    L.kq_linear_workspace_size.argtypes = [vp, i64]
    L.kq_linear_workspace_size.restype = sz
    L.kq_packed_linear.argtypes = [vp, ctypes.POINTER(LinearArgs), vp]
    L.kq_packed_linear.restype = ctypes.c_int
    L.kq_packed_linear_gelu_gate.argtypes = [vp, ctypes.POINTER(LinearArgs), vp]
    L.kq_packed_linear_gelu_gate.restype = ctypes.c_int
    L.kq_ffn_workspace_size.argtypes = [vp, vp, i64]
    L.kq_ffn_workspace_size.restype = sz
    L.kq_gated_feed_forward.argtypes = [vp, vp, ctypes.POINTER(FfnArgs), vp]
    L.kq_gated_feed_forward.restype = ctypes.c_int
    L.kq_weight_export_size.argtypes = [vp]
    L.kq_weight_export_size.restype = sz
    L.kq_weight_export.argtypes = [vp, vp, sz, vp]
    L.kq_weight_export.restype = ctypes.c_int
    L.kq_weight_import.argtypes = [vp, sz, vp, ctypes.POINTER(vp)]
    L.kq_weight_import.restype = ctypes.c_int
    L.kq_greedy_workspace_size.argtypes = [i64, i64]
    L.kq_greedy_workspace_size.restype = sz
    L.kq_greedy_token.argtypes = [vp, i64, i64, vp, vp, sz, vp]
    L.kq_greedy_token.restype = ctypes.c_int
    for name in ("kq_gelu_multiply", "kq_silu_multiply"):
        getattr(L, name).argtypes = [vp, vp, i64, vp, vp]
        getattr(L, name).restype = ctypes.c_int
    L.kq_greedy_linear_workspace_size.argtypes = [vp, i64]
    L.kq_greedy_linear_workspace_size.restype = sz
    L.kq_packed_linear_greedy.argtypes = [vp, ctypes.POINTER(LinearArgs), vp, vp]
    L.kq_packed_linear_greedy.restype = ctypes.c_int
    L.kq_rms_norm.argtypes = [ctypes.POINTER(RmsArgs), vp]
    L.kq_rms_norm.restype = ctypes.c_int
    L.kq_rms_linear_workspace_size.argtypes = [vp, i64]
    L.kq_rms_linear_workspace_size.restype = sz
    L.kq_packed_linear_rms.argtypes = [vp, ctypes.POINTER(LinearArgs), ctypes.POINTER(NormDesc), i32, vp]
    L.kq_packed_linear_rms.restype = ctypes.c_int
    L.kq_quantize_weight.argtypes = [vp, ctypes.c_int, i64, i64, i32, i32, i32, vp, vp, vp, vp]
    L.kq_quantize_weight.restype = ctypes.c_int
    L.kq_debug_read_floor.argtypes = [vp, ctypes.c_size_t, vp, vp]
    L.kq_debug_read_floor.restype = ctypes.c_int
    L.kq_debug_read_floor_shape.argtypes = [vp, ctypes.c_size_t, i32, i32, i32, vp, vp]
    L.kq_debug_read_floor_shape.restype = ctypes.c_int
    L.kq_debug_mfma_ceiling_workgroups.argtypes = []
    L.kq_debug_mfma_ceiling_workgroups.restype = ctypes.c_int32
    L.kq_debug_mfma_ceiling.argtypes = [i32, vp, vp, vp]
    L.kq_debug_mfma_ceiling.restype = ctypes.c_int
    L.kq_packed_linear_noalloc.argtypes = [vp, ctypes.POINTER(LinearArgs), vp]
    L.kq_packed_linear_noalloc.restype = ctypes.c_int
    L.kq_lowbit_parity_linear.argtypes = [vp, ctypes.POINTER(LinearArgs), vp]
    L.kq_lowbit_parity_linear.restype = ctypes.c_int
    L.kq_debug_route.argtypes = [vp, ctypes.POINTER(LinearArgs), i32]
    L.kq_debug_route.restype = i32
    L.kq_debug_route_shape.argtypes = [i32, i32, i64, i64, i32, i32, i64, ctypes.c_int, f32, i32]
    L.kq_debug_route_shape.restype = i32
    L.kq_debug_quantize.argtypes = [vp, vp, ctypes.c_int, i64, f32, vp, vp, vp, vp, vp]
    L.kq_debug_quantize.restype = ctypes.c_int
    L.kq_debug_partials.argtypes = [vp, ctypes.POINTER(LinearArgs), vp, vp]
    L.kq_debug_partials.restype = ctypes.c_int
    L.kq_layout_bytes.argtypes = [i32, i32, i64, i64]
    L.kq_layout_bytes.restype = sz
    L.kq_layout_encode_host.argtypes = [i32, i64, i64, vp, vp]
    L.kq_layout_encode_host.restype = ctypes.c_int
    L.kq_layout_decode_host.argtypes = [i32, i64, i64, vp, vp]
    L.kq_layout_decode_host.restype = ctypes.c_int
    _lib = L
    return L


def check(status: int) -> None:
    if status != KQ_OK:
        raise KqError(status, load().kq_last_error().decode())
