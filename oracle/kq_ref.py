"""numpy front end to the CPU oracle ``oracle/libkq_ref.so`` (built from ``oracle/kq_ref.cpp``).

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it
as the checker. Nothing under ``kidi_amd/`` imports it. Every function states the reference file:line it follows;
the C++ source holds the closed forms and the pinning status of each function.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkq_ref.so")

F32, F16, BF16, U8, I8, ZP_U8 = 0, 1, 2, 3, 4, 5
PATH_BLOCKWISE, PATH_SYMMETRIC, PATH_PORTABLE = 0, 1, 2

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (g++ only; no GPU, no ROCm)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        i64, i32, f32, vp = ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_void_p
        L.kqr_select_path.argtypes = [i32, i64, i64, i64, i32, f32]
        L.kqr_select_path.restype = i32
        L.kqr_half_to_float.argtypes = [ctypes.c_uint16]
        L.kqr_half_to_float.restype = f32
        L.kqr_pack_weight.argtypes = [vp, i32, i64, i64, i32, i64, i32, vp, vp, vp]
        L.kqr_pack_weight.restype = i32
        L.kqr_unpack_codes.argtypes = [vp, i64, i64, i32, vp]
        L.kqr_unpack_codes.restype = i32
        L.kqr_qat_to_signed.argtypes = [vp, i64, i32]
        L.kqr_qat_to_signed.restype = None
        L.kqr_quantize_dynamic.argtypes = [vp, i64, i64, i64, i32, vp, vp, vp, vp]
        L.kqr_quantize_dynamic.restype = i32
        L.kqr_quantize_static.argtypes = [vp, i64, i64, i64, f32, vp, vp]
        L.kqr_quantize_static.restype = i32
        L.kqr_partials.argtypes = [vp, vp, i64, i64, i64, i64, vp, vp]
        L.kqr_partials.restype = i32
        L.kqr_packed_linear.argtypes = [vp, i32, i64, i64, vp, i64, i32, i64, vp, i32, vp, i32, f32, f32, vp, i32]
        L.kqr_packed_linear.restype = i32
        L.kqr_gelu_gate.argtypes = [vp, i64, i64, vp]
        L.kqr_gelu_gate.restype = None
        L.kqr_silu_gate.argtypes = [vp, i64, i64, vp]
        L.kqr_silu_gate.restype = None
        L.kqr_rms_norm.argtypes = [vp, i32, i64, i64, vp, vp, vp, f32, vp, vp]
        L.kqr_rms_norm.restype = i32
        L.kqr_parity_linear.argtypes = [vp, i64, i64, vp, i64, i32, i64, vp, f32, f32, vp]
        L.kqr_parity_linear.restype = i32
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _float_dtype(a: np.ndarray, bf16: bool = False) -> int:
    if a.dtype == np.float32:
        return F32
    if a.dtype == np.float16:
        return F16
    if a.dtype == np.uint16:
        return BF16 if bf16 else F16
    raise TypeError(f"unsupported float storage {a.dtype}")


def select_path(bits: int, group: int, K: int, N: int, has_zero: bool, input_scale: float) -> int:
    """CpuBackend::prepare selection for PACKED_LINEAR (runtime/ynn/operators.cpp:2739-2900)."""
    return lib().kqr_select_path(bits, group, K, N, int(has_zero), input_scale)


def half_to_float(h: int) -> float:
    return lib().kqr_half_to_float(h)


def pack_weight(weight: np.ndarray, bits: int = 4, group_size: int = 128, asymmetric_clip: bool = False,
                bf16: bool = False):
    """ops::pack_weight (src/kidi/ops/quantization.cpp:12-133). ``weight`` is float32/float16, or uint16 holding
    bf16 bit patterns when ``bf16``. Returns (values u8 [N, K/(8/bits)], scales f32 [N, K/g], zeros f32|None)."""
    w = np.ascontiguousarray(weight)
    if w.ndim != 2:
        raise ValueError("invalid packed weight dimensions, precision or group size")
    rows, width = w.shape
    per = 8 // bits if bits in (2, 4, 8) else 1
    groups = width // group_size if group_size > 0 else 0
    values = np.zeros((rows, max(width // per, 0)), np.uint8)
    scales = np.zeros((rows, groups), np.float32)
    zeros = np.zeros((rows, groups), np.float32) if (asymmetric_clip and bits == 4) else None
    rc = lib().kqr_pack_weight(_p(w), _float_dtype(w, bf16), rows, width, bits, group_size, int(asymmetric_clip),
                               _p(values), _p(scales), _p(zeros))
    if rc != 0:
        raise ValueError("invalid packed weight dimensions, precision, group size or non-finite weight")
    return values, scales, zeros


def unpack_codes(values: np.ndarray, width: int, bits: int) -> np.ndarray:
    """Signed codes [N, K] (eager_test.cpp:318-320)."""
    v = np.ascontiguousarray(values, dtype=np.uint8)
    codes = np.zeros((v.shape[0], width), np.int8)
    if lib().kqr_unpack_codes(_p(v), v.shape[0], width, bits, _p(codes)) != 0:
        raise ValueError("bits")
    return codes


def qat_to_signed(values: np.ndarray, bits: int) -> np.ndarray:
    """model/gemma4.cpp:358-369 XOR conversion (returns a converted copy)."""
    out = np.ascontiguousarray(values, dtype=np.uint8).copy()
    lib().kqr_qat_to_signed(_p(out), out.size, bits)
    return out


def quantize_dynamic(x: np.ndarray, group: int, bits: int):
    """Per-(row, block) dynamic activation quantization (hnsw_test.cpp:490-520).
    Returns (q int8 [M, K], scale f32 [M, B], sum int32 [M, B], zero_point int32 [M, B])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    B = K // group
    q = np.zeros((M, K), np.int8)
    s = np.zeros((M, B), np.float32)
    Q = np.zeros((M, B), np.int32)
    zp = np.zeros((M, B), np.int32)
    if lib().kqr_quantize_dynamic(_p(x), M, K, group, bits, _p(q), _p(s), _p(Q), _p(zp)) != 0:
        raise ValueError("group")
    return q, s, Q, zp


def quantize_static(x: np.ndarray, group: int, input_scale: float):
    """Calibrated quantization q = clamp(nearbyint(x / input_scale), -128, 127) (eager_test.cpp:97-98)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    q = np.zeros((M, K), np.int8)
    Q = np.zeros((M, K // group), np.int32)
    if lib().kqr_quantize_static(_p(x), M, K, group, input_scale, _p(q), _p(Q)) != 0:
        raise ValueError("group or scale")
    return q, Q


def partials(q: np.ndarray, codes: np.ndarray, group: int):
    """P [M, N, B] = sum_{k in b} q*c and C [N, B] = sum_{k in b} c (exact int32)."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    c = np.ascontiguousarray(codes, dtype=np.int8)
    M, K = q.shape
    N = c.shape[0]
    B = K // group
    P = np.zeros((M, N, B), np.int32)
    C = np.zeros((N, B), np.int32)
    if lib().kqr_partials(_p(q), _p(c), M, N, K, group, _p(P), _p(C)) != 0:
        raise ValueError("group")
    return P, C


def packed_linear(x: np.ndarray, values: np.ndarray, scales: np.ndarray, bits: int, group_size: int,
                  input_scale: float = 0.0, output_scale: float = 0.0, zeros: np.ndarray | None = None,
                  zero_points: np.ndarray | None = None, x_bf16: bool = False, threads: int = 1):
    """Context::packed_linear on the CPU backend (ops/context.cpp:821-939 -> runtime/ynn/operators.cpp).
    ``x`` float32 [M, K] (or uint16 bf16 bits with ``x_bf16``); ``scales`` float32/float16; ``zeros`` additive
    float32/float16, or ``zero_points`` uint8 [N, B] in 0..15 (zero = (8 - zp) * scale). Returns (y, path)."""
    x = np.ascontiguousarray(x)
    M, K = x.shape
    v = np.ascontiguousarray(values)
    N = v.shape[0]
    s = np.ascontiguousarray(scales)
    if zeros is not None and zero_points is not None:
        raise ValueError("give zeros or zero_points, not both")
    z = None
    zdt = -1
    if zeros is not None:
        z = np.ascontiguousarray(zeros)
        zdt = _float_dtype(z)
    elif zero_points is not None:
        z = np.ascontiguousarray(zero_points, dtype=np.uint8)
        zdt = ZP_U8
    y = np.zeros((M, N), np.float32)
    xdt = BF16 if x_bf16 else F32
    if not x_bf16:
        x = x.astype(np.float32, copy=False)
    path = lib().kqr_packed_linear(_p(x), xdt, M, K, _p(v), N, bits, group_size, _p(s), _float_dtype(s), _p(z), zdt,
                                   input_scale, output_scale, _p(y), threads)
    if path < 0:
        raise ValueError("packed linear shape or dtype mismatch")
    return y, path


def parity_linear(x: np.ndarray, values: np.ndarray, scales: np.ndarray, bits: int, group_size: int,
                  input_scale: float, output_scale: float) -> np.ndarray:
    """Kidi's LOWBIT_PARITY projection (runtime/parity_math.cpp:226-291): calibrated input grid, c * s weights, serial
    FMA per output, output grid. Raises ValueError("INVALID_ARGUMENT" / "UNSUPPORTED") as the reference fails."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    v = np.ascontiguousarray(values, dtype=np.uint8)
    N = v.shape[0]
    s = np.ascontiguousarray(scales, dtype=np.float32)
    y = np.zeros((M, N), np.float32)
    st = lib().kqr_parity_linear(_p(x), M, K, _p(v), N, bits, group_size, _p(s), input_scale, output_scale, _p(y))
    if st == 1:
        raise ValueError("INVALID_ARGUMENT")
    if st == 2:
        raise ValueError("UNSUPPORTED")
    return y


def gelu_gate(gate_up: np.ndarray) -> np.ndarray:
    """gelu_tanh(gate) * up over [..., 2I] halves (ops/context.cpp:957-963, eager_test.cpp:142-159)."""
    g = np.ascontiguousarray(gate_up, dtype=np.float32)
    rows = g.size // g.shape[-1]
    width = g.shape[-1] // 2
    out = np.zeros(g.shape[:-1] + (width,), np.float32)
    lib().kqr_gelu_gate(_p(g), rows, width, _p(out))
    return out


def silu_gate(gate_up: np.ndarray) -> np.ndarray:
    """g / (1 + exp(-g)) * up over [..., 2I] halves (ops/context.cpp:964-969, eager_test.cpp:176-179)."""
    g = np.ascontiguousarray(gate_up, dtype=np.float32)
    rows = g.size // g.shape[-1]
    width = g.shape[-1] // 2
    out = np.zeros(g.shape[:-1] + (width,), np.float32)
    lib().kqr_silu_gate(_p(g), rows, width, _p(out))
    return out


def gated_feed_forward(x: np.ndarray, gate_up_values: np.ndarray, gate_up_scales: np.ndarray, down_values: np.ndarray,
                       down_scales: np.ndarray, bits: int, gate_up_group: int, down_group: int,
                       gate_up_input_scale: float, gate_up_output_scale: float, down_input_scale: float,
                       down_output_scale: float, silu: bool = False, gate_up_zero_points=None, down_zero_points=None,
                       x_bf16: bool = False, threads: int = 1):
    """Context::gated_feed_forward as its composed form (ops/context.cpp:977-984): the gate/up projection (rows
    [gate; up]), GELU-tanh or SiLU gating, then the down projection of h (whose calibrated codes are
    clamp(rint(h / down_input_scale)), what PackedFeedForward's mid tiles hold, runtime/ynn/operators.cpp:1437-1444).
    Returns (y, h)."""
    gu, _ = packed_linear(x, gate_up_values, gate_up_scales, bits, gate_up_group, gate_up_input_scale,
                          gate_up_output_scale, zero_points=gate_up_zero_points, x_bf16=x_bf16, threads=threads)
    h = silu_gate(gu) if silu else gelu_gate(gu)
    y, _ = packed_linear(h, down_values, down_scales, bits, down_group, down_input_scale, down_output_scale,
                         zero_points=down_zero_points, threads=threads)
    return y, h


def greedy_token(logits: np.ndarray) -> np.ndarray:
    """GREEDY_TOKEN (runtime/ynn/operators.cpp:117-178): per row of [..., width] logits the first index of the maximum
    (strict >, so -0 and 0 tie to the earlier), -1 when the row holds a NaN or an infinity (eager_test.cpp:231-252)."""
    x = np.asarray(logits, dtype=np.float32)
    if x.ndim == 0 or x.shape[-1] == 0:
        raise ValueError("greedy selection requires [..., width > 0] logits")
    rows = x.reshape(-1, x.shape[-1])
    out = np.empty(rows.shape[0], np.int32)
    for r, row in enumerate(rows):
        out[r] = -1 if not np.all(np.isfinite(row)) else int(np.argmax(row))  # argmax returns the first maximum
    return out.reshape(x.shape[:-1])


def rms_norm(x: np.ndarray, weight: np.ndarray, epsilon: float, residual: np.ndarray | None = None,
             scale: float | None = None, x_bf16: bool = False):
    """RMS normalization over the last axis (Context::rms_norm / rms_norm_residual, ops/context.cpp:1043-1049,
    :1103-1122; RmsNorm, runtime/ynn/operators.cpp:553-620): y = x * inv * weight, or with a residual
    (r + x * inv * weight) [* scale], inv = 1 / sqrt(sum(x^2) / width + epsilon) in the fixed summation order of
    kq_ref.cpp. x (and residual) are float32, or bf16 bit patterns (uint16) with x_bf16. Returns (y, inv per row)."""
    xa = np.ascontiguousarray(x, dtype=np.uint16 if x_bf16 else np.float32)
    width = xa.shape[-1]
    rows = xa.size // width if width else 0
    w = np.ascontiguousarray(weight, dtype=np.float32)
    r = None if residual is None else np.ascontiguousarray(residual, dtype=xa.dtype)
    if r is not None and r.shape != xa.shape:
        raise ValueError("residual shape mismatch")
    s = None if scale is None else np.array([scale], np.float32)
    y = np.zeros(xa.shape, np.float32)
    inv = np.zeros(max(rows, 1), np.float32)
    rc = lib().kqr_rms_norm(_p(xa), BF16 if x_bf16 else F32, rows, width, _p(w), _p(r), _p(s), epsilon, _p(y), _p(inv))
    if rc != 0:
        raise ValueError("invalid RMS normalization operands")
    return y, inv[:rows]


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16); NaN stays NaN."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rounding = ((b >> 16) & 1) + 0x7FFF
    out = ((b + rounding) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    out[nan] = 0x7FC0
    return out


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
