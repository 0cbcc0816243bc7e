"""Deterministic synthetic inputs shaped like the benchmark configurations (numpy only, no GPU)."""

from __future__ import annotations

import numpy as np


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Kidi layout: element k of a row in bits (k % (8/bits)) * bits of byte k / (8/bits), two's complement."""
    codes = np.asarray(codes, dtype=np.int64)
    N, K = codes.shape
    per = 8 // bits
    if bits == 8:
        return codes.astype(np.int8).view(np.uint8).reshape(N, K)
    out = np.zeros((N, K // per), np.uint8)
    mask = (1 << bits) - 1
    for i in range(per):
        out |= ((codes[:, i::per] & mask) << (i * bits)).astype(np.uint8)
    return out


def weights(rng: np.random.Generator, N: int, K: int, bits: int, group: int, zero_points: bool = False,
            scale_dtype=np.float16, code_range=None):
    """Codes uniform over the bit width's range (or code_range), fp16 scales in [0.002, 0.02], optional uint4
    zero points in [0, 15]. Returns (values u8 [N, K/(8/bits)], scales [N, B], zero_points u8 [N, B] or None,
    codes int8 [N, K])."""
    lo, hi = code_range if code_range else (-(1 << (bits - 1)), (1 << (bits - 1)) - 1)
    codes = rng.integers(lo, hi + 1, size=(N, K)).astype(np.int8)
    scales = rng.uniform(0.002, 0.02, size=(N, K // group)).astype(scale_dtype)
    zp = rng.integers(0, 16, size=(N, K // group)).astype(np.uint8) if zero_points else None
    return pack_codes(codes, bits), scales, zp, codes


def activations(rng: np.random.Generator, M: int, K: int, outliers: float = 0.0) -> np.ndarray:
    """bf16-representable N(0,1) activations (float32 holding bf16 values), optional outliers at x20."""
    x = rng.standard_normal((M, K)).astype(np.float32)
    if outliers > 0:
        count = max(1, int(round(outliers * M * K)))
        idx = rng.choice(M * K, size=count, replace=False)
        x.reshape(-1)[idx] *= 20.0
    b = x.view(np.uint32)
    b = ((b + (((b >> 16) & 1) + 0x7FFF)) >> 16) << 16
    return b.astype(np.uint32).view(np.float32)


def expected_partials(ref, q, codes, zpa, bits, group, zero_points=None, dynamic=True):
    """P' as the kernels define it: sum q*c, plus (8 - zp) * Q for uint4 zero points, minus zp_a * C for 8-bit."""
    P, C = ref.partials(q, codes, group)
    P = P.astype(np.int64)
    M, K = q.shape
    B = K // group
    Q = q.astype(np.int64).reshape(M, B, group).sum(axis=2)
    if zero_points is not None:
        P = P + (8 - zero_points.astype(np.int64))[None, :, :] * Q[:, None, :]
    if bits == 8 and dynamic:
        P = P - zpa.astype(np.int64)[:, None, :] * C.astype(np.int64)[None, :, :]
    return P
