"""Writes the golden fixtures of the quantized linear layer: small seeded cases, one per kernel path, with the
oracle's outputs (activation codes, block statistics, integer partials P' and fp32 y).

    python tests/golden/make_golden.py        # rewrites tests/golden/*.npz

The oracle (oracle/kq_ref.cpp) follows the reference's closed forms; every fixture is also checked against a
float64 restatement of y = sum_b a_s * (w_s * P + z_w * Q) in tests/test_golden.py, which does not go through the
oracle's own epilogue. Inputs are generated here with numpy's PCG64 from fixed seeds; the shapes sit in the domain
of each kernel path of the HIP library (decode M <= 4, skinny M <= 16, int8 MFMA GEMMs M > 16 with g = 128 and with
g = 32 / 64, row-major path for g the tiles cannot carry, calibrated 2/4/8-bit, GELU gate); the rms_* fixtures hold
an RMS normalization (plain, or after the residual form) and the projection of its output."""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import kq_ref  # noqa: E402  (test infrastructure)
from tests.cases import activations, expected_partials, weights  # noqa: E402

# name: (bits, group, M, K, N, zeros, input_scale, output_scale, x_bf16, outliers, gelu, seed)
CASES = {
    "c1_sym_g32_decode": (4, 32, 1, 512, 256, None, 0.0, 0.0, True, 0.0, False, 11),
    "c2_asym_g128_decode": (4, 128, 4, 1024, 128, "zp", 0.0, 0.0, True, 0.001, False, 12),
    "asym_g128_skinny": (4, 128, 9, 512, 128, "zp", 0.0, 0.0, False, 0.0, False, 13),
    "c3_asym_g128_prefill": (4, 128, 20, 1024, 144, "zp", 0.0, 0.0, True, 0.001, False, 14),
    "sym_g128_prefill_static": (4, 128, 24, 512, 64, None, 0.05, 0.0, False, 0.0, False, 15),
    "float_zero_g128": (4, 128, 3, 512, 128, "f16", 0.0, 0.0, False, 0.0, False, 16),
    "int8_g32_dynamic": (8, 32, 2, 256, 64, None, 0.0, 0.0, False, 0.001, False, 17),
    "int8_g32_calibrated": (8, 32, 3, 256, 64, None, 0.03, 0.125, False, 0.0, False, 18),
    "int2_g32_calibrated": (2, 32, 2, 512, 64, None, 0.05, 0.0, False, 0.0, False, 19),
    "asym_g96_rowmajor": (4, 96, 2, 384, 64, "zp", 0.0, 0.0, False, 0.0, False, 20),
    "gelu_gate_g128": (4, 128, 2, 512, 128, "zp", 0.0, 0.0, False, 0.0, True, 21),
    "gelu_gate_g128_prefill": (4, 128, 33, 512, 64, "zp", 0.0, 0.0, True, 0.0, True, 22),
    "sym_g32_prefill": (4, 32, 40, 512, 256, None, 0.0, 0.0, True, 0.001, False, 23),
    "g64_prefill_static": (4, 64, 20, 512, 128, None, 0.05, 0.0, False, 0.0, False, 24),
}

# RMS normalization before a projection (Context::rms_norm / rms_norm_residual, ops/context.cpp:1043-1049,
# :1103-1122): name: (M, K, N, bits, group, zero points, residual form, seed)
RMS_CASES = {
    "rms_residual_decode": (2, 1024, 256, 4, 128, True, True, 31),
    "rms_plain_prefill": (40, 1024, 256, 4, 128, True, False, 32),
}


def make_rms(case) -> dict:
    M, K, N, bits, group, zeros, residual, seed = case
    rng = np.random.default_rng(seed)
    values, scales, zp, _ = weights(rng, N, K, bits, group, zero_points=zeros)
    x = activations(rng, M, K, 0.001)
    r = activations(rng, M, K)
    w_in = rng.uniform(0.5, 1.5, K).astype(np.float32)
    w_res = rng.uniform(-1.5, 1.5, K).astype(np.float32)
    eps, eps_res, scale = 1e-6, 1e-5, 0.78125
    out = dict(bits=bits, group=group, x=x, values=values, scales=scales, w_in=w_in, eps=np.float32(eps))
    if zp is not None:
        out["zero_points"] = zp
    src = x
    if residual:
        hidden, _ = kq_ref.rms_norm(x, w_res, eps_res, residual=r, scale=scale)
        out.update(residual=r, w_res=w_res, eps_res=np.float32(eps_res), res_scale=np.float32(scale), hidden=hidden)
        src = hidden
    normed, inv = kq_ref.rms_norm(src, w_in, eps)
    y, path = kq_ref.packed_linear(normed, values, scales, bits, group, zero_points=zp)
    out.update(normed=normed, inv=inv, y=y, path=path)
    return out


def make(name: str, case) -> dict:
    bits, group, M, K, N, zeros, in_s, out_s, x_bf16, outliers, gelu, seed = case
    rng = np.random.default_rng(seed)
    values, scales, zp, codes = weights(rng, N, K, bits, group, zero_points=zeros in ("zp", "f16"))
    zf = None
    if zeros == "f16":
        zf = rng.uniform(-0.05, 0.05, size=scales.shape).astype(np.float16)
        zp = None
    x = activations(rng, M, K, outliers)
    y, path = kq_ref.packed_linear(x, values, scales, bits, group, in_s, out_s, zeros=zf, zero_points=zp)
    if in_s == 0:
        q, s, Q, zpa = kq_ref.quantize_dynamic(x, group, bits)
    else:
        (q, Q), s, zpa = kq_ref.quantize_static(x, group, in_s), np.zeros((M, K // group), np.float32), None
    P = expected_partials(kq_ref, q, codes, zpa, bits, group, zero_points=zp, dynamic=in_s == 0)
    out = dict(bits=bits, group=group, input_scale=np.float32(in_s), output_scale=np.float32(out_s),
               x_bf16=x_bf16, gelu=gelu, path=path, x=x, values=values, scales=scales, q=q,
               act_scale=s, act_sum=Q, P=P.astype(np.int32), y=y)
    if zp is not None:
        out["zero_points"] = zp
    if zf is not None:
        out["zeros"] = zf
    if zpa is not None:
        out["act_zero"] = zpa
    if gelu:
        out["h"] = kq_ref.gelu_gate(y)
    return out


def main() -> None:
    for name, case in CASES.items():
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **make(name, case))
        print(name)
    for name, case in RMS_CASES.items():
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **make_rms(case))
        print(name)


if __name__ == "__main__":
    main()
