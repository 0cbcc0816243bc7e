"""Every BASELINE configuration at its stated size on the GPU, against the CPU oracle, through the C ABI.

For each configuration the test asserts which kernel the call runs (kq_debug_route), that the production kernel's y
equals the parity-dump variant's y bit for bit (so the instances the dump does not use are tied to the bit-exact
partials), that the whole fp32 output is within max|dy| <= 2e-3 * max|y_ref| of the oracle, and that the int32
per-group partials are bit-exact on sampled rows and columns (all of M x N x K/g is too large to move to the host
at prefill sizes). Shapes, formats and seeds follow BASELINE.json's configs list:
  configs[0]  symmetric int4 g=32, M=1, K=2048, N=8192
  configs[1]  asymmetric int4 g=128 (fp16 scales, uint4 zero points), up K=2048 N=8192 and down K=8192 N=2048, M=1, 4
  configs[2]  prefill, asymmetric int4 g=128, K=2048, N=8192, M=2048 and M=512
  configs[3]  fused QKV N=2560 int4 g=32, gate/up N=16384 int4 g=128 asym + GELU-tanh, down K=8192 N=2048, M=1, 2048
  configs[4]  2-bit g=32 calibrated, 4-bit g=128 asym, 8-bit g=32 sym (K=2048, N=8192, M=1); int8 g=32 head
              N=262,144 at M=1 and M=8 with greedy selection
"""

import os

import numpy as np
import pytest

from tests.cases import activations, expected_partials, weights

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
TOL = 2e-3
THREADS = max(1, min(16, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    _native.load()
    return torch.device("cuda:0")


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def check_close(y, y_ref, tol=TOL):
    y = y.detach().cpu().numpy() if hasattr(y, "detach") else y
    scale = max(float(np.max(np.abs(y_ref))), 1e-30)
    err = float(np.max(np.abs(y - y_ref)))
    assert err <= tol * scale, f"max|dy| = {err:.3g} > {tol} * {scale:.3g}"


def sample(n, count, rng):
    """Sorted sample of indices 0..n-1 holding both ends and a contiguous run."""
    picks = {0, n - 1, *range(min(n, 48), min(n, 48 + 16))}
    picks.update(int(v) for v in rng.choice(n, size=min(n, count), replace=False))
    return np.array(sorted(picks))


def run_config(ref, dev, name, bits, group, M, K, N, zero_points, in_s, seed, route, outliers=0.001):
    """One configuration: returns (dw, x, xt, y_gpu, y_ref) after the route, dump-equality, output and partial
    checks."""
    from kidi_amd.ops import DeviceWeight

    print(f"config {name}: bits={bits} g={group} M={M} K={K} N={N} zp={zero_points} in_s={in_s} seed={seed}", flush=True)
    rng = np.random.default_rng(seed)
    values, scales, zp, codes = weights(rng, N, K, bits, group, zero_points=zero_points)
    x = activations(rng, M, K, outliers)
    dw = DeviceWeight(to_dev(values, dev), to_dev(scales, dev), bits, group, to_dev(zp, dev) if zp is not None else None)
    xt = to_dev(x, dev).to(torch.bfloat16)
    assert dw.route(xt, in_s) == route
    y = dw.linear(xt, in_s)
    y_d, P_d = dw.debug_partials(xt, in_s)
    torch.cuda.synchronize()
    y_np = y.cpu().numpy()
    np.testing.assert_array_equal(y_np, y_d.cpu().numpy())  # production instance == dump instance
    y_ref, path = ref.packed_linear(x, values, scales, bits, group, in_s, zero_points=zp, threads=THREADS)
    assert path == (ref.PATH_BLOCKWISE if in_s == 0 else ref.PATH_SYMMETRIC)
    check_close(y_np, y_ref)
    rows = sample(M, 6, rng)
    cols = sample(N, 64, rng)
    P = P_d[torch.from_numpy(rows).to(dev)][:, torch.from_numpy(cols).to(dev)].cpu().numpy().astype(np.int64)
    del P_d
    if in_s == 0:
        q, _, _, zpa = ref.quantize_dynamic(x[rows], group, bits)
    else:
        (q, _), zpa = ref.quantize_static(x[rows], group, in_s), None
    P_ref = expected_partials(ref, q, codes[cols], zpa, bits, group,
                              zero_points=zp[cols] if zp is not None else None, dynamic=in_s == 0)
    np.testing.assert_array_equal(P, P_ref)
    return dw, x, xt, y, y_ref


def test_config0_symmetric_g32_decode(dev, ref):
    run_config(ref, dev, "configs[0]", 4, 32, 1, 2048, 8192, False, 0.0, 100, "decode_kernel", outliers=0.0)


@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("K,N", [(2048, 8192), (8192, 2048)])
def test_config1_asymmetric_g128_decode(dev, ref, M, K, N):
    run_config(ref, dev, f"configs[1] K={K} N={N}", 4, 128, M, K, N, True, 0.0, 110 + M + K // 1024, "decode_kernel")


@pytest.mark.parametrize("M", [512, 2048])
def test_config2_prefill(dev, ref, M):
    run_config(ref, dev, f"configs[2] M={M}", 4, 128, M, 2048, 8192, True, 0.0, 120 + M, "gemm8_kernel", outliers=0.0)


@pytest.mark.parametrize("M", [1, 2048])
def test_config3_fused_qkv(dev, ref, M):
    run_config(ref, dev, f"configs[3] QKV M={M}", 4, 32, M, 2048, 2048 + 256 + 256, False, 0.0, 130 + M,
               "decode_kernel" if M == 1 else "gemm8w_kernel")


@pytest.mark.parametrize("M", [1, 2048])
def test_config3_gate_up_gelu(dev, ref, M):
    """The gate/up projection (N = 2 x 8192) through every check, then the GELU-gated form against the oracle's
    gelu_gate of the oracle's projection, and against the oracle's gelu_gate of the GPU's own projection."""
    dw, x, xt, y, y_ref = run_config(ref, dev, f"configs[3] gate/up M={M}", 4, 128, M, 2048, 2 * 8192, True, 0.0,
                                     140 + M, "decode_kernel" if M == 1 else "gemm8_kernel")
    assert dw.route(xt, 0.0, gelu_gate=True) == ("decode_kernel" if M == 1 else "gemm8_kernel")
    h = dw.linear(xt, gelu_gate=True)
    torch.cuda.synchronize()
    h_np = h.cpu().numpy()
    check_close(h_np, ref.gelu_gate(y_ref), tol=5e-3)
    check_close(h_np, ref.gelu_gate(y.cpu().numpy()), tol=1e-5)


@pytest.mark.parametrize("M", [1, 2048])
def test_config3_down(dev, ref, M):
    run_config(ref, dev, f"configs[3] down M={M}", 4, 128, M, 8192, 2048, True, 0.0, 150 + M,
               "decode_kernel" if M == 1 else "gemm8_kernel")


@pytest.mark.parametrize("name,bits,group,zp,in_s", [("int2_g32_calibrated", 2, 32, False, 0.03),
                                                      ("int4_g128_asym", 4, 128, True, 0.0),
                                                      ("int8_g32_sym", 8, 32, False, 0.0)])
def test_config4_mixed(dev, ref, name, bits, group, zp, in_s):
    run_config(ref, dev, f"configs[4] {name}", bits, group, 1, 2048, 8192, zp, in_s, 160 + bits, "decode_kernel")


@pytest.mark.parametrize("M", [1, 8])
def test_config4_head_greedy(dev, ref, M):
    """int8 g=32 head, N = 262,144: the projection through every check, then greedy selection fused into the head
    (logits kept on chip) picks the oracle's greedy token of the GPU's logits, and that token's oracle logit is the
    oracle's maximum within tolerance."""
    dw, x, xt, y, y_ref = run_config(ref, dev, f"configs[4] head M={M}", 8, 32, M, 2048, 262144, False, 0.0, 170 + M,
                                     "decode_kernel")
    tokens, logits = dw.linear_greedy(xt)
    torch.cuda.synchronize()
    assert logits is None
    tok = tokens.cpu().numpy()
    np.testing.assert_array_equal(tok, ref.greedy_token(y.cpu().numpy()))
    scale = float(np.max(np.abs(y_ref)))
    for r in range(M):
        assert y_ref[r, tok[r]] >= y_ref[r].max() - TOL * scale


@pytest.mark.parametrize("M", [512, 2048])
def test_config2_published_f16_zero(dev, ref, M):
    """configs[2] shape in the published package format (benchmarks/gemma4/arm/run.py:151, :694-695): F16
    weight_scale and F16 weight_zero = round_f16((8 - zp) * scale), an additive float zero that is not exactly
    (8 - zp) * scale. It reaches the MFMA prefill GEMM (float-zero variant); the projection is within 2e-3 of the oracle
    and the int32 partials sum q * c with the signed codes c = u - 8."""
    from kidi_amd.ops import DeviceWeight

    K, N = 2048, 8192
    rng = np.random.default_rng(180 + M)
    values, scales, zp, codes = weights(rng, N, K, 4, 128, zero_points=True)
    zf = ((8.0 - zp.astype(np.float32)) * scales.astype(np.float32)).astype(np.float16)
    assert np.any(zf.astype(np.float32) != (8.0 - zp.astype(np.float32)) * scales.astype(np.float32))
    x = activations(rng, M, K, 0.001)
    dw = DeviceWeight(to_dev(values, dev), to_dev(scales, dev), 4, 128, to_dev(zf, dev))
    xt = to_dev(x, dev).to(torch.bfloat16)
    assert dw.route(xt) == "gemm8_kernel"
    y = dw.linear(xt)
    y_d, P_d = dw.debug_partials(xt)
    torch.cuda.synchronize()
    y_np = y.cpu().numpy()
    np.testing.assert_array_equal(y_np, y_d.cpu().numpy())
    y_ref, path = ref.packed_linear(x, values, scales, 4, 128, zeros=zf, threads=THREADS)
    assert path == ref.PATH_BLOCKWISE
    check_close(y_np, y_ref)
    rows, cols = sample(M, 6, rng), sample(N, 64, rng)
    P = P_d[torch.from_numpy(rows).to(dev)][:, torch.from_numpy(cols).to(dev)].cpu().numpy().astype(np.int64)
    q, _, _, zpa = ref.quantize_dynamic(x[rows], 128, 4)
    np.testing.assert_array_equal(P, expected_partials(ref, q, codes[cols], zpa, 4, 128))
