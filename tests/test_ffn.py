"""Gated feed-forward (Context::gated_feed_forward, ops/context.cpp:970-996; PackedFeedForward,
runtime/ynn/operators.cpp:1321-1517): gate/up projection, GELU-tanh or SiLU gating, down projection of h.

Cases: the reference's own fused-versus-composed check (tests/kidi/runtime/ynn/graph_test.cpp:115-157: K = 128,
I = 2056, per-channel scales, bits 2/4/8, M = 1 and 17, scales 0.125 / 0.0625 / 0.03125 / 0.125, GELU and SiLU,
deterministic inputs) and the BASELINE decoder-layer shapes (gate/up N = 2 x 8192, down K = 8192, g = 128, dynamic).

CPU: the oracle's composition agrees with a float64 restatement built from the closed forms (exact calibrated gate/up
projection, float64 gating, down projection from h's codes). GPU: kq_gated_feed_forward through the C ABI against the
oracle (within 2e-3 * max|y_ref|) and against the library's own composed calls (bit-equal, the reference's
fused == composed check)."""

import numpy as np
import pytest

from tests.cases import activations, pack_codes, weights

torch = pytest.importorskip("torch")

INPUT, INTER = 128, 2056
SCALES = (0.125, 0.0625, 0.03125, 0.125)  # gate_up in, gate_up out, down in, down out (graph_test.cpp:123-127)


def graph_case(bits: int, M: int):
    """graph_test.cpp:119-134 inputs: x, gate_up bytes, down bytes and the per-channel scales of :76-79."""
    per = 8 // bits
    x = np.array([((i * 5) % 19 - 9) * 0.0625 for i in range(M * INPUT)], np.float32).reshape(M, INPUT)
    gu = np.array([(i * 11 + 7) & 0xFF for i in range(2 * INTER * (INPUT // per))], np.uint8).reshape(2 * INTER, -1)
    dn = np.array([(i * 17 + 3) & 0xFF for i in range(INPUT * (INTER // per))], np.uint8).reshape(INPUT, -1)
    gus = (0.00390625 * (1 + np.arange(2 * INTER) % 5)).astype(np.float32).reshape(-1, 1)
    dns = (0.00390625 * (1 + np.arange(INPUT) % 7)).astype(np.float32).reshape(-1, 1)
    return x, gu, gus, dn, dns


def signed_codes(values: np.ndarray, K: int, bits: int) -> np.ndarray:
    if bits == 8:
        return values.view(np.int8).astype(np.int64)
    per, mask, sign = 8 // bits, (1 << bits) - 1, 1 << (bits - 1)
    out = np.zeros((values.shape[0], K), np.int64)
    for i in range(per):
        raw = (values.astype(np.int64) >> (i * bits)) & mask
        out[:, i::per] = (raw ^ sign) - sign
    return out


def calibrated_linear64(x, values, scales, bits, in_s, out_s):
    """Per-channel calibrated projection in exact arithmetic: q = clamp(rint(x / in_s)) (fp32 division),
    y = in_s * s * sum q c, then clamp(rint(y / out_s)) * out_s (eager_test.cpp:94-103)."""
    K = x.shape[1]
    q = np.clip(np.rint(x.astype(np.float32) / np.float32(in_s)), -128, 127).astype(np.int64)
    c = signed_codes(values, K, bits)
    y = (q @ c.T).astype(np.float64) * scales.astype(np.float64).reshape(1, -1) * in_s
    if out_s > 0:
        y = np.clip(np.rint(y / out_s), -128, 127) * out_s
    return y


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("M", [1, 17])
@pytest.mark.parametrize("silu", [False, True])
def test_oracle_ffn_closed_form(ref, bits, M, silu):
    x, gu, gus, dn, dns = graph_case(bits, M)
    y, h = ref.gated_feed_forward(x, gu, gus, dn, dns, bits, INPUT, INTER, *SCALES, silu=silu)
    gate_up = calibrated_linear64(x, gu, gus, bits, SCALES[0], SCALES[1])
    gate_up_o, _ = ref.packed_linear(x, gu, gus, bits, INPUT, SCALES[0], SCALES[1])
    np.testing.assert_array_equal(gate_up_o, gate_up.astype(np.float32))  # power-of-two scales: exact
    g, up = gate_up[:, :INTER], gate_up[:, INTER:]
    act = g / (1 + np.exp(-g)) if silu else 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3)))
    h64 = act * up
    assert np.max(np.abs(h - h64)) <= 1e-5 * max(np.max(np.abs(h64)), 1.0)
    y64 = calibrated_linear64(h, dn, dns, bits, SCALES[2], SCALES[3])  # from the oracle's own h: exact codes
    np.testing.assert_allclose(y, y64.astype(np.float32), rtol=0, atol=1e-6 * max(np.max(np.abs(y64)), 1.0))


def test_oracle_silu_formula(ref):
    g = np.linspace(-30, 30, 601, dtype=np.float32)
    up = np.cos(np.arange(601, dtype=np.float32))
    h = ref.silu_gate(np.concatenate([g, up])[None])[0]
    expect = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * up
    assert np.max(np.abs(h - expect)) <= 1e-5  # eager_test.cpp:176-181


def test_context_rejects_mismatched_shapes():
    pytest.importorskip("kidi_amd._native")
    try:
        from kidi_amd.ops import Context, Failure
    except ImportError as e:  # library not built
        pytest.skip(str(e))
    x, gu, gus, dn, dns = graph_case(4, 1)
    ctx = Context("cpu")
    t = torch.from_numpy
    with pytest.raises(Failure) as e:  # down has the wrong row count
        ctx.gated_feed_forward(t(x), t(gu), t(gus), t(dn[:-1]), t(dns[:-1]), 4, INPUT, INTER, *SCALES)
    assert e.value.code == "INVALID_ARGUMENT"
    with pytest.raises(Failure) as e:  # negative scale
        ctx.gated_feed_forward(t(x), t(gu), t(gus), t(dn), t(dns), 4, INPUT, INTER, 0.125, -1.0, 0.03125, 0.125)
    assert e.value.code == "INVALID_ARGUMENT"


# ---- GPU --------------------------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    _native.load()
    return torch.device("cuda:0")


def _dw(values, scales, bits, group, dev, zero_points=None):
    from kidi_amd.ops import DeviceWeight

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return DeviceWeight(t(values), t(scales), bits, group, t(zero_points) if zero_points is not None else None)


def _close(y, y_ref, tol=2e-3):
    scale = max(float(np.max(np.abs(y_ref))), 1e-30)
    err = float(np.max(np.abs(y - y_ref)))
    assert err <= tol * scale, f"max|dy| = {err:.3g} > {tol} * {scale:.3g}"


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("M", [1, 17])
@pytest.mark.parametrize("silu", [False, True])
def test_ffn_graph_cases_gpu(dev, ref, bits, M, silu):
    from kidi_amd.ops import gated_feed_forward

    print(f"ffn graph case bits={bits} M={M} silu={silu}", flush=True)
    x, gu, gus, dn, dns = graph_case(bits, M)
    y_ref, _ = ref.gated_feed_forward(x, gu, gus, dn, dns, bits, INPUT, INTER, *SCALES, silu=silu)
    gw, dw = _dw(gu, gus, bits, INPUT, dev), _dw(dn, dns, bits, INTER, dev)
    xt = torch.from_numpy(x).to(dev)
    y = gated_feed_forward(gw, dw, xt, *SCALES, silu=silu)
    _close(y.cpu().numpy(), y_ref)
    # fused == composed (graph_test.cpp:137-154): the library's own projection + gating + projection calls
    gate_up = gw.linear(xt, SCALES[0], SCALES[1])
    g, up = gate_up[:, :INTER], gate_up[:, INTER:]
    h = g / (1 + torch.exp(-g)) * up if silu else gw.linear(xt, SCALES[0], SCALES[1], gelu_gate=True)
    composed = dw.linear(h.contiguous(), SCALES[2], SCALES[3])
    if silu:  # torch's exp is not the kernel's: h may differ by an ulp, so compare to the bar above
        _close(y.cpu().numpy(), composed.cpu().numpy())
    else:
        assert torch.equal(y, composed)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 20])
def test_ffn_baseline_shapes_gpu(dev, ref, M):
    """gate/up N = 2 x 8192, K = 2048 and down K = 8192, N = 2048, asymmetric int4 g = 128,
    bf16 activations, dynamic quantization of x and h."""
    from kidi_amd.ops import gated_feed_forward

    print(f"ffn baseline M={M}", flush=True)
    rng = np.random.default_rng(40 + M)
    I, K = 8192, 2048
    guv, gus, guz, _ = weights(rng, 2 * I, K, 4, 128, zero_points=True)
    dnv, dns, dnz, _ = weights(rng, K, I, 4, 128, zero_points=True)
    x = activations(rng, M, K, outliers=0.001)
    y_ref, _ = ref.gated_feed_forward(x, guv, gus, dnv, dns, 4, 128, 128, 0.0, 0.0, 0.0, 0.0,
                                      gate_up_zero_points=guz, down_zero_points=dnz, threads=8)
    gw, dw = _dw(guv, gus, 4, 128, dev, guz), _dw(dnv, dns, 4, 128, dev, dnz)
    y = gated_feed_forward(gw, dw, torch.from_numpy(x).to(dev).to(torch.bfloat16), 0.0, 0.0, 0.0, 0.0)
    _close(y.cpu().numpy(), y_ref)


@pytest.mark.gpu
def test_ffn_rejects_mismatched_weights_gpu(dev):
    from kidi_amd.ops import Failure, gated_feed_forward

    x, gu, gus, dn, dns = graph_case(4, 1)
    gw = _dw(gu, gus, 4, INPUT, dev)
    dw8 = _dw(pack_codes(np.zeros((INPUT, INTER), np.int64), 8), dns, 8, INTER, dev)  # 8-bit down, 4-bit gate/up
    with pytest.raises(Failure) as e:
        gated_feed_forward(gw, dw8, torch.from_numpy(x).to(dev), *SCALES)
    assert e.value.code == "INVALID_ARGUMENT"
    # m = 0 is a no-op
    y = gated_feed_forward(gw, _dw(dn, dns, 4, INTER, dev), torch.zeros((0, INPUT), device=dev), *SCALES)
    assert y.shape == (0, INPUT)
