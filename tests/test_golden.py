"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture exactly, and each fixture agrees with a float64 restatement of the closed
form y = sum_b a_s * (w_s * P + z_w * Q) (runtime/ynn/operators.cpp:1118-1169 for the dynamic path,
eager_test.cpp:94-103 for the calibrated one) built from the fixture's own codes with numpy, so a dropped zero
term, a wrong sign or a transposed operand in the oracle fails here. GPU: the HIP path through the C ABI matches the
fixtures: activation codes, block statistics and integer partials bit-exact, y within 2e-3 * max|y|."""

import glob
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))
# projection fixtures (the rms_* ones hold a normalization before the projection: tests/test_rms_norm.py)
NAMES = [n for n in (os.path.splitext(os.path.basename(f))[0] for f in FIXTURES) if not n.startswith("rms_")]


def load(name):
    with np.load(os.path.join(HERE, "golden", name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def signed_codes(values, K, bits):
    """Kidi layout -> signed codes (element k in bits (k % (8/b)) * b of byte k / (8/b), eager_test.cpp:318-320)."""
    if bits == 8:
        return values.view(np.int8).astype(np.int64)
    per = 8 // bits
    mask = (1 << bits) - 1
    sign = 1 << (bits - 1)
    out = np.zeros((values.shape[0], K), np.int64)
    for i in range(per):
        raw = (values.astype(np.int64) >> (i * bits)) & mask
        out[:, i::per] = (raw ^ sign) - sign
    return out


def test_fixtures_present():
    assert len(NAMES) >= 14


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(ref, name):
    f = load(name)
    bits, group = int(f["bits"]), int(f["group"])
    in_s, out_s = float(f["input_scale"]), float(f["output_scale"])
    y, path = ref.packed_linear(f["x"], f["values"], f["scales"], bits, group, in_s, out_s,
                                zeros=f.get("zeros"), zero_points=f.get("zero_points"))
    assert path == int(f["path"])
    np.testing.assert_array_equal(y, f["y"])
    if in_s == 0:
        q, s, Q, zpa = ref.quantize_dynamic(f["x"], group, bits)
        np.testing.assert_array_equal(s, f["act_scale"])
        np.testing.assert_array_equal(zpa, f["act_zero"]) if "act_zero" in f else None
    else:
        q, Q = ref.quantize_static(f["x"], group, in_s)
    np.testing.assert_array_equal(q, f["q"])
    np.testing.assert_array_equal(Q, f["act_sum"])
    if "h" in f:
        np.testing.assert_array_equal(ref.gelu_gate(f["y"]), f["h"])


@pytest.mark.parametrize("name", NAMES)
def test_fixture_closed_form(name):
    """float64 restatement from the fixture's codes and activation codes (no oracle call)."""
    f = load(name)
    bits, group = int(f["bits"]), int(f["group"])
    in_s, out_s = float(f["input_scale"]), float(f["output_scale"])
    x, q = f["x"].astype(np.float64), f["q"].astype(np.int64)
    M, K = x.shape
    B = K // group
    c = signed_codes(f["values"], K, bits)
    N = c.shape[0]
    ws = f["scales"].astype(np.float64)
    # integer partials P = sum q*c per group, Q = sum q: recomputed here and against the fixture's P'
    P = np.einsum("mbk,nbk->mnb", q.reshape(M, B, group), c.reshape(N, B, group))
    Q = q.reshape(M, B, group).sum(axis=2)
    np.testing.assert_array_equal(Q, f["act_sum"])
    Pk = P.copy()
    if "zero_points" in f:
        Pk = Pk + (8 - f["zero_points"].astype(np.int64))[None] * Q[:, None, :]
    if bits == 8 and in_s == 0:
        Pk = Pk - f["act_zero"].astype(np.int64)[:, None, :] * c.reshape(N, B, group).sum(axis=2)[None]
    np.testing.assert_array_equal(Pk, f["P"].astype(np.int64))
    # quantizer: the codes reconstruct x to half a step
    if in_s == 0 and bits != 8:
        a_s = np.repeat(f["act_scale"].astype(np.float64), group, axis=1)
        assert np.all(np.abs(a_s * q - x) <= (0.5 + 1e-4) * a_s + 1e-30)  # x*(127/max) vs x/(max/127)
        assert np.all(np.abs(q) <= 127)
    elif in_s > 0:
        # q = clamp(nearbyint(x / in_s), -128, 127) with the division in fp32 (eager_test.cpp:97-98)
        expect = np.clip(np.rint(f["x"].astype(np.float32) / np.float32(in_s)), -128, 127)
        np.testing.assert_array_equal(expect, q)
    # y
    if in_s > 0:
        y = in_s * np.einsum("nb,mnb->mn", ws, P)
        if out_s > 0:
            y = np.clip(np.rint(y / out_s), -128, 127) * out_s
            assert np.mean(np.abs(y - f["y"]) > 1e-6) <= 0.01  # rounding-boundary ties only
            assert np.max(np.abs(y - f["y"])) <= out_s * (1 + 1e-6)
            return
    else:
        a_s = f["act_scale"].astype(np.float64)
        if bits == 8:
            zc = P - f["act_zero"].astype(np.int64)[:, None, :] * c.reshape(N, B, group).sum(axis=2)[None]
            y = np.einsum("mb,nb,mnb->mn", a_s, ws, zc)
        else:
            if "zero_points" in f:
                z = (8 - f["zero_points"].astype(np.float64)) * ws
            elif "zeros" in f:
                z = f["zeros"].astype(np.float64)
            else:
                z = np.zeros_like(ws)
            y = np.einsum("mb,nb,mnb->mn", a_s, ws, P) + np.einsum("mb,nb,mb->mn", a_s, z, Q)
    scale = max(np.max(np.abs(y)), 1e-30)
    assert np.max(np.abs(y - f["y"])) <= 1e-5 * scale
    if "h" in f:
        I = y.shape[1] // 2
        g, up = y[:, :I], y[:, I:]
        h = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3))) * up
        assert np.max(np.abs(h - f["h"])) <= 1e-5 * max(np.max(np.abs(h)), 1e-30)


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_hip_matches_fixture(name):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native
    from kidi_amd.ops import DeviceWeight

    _native.load()
    print(f"golden {name}", flush=True)
    dev = torch.device("cuda:0")
    f = load(name)
    bits, group = int(f["bits"]), int(f["group"])
    in_s, out_s = float(f["input_scale"]), float(f["output_scale"])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    z = f.get("zeros", f.get("zero_points"))
    dw = DeviceWeight(t(f["values"]), t(f["scales"]), bits, group, t(z) if z is not None else None)
    x = t(f["x"])
    if bool(f["x_bf16"]):
        x = x.to(torch.bfloat16)
    tol = 2e-3
    if bool(f["gelu"]):
        h = dw.linear(x, in_s, out_s, gelu_gate=True).cpu().numpy()
        assert np.max(np.abs(h - f["h"])) <= 5e-3 * np.max(np.abs(f["h"]))
    if int(f["path"]) == 2:  # portable path: no integer pipeline to compare
        y = dw.linear(x, in_s, out_s).cpu().numpy()
        assert np.max(np.abs(y - f["y"])) <= tol * np.max(np.abs(f["y"]))
        return
    codes, s, Q, zpa = dw.debug_quantize(x, in_s)
    np.testing.assert_array_equal(codes.cpu().numpy(), f["q"])
    np.testing.assert_array_equal(Q.cpu().numpy(), f["act_sum"])
    if in_s == 0:
        np.testing.assert_array_equal(s.cpu().numpy(), f["act_scale"])
        if "act_zero" in f:
            np.testing.assert_array_equal(zpa.cpu().numpy(), f["act_zero"])
    y_d, P = dw.debug_partials(x, in_s, out_s)
    np.testing.assert_array_equal(P.cpu().numpy(), f["P"])
    y = dw.linear(x, in_s, out_s).cpu().numpy()
    np.testing.assert_array_equal(y, y_d.cpu().numpy())
    if out_s > 0:  # calibrated outputs: steps of out_s, exact but for rounding-boundary ties
        assert np.mean(np.abs(y - f["y"]) > 0) <= 0.01 and np.max(np.abs(y - f["y"])) <= out_s * (1 + 1e-6)
    else:
        assert np.max(np.abs(y - f["y"])) <= tol * np.max(np.abs(f["y"]))
