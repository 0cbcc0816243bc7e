"""RMS normalization (Context::rms_norm / rms_norm_residual, ops/context.cpp:1043-1049, :1103-1122; RmsNorm,
runtime/ynn/operators.cpp:553-620) and its fusion into the projection's activation quantization (the norm that
precedes each projection group of the decoder layer, layers/gemma4.cpp:405-413).

CPU: the oracle against the reference's KAT (tests/kidi/layers/eager_test.cpp:388-412), the fused-residual identity
(tests/kidi/runtime/cuda/operators_test.cpp:346-350), a float64 closed form, power-of-two weight scaling and an
independent numpy restatement of the fixed summation order. GPU: kq_rms_norm bit-exact against the oracle;
kq_packed_linear_rms bit-equal to kq_rms_norm followed by kq_packed_linear (decode, prefill and fallback paths),
its hidden output bit-exact, and y within 2e-3 * max|y_ref| of the oracle's composition."""

import numpy as np
import pytest

from tests.cases import activations, weights

torch = pytest.importorskip("torch")

KAT_X = np.array([[1, 2, 3, 4], [0, 0, 0, 0]], np.float32)
KAT_W = np.array([1, -2, 0.5, 3], np.float32)


def canonical_sum_squares(row: np.ndarray) -> np.float32:
    """The fixed order, vectorized: 8-column pieces in column order, a pairwise tree over a segment's 64 pieces,
    segments in order (all in float32)."""
    width = row.shape[0]
    segs = -(-width // 512)
    padded = np.zeros(segs * 512, np.float32)
    padded[:width] = row
    sq = (padded * padded).reshape(segs, 64, 8)
    piece = sq[:, :, 0].copy()
    for i in range(1, 8):
        piece = (piece + sq[:, :, i]).astype(np.float32)
    while piece.shape[1] > 1:
        piece = (piece[:, 0::2] + piece[:, 1::2]).astype(np.float32)
    total = np.float32(piece[0, 0])
    for s in range(1, segs):
        total = np.float32(total + piece[s, 0])
    return total


def test_oracle_rms_kat(ref):
    """eager_test.cpp:388-412: plain, doubled weight, residual, residual scaled by 0.5; zero row exactly 0."""
    expected = KAT_X[0] * KAT_W / np.sqrt(np.float32(7.5) + np.float32(1e-6))
    y, _ = ref.rms_norm(KAT_X, KAT_W, 1e-6)
    assert np.max(np.abs(y[0] - expected)) <= 1e-5
    assert np.all(y[1] == 0)
    y2, _ = ref.rms_norm(KAT_X, 2 * KAT_W, 1e-6)
    assert np.max(np.abs(y2[0] - 2 * expected)) <= 1e-5
    np.testing.assert_array_equal(y2, 2 * y)  # power-of-two weight scaling is exact
    yr, _ = ref.rms_norm(KAT_X, KAT_W, 1e-6, residual=KAT_X)
    assert np.max(np.abs(yr[0] - (KAT_X[0] + expected))) <= 1e-5
    ys, _ = ref.rms_norm(KAT_X, KAT_W, 1e-6, residual=KAT_X, scale=0.5)
    assert np.max(np.abs(ys[0] - 0.5 * (KAT_X[0] + expected))) <= 1e-5


def test_oracle_rms_invalid(ref):
    with pytest.raises(ValueError):
        ref.rms_norm(KAT_X, KAT_W, 0.0)  # eager_test.cpp:413-419: epsilon 0 is INVALID_ARGUMENT
    with pytest.raises(ValueError):
        ref.rms_norm(KAT_X, KAT_W, float("nan"))


@pytest.mark.parametrize("scaled", [False, True])
def test_oracle_rms_residual_identity(ref, scaled):
    """cuda/operators_test.cpp:346-350: rms_norm_residual(x, w, r, eps[, s]) == (rms_norm(x, w, eps) + r)[* s]
    exactly, here on bf16 [2, 3, 4, 64] operands with the scalar 0.78125."""
    rng = np.random.default_rng(3)
    x = ref.f32_to_bf16_bits(rng.standard_normal((2, 3, 4, 64)).astype(np.float32))
    r = ref.f32_to_bf16_bits(rng.standard_normal((2, 3, 4, 64)).astype(np.float32))
    w = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    s = 0.78125 if scaled else None
    fused, _ = ref.rms_norm(x, w, 1e-6, residual=r, scale=s, x_bf16=True)
    plain, _ = ref.rms_norm(x, w, 1e-6, x_bf16=True)
    added = plain + ref.bf16_bits_to_f32(r).reshape(plain.shape)
    np.testing.assert_array_equal(fused, added * np.float32(s) if scaled else added)


@pytest.mark.parametrize("width", [1, 7, 512, 1000, 2048, 8192])
def test_oracle_rms_closed_form(ref, width):
    rng = np.random.default_rng(width)
    x = (rng.standard_normal((3, width)) * np.array([[1.0], [1e-3], [50.0]])).astype(np.float32)
    w = rng.uniform(-2, 2, width).astype(np.float32)
    y, inv = ref.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    inv64 = 1.0 / np.sqrt((x64 * x64).mean(axis=1) + 1e-6)
    np.testing.assert_allclose(inv, inv64, rtol=4e-7 * max(1.0, np.log2(width)), atol=0)
    y64 = x64 * inv64[:, None] * w.astype(np.float64)[None]
    assert np.max(np.abs(y - y64)) <= 1e-6 * np.max(np.abs(y64))
    for r in range(3):  # the documented summation order, restated independently
        expect = np.float32(1) / np.sqrt(np.float32(canonical_sum_squares(x[r]) / np.float32(width)) + np.float32(1e-6))
        assert inv[r] == np.float32(expect)


def test_context_rms_validation():
    """Context::rms_norm_residual's operand checks (ops/context.cpp:1106-1112) raise INVALID_ARGUMENT before any
    device work."""
    from kidi_amd.ops import Context, Failure

    ctx = Context("cuda")
    x = torch.ones((2, 4))
    w = torch.ones(4)
    for bad in (lambda: ctx.rms_norm(x, w, 0.0), lambda: ctx.rms_norm(x, torch.ones(3), 1e-6),
                lambda: ctx.rms_norm(x, w.double(), 1e-6),
                lambda: ctx.rms_norm_residual(x, w, torch.ones((2, 5)), 1e-6),
                lambda: ctx.rms_norm_residual(x, w, x, 1e-6, torch.ones(2))):
        with pytest.raises(Failure) as e:
            bad()
        assert e.value.code == "INVALID_ARGUMENT"


# ---------------------------------------------------------------- GPU ------------------------------------------------


def _dev():
    return torch.device("cuda:0")


@pytest.mark.gpu
def test_gpu_rms_kat():
    from kidi_amd.ops import Context

    ctx = Context("cuda")
    x = torch.from_numpy(KAT_X).cuda()
    w = torch.from_numpy(KAT_W).cuda()
    expected = torch.from_numpy(KAT_X[0] * KAT_W / np.sqrt(np.float32(7.5) + np.float32(1e-6)))
    y = ctx.rms_norm(x, w, 1e-6).cpu()
    assert torch.max(torch.abs(y[0] - expected)) <= 1e-5 and torch.all(y[1] == 0)
    y2 = ctx.rms_norm(x, 2 * w, 1e-6).cpu()
    assert torch.equal(y2, 2 * y)
    yr = ctx.rms_norm_residual(x, w, x, 1e-6).cpu()
    assert torch.max(torch.abs(yr[0] - (x[0].cpu() + expected))) <= 1e-5
    ys = ctx.rms_norm_residual(x, w, x, 1e-6, torch.tensor([0.5], device="cuda")).cpu()
    assert torch.max(torch.abs(ys[0] - 0.5 * (x[0].cpu() + expected))) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("width", [4, 1000, 2048, 8192])
@pytest.mark.parametrize("rows", [1, 37])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("form", ["plain", "residual", "scaled"])
def test_gpu_rms_norm_exact(ref, width, rows, bf16, form):
    from kidi_amd.ops import rms_norm

    rng = np.random.default_rng(width * 7 + rows)
    x = activations(rng, rows, width, outliers=0.001)
    x[rows // 2] = 0.0  # an all-zero row
    r = activations(rng, rows, width)
    w = rng.uniform(-2, 2, width).astype(np.float32)
    res = None if form == "plain" else r
    s = 0.78125 if form == "scaled" else None
    if bf16:
        y_ref, _ = ref.rms_norm(ref.f32_to_bf16_bits(x), w, 1e-6, residual=None if res is None else ref.f32_to_bf16_bits(r),
                                scale=s, x_bf16=True)
    else:
        y_ref, _ = ref.rms_norm(x, w, 1e-6, residual=res, scale=s)
    dt = torch.bfloat16 if bf16 else torch.float32
    xt = torch.from_numpy(x).to(_dev()).to(dt)
    rt = torch.from_numpy(r).to(_dev()).to(dt) if res is not None else None
    st = torch.tensor([s], dtype=torch.float32, device=_dev()) if s is not None else None
    y = rms_norm(xt, torch.from_numpy(w).to(_dev()), 1e-6, residual=rt, output_scale=st)
    np.testing.assert_array_equal(y.cpu().numpy(), y_ref)


# shapes of the fused projection: (name, bits, g, K, N, M, zero points, calibrated input scale, gelu)
FUSED = [
    ("decode-up-M1", 4, 128, 2048, 8192, 1, True, 0.0, False),
    ("decode-up-M4", 4, 128, 2048, 2048, 4, True, 0.0, False),
    ("decode-up-M8", 4, 128, 2048, 1024, 8, True, 0.0, False),
    ("decode-qkv-g32", 4, 32, 2048, 2560, 1, False, 0.0, False),
    ("decode-int8", 8, 32, 2048, 1024, 2, False, 0.0, False),
    ("decode-calibrated", 4, 128, 1024, 512, 3, False, 0.0625, False),
    ("decode-gelu", 4, 128, 2048, 2 * 1024, 1, True, 0.0, True),
    ("prefill", 4, 128, 2048, 1024, 300, True, 0.0, False),
    ("prefill-gelu", 4, 128, 1024, 2 * 512, 64, True, 0.0, True),
    ("fallback-K8192", 4, 128, 8192, 256, 2, True, 0.0, False),
    ("fallback-skinny-g64", 4, 64, 1536, 256, 12, False, 0.0, False),
    ("fallback-generic", 8, 32, 512, 384, 40, False, 0.0, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", FUSED, ids=[c[0] for c in FUSED])
@pytest.mark.parametrize("residual", [False, True])
def test_gpu_linear_rms(ref, case, residual):
    from kidi_amd.ops import DeviceWeight, rms_norm

    name, bits, g, K, N, M, zp, in_s, gelu = case
    rng = np.random.default_rng(len(name) * 31 + M)
    values, scales, zpa, _ = weights(rng, N, K, bits, g, zero_points=zp)
    x = activations(rng, M, K, outliers=0.001)
    r = activations(rng, M, K)
    w_in = rng.uniform(0.5, 1.5, K).astype(np.float32)
    w_res = rng.uniform(-1.5, 1.5, K).astype(np.float32)
    dev = _dev()
    dw = DeviceWeight(torch.from_numpy(values).to(dev), torch.from_numpy(scales).to(dev), bits, g,
                      torch.from_numpy(zpa).to(dev) if zp else None)
    xt = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    rt = torch.from_numpy(r).to(dev).to(torch.bfloat16)
    wt, wrt = torch.from_numpy(w_in).to(dev), torch.from_numpy(w_res).to(dev)
    st = torch.tensor([0.78125], device=dev)
    print(f"case {name} residual={residual}", flush=True)
    if residual:
        y, hidden = dw.linear_rms(xt, wt, 1e-6, residual=rt, residual_weight=wrt, residual_scale=st,
                                  residual_epsilon=1e-5, input_scale=in_s, gelu_gate=gelu)
        h_c = rms_norm(xt, wrt, 1e-5, residual=rt, output_scale=st)
        n_c = rms_norm(h_c, wt, 1e-6)
    else:
        y, hidden = dw.linear_rms(xt, wt, 1e-6, input_scale=in_s, gelu_gate=gelu)
        n_c = rms_norm(xt, wt, 1e-6)
    y_c = dw.linear(n_c, input_scale=in_s, gelu_gate=gelu)
    torch.cuda.synchronize()
    # fused == kq_rms_norm then kq_packed_linear, bit for bit
    np.testing.assert_array_equal(y.cpu().numpy(), y_c.cpu().numpy())
    # oracle: the normalization, then the projection of its F32 output
    xb = ref.f32_to_bf16_bits(x)
    if residual:
        h_ref, _ = ref.rms_norm(xb, w_res, 1e-5, residual=ref.f32_to_bf16_bits(r), scale=0.78125, x_bf16=True)
        np.testing.assert_array_equal(hidden.cpu().numpy(), h_ref)
        n_ref, _ = ref.rms_norm(h_ref, w_in, 1e-6)
    else:
        assert hidden is None
        n_ref, _ = ref.rms_norm(xb, w_in, 1e-6, x_bf16=True)
    np.testing.assert_array_equal(n_c.cpu().numpy(), n_ref)
    y_ref, _ = ref.packed_linear(n_ref, values, scales, bits, g, in_s, zero_points=zpa, threads=8)
    if gelu:
        y_ref = ref.gelu_gate(y_ref)
    err = float(np.max(np.abs(y.cpu().numpy() - y_ref)))
    assert err <= 2e-3 * float(np.max(np.abs(y_ref))), (name, err)


# ---------------------------------------------------------------- golden fixtures -------------------------------------

RMS_FIXTURES = ["rms_residual_decode", "rms_plain_prefill"]


def _fixture(name):
    import os

    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name + ".npz")
    with np.load(path, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", RMS_FIXTURES)
def test_oracle_reproduces_rms_fixture(ref, name):
    f = _fixture(name)
    src = f["x"]
    if "hidden" in f:
        h, _ = ref.rms_norm(f["x"], f["w_res"], float(f["eps_res"]), residual=f["residual"], scale=float(f["res_scale"]))
        np.testing.assert_array_equal(h, f["hidden"])
        src = h
    n, inv = ref.rms_norm(src, f["w_in"], float(f["eps"]))
    np.testing.assert_array_equal(n, f["normed"])
    np.testing.assert_array_equal(inv, f["inv"])
    y, path = ref.packed_linear(n, f["values"], f["scales"], int(f["bits"]), int(f["group"]), zero_points=f.get("zero_points"))
    assert path == int(f["path"])
    np.testing.assert_array_equal(y, f["y"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", RMS_FIXTURES)
def test_gpu_rms_fixture(name):
    """The fused projection reproduces the fixture: h and the normalized input bit-exact (kq_rms_norm), y within
    2e-3 * max|y| (kq_packed_linear_rms)."""
    from kidi_amd.ops import DeviceWeight, rms_norm

    f = _fixture(name)
    dev = _dev()
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    zp = f.get("zero_points")
    dw = DeviceWeight(t(f["values"]), t(f["scales"]), int(f["bits"]), int(f["group"]), t(zp) if zp is not None else None)
    x = t(f["x"]).to(torch.bfloat16)
    if "hidden" in f:
        r = t(f["residual"]).to(torch.bfloat16)
        st = torch.tensor([float(f["res_scale"])], device=dev)
        y, h = dw.linear_rms(x, t(f["w_in"]), float(f["eps"]), residual=r, residual_weight=t(f["w_res"]), residual_scale=st,
                             residual_epsilon=float(f["eps_res"]))
        np.testing.assert_array_equal(h.cpu().numpy(), f["hidden"])
        h2 = rms_norm(x, t(f["w_res"]), float(f["eps_res"]), residual=r, output_scale=st)
        n = rms_norm(h2, t(f["w_in"]), float(f["eps"]))
    else:
        y, _ = dw.linear_rms(x, t(f["w_in"]), float(f["eps"]))
        n = rms_norm(x, t(f["w_in"]), float(f["eps"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(n.cpu().numpy(), f["normed"])
    err = float(np.max(np.abs(y.cpu().numpy() - f["y"])))
    assert err <= 2e-3 * float(np.max(np.abs(f["y"]))), err
