"""Load-time weight quantization on the device (kq_quantize_weight, ops.pack_weight, Context.prepare_linear_weights)
against the oracle's ops::pack_weight (src/kidi/ops/quantization.cpp:12-133): codes, scales and zeros bit-exact.

The CPU tests cover the argument checks (no device call is made for invalid arguments); the GPU tests cover the
packer KATs of tests/arm_gemma_benchmark_test.py:83-101, seeded F32 / F16 / BF16 weights at 2, 4 and 8 bits,
symmetric and asymmetric, ties and zero groups, the non-finite and underflow errors, and the Context.linear
redirect (ops/context.cpp:742-773, :783-812)."""

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

f32 = np.float32


@pytest.fixture(scope="module")
def native():
    from kidi_amd import _native

    _native.load()
    return _native


@pytest.mark.parametrize("bad", ["bits", "group0", "ragged", "subbyte", "dtype", "rows", "null"])
def test_quantize_weight_rejects_invalid(native, bad):
    """quantization.cpp:15-20 checks, answered on the host before any device work."""
    lib = native.load()
    rows, cols, bits, group, dt = 4, 64, 4, 32, native.KQ_F32
    dummy = ctypes.c_void_p(16)
    w = v = s = dummy
    if bad == "bits":
        bits = 3
    elif bad == "group0":
        group = 0
    elif bad == "ragged":
        group = 24
    elif bad == "subbyte":
        bits, group = 2, 6  # a group must cover whole bytes
        cols = 66
    elif bad == "dtype":
        dt = native.KQ_U8
    elif bad == "rows":
        rows = 0
    elif bad == "null":
        w = None
    status = lib.kq_quantize_weight(w, dt, rows, cols, bits, group, 0, v, s, None, None)
    assert status == native.KQ_INVALID_ARGUMENT
    assert lib.kq_last_error()


def test_python_pack_weight_rejects_invalid():
    from kidi_amd.ops import Failure, pack_weight

    with pytest.raises(Failure) as e:
        pack_weight(torch.zeros((2, 6), dtype=torch.float32), 4, 4)
    assert e.value.code == "INVALID_ARGUMENT"
    with pytest.raises(Failure):
        pack_weight(torch.zeros((2, 8), dtype=torch.float64), 4, 4)
    with pytest.raises(Failure):
        pack_weight(torch.zeros((8,), dtype=torch.float32), 4, 4)


def test_context_linear_without_binding_is_unsupported():
    from kidi_amd.ops import Context, Failure

    ctx = Context("cpu")
    with pytest.raises(Failure) as e:
        ctx.linear(torch.zeros((1, 8)), torch.zeros((4, 8)))
    assert e.value.code == "UNSUPPORTED"
    with pytest.raises(Failure) as e:
        ctx.prepare_linear_weights(torch.zeros((4, 8)), 3, 4)
    assert e.value.code == "INVALID_ARGUMENT"


# ---------------------------------------------------------------------------------------------- GPU


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    _native.load()
    return torch.device("cuda:0")


def _device_pack(w_np, bits, group, asym, dev, dtype=torch.float32):
    from kidi_amd.ops import pack_weight

    if dtype == torch.bfloat16:
        t = torch.from_numpy(np.ascontiguousarray(w_np).view(np.int16)).view(torch.bfloat16).to(dev)
    else:
        t = torch.from_numpy(np.ascontiguousarray(w_np)).to(dev)
    p = pack_weight(t, bits, group, asym)
    return (p.values.cpu().numpy(), p.scales.cpu().numpy(), None if p.zeros is None else p.zeros.cpu().numpy())


def _assert_same(got, want):
    gv, gs, gz = got
    v, s, z = want
    np.testing.assert_array_equal(gv, v)
    np.testing.assert_array_equal(gs.view(np.uint32), s.view(np.uint32))
    if z is None:
        assert gz is None
    else:
        np.testing.assert_array_equal(gz.view(np.uint32), z.view(np.uint32))


@pytest.mark.gpu
def test_packer_kats_gpu(dev, ref):
    """arm_gemma_benchmark_test.py:83-101 on the device: ties away from zero, nibble order, grouped scales."""
    v, s, z = _device_pack(np.array([[-7, -1, 0, 1, 7, -3.5], [0, 0, 0, 0, 0, 0]], f32), 4, 6, False, dev)
    np.testing.assert_array_equal(s, [[1.0], [1.0]])
    assert z is None
    np.testing.assert_array_equal(ref.unpack_codes(v, 6, 4), [[-7, -1, 0, 1, 7, -4], [0] * 6])
    below_half = np.nextafter(f32(0.5), f32(0))
    v, _, _ = _device_pack(np.array([[below_half, 7.0]], f32), 4, 2, False, dev)
    np.testing.assert_array_equal(ref.unpack_codes(v, 2, 4), [[0, 7]])
    v, s, _ = _device_pack(np.array([[-7.0, 3.5, 14.0, -7.0]], f32), 4, 2, False, dev)
    np.testing.assert_array_equal(s, [[1.0, 2.0]])
    np.testing.assert_array_equal(ref.unpack_codes(v, 4, 4), [[-7, 4, 7, -4]])
    v, s, _ = _device_pack(np.array([[-127.0, 0.0, 63.5, 127.0]], f32), 8, 4, False, dev)
    np.testing.assert_array_equal(s, [[1.0]])
    np.testing.assert_array_equal(v.view(np.int8), [[-127, 0, 64, 127]])
    w = np.array([[-0.2, 0.0, 0.5, 1.0]], f32)
    _assert_same(_device_pack(w, 4, 2, True, dev), ref.pack_weight(w, 4, 2, asymmetric_clip=True))


def _seeded(rng, rows, cols, group):
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(f32)
    w[0, :group] = 0.0  # a zero group: scale 1
    if rows > 1:  # exact ties at multiples of scale / 2
        w[1, :group] = (np.arange(group) % 15 - 7).astype(f32) * f32(0.5)
    if rows > 2:
        w[2, :group] = 1e-38  # tiny but representable scale
    if rows > 3:
        w[3, : group // 2] = 3.0e4  # a large outlier group
    return w


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits,group,asym", [(2, 4, False), (2, 32, False), (4, 2, False), (4, 32, False),
                                             (4, 128, False), (4, 32, True), (4, 128, True), (8, 32, False),
                                             (8, 128, False)])
def test_pack_weight_matches_oracle(dev, ref, dtype, bits, group, asym):
    rng = np.random.default_rng(bits * 1000 + group + 7 * asym)
    rows, cols = 37, 512
    w = _seeded(rng, rows, cols, group)
    if dtype == torch.float16:
        w_in = w.astype(np.float16)
        want = ref.pack_weight(w_in, bits, group, asymmetric_clip=asym)
    elif dtype == torch.bfloat16:
        w_in = (w.view(np.uint32) >> 16).astype(np.uint16)  # truncated bf16 bit patterns
        want = ref.pack_weight(w_in, bits, group, asymmetric_clip=asym, bf16=True)
    else:
        w_in = w
        want = ref.pack_weight(w_in, bits, group, asymmetric_clip=asym)
    _assert_same(_device_pack(w_in, bits, group, asym, dev, dtype), want)


@pytest.mark.gpu
def test_pack_weight_large_matches_oracle(dev, ref):
    """A projection-sized weight (2048 x 2048, g = 128, asymmetric): every byte, scale and zero bit-exact."""
    rng = np.random.default_rng(77)
    w = (rng.standard_normal((2048, 2048)) * 0.02).astype(f32)
    _assert_same(_device_pack(w, 4, 128, True, dev), ref.pack_weight(w, 4, 128, asymmetric_clip=True))


@pytest.mark.gpu
@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
@pytest.mark.parametrize("asym", [False, True])
def test_pack_weight_rejects_non_finite_gpu(dev, bad, asym):
    from kidi_amd.ops import Failure, pack_weight

    w = torch.zeros((4, 64), dtype=torch.float32)
    w[3, 17] = bad
    with pytest.raises(Failure) as e:
        pack_weight(w.to(dev), 4, 32, asym)
    assert e.value.code == "INVALID_ARGUMENT" and "non-finite" in str(e.value)
    # the library stays usable: the next call succeeds and is exact
    ok = pack_weight(torch.ones((4, 64), device=dev), 4, 32, asym)
    torch.cuda.synchronize()
    assert ok.values.shape == (4, 32)


@pytest.mark.gpu
def test_pack_weight_scale_underflow_gpu(dev, ref):
    """A symmetric scale that rounds to zero (max|w| = the smallest subnormal, / 7) is INVALID_ARGUMENT, as the
    reference's 'quantization scale underflow'."""
    from kidi_amd.ops import Failure, pack_weight

    w = np.zeros((2, 8), f32)
    w[1, 3] = np.float32(1e-45)
    with pytest.raises(ValueError):
        ref.pack_weight(w, 4, 4)
    with pytest.raises(Failure) as e:
        pack_weight(torch.from_numpy(w).to(dev), 4, 4)
    assert "underflow" in str(e.value)


@pytest.mark.gpu
def test_prepare_linear_weights_redirect(dev, ref):
    """Context.prepare_linear_weights + Context.linear: a bound float weight runs the packed projection with
    dynamic activations on the device-packed weight; the result equals packing with the oracle and projecting
    with the same library; a second binding with another layout is INVALID_ARGUMENT; a multi-row input without
    packed_prefill (the reference's dense fallback) is UNSUPPORTED here."""
    from kidi_amd.ops import Context, DeviceWeight, Failure

    rng = np.random.default_rng(41)
    w = (rng.standard_normal((256, 512)) * 0.05).astype(f32)
    x = rng.standard_normal((1, 512)).astype(f32)
    ctx = Context(dev)
    wt = torch.from_numpy(w).to(dev)
    ctx.prepare_linear_weights(wt, 4, 128, asymmetric_clip=True)
    ctx.prepare_linear_weights(wt, 4, 128, asymmetric_clip=True)  # same layout: no-op
    with pytest.raises(Failure) as e:
        ctx.prepare_linear_weights(wt, 8, 128)
    assert e.value.code == "INVALID_ARGUMENT"
    y = ctx.linear(torch.from_numpy(x).to(dev), wt).cpu().numpy()
    v, s, z = ref.pack_weight(w, 4, 128, asymmetric_clip=True)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    y_ref = DeviceWeight(t(v), t(s), 4, 128, t(z)).linear(t(x)).cpu().numpy()
    np.testing.assert_array_equal(y, y_ref)
    with pytest.raises(Failure) as e:
        ctx.linear(torch.from_numpy(np.tile(x, (3, 1))).to(dev), wt)
    assert e.value.code == "UNSUPPORTED"
    ctx.decode_projections = True
    y3 = ctx.linear(torch.from_numpy(np.tile(x, (3, 1))).to(dev), wt).cpu().numpy()
    assert y3.shape == (3, 256)


def test_runtime_packing_choice():
    """gemma4.cpp:435-447: 4-bit groups where the width divides, 8-bit per-row otherwise, embeddings skipped,
    the asymmetric clip only for grouped 4-bit weights."""
    from kidi_amd.checkpoint import prepare_runtime_packing

    calls = []

    class Recorder:
        def prepare_linear_weights(self, weight, bits, group, packed_prefill, asym):
            calls.append((tuple(weight.shape), bits, group, packed_prefill, asym))

    state = {"embed_tokens.weight": torch.zeros(8, 256), "q_proj.weight": torch.zeros(64, 256),
             "odd.weight": torch.zeros(16, 200), "norm.weight": torch.zeros(256)}
    chosen = prepare_runtime_packing(Recorder(), state, 4, 128, packed_prefill=True, asymmetric_clip=True)
    assert chosen == [("q_proj.weight", 4, 128), ("odd.weight", 8, 200)]
    assert calls == [((64, 256), 4, 128, True, True), ((16, 200), 8, 200, True, False)]
    assert prepare_runtime_packing(Recorder(), state, 0) == []
