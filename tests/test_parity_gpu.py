"""GPU parity of the HIP path against the CPU oracle, through the C ABI (ctypes) on the same seeded inputs.

Bar: int8 activation codes, block sums and int32 per-group partials bit-exact; fp32 outputs within
max|dy| <= 2e-3 * max|y_ref|; exact equality where the reference pins exact values (calibrated KATs)."""

import numpy as np
import pytest

from tests.cases import activations, expected_partials, pack_codes, weights

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
TOL = 2e-3


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    _native.load()
    return torch.device("cuda:0")


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def device_weight(values, scales, bits, group, dev, zeros=None, zero_points=None, on_device=True):
    from kidi_amd.ops import DeviceWeight

    conv = (lambda a: to_dev(a, dev)) if on_device else (lambda a: torch.from_numpy(np.ascontiguousarray(a)))
    z = zeros if zeros is not None else zero_points
    return DeviceWeight(conv(values), conv(scales), bits, group, conv(z) if z is not None else None)


def check_close(y, y_ref, tol=TOL):
    y = y.detach().cpu().numpy() if hasattr(y, "detach") else y
    scale = max(float(np.max(np.abs(y_ref))), 1e-30)
    err = float(np.max(np.abs(y - y_ref))) if y.size else 0.0
    assert err <= tol * scale, f"max|dy| = {err:.3g} > {tol} * {scale:.3g}"


CASES = [
    # (bits, group, M, K, N, zeros, input_scale, x_bf16, outliers)
    (4, 32, 1, 256, 512, None, 0.0, False, 0.0),
    (4, 32, 3, 512, 256, None, 0.0, True, 0.0),
    (4, 128, 1, 512, 272, "zp", 0.0, True, 0.001),
    (4, 128, 4, 1024, 256, "zp", 0.0, True, 0.001),
    (4, 64, 2, 512, 320, "zp", 0.0, False, 0.0),
    (4, 256, 1, 1024, 256, None, 0.0, False, 0.0),
    (4, 128, 5, 512, 256, "f16", 0.0, False, 0.0),
    (8, 32, 1, 256, 128, None, 0.0, True, 0.0),
    (8, 32, 8, 512, 192, None, 0.0, False, 0.001),
    (8, 128, 3, 512, 64, None, 0.0, False, 0.0),
    (2, 32, 1, 512, 256, None, 0.05, False, 0.0),
    # decode rows 9..16 (skinny kernel), groups spanning tiles, large groups (whole-wave quantizer)
    (4, 128, 16, 512, 256, "zp", 0.0, True, 0.001),
    (8, 32, 12, 256, 128, None, 0.0, False, 0.0),
    (2, 32, 16, 512, 256, None, 0.05, False, 0.0),
    (4, 256, 9, 1024, 256, None, 0.0, False, 0.0),
    (4, 512, 2, 1024, 256, "zp", 0.0, True, 0.0),
    (8, 192, 3, 384, 128, None, 0.0, False, 0.0),
    (4, 128, 7, 512, 256, "f16", 0.0, True, 0.0),
    # decode kernel (M <= 4, K a multiple of 512, g in {32, 64, 128})
    (8, 32, 2, 1024, 192, None, 0.0, True, 0.001),
    (8, 128, 3, 512, 128, None, 0.03, False, 0.0),
    (8, 64, 4, 1536, 64, None, 0.0, False, 0.0),
    (4, 32, 4, 2048, 256, None, 0.0, False, 0.0),
    (4, 64, 1, 1024, 288, "zp", 0.0, True, 0.001),
    (4, 128, 1, 512, 256, "f16", 0.0, False, 0.0),
    (2, 64, 3, 1024, 128, None, 0.05, True, 0.0),
    (2, 128, 1, 512, 48, None, 0.05, False, 0.0),
    (2, 128, 6, 512, 128, None, 0.05, True, 0.0),
    (4, 32, 2, 256, 256, None, 0.05, False, 0.0),
    (8, 64, 1, 256, 128, None, 0.03, False, 0.0),
    # decode kernel, 5..8 rows (two MFMA row halves)
    (8, 32, 8, 2048, 256, None, 0.0, False, 0.001),
    (4, 128, 6, 1024, 272, "zp", 0.0, True, 0.001),
    (4, 32, 5, 512, 256, None, 0.0, False, 0.0),
    (2, 32, 7, 512, 128, None, 0.05, False, 0.0),
    (8, 64, 8, 512, 64, None, 0.03, False, 0.0),
    # prefill GEMM shapes (M > 8, ragged M and N)
    (4, 128, 130, 512, 272, "zp", 0.0, True, 0.001),
    (4, 32, 129, 256, 256, None, 0.0, False, 0.0),
    (4, 64, 200, 256, 384, "zp", 0.0, False, 0.0),
    (4, 256, 64, 512, 256, None, 0.0, False, 0.0),
    (4, 128, 40, 256, 256, "f16", 0.0, False, 0.0),
    (8, 32, 150, 256, 200, None, 0.0, False, 0.001),
    (8, 128, 17, 256, 64, None, 0.0, True, 0.0),
    (2, 32, 140, 512, 144, None, 0.05, False, 0.0),
    (2, 128, 33, 512, 128, None, 0.05, False, 0.0),
    (4, 32, 257, 256, 128, None, 0.05, False, 0.0),
    # int8 MFMA GEMM (4-bit, g = 128, K a multiple of 512): several row blocks, ragged N, static and symmetric
    (4, 128, 300, 1024, 400, None, 0.0, False, 0.0),
    (4, 128, 513, 512, 256, "zp", 0.0, True, 0.001),
    (4, 128, 17, 2048, 128, None, 0.05, False, 0.0),
    (4, 128, 64, 512, 1040, "zp", 0.0, True, 0.0),
    (4, 128, 260, 1536, 144, "zp", 0.0, False, 0.001),
    # 128-row tiles (fewer 256-row tiles than CUs): ragged M and N, calibrated inputs, float zeros
    (4, 128, 300, 1024, 2048, "zp", 0.0, True, 0.001),
    (4, 128, 250, 512, 2052, None, 0.05, False, 0.0),
    (4, 128, 129, 512, 2560, "f16", 0.0, True, 0.0),
    # split K (2 or 4 ranges per output tile, summed in range order by a reduction kernel)
    (4, 128, 64, 4096, 256, "zp", 0.0, True, 0.0),
    (4, 128, 300, 8192, 256, None, 0.0, False, 0.001),
    (4, 128, 40, 8192, 144, None, 0.05, False, 0.0),
    (4, 128, 64, 4096, 256, "f16", 0.0, True, 0.001),  # additive float zeros on the fp32 MFMA, K split in 4
    # 4-bit g = 32 / 64 prefill (gemm8_kernel from the prefill copy: one or two groups per 64-column step):
    # fused-QKV-like K, ragged M and N, zero points, additive float zeros, calibrated inputs, a single item step pair
    (4, 32, 300, 2048, 640, None, 0.0, True, 0.001),
    (4, 32, 64, 1024, 272, "zp", 0.0, True, 0.0),
    (4, 64, 140, 1536, 400, "zp", 0.0, False, 0.001),
    (4, 64, 33, 512, 128, None, 0.05, False, 0.0),
    (4, 32, 129, 128, 256, None, 0.0, False, 0.0),
    (4, 32, 260, 1024, 256, "f16", 0.0, True, 0.001),
    (4, 64, 100, 512, 144, "f16", 0.0, False, 0.0),
    # 4-bit g = 32 / 64 with N % 4 != 0 (no 16-byte output stores): the two-stage LDS kernel gemm_i4g_kernel
    (4, 32, 100, 512, 270, None, 0.0, False, 0.0),
    (4, 64, 70, 1024, 142, "zp", 0.0, True, 0.001),
    # group sizes the tiles cannot carry (row-major integer path)
    (4, 96, 3, 384, 256, "zp", 0.0, False, 0.0),
    (8, 48, 2, 288, 96, None, 0.0, False, 0.0),
    (8, 48, 20, 192, 64, None, 0.0, False, 0.0),
]


def _make(ref, case, seed):
    bits, group, M, K, N, zeros, input_scale, x_bf16, outliers = case
    rng = np.random.default_rng(seed)
    values, scales, zp, codes = weights(rng, N, K, bits, group, zero_points=zeros in ("zp", "f16"))
    zf = None
    if zeros == "f16":
        # an additive F16 zero that is not (8 - zp) * scale: stays a float zero on the device
        zf = rng.uniform(-0.05, 0.05, size=scales.shape).astype(np.float16)
        zp = None
    x = activations(rng, M, K, outliers)
    return bits, group, M, K, N, values, scales, zp, zf, codes, x, input_scale, x_bf16


@pytest.mark.parametrize("index", range(len(CASES)),
                         ids=[f"b{c[0]}g{c[1]}m{c[2]}k{c[3]}n{c[4]}{c[5] or ''}s{c[6]}" for c in CASES])
def test_projection_parity(dev, ref, index):
    case = CASES[index]
    print(f"case {case}", flush=True)
    bits, group, M, K, N, values, scales, zp, zf, codes, x, in_s, x_bf16 = _make(ref, case, 1000 + index)
    y_ref, path = ref.packed_linear(x, values, scales, bits, group, in_s, 0.0, zeros=zf, zero_points=zp)
    assert path != ref.PATH_PORTABLE
    dw = device_weight(values, scales, bits, group, dev, zeros=zf, zero_points=zp)
    xt = to_dev(x, dev)
    if x_bf16:
        xt = xt.to(torch.bfloat16)
    # activation codes and block statistics: bit-exact
    if in_s == 0:
        q_ref, s_ref, Q_ref, zpa_ref = ref.quantize_dynamic(x, group, bits)
    else:
        (q_ref, Q_ref), s_ref, zpa_ref = ref.quantize_static(x, group, in_s), None, None
    codes_d, s_d, Q_d, z_d = dw.debug_quantize(xt, in_s)
    np.testing.assert_array_equal(codes_d.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(Q_d.cpu().numpy(), Q_ref)
    if in_s == 0:
        np.testing.assert_array_equal(s_d.cpu().numpy(), s_ref)
        np.testing.assert_array_equal(z_d.cpu().numpy(), zpa_ref)
    # int32 per-group partials: bit-exact
    y_d, P_d = dw.debug_partials(xt, in_s)
    P_ref = expected_partials(ref, q_ref, codes, zpa_ref, bits, group, zero_points=zp, dynamic=in_s == 0)
    np.testing.assert_array_equal(P_d.cpu().numpy().astype(np.int64), P_ref)
    # fp32 outputs
    check_close(y_d, y_ref)
    y = dw.linear(xt, in_s)
    torch.cuda.synchronize()
    check_close(y, y_ref)
    np.testing.assert_array_equal(y.cpu().numpy(), y_d.cpu().numpy())  # the dump variant computes the same y


def test_eager_calibrated_projection_exact_gpu(dev, ref):
    """tests/kidi/layers/eager_test.cpp:64-111 through the HIP path: exact equality, bits 2/4/8, g = K = 256."""
    WIDTH = 256
    for bits in (2, 4, 8):
        per = 8 // bits
        for columns in (3, 35, 67, 257, 513):
            idx = np.arange(columns * WIDTH, dtype=np.int64)
            integers = ((idx * 13 + idx // WIDTH * 7 + idx // (WIDTH * 3) + 3) % (1 << bits)) - (1 << (bits - 1))
            weight = pack_codes(integers.reshape(columns, WIDTH), bits)
            factors = np.full((columns, 1), 0.001953125, np.float32)
            values = ((np.arange(WIDTH) % 17) - 8).astype(np.float32) * np.float32(0.125)
            values[0], values[1] = -1000.0, 1000.0
            y_ref, _ = ref.packed_linear(values[None, :], weight, factors, bits, WIDTH, 0.25, 0.125)
            dw = device_weight(weight, factors, bits, WIDTH, dev)
            y = dw.linear(to_dev(values[None, :], dev), 0.25, 0.125).cpu().numpy()
            np.testing.assert_array_equal(y, y_ref)


def test_cuda_kat_gpu(dev):
    """tests/kidi/runtime/cuda/operators_test.cpp:815-831 bytes, g=2 (row-major path); hand-worked values."""
    w = np.array([[0xE1, 0xC3], [0x54, 0x7A]], np.uint8)
    s = np.array([[0.25, 0.5], [0.125, 0.25]], np.float32)
    x = np.array([[0.25, -0.5, 0.75, -1], [-0.25, 0.5, -0.75, 1]], np.float32)
    dw = device_weight(w, s, 4, 2, dev)
    y = dw.linear(to_dev(x, dev), 0.25, 0.125).cpu().numpy()
    np.testing.assert_array_equal(y, np.array([[3.5, -3.0], [-3.5, 3.0]], np.float32))


@pytest.mark.parametrize("bits,group,N,M,in_s", [(4, 128, 35, 3, 0.0), (4, 4, 2, 1, 0.0), (2, 32, 256, 2, 0.0),
                                                 (8, 32, 63, 2, 0.0), (4, 128, 256, 2, 0.5)])
def test_portable_path(dev, ref, bits, group, N, M, in_s):
    """Float path (PortablePackedLinearOp) domains: N < 256 without zeros, g < 32, dynamic 2-bit, 8-bit N < 64,
    calibrated with zeros. The GPU sums k in the oracle's order without contraction: equal to the last bit."""
    rng = np.random.default_rng(N * 7 + bits)
    K = 256
    values, scales, zp, _ = weights(rng, N, K, bits, group, zero_points=in_s > 0)
    x = activations(rng, M, K)
    y_ref, path = ref.packed_linear(x, values, scales, bits, group, in_s, 0.0, zero_points=zp)
    assert path == ref.PATH_PORTABLE
    dw = device_weight(values, scales, bits, group, dev, zero_points=zp)
    y = dw.linear(to_dev(x, dev), in_s).cpu().numpy()
    np.testing.assert_array_equal(y, y_ref)


def test_eager_pack_weight_group4_gpu(dev, ref):
    """eager_test.cpp:300-345 on the device: pack_weight g=4, portable projection within 1e-3, 33 rows."""
    weights_ = np.array([0, -7, 7, 1, 0, 14, -14, 2, 0, 0, 0, 0, 7, -7, 1, -1], np.float32).reshape(2, 8)
    act = np.array([0, 1, 2, 3, 4, 5, 6, 255], np.float32)
    for bits in (2, 4, 8):
        v, s, _ = ref.pack_weight(weights_, bits, 4)
        y_ref, _ = ref.packed_linear(act[None, :], v, s, bits, 4)
        dw = device_weight(v, s, bits, 4, dev)
        y = dw.linear(to_dev(np.tile(act, (33, 1)), dev)).cpu().numpy()
        assert np.all(np.abs(y - y_ref[0][None, :]) <= 1e-3)


def test_output_calibration(dev, ref):
    """output_scale > 0 rounds y to int8 steps: codes agree except where y_ref sits within fp32 noise of a
    rounding boundary, and then by one step."""
    rng = np.random.default_rng(9)
    values, scales, zp, _ = weights(rng, 512, 1024, 4, 128, zero_points=True)
    x = activations(rng, 2, 1024)
    out_s = 0.01
    y_ref, _ = ref.packed_linear(x, values, scales, 4, 128, 0.0, out_s, zero_points=zp)
    y = device_weight(values, scales, 4, 128, dev, zero_points=zp).linear(to_dev(x, dev), 0.0, out_s).cpu().numpy()
    steps = np.rint((y - y_ref) / out_s)
    assert np.all(np.abs(steps) <= 1)
    assert np.mean(steps == 0) > 0.99


def test_host_source_and_repeat(dev, ref):
    """Weights packed from host memory equal weights packed from device memory; repeated calls are identical."""
    rng = np.random.default_rng(4)
    values, scales, zp, _ = weights(rng, 256, 512, 4, 128, zero_points=True)
    x = to_dev(activations(rng, 1, 512), dev)
    a = device_weight(values, scales, 4, 128, dev, zero_points=zp, on_device=False).linear(x)
    b = device_weight(values, scales, 4, 128, dev, zero_points=zp, on_device=True)
    y1, y2 = b.linear(x), b.linear(x)
    torch.cuda.synchronize()
    assert torch.equal(a, y1) and torch.equal(y1, y2)


def test_pack_weight_asymmetric_zeros_become_zero_points(dev, ref):
    """ops::pack_weight asymmetric output (F32 zeros = (8 - zp) * scale) runs the integer zero-point fold."""
    rng = np.random.default_rng(21)
    w = (rng.standard_normal((256, 512)) * 0.05).astype(np.float32)
    v, s, z = ref.pack_weight(w, 4, 128, asymmetric_clip=True)
    x = activations(rng, 3, 512)
    y_ref, path = ref.packed_linear(x, v, s, 4, 128, zeros=z)
    assert path == ref.PATH_BLOCKWISE
    dw = device_weight(v, s, 4, 128, dev, zeros=z)
    check_close(dw.linear(to_dev(x, dev)), y_ref)
    zp = np.rint(8 - z / s).astype(np.uint8)
    _, P = dw.debug_partials(to_dev(x, dev))
    q, _, _, _ = ref.quantize_dynamic(x, 128, 4)
    np.testing.assert_array_equal(P.cpu().numpy(), expected_partials(ref, q, ref.unpack_codes(v, 512, 4), None, 4, 128,
                                                                      zero_points=zp))


def test_zero_block_and_empty(dev, ref):
    """An all-zero activation block quantizes to codes 0 / scale 0 and contributes nothing; M = 0 is a no-op."""
    rng = np.random.default_rng(5)
    values, scales, zp, _ = weights(rng, 256, 256, 4, 32, zero_points=True)
    x = activations(rng, 2, 256)
    x[0, 32:64] = 0.0
    x[1, :] = 0.0
    y_ref, _ = ref.packed_linear(x, values, scales, 4, 32, zero_points=zp)
    dw = device_weight(values, scales, 4, 32, dev, zero_points=zp)
    y = dw.linear(to_dev(x, dev)).cpu().numpy()
    check_close(y, y_ref)
    assert np.all(y[1] == 0)
    empty = dw.linear(torch.zeros((0, 256), device=dev))
    assert tuple(empty.shape) == (0, 256)


@pytest.mark.parametrize("M,I,K", [(1, 256, 512), (4, 256, 512), (8, 256, 512), (16, 256, 512), (200, 256, 512),
                                   (300, 272, 512), (40, 256, 2048), (40, 256, 4096)])
def test_gelu_gate_fused(dev, ref, M, I, K):
    """gate/up projection + GELU-tanh in one pass equals the oracle's projection followed by gelu_gate."""
    rng = np.random.default_rng(M)
    values, scales, zp, _ = weights(rng, 2 * I, K, 4, 128, zero_points=True)
    x = activations(rng, M, K)
    y_full, _ = ref.packed_linear(x, values, scales, 4, 128, zero_points=zp)
    h_ref = ref.gelu_gate(y_full)
    from kidi_amd.ops import Context

    ctx = Context(dev)
    h = ctx.packed_linear_gelu_gate(to_dev(x, dev), to_dev(values, dev), to_dev(scales, dev), 4, 128,
                                    zeros=to_dev(zp, dev))
    check_close(h, h_ref, tol=5e-3)


def test_fused_qkv_concat(dev, ref):
    """Fused QKV (one weight of N = 2048 + 256 + 256 rows, g = 32) equals the three projections side by side."""
    rng = np.random.default_rng(31)
    K = 2048
    parts = [weights(rng, n, K, 4, 32) for n in (2048, 256, 256)]
    x = activations(rng, 1, K)
    from kidi_amd.ops import DeviceWeight

    fused = DeviceWeight(None, None, 4, 32, concat=[(to_dev(v, dev), to_dev(s, dev), None) for v, s, _, _ in parts])
    y = fused.linear(to_dev(x, dev)).cpu().numpy()
    y_ref = np.concatenate([ref.packed_linear(x, v, s, 4, 32)[0] for v, s, _, _ in parts], axis=1)
    check_close(y, y_ref)


def test_context_mirror(dev, ref):
    """Context.packed_linear: host tensors in, host tensors out; validation errors carry Kidi's error codes."""
    from kidi_amd.ops import Context, Failure

    rng = np.random.default_rng(8)
    values, scales, zp, _ = weights(rng, 256, 256, 4, 128, zero_points=True)
    x = activations(rng, 2, 256)
    ctx = Context(dev)
    v, s, z = torch.from_numpy(values), torch.from_numpy(scales), torch.from_numpy(zp)
    ctx.bind_packed_zero(s, z)
    y = ctx.packed_linear(torch.from_numpy(x), v, s, 4, 128)
    y_ref, _ = ref.packed_linear(x, values, scales, 4, 128, zero_points=zp)
    check_close(y.numpy(), y_ref)
    with pytest.raises(Failure) as e:
        ctx.packed_linear(torch.from_numpy(x), v, s, 4, 96)
    assert e.value.code == "INVALID_ARGUMENT"
    with pytest.raises(Failure) as e:
        ctx.packed_linear(torch.from_numpy(x), v, s, 4, 128, input_scale=-1.0)
    assert e.value.code == "INVALID_ARGUMENT"


@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("shape", [(2048, 8192), (8192, 2048)])
def test_baseline_decode_shapes(dev, ref, M, shape):
    """Config 2 at full size: asymmetric int4 g=128, bf16 activations with 0.1% outliers x20."""
    K, N = shape
    rng = np.random.default_rng(2)
    values, scales, zp, codes = weights(rng, N, K, 4, 128, zero_points=True)
    x = activations(rng, M, K, outliers=0.001)
    y_ref, _ = ref.packed_linear(x, values, scales, 4, 128, zero_points=zp, threads=8)
    dw = device_weight(values, scales, 4, 128, dev, zero_points=zp)
    xt = to_dev(x, dev).to(torch.bfloat16)
    y_d, P_d = dw.debug_partials(xt)
    q, _, _, _ = ref.quantize_dynamic(x, 128, 4)
    np.testing.assert_array_equal(P_d.cpu().numpy().astype(np.int64),
                                  expected_partials(ref, q, codes, None, 4, 128, zero_points=zp))
    check_close(dw.linear(xt), y_ref)


def test_prefill_f32_scales(dev, ref):
    """GEMM path with F32 scales and F32 activations: partials bit-exact, outputs within tolerance."""
    rng = np.random.default_rng(77)
    M, K, N = 96, 1024, 256
    values, scales, zp, codes = weights(rng, N, K, 4, 128, zero_points=True, scale_dtype=np.float32)
    x = activations(rng, M, K)
    y_ref, _ = ref.packed_linear(x, values, scales, 4, 128, zero_points=zp)
    dw = device_weight(values, scales, 4, 128, dev, zero_points=zp)
    y_d, P_d = dw.debug_partials(to_dev(x, dev))
    q, _, _, _ = ref.quantize_dynamic(x, 128, 4)
    np.testing.assert_array_equal(P_d.cpu().numpy().astype(np.int64),
                                  expected_partials(ref, q, codes, None, 4, 128, zero_points=zp))
    check_close(y_d, y_ref)
    check_close(dw.linear(to_dev(x, dev)), y_ref)


def test_baseline_prefill_rows(dev, ref):
    """Config 3 (M=2048, K=2048, N=8192, asymmetric g=128): rows are independent, so a sample of 16 rows of the
    full GEMM output is checked against the oracle on those rows; all rows are finite."""
    M, K, N = 2048, 2048, 8192
    rng = np.random.default_rng(3)
    values, scales, zp, _ = weights(rng, N, K, 4, 128, zero_points=True)
    x = activations(rng, M, K)
    dw = device_weight(values, scales, 4, 128, dev, zero_points=zp)
    y = dw.linear(to_dev(x, dev).to(torch.bfloat16)).cpu().numpy()
    assert np.all(np.isfinite(y))
    rows = np.sort(rng.choice(M, size=16, replace=False))
    y_ref, _ = ref.packed_linear(x[rows], values, scales, 4, 128, zero_points=zp, threads=8)
    check_close(y[rows], y_ref)


def test_fused_qkv_prefill_rows(dev, ref):
    """configs[3] fused QKV at prefill size (M = 2048, K = 2048, N = 2048 + 256 + 256, 4-bit g = 32): sampled rows
    against the oracle (the g = 32 prefill GEMM)."""
    M, K, N, g = 2048, 2048, 2560, 32
    rng = np.random.default_rng(33)
    values, scales, _, _ = weights(rng, N, K, 4, g)
    x = activations(rng, M, K, 0.001)
    dw = device_weight(values, scales, 4, g, dev)
    y = dw.linear(to_dev(x, dev).to(torch.bfloat16))
    torch.cuda.synchronize()
    rows = np.array([0, 1, 127, 128, 1000, M - 1])
    xb = ref.f32_to_bf16_bits(x[rows])
    y_ref, path = ref.packed_linear(xb, values, scales, 4, g, x_bf16=True, threads=8)
    assert path == ref.PATH_BLOCKWISE
    check_close(y[torch.from_numpy(rows).to(dev)], y_ref)


# g = 32 prefill in 128 x 160 tiles (gemm8w_kernel: where 256 x 128 tiles leave CUs idle): M, K, N, zeros, input
# scale, x as bf16, F32 weight scales
WIDE_CASES = [
    (2048, 2048, 2560, None, 0.0, True, False),   # configs[3] fused QKV
    (2000, 1024, 2496, "zp", 0.0, False, False),  # ragged M (a partial last row tile), two dead column blocks
    (1536, 512, 2560, None, 0.05, True, False),   # calibrated inputs
    (2048, 1024, 2400, None, 0.0, True, True),    # F32 weight scales, 15 column tiles
    (4096, 512, 2560, None, 0.0, True, False),    # two tiles per workgroup (the copy ring runs across items)
    (2048, 128, 2560, None, 0.0, True, False),    # two k steps: fewer than the four ring stages
    (4096, 256, 2560, "zp", 0.0, False, False),   # four k steps per item, two items per workgroup
]


@pytest.mark.parametrize("index", range(len(WIDE_CASES)), ids=[f"m{c[0]}k{c[1]}n{c[2]}" for c in WIDE_CASES])
def test_wide_tile_prefill(dev, ref, index):
    """The g = 32 prefill in 128 x 160 tiles: routed there, y bit-identical to the parity-dump instance's (256 x 128
    tiles, whose int32 partials are checked bit-exact against the oracle here on sampled rows and columns, and the
    same per-element operation order), and sampled rows within tolerance of the oracle."""
    M, K, N, zeros, in_s, x_bf16, f32_scales = WIDE_CASES[index]
    print(f"wide case M={M} K={K} N={N} zeros={zeros} in_s={in_s}", flush=True)
    rng = np.random.default_rng(700 + index)
    values, scales, zp, codes = weights(rng, N, K, 4, 32, zero_points=zeros == "zp",
                                        scale_dtype=np.float32 if f32_scales else np.float16)
    x = activations(rng, M, K, 0.001)
    dw = device_weight(values, scales, 4, 32, dev, zero_points=zp)
    xt = to_dev(x, dev)
    if x_bf16:
        xt = xt.to(torch.bfloat16)
    assert dw.route(xt, in_s) == "gemm8w_kernel"
    y = dw.linear(xt, in_s)
    y_d, P_d = dw.debug_partials(xt, in_s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), y_d.cpu().numpy())
    rows = np.array(sorted({0, 1, 127, 128, 129, M // 2, M - 1}))
    xr = ref.f32_to_bf16_bits(x[rows]) if x_bf16 else x[rows]
    y_ref, path = ref.packed_linear(xr, values, scales, 4, 32, in_s, zero_points=zp, x_bf16=x_bf16, threads=8)
    assert path == (ref.PATH_BLOCKWISE if in_s == 0 else ref.PATH_SYMMETRIC)
    check_close(y[torch.from_numpy(rows).to(dev)], y_ref)
    cols = np.array(sorted({0, 31, 32, 159, 160, N - 1, *rng.choice(N, 24, replace=False).tolist()}))
    xq = (ref.bf16_bits_to_f32(xr) if x_bf16 else xr)
    if in_s == 0:
        q, _, _, zpa = ref.quantize_dynamic(xq, 32, 4)
    else:
        (q, _), zpa = ref.quantize_static(xq, 32, in_s), None
    P = P_d[torch.from_numpy(rows).to(dev)][:, torch.from_numpy(cols).to(dev)].cpu().numpy().astype(np.int64)
    np.testing.assert_array_equal(P, expected_partials(ref, q, codes[cols], zpa, 4, 32,
                                                       zero_points=zp[cols] if zp is not None else None,
                                                       dynamic=in_s == 0))


def test_wide_tile_output_calibration(dev, ref):
    """Calibrated outputs (output_scale > 0) from the 128 x 160 g = 32 tiles: bit-identical to the dump instance and
    within one int8 step of the oracle, on sampled rows."""
    M, K, N, out_s = 2048, 512, 2560, 0.01
    rng = np.random.default_rng(750)
    values, scales, _, _ = weights(rng, N, K, 4, 32)
    x = activations(rng, M, K, 0.0)
    dw = device_weight(values, scales, 4, 32, dev)
    xt = to_dev(x, dev).to(torch.bfloat16)
    assert dw.route(xt) == "gemm8w_kernel"
    y = dw.linear(xt, 0.0, out_s)
    y_d, _ = dw.debug_partials(xt, 0.0, out_s)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), y_d.cpu().numpy())
    rows = np.array([0, 5, 127, 128, 1500, M - 1])
    y_ref, _ = ref.packed_linear(x[rows], values, scales, 4, 32, 0.0, out_s, threads=8)
    steps = np.rint((y[torch.from_numpy(rows).to(dev)].cpu().numpy() - y_ref) / out_s)
    assert np.all(np.abs(steps) <= 1)
    assert np.mean(steps == 0) > 0.99
    assert np.any(y_ref != 0)


@pytest.mark.parametrize("group", [32, 64, 128])
@pytest.mark.parametrize("scale_kind", ["f32", "f16_extreme"])
def test_prefill_scale_forms(dev, ref, group, scale_kind):
    """Prefill GEMMs (g = 128 and g = 32 / 64 kernels) with F32 weight scales (the conversion epilogue) and with F16
    scales spanning subnormals to large values (the biased-accumulator epilogue, exact t = s * P' for any F16 s):
    int32 partials bit-exact, outputs within tolerance of the oracle."""
    rng = np.random.default_rng(500 + group)
    M, K, N = 40, 512, 256
    if scale_kind == "f32":
        values, scales, zp, codes = weights(rng, N, K, 4, group, zero_points=True, scale_dtype=np.float32)
    else:
        values, scales, zp, codes = weights(rng, N, K, 4, group, zero_points=True)
        mags = rng.choice(np.array([6.0e-8, 3.0e-5, 0.01, 1.0, 250.0, 6.0e4], np.float32), size=scales.shape)
        scales = (mags * rng.uniform(0.5, 1.0, scales.shape).astype(np.float32)).astype(np.float16)
    x = activations(rng, M, K, 0.001)
    y_ref, path = ref.packed_linear(x, values, scales, 4, group, zero_points=zp)
    assert path == ref.PATH_BLOCKWISE
    dw = device_weight(values, scales, 4, group, dev, zero_points=zp)
    y_d, P_d = dw.debug_partials(to_dev(x, dev))
    q, _, _, _ = ref.quantize_dynamic(x, group, 4)
    np.testing.assert_array_equal(P_d.cpu().numpy().astype(np.int64),
                                  expected_partials(ref, q, codes, None, 4, group, zero_points=zp))
    check_close(y_d, y_ref)
    y = dw.linear(to_dev(x, dev))
    torch.cuda.synchronize()
    check_close(y, y_ref)
    np.testing.assert_array_equal(y.cpu().numpy(), y_d.cpu().numpy())  # the dump variant computes the same y


@pytest.mark.parametrize("N", [16 * 511, 16 * 512, 16 * 1024, 16 * 1025 - 8])
@pytest.mark.parametrize("bits,group,zeros", [(4, 32, None), (4, 64, "zp"), (4, 128, "zp"), (8, 32, None)])
def test_decode_unit_plan_boundaries(dev, ref, N, bits, group, zeros):
    """M = 1 around the launch plan's boundaries (single row-tile units up to 1024 row tiles, pairs above; ragged
    last tile): int32 partials bit-exact, outputs within tolerance."""
    rng = np.random.default_rng(N + bits * 7 + group)
    M, K = 1, 512
    values, scales, zp, codes = weights(rng, N, K, bits, group, zero_points=zeros == "zp")
    x = activations(rng, M, K, 0.001)
    y_ref, path = ref.packed_linear(x, values, scales, bits, group, zero_points=zp)
    assert path == ref.PATH_BLOCKWISE
    dw = device_weight(values, scales, bits, group, dev, zero_points=zp)
    y_d, P_d = dw.debug_partials(to_dev(x, dev))
    q, _, _, zpa = ref.quantize_dynamic(x, group, bits)
    np.testing.assert_array_equal(P_d.cpu().numpy().astype(np.int64),
                                  expected_partials(ref, q, codes, zpa, bits, group, zero_points=zp))
    check_close(y_d, y_ref)
    y = dw.linear(to_dev(x, dev))
    torch.cuda.synchronize()
    check_close(y, y_ref)
