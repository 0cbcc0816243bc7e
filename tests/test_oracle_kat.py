"""Pins the CPU oracle (oracle/kq_ref.cpp) against the reference's own known-answer tests and against what the
mathematics fixes. Each test names the reference file:line it reproduces. CPU only."""

import numpy as np
import pytest

f32 = np.float32


# ---------------------------------------------------------------------------------------------------------------
# tests/kidi/layers/eager_test.cpp:64-111 -- calibrated projection, exact equality, bits 2/4/8, K=256 per-channel.
@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("columns", [3, 35, 67, 257, 513])
def test_eager_calibrated_projection_exact(ref, bits, columns):
    WIDTH = 256
    per = 8 // bits
    idx = np.arange(columns * WIDTH, dtype=np.int64)
    integers = ((idx * 13 + idx // WIDTH * 7 + idx // (WIDTH * 3) + 3) % (1 << bits)) - (1 << (bits - 1))
    packed = np.zeros(columns * WIDTH // per, np.uint8)
    for i in range(per):
        packed |= ((integers[i::per] & ((1 << bits) - 1)) << (i * bits)).astype(np.uint8)
    weight = packed.reshape(columns, WIDTH // per)
    factors = np.full((columns, 1), 0.001953125, f32)
    values = ((np.arange(WIDTH) % 17) - 8).astype(f32) * f32(0.125)
    values[0], values[1] = -1000.0, 1000.0
    y, path = ref.packed_linear(values[None, :], weight, factors, bits, WIDTH, 0.25, 0.125)
    assert path == ref.PATH_SYMMETRIC
    # expected = clamp(nearbyint(sum * factor * 0.25 / 0.125), -128, 127) * 0.125, sum over clamp(nearbyint(x/0.25))
    codes_x = np.clip(np.rint(values / f32(0.25)), -128, 127).astype(np.int64)
    ints = integers.reshape(columns, WIDTH)
    sums = (ints * codes_x[None, :]).sum(axis=1)
    expected = np.clip(np.rint(sums.astype(f32) * factors[:, 0] * f32(0.25) / f32(0.125)), -128, 127).astype(f32) * f32(0.125)
    np.testing.assert_array_equal(y[0], expected)


# tests/kidi/runtime/cuda/operators_test.cpp:815-831 -- 4-bit bytes E1 C3 54 7A, g=2, in 0.25, out 0.125. The
# expected values below are worked by hand from the byte layout (low nibble = even element, two's complement):
# rows of codes [1,-2,3,-4] and [4,5,-6,7]; x/0.25 = [1,-2,3,-4], [-1,2,-3,4].
def test_cuda_packed_kat_by_hand(ref):
    w = np.array([[0xE1, 0xC3], [0x54, 0x7A]], np.uint8)
    s = np.array([[0.25, 0.5], [0.125, 0.25]], f32)
    x = np.array([[0.25, -0.5, 0.75, -1], [-0.25, 0.5, -0.75, 1]], f32)
    y, path = ref.packed_linear(x, w, s, 4, 2, 0.25, 0.125)
    assert path == ref.PATH_SYMMETRIC
    # m=0,n=0: P=[1+4, 9+16]=[5,25] -> (5*.25 + 25*.5)*.25 = 3.4375 -> /0.125 = 27.5 -> rint 28 -> 3.5
    # m=0,n=1: P=[4-10, -18-28]=[-6,-46] -> (-6*.125 - 46*.25)*.25 = -3.0625 -> -24.5 -> rint -24 -> -3.0
    # m=1 is m=0 negated: 3.5 -> -27.5 -> -28 -> -3.5 ; -3.0625 -> 24.5 -> 24 -> 3.0
    np.testing.assert_array_equal(y, np.array([[3.5, -3.0], [-3.5, 3.0]], f32))


# tests/kidi/layers/precision_test.cpp:95-108 -- signed 4-bit unpack of 0xe1,0xc3 with scale 0.5 on x=[1,2,3,4] is -5.
def test_precision_signed_nibbles(ref):
    y, path = ref.packed_linear(np.array([[1, 2, 3, 4]], f32), np.array([[0xE1, 0xC3]], np.uint8),
                                np.array([[0.5]], f32), 4, 4)
    assert path == ref.PATH_PORTABLE
    assert y[0, 0] == -5.0
    np.testing.assert_array_equal(ref.unpack_codes(np.array([[0xE1, 0xC3]], np.uint8), 4, 4), [[1, -2, 3, -4]])


# tests/arm_gemma_benchmark_test.py:83-101 -- packer KATs (ties away from zero, nibble order, grouped scales).
def test_pack_weight_python_kats(ref):
    v, s, z = ref.pack_weight(np.array([[-7, -1, 0, 1, 7, -3.5], [0, 0, 0, 0, 0, 0]], f32), 4, 6)
    np.testing.assert_array_equal(s, [[1.0], [1.0]])
    assert z is None
    np.testing.assert_array_equal(ref.unpack_codes(v, 6, 4), [[-7, -1, 0, 1, 7, -4], [0] * 6])
    below_half = np.nextafter(f32(0.5), f32(0))
    v, _, _ = ref.pack_weight(np.array([[below_half, 7.0]], f32), 4, 2)
    np.testing.assert_array_equal(ref.unpack_codes(v, 2, 4), [[0, 7]])
    v, s, _ = ref.pack_weight(np.array([[-7.0, 3.5, 14.0, -7.0]], f32), 4, 2)
    np.testing.assert_array_equal(s, [[1.0, 2.0]])
    np.testing.assert_array_equal(ref.unpack_codes(v, 4, 4), [[-7, 4, 7, -4]])
    v, s, _ = ref.pack_weight(np.array([[-127.0, 0.0, 63.5, 127.0]], f32), 8, 4)
    np.testing.assert_array_equal(s, [[1.0]])
    np.testing.assert_array_equal(v.view(np.int8), [[-127, 0, 64, 127]])
    v, s, z = ref.pack_weight(np.array([[-0.2, 0.0, 0.5, 1.0]], f32), 4, 2, asymmetric_clip=True)
    assert v.shape == (1, 2) and s.shape == (1, 2) and z.shape == (1, 2)
    with pytest.raises(ValueError):
        ref.pack_weight(np.array([[np.nan, 0.0]], f32), 4, 2)


# tests/kidi/layers/eager_test.cpp:300-345 -- pack_weight g=4 layout/decode and the portable projection (1e-3),
# invalid group 3 rejected, 33-row tiling equals the single row (0.1).
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_eager_pack_weight_group4(ref, bits):
    weights = np.array([0, -7, 7, 1, 0, 14, -14, 2, 0, 0, 0, 0, 7, -7, 1, -1], f32).reshape(2, 8)
    v, s, _ = ref.pack_weight(weights, bits, 4)
    act = np.array([0, 1, 2, 3, 4, 5, 6, 255], f32)
    y, path = ref.packed_linear(act[None, :], v, s, bits, 4)
    assert path == ref.PATH_PORTABLE
    flat = v.reshape(-1)
    for row in range(2):
        expected = f32(0)
        for ch in range(8):
            off = row * 8 + ch
            raw = (int(flat[off // (8 // bits)]) >> ((off % (8 // bits)) * bits)) & ((1 << bits) - 1)
            integer = (raw ^ (1 << (bits - 1))) - (1 << (bits - 1))
            expected += act[ch] * f32(integer) * s[row, ch // 4]
        assert np.isfinite(y[0, row]) and abs(y[0, row] - expected) <= 1e-3
    with pytest.raises(ValueError):
        ref.pack_weight(weights, bits, 3)
    many, _ = ref.packed_linear(np.tile(act, (33, 1)), v, s, bits, 4)
    assert np.all(np.abs(many - y[0][None, :]) <= 0.1)


# tests/kidi/layers/eager_test.cpp:347-378 -- default pack_weight (4-bit, g=128) on N=35 takes the portable path
# and matches the float matmul within 0.05 for rows {1, 3, 33}.
def test_eager_int4_g128_portable(ref):
    WIDTH, COLUMNS = 256, 35
    col = np.arange(COLUMNS)[:, None]
    ch = np.arange(WIDTH)[None, :]
    weights = (((col * 7 + ch) % 15) - 7).astype(f32) * np.where(ch < 128, f32(0.125), f32(0.25))
    v, s, _ = ref.pack_weight(weights)
    for rows in (1, 3, 33):
        act = (np.arange(rows * WIDTH) % 256).astype(f32).reshape(rows, WIDTH)
        y, path = ref.packed_linear(act, v, s, 4, 128)
        assert path == ref.PATH_PORTABLE
        expected = act.astype(np.float64) @ weights.astype(np.float64).T
        assert np.all(np.isfinite(y)) and np.max(np.abs(y - expected)) <= 0.05


# tests/kidi/layers/eager_test.cpp:431-452 -- GELU(tanh) saturates exactly and follows the formula to 1e-5.
def test_gelu_tanh(ref):
    g = np.array([-1000, -20, 20, 1000], f32)
    out = ref.gelu_gate(np.concatenate([g, np.ones(4, f32)])[None, :])[0]
    np.testing.assert_array_equal(out, [0, 0, 20, 1000])
    x = np.linspace(-6, 6, 97).astype(f32)
    got = ref.gelu_gate(np.concatenate([x, np.ones_like(x)])[None, :])[0]
    want = 0.5 * x.astype(np.float64) * (1 + np.tanh(np.sqrt(2 / np.pi) * (x + 0.044715 * x.astype(np.float64) ** 3)))
    assert np.max(np.abs(got - want)) <= 1e-5


# ---------------------------------------------------------------------------------------------------------------
# What the mathematics fixes.

def test_half_to_float_exhaustive(ref):
    """Every binary16 pattern converts exactly (numpy's float16 is IEEE binary16)."""
    lib = ref.lib()
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.kqr_half_to_float(int(b)) for b in bits[::7]], np.float32)
    w = want[::7]
    same = (got == w) | (np.isnan(got) & np.isnan(w))
    assert same.all()


def test_dynamic_quantizer_rounding_kat(ref):
    """Symmetric dynamic form: with max=127 the inverse is 1, so ties go to even (nearbyint): 2.5->2, -3.5->-4."""
    x = np.array([[127.0, 2.5, -3.5, 0.5, -127.0, 1.5, 0.0, -0.5]], f32)
    q, s, Q, zp = ref.quantize_dynamic(x, 8, 4)
    np.testing.assert_array_equal(q, [[127, 2, -4, 0, -127, 2, 0, 0]])
    assert s[0, 0] == f32(1.0) and Q[0, 0] == q.sum() and zp[0, 0] == 0
    # all-zero block: codes 0, scale 0 (defined here; the restated form is 0*inf there)
    q, s, Q, _ = ref.quantize_dynamic(np.zeros((1, 32), f32), 32, 4)
    assert not q.any() and s[0, 0] == 0 and Q[0, 0] == 0


def test_dynamic_quantizer_asymmetric_kat(ref):
    """8-bit asymmetric form (hnsw_test.cpp:492-511) worked by hand for x=[-1,0,1,2]:
    rdiff=3, inverse=85, min_error=-213, max_error=297 -> fzp=-128+85=-43, q=round(85x)-43."""
    q, s, Q, zp = ref.quantize_dynamic(np.array([[-1.0, 0.0, 1.0, 2.0]], f32), 4, 8)
    np.testing.assert_array_equal(q, [[-128, -43, 42, 127]])
    assert zp[0, 0] == -43 and Q[0, 0] == -2 and s[0, 0] == f32(3.0) / f32(255.0)
    q, s, Q, zp = ref.quantize_dynamic(np.zeros((1, 4), f32), 4, 8)
    assert (q == -128).all() and zp[0, 0] == -128 and s[0, 0] == 1.0


def test_dynamic_quantizer_invariants(ref):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 512)).astype(f32)
    x[1, 40] = 30.0
    for g in (32, 128):
        q, s, Q, _ = ref.quantize_dynamic(x, g, 4)
        xb = x.reshape(5, -1, g)
        qb = q.reshape(5, -1, g).astype(np.int64)
        assert np.abs(qb).max() <= 127
        np.testing.assert_array_equal(np.abs(qb).max(axis=2), 127)  # the block maximum maps to +-127
        np.testing.assert_array_equal(qb.sum(axis=2), Q)
        err = np.abs(xb - qb * s[..., None])
        assert np.all(err <= s[..., None] * 0.5000001 + 1e-12)
        np.testing.assert_array_equal(s, np.abs(xb).max(axis=2) / f32(127))
    q8, s8, Q8, zp8 = ref.quantize_dynamic(x, 32, 8)
    rec = (q8.reshape(5, -1, 32).astype(np.int64) - zp8[..., None]) * s8[..., None]
    assert np.all(np.abs(rec - x.reshape(5, -1, 32)) <= s8[..., None] * 0.5001)


def test_static_quantizer(ref):
    x = np.array([[-100, -1.25, -0.75, -0.25, 0.25, 0.75, 1.25, 100]], f32)
    q, Q = ref.quantize_static(x, 8, 0.5)
    # eager_test.cpp:425-430 static_round KAT: codes of x/0.5 with ties to even, clamped to [-128, 127]
    np.testing.assert_array_equal(q, [[-128, -2, -2, 0, 0, 2, 2, 127]])
    np.testing.assert_array_equal(q.astype(f32) * f32(0.5), [[-64, -1, -1, 0, 0, 1, 1, 63.5]])
    assert Q[0, 0] == q.sum()


def test_partials_brute_force(ref):
    rng = np.random.default_rng(5)
    q = rng.integers(-128, 128, (3, 96)).astype(np.int8)
    c = rng.integers(-8, 8, (7, 96)).astype(np.int8)
    P, C = ref.partials(q, c, 32)
    for m in range(3):
        for n in range(7):
            for b in range(3):
                sl = slice(32 * b, 32 * b + 32)
                assert P[m, n, b] == int(np.dot(q[m, sl].astype(np.int64), c[n, sl].astype(np.int64)))
    np.testing.assert_array_equal(C, c.reshape(7, 3, 32).astype(np.int64).sum(axis=2))


def test_pack_weight_asymmetric_exact_grid(ref):
    """A group on the exact 16-level grid 0..1.5 quantizes losslessly with the full range (frac 1.0):
    scale 0.1, zp 0, zero = 8 * scale, codes u - 8."""
    w = (np.arange(16, dtype=f32) * f32(0.1))[None, :]
    v, s, z = ref.pack_weight(w, 4, 16, asymmetric_clip=True)
    assert s[0, 0] == max((f32(2) * f32(1) * f32(0.75)) / f32(15), f32(1e-8))
    assert z[0, 0] == f32(8) * s[0, 0]
    np.testing.assert_array_equal(ref.unpack_codes(v, 16, 4)[0], np.arange(16) - 8)


def test_pack_weight_asymmetric_argmin(ref):
    """The stored (scale, zero) reconstructs every group with an MSE no worse (up to float rounding) than any of
    the 11 clip candidates, computed independently in float64; and w_hat = c*s + z stays on the grid."""
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((6, 256)) * 0.05 + rng.standard_normal((6, 1)) * 0.02).astype(f32)
    w[2, 5] = 0.9  # an outlier that makes clipping pay
    v, s, z = ref.pack_weight(w, 4, 128, asymmetric_clip=True)
    codes = ref.unpack_codes(v, 256, 4).astype(np.float64)
    for r in range(6):
        for g in range(2):
            wg = w[r, g * 128:(g + 1) * 128].astype(np.float64)
            rec = codes[r, g * 128:(g + 1) * 128] * s[r, g] + z[r, g]
            mse = np.mean((wg - rec) ** 2)
            mn, mx = wg.min(), wg.max()
            best = np.inf
            for frac in (1.0, .95, .9, .85, .8, .75, .7, .65, .6, .55, .5):
                center, half = 0.5 * (mx + mn), 0.5 * (mx - mn)
                sc = max(2 * frac * half / 15, 1e-8)
                zp = np.clip(np.rint(-(center - frac * half) / sc), 0, 15)
                qq = np.clip(np.rint(wg / sc + zp), 0, 15)
                best = min(best, np.mean((wg - (qq - zp) * sc) ** 2))
            assert mse <= best * (1 + 1e-4) + 1e-12
            zp_back = 8 - z[r, g] / s[r, g]
            assert abs(zp_back - round(zp_back)) < 1e-4 and 0 <= round(zp_back) <= 15


def test_pack_weight_symmetric_roundtrip(ref):
    rng = np.random.default_rng(2)
    w = rng.standard_normal((4, 256)).astype(f32)
    for bits, limit in ((2, 1), (4, 7), (8, 127)):
        v, s, _ = ref.pack_weight(w, bits, 32)
        c = ref.unpack_codes(v, 256, bits).astype(np.float64)
        assert np.abs(c).max() <= limit
        rec = c * np.repeat(s, 32, axis=1)
        assert np.all(np.abs(rec - w) <= np.repeat(s, 32, axis=1) * 0.5 + 1e-6)
        np.testing.assert_array_equal(s, np.abs(w.reshape(4, -1, 32)).max(axis=2) / f32(limit))
    # bf16 and f16 sources decode exactly before packing
    wb = ref.f32_to_bf16_bits(w)
    v1, s1, _ = ref.pack_weight(wb, 4, 32, bf16=True)
    v2, s2, _ = ref.pack_weight(ref.bf16_bits_to_f32(wb), 4, 32)
    np.testing.assert_array_equal(v1, v2)
    np.testing.assert_array_equal(s1, s2)
    v3, s3, _ = ref.pack_weight(w.astype(np.float16), 4, 32)
    v4, s4, _ = ref.pack_weight(w.astype(np.float16).astype(f32), 4, 32)
    np.testing.assert_array_equal(v3, v4)
    np.testing.assert_array_equal(s3, s4)


def test_qat_xor_roundtrip(ref):
    raw = np.arange(256, dtype=np.uint8)
    for bits, mask in ((4, 0x88), (2, 0xAA)):
        conv = ref.qat_to_signed(raw, bits)
        np.testing.assert_array_equal(conv, raw ^ mask)
        np.testing.assert_array_equal(ref.qat_to_signed(conv, bits), raw)
    # 4-bit offset code 8 (0x88 = two offset nibbles of 8) is signed zero; offset 0 is -8
    assert ref.unpack_codes(ref.qat_to_signed(np.array([[0x88]], np.uint8), 4), 2, 4).tolist() == [[0, 0]]
    assert ref.unpack_codes(ref.qat_to_signed(np.array([[0x00]], np.uint8), 4), 2, 4).tolist() == [[-8, -8]]
    np.testing.assert_array_equal(ref.qat_to_signed(raw, 8), raw)


def test_select_path_matches_supports(ref):
    """BlockwiseLinear::supports (operators.cpp:1038-1059) and SymmetricPackedLinear::supports (:1185-1204)."""
    B, S, P = ref.PATH_BLOCKWISE, ref.PATH_SYMMETRIC, ref.PATH_PORTABLE
    assert ref.select_path(4, 128, 2048, 8192, False, 0) == B
    assert ref.select_path(4, 128, 2048, 255, False, 0) == P      # N < 256 without zeros
    assert ref.select_path(4, 128, 2048, 35, True, 0) == B        # zeros lift the N bound
    assert ref.select_path(4, 2048, 2048, 8192, False, 0) == P    # per-channel (g == K) without zeros
    assert ref.select_path(4, 16, 2048, 8192, True, 0) == P       # g < 32
    assert ref.select_path(4, 48, 2016, 8192, True, 0) == P       # g % 32 != 0
    assert ref.select_path(8, 48, 2016, 64, False, 0) == B        # 8-bit: g % 16 == 0, N >= 64
    assert ref.select_path(8, 32, 2048, 63, False, 0) == P
    assert ref.select_path(8, 32, 2048, 64, True, 0) == P         # 8-bit never takes zeros
    assert ref.select_path(2, 32, 2048, 8192, False, 0) == P      # no dynamic 2-bit
    assert ref.select_path(2, 32, 2048, 8192, False, 0.5) == S
    assert ref.select_path(4, 2, 4, 2, False, 0.25) == S
    assert ref.select_path(4, 128, 2048, 8192, True, 0.5) == P    # calibrated with zeros: portable


def test_dynamic_linear_closed_form(ref):
    """BlockwiseLinear closed form assembled correctly: equals, to fp32 rounding, the float64 dot of the dequantized
    activation codes and weights (catches a dropped zero term, a wrong sign or a transposed operand)."""
    rng = np.random.default_rng(7)
    M, K, N, g = 3, 256, 260, 32
    x = rng.standard_normal((M, K)).astype(f32)
    codes = rng.integers(-8, 8, (N, K))
    v = np.zeros((N, K // 2), np.uint8)
    v |= (codes[:, 0::2] & 15).astype(np.uint8)
    v |= ((codes[:, 1::2] & 15) << 4).astype(np.uint8)
    s = rng.uniform(0.002, 0.02, (N, K // g)).astype(np.float16)
    zp = rng.integers(0, 16, (N, K // g)).astype(np.uint8)
    for zeros in (None, "zp", "f32"):
        kw = {}
        z64 = np.zeros((N, K // g))
        if zeros == "zp":
            kw["zero_points"] = zp
            z64 = (8.0 - zp) * s.astype(np.float64)
        elif zeros == "f32":
            zf = rng.uniform(-0.1, 0.1, (N, K // g)).astype(f32)
            kw["zeros"] = zf
            z64 = zf.astype(np.float64)
        y, path = ref.packed_linear(x, v, s, 4, g, **kw)
        assert path == ref.PATH_BLOCKWISE
        q, a_s, _, _ = ref.quantize_dynamic(x, g, 4)
        xd = q.astype(np.float64) * np.repeat(a_s, g, axis=1)
        wd = codes * np.repeat(s.astype(np.float64), g, axis=1) + np.repeat(z64, g, axis=1)
        want = xd @ wd.T
        assert np.max(np.abs(y - want)) <= 1e-5 * np.max(np.abs(want))
    # 8-bit: asymmetric activations, x = (q - zp) * scale
    c8 = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s8 = rng.uniform(0.002, 0.02, (N, K // g)).astype(f32)
    y, path = ref.packed_linear(x, c8.view(np.uint8), s8, 8, g)
    assert path == ref.PATH_BLOCKWISE
    q, a_s, _, zpa = ref.quantize_dynamic(x, g, 8)
    xd = (q.astype(np.float64) - np.repeat(zpa, g, axis=1)) * np.repeat(a_s, g, axis=1)
    want = xd @ (c8.astype(np.float64) * np.repeat(s8, g, axis=1)).T
    assert np.max(np.abs(y - want)) <= 1e-5 * np.max(np.abs(want))


def _graph_test_operands(bits, m_rows):
    """tests/kidi/runtime/ynn/graph_test.cpp:120-135: INPUT_SIZE 128, INTERMEDIATE 2056, gate_up bytes
    (i * 11 + 7) & 0xFF, x = ((i * 5) % 19 - 9) / 16, per-channel scales (1 + i % 5) / 256."""
    K, I = 128, 2056
    per = 8 // bits
    x = ((np.arange(m_rows * K) * 5) % 19 - 9).astype(np.float32).reshape(m_rows, K) * np.float32(0.0625)
    gu = ((np.arange(2 * I * (K // per)) * 11 + 7) & 0xFF).astype(np.uint8).reshape(2 * I, K // per)
    s = (np.float32(0.00390625) * (1 + np.arange(2 * I) % 5).astype(np.float32)).reshape(2 * I, 1)
    return x, gu, s


def test_lowbit_parity_kat(ref):
    """tests/kidi/layers/precision_test.cpp:59-64, :87-92: LOWBIT_PARITY on x [0.15, -0.2], 8-bit weights
    [[2, -2], [1, 1]], scales [0.5, 0.25], g = 2, input and output scales 0.1 -> [0.4, 0]."""
    x = np.array([[0.15, -0.2]], np.float32)
    w = np.array([[2, 254], [1, 1]], np.uint8)
    s = np.array([[0.5], [0.25]], np.float32)
    y = ref.parity_linear(x, w, s, 8, 2, 0.1, 0.1)
    assert abs(y[0, 0] - 0.4) < 1e-5 and abs(y[0, 1]) < 1e-5


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("m_rows", [1, 17])
def test_lowbit_parity_matches_calibrated_path(ref, bits, m_rows):
    """graph_test.cpp:158-177: the calibrated SymmetricPackedLinear output equals LOWBIT_PARITY within 1e-5 (input
    scale 0.125, output scale 0.0625, g = K = 128)."""
    x, gu, s = _graph_test_operands(bits, m_rows)
    fast, path = ref.packed_linear(x, gu, s, bits, 128, 0.125, 0.0625)
    assert path == ref.PATH_SYMMETRIC
    parity = ref.parity_linear(x, gu, s, bits, 128, 0.125, 0.0625)
    assert np.max(np.abs(fast - parity)) <= 1e-5


def test_lowbit_parity_serial_fma_and_domain(ref):
    """The serial form: a float64 dot of grid-rounded x and c * s matches to the float32 rounding of the running FMA
    chain; non-positive scales are INVALID_ARGUMENT, a zero input or output scale UNSUPPORTED (parity_math.cpp:239-240,
    ops/context.cpp:919-929)."""
    rng = np.random.default_rng(3)
    K, N, g = 256, 64, 32
    codes = rng.integers(-8, 8, size=(N, K)).astype(np.int8)
    from tests.cases import pack_codes

    v = pack_codes(codes, 4)
    s = rng.uniform(0.01, 0.02, size=(N, K // g)).astype(np.float32)
    x = rng.standard_normal((3, K)).astype(np.float32)
    in_s, out_s = 0.05, 1e-4
    y = ref.parity_linear(x, v, s, 4, g, in_s, out_s)
    xr = np.clip(np.rint(x / np.float32(in_s)), -128, 127).astype(np.float64) * np.float32(in_s)
    w = codes.astype(np.float64) * np.repeat(s.astype(np.float64), g, axis=1)
    exact = np.clip(np.rint((xr @ w.T) / out_s), -128, 127) * out_s
    assert np.max(np.abs(y - exact)) <= out_s * 1.0001  # at most one output step where the chain rounds across
    bad = s.copy()
    bad[3, 1] = 0.0
    with pytest.raises(ValueError, match="INVALID_ARGUMENT"):
        ref.parity_linear(x, v, bad, 4, g, in_s, out_s)
    with pytest.raises(ValueError, match="UNSUPPORTED"):
        ref.parity_linear(x, v, s, 4, g, 0.0, out_s)
    with pytest.raises(ValueError, match="UNSUPPORTED"):
        ref.parity_linear(x, v, s, 4, g, in_s, 0.0)
