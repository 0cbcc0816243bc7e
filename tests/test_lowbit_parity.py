"""Kidi's LOWBIT_PARITY projection (runtime::parity::packed_linear, src/kidi/runtime/parity_math.cpp:226-291) on the
GPU through Context.set_precision("lowbit-parity") and kq_lowbit_parity_linear, against the CPU oracle: equal to the
last bit (both sum each output as one serial FMA chain in column order), the reference's KAT, its cross-check against
the calibrated projection, and its UNSUPPORTED / INVALID_ARGUMENT domain."""

import numpy as np
import pytest

from tests.cases import activations, pack_codes, weights
from tests.test_oracle_kat import _graph_test_operands

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd.ops import Context

    c = Context("cuda:0")
    c.set_precision("lowbit-parity")
    return c


def test_kat(ctx):
    """precision_test.cpp:87-92: [0.4, 0]."""
    x = torch.tensor([[0.15, -0.2]], dtype=torch.float32)
    w = torch.tensor([[2, 254], [1, 1]], dtype=torch.uint8)
    s = torch.tensor([[0.5], [0.25]], dtype=torch.float32)
    y = ctx.packed_linear(x, w, s, 8, 2, 0.1, 0.1).numpy()
    assert abs(y[0, 0] - 0.4) < 1e-5 and abs(y[0, 1]) < 1e-5


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("m_rows", [1, 17])
def test_graph_test_operands(ctx, ref, bits, m_rows):
    """graph_test.cpp:158-177 operands: equal to the oracle, and within 1e-5 of the calibrated PACKED_LINEAR path of
    this library (CHECKPOINT precision)."""
    from kidi_amd.ops import Context

    x, gu, s = _graph_test_operands(bits, m_rows)
    y = ctx.packed_linear(torch.from_numpy(x), torch.from_numpy(gu), torch.from_numpy(s), bits, 128, 0.125, 0.0625).numpy()
    np.testing.assert_array_equal(y, ref.parity_linear(x, gu, s, bits, 128, 0.125, 0.0625))
    fast = Context("cuda:0").packed_linear(torch.from_numpy(x), torch.from_numpy(gu), torch.from_numpy(s), bits, 128,
                                           0.125, 0.0625).numpy()
    assert np.max(np.abs(fast - y)) <= 1e-5


@pytest.mark.parametrize("bits,group,M,K,N", [(4, 32, 1, 512, 256), (4, 128, 3, 1024, 272), (8, 32, 8, 256, 128),
                                              (2, 64, 20, 512, 96), (4, 96, 9, 384, 64), (8, 16, 2, 64, 40)])
def test_random_operands_bit_exact(ctx, ref, bits, group, M, K, N):
    """Random codes, F32 scales and N(0,1) inputs, tiled and row-major weights, M below and above the reference's
    sgemm threshold (8): the GPU's serial FMA chain equals the oracle's to the last bit."""
    rng = np.random.default_rng(M * 131 + K + bits)
    values, scales, _, _ = weights(rng, N, K, bits, group, scale_dtype=np.float32)
    x = activations(rng, M, K, 0.001)
    in_s, out_s = 0.03, 0.002
    y = ctx.packed_linear(torch.from_numpy(x), torch.from_numpy(values), torch.from_numpy(scales), bits, group, in_s,
                          out_s).numpy()
    np.testing.assert_array_equal(y, ref.parity_linear(x, values, scales, bits, group, in_s, out_s))


def test_bound_zeros_not_applied(ctx, ref):
    """LOWBIT_PARITY does not pass the bound zero tensor (ops/context.cpp:917-932): the output ignores it."""
    rng = np.random.default_rng(7)
    values, scales, zp, _ = weights(rng, 64, 256, 4, 128, zero_points=True, scale_dtype=np.float32)
    x = activations(rng, 2, 256)
    v, s = torch.from_numpy(values), torch.from_numpy(scales)
    plain = ctx.packed_linear(torch.from_numpy(x), v, s, 4, 128, 0.05, 0.01).numpy()
    ctx.bind_packed_zero(s, torch.from_numpy((8.0 - zp.astype(np.float32)) * scales))
    bound = ctx.packed_linear(torch.from_numpy(x), v, s, 4, 128, 0.05, 0.01).numpy()
    np.testing.assert_array_equal(plain, bound)
    np.testing.assert_array_equal(plain, ref.parity_linear(x, values, scales, 4, 128, 0.05, 0.01))


def test_domain(ctx):
    """UNSUPPORTED outside the reference's domain, INVALID_ARGUMENT for bad scales, with the reference's messages."""
    from kidi_amd.ops import Context, Failure

    rng = np.random.default_rng(1)
    codes = rng.integers(-8, 8, size=(32, 64)).astype(np.int8)
    w = torch.from_numpy(pack_codes(codes, 4))
    s = torch.full((32, 2), 0.01, dtype=torch.float32)
    x = torch.randn((2, 64), dtype=torch.float32)
    cases = [
        (dict(input=x.to(torch.bfloat16)), "UNSUPPORTED"),          # input must be F32
        (dict(scales=s.to(torch.float16)), "UNSUPPORTED"),          # scales must be F32
        (dict(input_scale=0.0), "UNSUPPORTED"),                     # calibrated only
        (dict(output_scale=0.0), "UNSUPPORTED"),
        (dict(input_scale=-1.0), "INVALID_ARGUMENT"),
        (dict(group=48), "UNSUPPORTED"),                            # width % g != 0
        (dict(scales=torch.zeros((32, 2), dtype=torch.float32)), "INVALID_ARGUMENT"),
    ]
    for change, code in cases:
        a = dict(input=x, scales=s, input_scale=0.05, output_scale=0.01, group=32)
        a.update(change)
        with pytest.raises(Failure) as e:
            ctx.packed_linear(a["input"], w, a["scales"], 4, a["group"], a["input_scale"], a["output_scale"])
        assert e.value.code == code, change
    with pytest.raises(Failure) as e:
        Context("cuda:0").set_precision("fp32")
    assert e.value.code == "UNSUPPORTED"
