"""GELU_MULTIPLY / SILU_MULTIPLY, the slice form of the gated feed-forward (Context::gelu_multiply / silu_multiply,
ops/context.cpp:944-957; layers/gemma4.cpp:213-225): on the two halves of a gate/up projection they equal the fused
gating bit for bit (same expressions), and the oracle's GELU-tanh / SiLU gates within 1e-5 of max|ref|; odd counts,
unaligned buffers, host tensors and the reference's INVALID_ARGUMENT messages."""

import numpy as np
import pytest

from tests.cases import activations, weights

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ctx():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd.ops import Context

    return Context("cuda:0")


def close(y, ref, tol=1e-5):
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    assert float(np.max(np.abs(y - ref))) <= tol * scale


@pytest.mark.parametrize("M", [1, 20])
def test_gelu_multiply_equals_fused_gating(ctx, ref, M):
    from kidi_amd.ops import DeviceWeight

    rng = np.random.default_rng(300 + M)
    I, K = 1024, 512
    values, scales, zp, _ = weights(rng, 2 * I, K, 4, 128, zero_points=True)
    dw = DeviceWeight(*(torch.from_numpy(a).cuda() for a in (values, scales)), 4, 128, torch.from_numpy(zp).cuda())
    x = torch.from_numpy(activations(rng, M, K)).cuda()
    y = dw.linear(x)
    fused = dw.linear(x, gelu_gate=True)
    h = ctx.gelu_multiply(y[:, :I].contiguous(), y[:, I:].contiguous())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(h.cpu().numpy(), fused.cpu().numpy())
    close(h.cpu().numpy(), ref.gelu_gate(y.cpu().numpy()))


@pytest.mark.parametrize("silu", [False, True])
@pytest.mark.parametrize("n", [1, 7, 4096, 100003])
def test_against_oracle(ctx, ref, silu, n):
    rng = np.random.default_rng(n + silu)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = rng.standard_normal(n).astype(np.float32)
    fn = ctx.silu_multiply if silu else ctx.gelu_multiply
    h = fn(torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()).cpu().numpy()
    gate = ref.silu_gate if silu else ref.gelu_gate
    close(h, gate(np.concatenate([g, u])[None, :])[0])


def test_unaligned_and_host(ctx):
    rng = np.random.default_rng(9)
    base = torch.from_numpy(rng.standard_normal(2 * 1001 + 1).astype(np.float32)).cuda()
    g, u = base[1:1002], base[1002:]  # 4-byte aligned views: the scalar path
    aligned = ctx.gelu_multiply(g.clone(), u.clone())
    np.testing.assert_array_equal(ctx.gelu_multiply(g, u).cpu().numpy(), aligned.cpu().numpy())
    hg, hu = g.cpu(), u.cpu()
    on_host = ctx.silu_multiply(hg, hu)
    assert not on_host.is_cuda
    np.testing.assert_array_equal(on_host.numpy(), ctx.silu_multiply(g.clone(), u.clone()).cpu().numpy())


def test_invalid_arguments(ctx):
    from kidi_amd.ops import Failure

    a = torch.zeros((2, 8), device="cuda:0")
    for g, v, silu in [(a, torch.zeros((2, 9), device="cuda:0"), False), (a.half(), a.half(), True),
                       (a, a.to(torch.bfloat16), False)]:
        with pytest.raises(Failure) as e:
            (ctx.silu_multiply if silu else ctx.gelu_multiply)(g, v)
        assert e.value.code == "INVALID_ARGUMENT"
        assert str(e.value).endswith(("SiLU" if silu else "GELU") + " multiplication requires matching floating tensors")
