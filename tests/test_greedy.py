"""Greedy token selection: GREEDY_TOKEN (GreedyToken, runtime/ynn/operators.cpp:117-178; Context::greedy_token) and the
output head fused with it (kq_packed_linear_greedy).

Rule, pinned by the reference KAT tests/kidi/layers/eager_test.cpp:231-252: the first index of the row maximum (ties
to the lower index; -0 equals 0), -1 when the row holds a NaN or an infinity; a scalar input is INVALID_ARGUMENT.
CPU: the oracle against the KAT and a scalar loop. GPU: kq_greedy_token against the KAT and the oracle on tie-heavy
rows; the fused head returns the oracle's selection over its own logits (kept or not) at decode and prefill sizes."""

import numpy as np
import pytest

from tests.cases import activations, weights

torch = pytest.importorskip("torch")


def kat_rows(width: int) -> np.ndarray:
    """eager_test.cpp:232-240."""
    s = np.full(6 * width, -2.0, np.float32)
    s[1] = s[width - 1] = 4.0
    s[width:2 * width] = -np.inf
    s[2 * width + width - 1] = np.nan
    s[3 * width + 1] = np.inf
    s[6 * width - 1] = 3.0
    return s.reshape(6, width)


def kat_expected(width: int):
    return [1, -1, -1, -1, 0, width - 1]


def scalar_greedy(row) -> int:
    """The reference's chunk combination (operators.cpp:155-167) as one loop: best = -inf, winner = -1, strict >."""
    best, winner, invalid = -np.inf, -1, False
    for i, v in enumerate(row):
        if not np.isfinite(v):
            invalid = True
        elif v > best:
            best, winner = v, i
    return -1 if invalid else winner


@pytest.mark.parametrize("width", [7, 1027, 262144])
def test_oracle_kat(ref, width):
    assert list(ref.greedy_token(kat_rows(width))) == kat_expected(width)


def test_oracle_finite_ties_and_scalar_loop(ref):
    assert ref.greedy_token(np.array([[-3.0, 0.0, -0.0]], np.float32) * 2)[0] == 1  # eager_test.cpp:246-250
    rng = np.random.default_rng(5)
    rows = rng.integers(-3, 4, size=(40, 257)).astype(np.float32)  # many ties
    rows[3, 100] = np.nan
    rows[7, 0] = -np.inf
    np.testing.assert_array_equal(ref.greedy_token(rows), [scalar_greedy(r) for r in rows])


def test_context_rejects_scalar():
    try:
        from kidi_amd.ops import Context, Failure
    except ImportError as e:  # library not built
        pytest.skip(str(e))
    with pytest.raises(Failure) as e:
        Context("cpu").greedy_token(torch.zeros(()))
    assert e.value.code == "INVALID_ARGUMENT"


# ---- GPU --------------------------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    _native.load()
    return torch.device("cuda:0")


@pytest.mark.gpu
@pytest.mark.parametrize("width", [7, 1027, 262144])
def test_greedy_token_kat_gpu(dev, width):
    from kidi_amd.ops import Context

    print(f"greedy KAT width={width}", flush=True)
    ctx = Context(dev)
    t = ctx.greedy_token(torch.from_numpy(kat_rows(width)).to(dev))
    assert t.cpu().tolist() == kat_expected(width)
    finite = torch.tensor([[-3.0, 0.0, -0.0]], device=dev)
    assert ctx.greedy_token(finite + finite).cpu().tolist() == [1]


@pytest.mark.gpu
@pytest.mark.parametrize("rows,width", [(1, 1), (3, 4096), (5, 4097), (9, 3 * 4096 + 1), (2, 262144)])
def test_greedy_token_matches_oracle_gpu(dev, ref, rows, width):
    from kidi_amd.ops import greedy_token

    rng = np.random.default_rng(rows * 1000 + width)
    x = rng.integers(-5, 6, size=(rows, width)).astype(np.float32)  # ties in every row
    if rows > 2:
        x[1, width // 2] = np.nan
        x[2, -1] = np.inf
    t = greedy_token(torch.from_numpy(x).to(dev))
    np.testing.assert_array_equal(t.cpu().numpy(), ref.greedy_token(x))


def _head(dev, N, K=2048, seed=3):
    """int8 g = 32 symmetric output head (BASELINE config 5's head at a reduced N)."""
    from kidi_amd.ops import DeviceWeight

    rng = np.random.default_rng(seed)
    v, s, _, _ = weights(rng, N, K, 8, 32, code_range=(-127, 127))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    return DeviceWeight(t(v), t(s), 8, 32), (v, s)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 5, 8, 20])
def test_greedy_head_gpu(dev, ref, M):
    print(f"greedy head M={M}", flush=True)
    N, K = 32768, 2048
    dw, (v, s) = _head(dev, N, K)
    x = torch.from_numpy(activations(np.random.default_rng(M), M, K)).to(dev).to(torch.bfloat16)
    tokens, logits = dw.linear_greedy(x, keep_logits=True)
    lg = logits.cpu().numpy()
    np.testing.assert_array_equal(tokens.cpu().numpy(), ref.greedy_token(lg))  # selection over its own logits
    np.testing.assert_array_equal(lg, dw.linear(x).cpu().numpy())  # the same logits as the plain projection
    tokens2, none = dw.linear_greedy(x)  # logits not stored
    assert none is None
    np.testing.assert_array_equal(tokens2.cpu().numpy(), tokens.cpu().numpy())
    # against the oracle's logits: the chosen logit is the oracle maximum within the projection tolerance
    y_ref, _ = ref.packed_linear(x.float().cpu().numpy(), v, s, 8, 32, threads=8)
    pick = y_ref[np.arange(M), tokens.cpu().numpy()]
    assert np.all(y_ref.max(axis=1) - pick <= 2e-3 * np.max(np.abs(y_ref)))


@pytest.mark.gpu
def test_greedy_head_non_finite_gpu(dev, ref):
    print("greedy head non-finite", flush=True)
    N, K = 4096, 2048
    dw, _ = _head(dev, N, K, seed=9)
    x = torch.from_numpy(activations(np.random.default_rng(9), 3, K)).to(dev)
    x[1, 17] = float("inf")
    tokens, logits = dw.linear_greedy(x, keep_logits=True)
    lg = logits.cpu().numpy()
    assert not np.all(np.isfinite(lg[1]))
    np.testing.assert_array_equal(tokens.cpu().numpy(), ref.greedy_token(lg))
    assert tokens[1].item() == -1
    tokens2, _ = dw.linear_greedy(x)
    np.testing.assert_array_equal(tokens2.cpu().numpy(), tokens.cpu().numpy())
