"""Packed checkpoint ingestion and the persisted gfx950 layout (kidi_amd/checkpoint.py, kq_weight_export/import).

Fixture: tests/golden/gemma4_qat/ holds the data files of the reference's own QAT fixture (tests/data/gemma4-qat:
model.safetensors and config.json, a random four-layer Gemma 4 with mixed Q2/Q4/Q8 per-channel projections and static
activation calibration). CPU: per-module bit rules (gemma4.cpp:30-43), the QAT XOR conversion against the oracle and
its closed form (offset nibble - 2^(b-1) = two's complement nibble), the layout cache's header validation, atomic
store and switches. GPU: every projection of the fixture through the loader against the oracle on the converted
codes; export/import and cache round trips bit-identical; malformed blobs rejected."""

import json
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "gemma4_qat", "model.safetensors")
CONFIG = json.load(open(os.path.join(HERE, "golden", "gemma4_qat", "config.json")))


def _ck():
    try:
        from kidi_amd import checkpoint
    except ImportError as e:  # library not built
        pytest.skip(str(e))
    return checkpoint


def test_quant_bits_rules():
    ck = _ck()
    L = "model.language_model."
    assert ck.quant_bits(CONFIG, "lm_head") == 2                      # "^lm_head$"
    assert ck.quant_bits(CONFIG, L + "embed_tokens") == 2             # "language_model\.embed_tokens$"
    assert ck.quant_bits(CONFIG, L + "embed_tokens_per_layer") == 4
    assert ck.quant_bits(CONFIG, L + "layers.0.mlp.gate_proj") == 4   # default num_bits
    assert ck.quant_bits(CONFIG, L + "layers.3.mlp.down_proj") == 2   # "layers\.[23]\.mlp\."
    assert ck.quant_bits(CONFIG, L + "layers.1.per_layer_input_gate") == 8
    assert ck.quant_bits(CONFIG, L + "per_layer_model_projection") == 0  # modules_to_not_convert
    assert ck.quant_bits({}, "lm_head") == 0
    bad = {"quantization_config": {"num_bits": 3}}
    with pytest.raises(ck.Failure) as e:
        ck.quant_bits(bad, "x")
    assert e.value.code == "UNSUPPORTED"


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_qat_conversion(ref, bits):
    ck = _ck()
    rng = np.random.default_rng(bits)
    v = rng.integers(0, 256, size=(5, 12), dtype=np.uint8)
    conv = ck.qat_signed(v, bits)
    np.testing.assert_array_equal(conv, ref.qat_to_signed(v, bits))
    if bits < 8:  # offset code u (stored) is c + 2^(b-1): unsigned fields minus the offset = signed fields
        per, mask, half = 8 // bits, (1 << bits) - 1, 1 << (bits - 1)
        for i in range(per):
            u = (v.astype(np.int64) >> (i * bits)) & mask
            c = (conv.astype(np.int64) >> (i * bits)) & mask
            np.testing.assert_array_equal(u - half, (c ^ half) - half)


def _cache_spec(n=0):
    return (4, 128, 64 + n, 256, 0x1234 + n)


def test_layout_cache_store_load_and_invalidation(tmp_path, monkeypatch):
    ck = _ck()
    monkeypatch.delenv("KQ_LAYOUT_CACHE", raising=False)
    src = tmp_path / "model.safetensors"
    src.write_bytes(b"x" * 100)
    cache = ck.LayoutCache(tmp_path / "cache", src)
    assert cache.enabled and cache.writable
    payload = bytes(range(256)) * 3
    cache.store(_cache_spec(), payload)
    assert cache.load(_cache_spec()) == payload and cache.hits == 1
    assert cache.load(_cache_spec(1)) is None  # another spec
    files = os.listdir(tmp_path / "cache")
    assert len(files) == 1 and not any(".tmp." in f for f in files)
    # a truncated or corrupted file is a miss
    path = os.path.join(tmp_path / "cache", files[0])
    data = open(path, "rb").read()
    open(path, "wb").write(data[:-1])
    assert cache.load(_cache_spec()) is None
    open(path, "wb").write(b"NOTMAGIC" + data[8:])
    assert cache.load(_cache_spec()) is None
    open(path, "wb").write(data)
    assert cache.load(_cache_spec()) == payload
    # the source file changed: a new cache object rejects the old entry
    src.write_bytes(b"y" * 101)
    assert ck.LayoutCache(tmp_path / "cache", src).load(_cache_spec()) is None


def test_layout_cache_switches(tmp_path, monkeypatch):
    ck = _ck()
    src = tmp_path / "m.safetensors"
    src.write_bytes(b"z")
    for off in ("0", "off", "false", ""):
        monkeypatch.setenv("KQ_LAYOUT_CACHE", off)
        assert not ck.LayoutCache(tmp_path / "c", src).enabled
    monkeypatch.setenv("KQ_LAYOUT_CACHE", str(tmp_path / "elsewhere"))
    c = ck.LayoutCache(None, src)
    assert c.writable and c.directory == str(tmp_path / "elsewhere")
    monkeypatch.delenv("KQ_LAYOUT_CACHE")
    assert not ck.LayoutCache(None, src).enabled  # no directory configured
    assert not ck.LayoutCache(tmp_path / "c", tmp_path / "missing").enabled  # no source file
    ro = tmp_path / "ro"
    ro.mkdir()
    os.chmod(ro, 0o555)
    try:
        c = ck.LayoutCache(ro, src)
        assert c.readable and (not c.writable or os.geteuid() == 0)  # root ignores permission bits
    finally:
        os.chmod(ro, 0o755)


# ---- GPU --------------------------------------------------------------------------------------------------------

@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    _native.load()
    return torch.device("cuda:0")


def _fixture_modules():
    from safetensors import safe_open

    with safe_open(FIXTURE, framework="np") as f:
        return {k[:-len(".weight")]: (f.get_tensor(k), f.get_tensor(k + "_scale")) for k in f.keys()
                if k.endswith(".weight") and k + "_scale" in f.keys() and f.get_tensor(k).dtype in (np.uint8, np.int8)}


@pytest.mark.gpu
def test_qat_fixture_projections_gpu(dev, ref, tmp_path, monkeypatch):
    ck = _ck()
    monkeypatch.delenv("KQ_LAYOUT_CACHE", raising=False)
    print("qat fixture projections", flush=True)
    linears = ck.load_packed_linears(FIXTURE, device=dev)
    raw = _fixture_modules()
    assert set(linears) == set(raw) and len(linears) >= 20
    rng = np.random.default_rng(7)
    for name, lin in sorted(linears.items()):
        values, scales = raw[name]
        bits = ck.quant_bits(CONFIG, name)
        assert (lin.bits, lin.group_size) == (bits, values.shape[1] * (8 // bits) // scales.shape[1])
        codes = ck.qat_signed(values.view(np.uint8), bits) if values.dtype == np.uint8 else values.view(np.uint8)
        K = values.shape[1] * (8 // bits)
        x = (rng.standard_normal((3, K)) * max(lin.input_scale, 0.05) * 40).astype(np.float32)
        y_ref, _ = ref.packed_linear(x, codes, scales, bits, lin.group_size, lin.input_scale, lin.output_scale)
        y = lin(torch.from_numpy(x).to(dev)).cpu().numpy()
        if lin.output_scale > 0:  # calibrated outputs: steps of out_s, exact but for rounding-boundary ties
            assert np.max(np.abs(y - y_ref)) <= lin.output_scale * (1 + 1e-6), name
        else:
            assert np.max(np.abs(y - y_ref)) <= 2e-3 * max(np.max(np.abs(y_ref)), 1e-30), name


@pytest.mark.gpu
def test_export_import_and_cache_gpu(dev, tmp_path, monkeypatch):
    ck = _ck()
    from kidi_amd.ops import DeviceWeight

    monkeypatch.delenv("KQ_LAYOUT_CACHE", raising=False)
    print("layout export/import and cache", flush=True)
    first = ck.load_packed_linears(FIXTURE, device=dev, cache_dir=tmp_path / "cache")
    c1 = ck.load_packed_linears.last_cache
    assert c1.stores == len(first) and c1.hits == 0
    second = ck.load_packed_linears(FIXTURE, device=dev, cache_dir=tmp_path / "cache")
    c2 = ck.load_packed_linears.last_cache
    assert c2.hits == len(second) and c2.stores == 0
    rng = np.random.default_rng(3)
    for name in first:
        a, b = first[name], second[name]
        x = torch.from_numpy(rng.standard_normal((4, a.weight.cols)).astype(np.float32)).to(dev)
        assert torch.equal(a(x), b(x)), name
        blob = a.weight.export()
        assert DeviceWeight.import_blob(blob).export() == blob
    # a larger tiled weight with zero points survives the round trip too
    from tests.cases import weights

    v, s, zp, _ = weights(np.random.default_rng(1), 256, 1024, 4, 128, zero_points=True)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    w = DeviceWeight(t(v), t(s), 4, 128, t(zp))
    w2 = DeviceWeight.import_blob(w.export())
    x = torch.randn((3, 1024), device=dev)
    assert torch.equal(w.linear(x), w2.linear(x))
    assert (w2.bits, w2.group_size, w2.rows, w2.cols, w2.has_zeros) == (4, 128, 256, 1024, True)


@pytest.mark.gpu
def test_import_rejects_malformed_blob_gpu(dev):
    from kidi_amd.ops import DeviceWeight, Failure
    from tests.cases import weights

    v, s, _, _ = weights(np.random.default_rng(2), 32, 256, 4, 128)
    w = DeviceWeight(torch.from_numpy(v).to(dev), torch.from_numpy(s).to(dev), 4, 128)
    blob = w.export()
    for bad in (blob[:-1], b"XXXXXXXX" + blob[8:], blob[:20]):
        with pytest.raises(Failure) as e:
            DeviceWeight.import_blob(bad)
        assert e.value.code == "INVALID_MANIFEST"
