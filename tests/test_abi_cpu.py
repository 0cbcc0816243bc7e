"""C ABI checks that need no GPU: the library loads, exports every declared symbol, rejects invalid descriptors
with Kidi's error codes, selects operators like the reference, and its host-side tile layout round-trips."""

import ctypes
import os
import re

import numpy as np
import pytest

from tests.cases import pack_codes

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def native():
    from kidi_amd import _native

    _native.load()
    return _native


def test_exports_every_declared_symbol(native):
    header = open(os.path.join(ROOT, "include", "kq.h")).read()
    declared = set(re.findall(r"\b(kq_[a-z_]+)\s*\(", header))
    assert declared == set(native.EXPORTS)
    lib = native.load()
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.kq_arch() == b"gfx950"
    assert lib.kq_version() >= 1


def test_library_resolves_every_symbol_at_load(native):
    """The library binds with RTLD_NOW (a kernel whose launch stub the host pass dropped shows up here as an
    undefined symbol, not as a lazy-binding failure on the GPU box)."""
    import subprocess
    import sys

    code = f"import ctypes, os; ctypes.CDLL({native.LIB_PATH!r}, mode=os.RTLD_NOW)"
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]


def test_select_path_matches_oracle(native, ref):
    lib = native.load()
    for bits in (2, 4, 8):
        for group in (2, 4, 16, 32, 48, 64, 96, 128, 2048):
            for K in (256, 2048, 2016, 4):
                for N in (3, 63, 64, 255, 256, 8192):
                    for has_zero in (0, 1):
                        for scale in (0.0, 0.25):
                            if group <= 0 or K % group or group % (8 // bits):
                                continue
                            assert lib.kq_select_path(bits, group, K, N, has_zero, scale) == \
                                ref.select_path(bits, group, K, N, bool(has_zero), scale)


def _desc(native, values, scales, bits, group, zeros=None, zdt=None):
    d = native.PackDesc()
    d.bits, d.group_size = bits, group
    d.rows = values.shape[0]
    d.cols = values.shape[1] * (8 // bits) if bits in (2, 4, 8) else 0
    d.values = values.ctypes.data
    d.values_dtype = native.KQ_U8
    d.scales = scales.ctypes.data
    d.scales_dtype = native.KQ_F32 if scales.dtype == np.float32 else native.KQ_F16
    d.zeros = zeros.ctypes.data if zeros is not None else None
    d.zeros_dtype = zdt if zeros is not None else native.KQ_NONE
    d.memory = native.KQ_HOST
    return d


@pytest.mark.parametrize("bad", ["bits", "group", "shape", "dtype", "zp"])
def test_pack_rejects_invalid(native, bad):
    lib = native.load()
    v = np.zeros((4, 32), np.uint8)
    s = np.ones((4, 2), np.float32)
    z = None
    bits, group = 4, 32
    if bad == "bits":
        bits = 3
    elif bad == "group":
        group = 24  # K=64 not divisible
    elif bad == "shape":
        group = 0
    elif bad == "dtype":
        s = np.ones((4, 2), np.float64)
    elif bad == "zp":
        z = np.full((4, 2), 16, np.uint8)
    d = _desc(native, v, s, bits, group, z, native.KQ_ZP_U8)
    if bad == "dtype":
        d.scales_dtype = native.KQ_BF16
    h = ctypes.c_void_p()
    status = lib.kq_weight_pack(ctypes.byref(d), None, ctypes.byref(h))
    assert status == native.KQ_INVALID_ARGUMENT
    assert lib.kq_last_error()
    assert not h.value


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("shape", [(16, 512), (35, 256), (3, 64), (1, 8)])
def test_layout_roundtrip(native, ref, bits, shape):
    """Encoding Kidi's layout into tiles and decoding it again gives Kidi's signed codes (oracle unpack)."""
    lib = native.load()
    N, K = shape
    if K % (8 // bits):
        pytest.skip("width")
    rng = np.random.default_rng(bits * 1000 + N)
    codes = rng.integers(-(1 << (bits - 1)), 1 << (bits - 1), size=(N, K)).astype(np.int8)
    values = pack_codes(codes, bits)
    np.testing.assert_array_equal(ref.unpack_codes(values, K, bits), codes)
    nbytes = lib.kq_layout_bytes(bits, 32, N, K)
    assert nbytes % 1024 == 0 and nbytes >= N * K * bits // 8
    tiles = np.zeros(nbytes, np.uint8)
    assert lib.kq_layout_encode_host(bits, N, K, values.ctypes.data, tiles.ctypes.data) == 0
    back = np.zeros((N, K), np.int8)
    assert lib.kq_layout_decode_host(bits, N, K, tiles.ctypes.data, back.ctypes.data) == 0
    np.testing.assert_array_equal(back, codes)


def test_layout_lane_order(native):
    """The documented slot order: 4-bit tile 0, lane l = row + 16 L; dword 2j+h, low nibble of byte r = column
    64j + 32h + 8L + r (stored as c + 8), high nibble = column 64j + 32h + 8L + 4 + r."""
    lib = native.load()
    N, K, bits = 16, 128, 4
    codes = np.zeros((N, K), np.int64)
    row, col = 5, 64 + 32 + 8 * 2 + 4 + 1  # j=1, h=1, L=2, i=5 -> high nibble of byte r=1 of dword 3
    codes[row, col] = 3
    tiles = np.zeros(lib.kq_layout_bytes(bits, 32, N, K), np.uint8)
    lib.kq_layout_encode_host(bits, N, K, pack_codes(codes, bits).ctypes.data, tiles.ctypes.data)
    lane = row + 16 * 2
    slot = tiles[16 * lane:16 * lane + 16]
    expected = np.full(16, 0x88, np.uint8)  # every code 0 -> nibble 8
    expected[4 * 3 + 1] = 0x08 | ((3 + 8) << 4)
    np.testing.assert_array_equal(slot, expected)


def test_oracle_is_not_imported_by_product():
    """The product package neither imports nor links the CPU oracle."""
    pkg = os.path.join(ROOT, "kidi_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".hpp", ".h")):
                text = open(os.path.join(dirpath, f)).read()
                for needle in ("from oracle", "import oracle", "kq_ref", "libkq_ref"):
                    assert needle not in text, (f, needle)
