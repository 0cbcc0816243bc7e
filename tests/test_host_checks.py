"""Host-side checks of the C ABI that run before any device call (no GPU needed): persisted-blob validation in
kq_weight_import, the kernel route a call would take (kq_debug_route_shape), and the absence of environment
switches in the shipped launch plans."""

import ctypes
import os
import re
import struct

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# BlobHeader of kq_api.cpp: magic, version, bits, group, rows, cols, tiled, scale_type, zero_mode, zero_type,
# offsets of tiles, scales, zero_points, zeros, code_sums (-1 when absent), image bytes.
HEADER = struct.Struct("<8sIii4xqqiiiiqqqqqQ")
MAGIC, VERSION = b"KQGFX950", 1
KQ_INVALID_MANIFEST = 3


@pytest.fixture(scope="module")
def lib():
    from kidi_amd import _native

    return _native.load()


def align(v):
    return (v + 255) // 256 * 256


def layout(bits, group, rows, cols, scale_f16, zero_mode, zero_f16=False):
    """The image this build lays out for a tiled weight: 1 KiB tiles of 16 rows x 512/bits columns, then scales,
    zero-point nibbles, additive zeros and (8-bit) code sums, each [n_tiles][groups][16] and 256-byte aligned."""
    kt = 512 // bits
    n_tiles, k_tiles = -(-rows // 16), -(-cols // kt)
    groups_p = k_tiles * kt // group
    meta = n_tiles * groups_p * 16
    off = align(n_tiles * k_tiles * 1024)
    scales = off
    off = align(off + meta * (2 if scale_f16 else 4))
    zp = zeros = sums = -1
    if zero_mode == 1:
        zp, off = off, align(off + meta // 2)
    if zero_mode == 2:
        zeros, off = off, align(off + meta * (2 if zero_f16 else 4))
    if bits == 8:
        sums, off = off, align(off + meta * 4)
    return 0, scales, zp, zeros, sums, off


def blob(base=None, **override):
    """Header + image of a weight described by `base` (geometry and modes), with `override` applied to the header
    fields afterwards (so an override leaves the offsets and size of the base layout in place)."""
    b = dict(bits=4, group=128, rows=32, cols=256, tiled=1, scale_f16=1, zero_mode=1, zero_f16=0)
    b.update(base or {})
    bits, group, rows, cols, tiled = b["bits"], b["group"], b["rows"], b["cols"], b["tiled"]
    scale_f16, zero_mode, zero_f16 = b["scale_f16"], b["zero_mode"], b["zero_f16"]
    tiles, scales, zp, zeros, sums, nbytes = layout(bits, group, rows, cols, scale_f16, zero_mode, zero_f16)
    fields = dict(magic=MAGIC, version=VERSION, bits=bits, group=group, rows=rows, cols=cols, tiled=tiled,
                  scale_type=scale_f16, zero_mode=zero_mode, zero_type=zero_f16, tiles=tiles, scales=scales,
                  zero_points=zp, zeros=zeros, code_sums=sums, bytes=nbytes)
    fields.update(override)
    image_bytes = override.get("image_bytes", fields["bytes"])
    fields.pop("image_bytes", None)
    head = HEADER.pack(*[fields[k] for k in ("magic", "version", "bits", "group", "rows", "cols", "tiled", "scale_type",
                                             "zero_mode", "zero_type", "tiles", "scales", "zero_points", "zeros",
                                             "code_sums", "bytes")])
    return head + bytes(image_bytes)


def import_status(lib, data):
    buf = ctypes.create_string_buffer(data, len(data))
    out = ctypes.c_void_p()
    st = lib.kq_weight_import(buf, len(data), None, ctypes.byref(out))
    assert not out.value
    return st, lib.kq_last_error().decode()


def test_header_size_matches_library():
    assert HEADER.size == 104


def test_valid_blob_passes_validation(lib):
    """A well-formed header gets past every manifest check: without a GPU the first device call then fails with
    RUNTIME, never INVALID_MANIFEST."""
    for kw in ({}, dict(zero_mode=0), dict(zero_mode=2, zero_f16=1), dict(bits=8, group=32, zero_mode=0),
               dict(scale_f16=0, rows=48, cols=512)):
        st, msg = import_status(lib, blob(kw))
        assert st != KQ_INVALID_MANIFEST, (kw, msg)


@pytest.mark.parametrize("case", [
    dict(rows=64),                          # enlarged rows: offsets and size no longer match
    dict(cols=512),                         # enlarged cols
    dict(zero_points=-1),                   # ZERO_POINT weight without its zero points
    dict(zero_mode=2),                      # float zeros claimed, none present
    dict(zero_mode=7),                      # mode out of range
    dict(scale_type=3),                     # scale type out of range
    dict(zero_type=5),                      # zero type out of range
    dict(tiled=0),                          # a g = 128 weight is always tiled
    dict(group=96, tiled=1),                # g = 96 cannot be tiled
    dict(bits=8, group=32, zero_mode=0),    # an 8-bit tiled image needs code sums the 4-bit layout lacks
    dict(scales=256),                       # shifted offset
    dict(bytes=4096, image_bytes=4096),     # image shorter than the layout, header and blob consistent
    dict(image_bytes=100),                  # blob shorter than the header's image size
    dict(version=2),
    dict(magic=b"KQGFX942"),
    dict(group=100),                        # K % g != 0
    dict(bits=3),
])
def test_malformed_blob_rejected_before_device(lib, case):
    st, msg = import_status(lib, blob(**case))
    assert st == KQ_INVALID_MANIFEST, (case, msg)


def test_truncated_blob(lib):
    st, _ = import_status(lib, blob()[:50])
    assert st == KQ_INVALID_MANIFEST


# kq_debug_route values
NONE, DECODE, SKINNY, GEMM_I4, GEMM_I4G, GEMV, GEMM, ROWMAJOR, PORTABLE, GEMM8, GEMM8W = range(11)
F32, BF16 = 0, 2


def route(lib, bits, group, rows, cols, zero_mode, m, x=BF16, in_s=0.0, gelu=0, f16=1):
    return lib.kq_debug_route_shape(bits, group, rows, cols, zero_mode, f16, m, x, in_s, gelu)


def test_routes_of_baseline_shapes(lib):
    assert route(lib, 4, 128, 8192, 2048, 1, 1) == DECODE          # configs[1]
    assert route(lib, 4, 128, 2048, 8192, 1, 4) == DECODE
    assert route(lib, 4, 32, 8192, 2048, 0, 1) == DECODE           # configs[0]
    assert route(lib, 4, 128, 8192, 2048, 1, 2048) == GEMM8        # configs[2]
    assert route(lib, 4, 128, 8192, 2048, 1, 512) == GEMM8
    assert route(lib, 4, 32, 2560, 2048, 0, 2048) == GEMM8W        # configs[3] fused QKV (128 x 160 tiles)
    assert route(lib, 4, 128, 16384, 2048, 1, 2048, gelu=1) == GEMM8
    assert route(lib, 4, 128, 2048, 8192, 1, 2048) == GEMM8        # configs[3] down
    assert route(lib, 4, 128, 8192, 2048, 2, 2048) == GEMM8        # additive float zeros
    assert route(lib, 4, 128, 8192, 2048, 0, 2048, in_s=0.05) == GEMM8  # calibrated
    assert route(lib, 2, 32, 8192, 2048, 0, 1, in_s=0.03) == DECODE  # configs[4]
    assert route(lib, 8, 32, 262144, 2048, 0, 8) == DECODE
    assert route(lib, 4, 128, 8192, 2048, 1, 0) == NONE


def test_routes_of_other_shapes(lib):
    assert route(lib, 4, 64, 2560, 2048, 1, 300) == GEMM8          # g = 64 prefill
    assert route(lib, 4, 32, 2560, 2048, 2, 300) == GEMM8          # g = 32 with additive float zeros
    # g = 32 in 128 x 160 tiles only where 256 x 128 tiles leave CUs idle and the wide tiles fill 192-256 of them
    assert route(lib, 4, 32, 2560, 2048, 0, 1536) == GEMM8W        # 120 -> 192 tiles
    assert route(lib, 4, 32, 2560, 2048, 0, 1408) == GEMM8         # 11 x 16 = 176 wide tiles: fewer than 192
    assert route(lib, 4, 32, 2560, 2048, 0, 2049) == GEMM8         # 17 x 16 = 272 wide tiles: more than the CUs
    assert route(lib, 4, 32, 2560, 2048, 0, 3072) == GEMM8         # 240 tiles in one round against 384 in two
    assert route(lib, 4, 32, 2560, 2048, 0, 4096) == GEMM8W        # 2 rounds of 512 against 2 of 320 (one a quarter full)
    assert route(lib, 4, 32, 2560, 2048, 0, 6144) == GEMM8         # 3 rounds of 768 against 2 of 480
    assert route(lib, 4, 32, 2560, 2048, 2, 2048) == GEMM8         # additive float zeros stay on 256 x 128
    assert route(lib, 4, 32, 8192, 2048, 0, 2048) == GEMM8         # 512 tiles of 256 x 128 already fill the CUs
    assert route(lib, 4, 32, 2562, 2048, 0, 300) == GEMM_I4G       # N % 4 != 0: no 16-byte output stores
    assert route(lib, 4, 32, 2560, 2048, 0, 300, gelu=1) == GEMM   # gate/up pairing is for g = 128 weights
    assert route(lib, 4, 128, 256, 512, 1, 12) == SKINNY
    assert route(lib, 4, 96, 256, 384, 1, 3) == ROWMAJOR
    assert route(lib, 2, 32, 256, 512, 0, 1) == PORTABLE           # dynamic 2-bit: Kidi's portable path
    assert route(lib, 4, 128, 256, 512, 1, 2, in_s=0.5) == PORTABLE  # calibrated with zeros
    assert route(lib, 8, 32, 200, 256, 0, 150) == GEMM
    assert route(lib, 4, 256, 256, 1024, 0, 64) == GEMM
    assert route(lib, 4, 96, 48, 384, 1, 3, gelu=1) == ROWMAJOR
    assert route(lib, 4, 128, 2 * 24, 512, 1, 2, gelu=1) != DECODE  # gate/up split inside a 16-row tile
    assert route(lib, 4, 128, 8192, 2048, 1, 1, gelu=1) == DECODE  # even rows, whole tiles
    assert route(lib, 4, 128, 8191, 2048, 1, 1, gelu=1) == -1                # odd rows: invalid


def test_gemm8_activation_panel_bounds(lib):
    """gemm8's activation buffer is addressed with 32-bit offsets: M_p * K < 2^31, else the next route."""
    K = 2048
    M = (1 << 31) // K
    assert route(lib, 4, 128, 256, K, 1, M - 256) == GEMM8
    assert route(lib, 4, 128, 256, K, 1, M) != GEMM8


def test_no_environment_switches_in_launch_plans():
    """Launch plans of the shipped library do not read the environment (no tuning overrides)."""
    csrc = os.path.join(ROOT, "kidi_amd", "csrc")
    for name in os.listdir(csrc):
        text = open(os.path.join(csrc, name)).read()
        assert not re.search(r"\bgetenv\s*\(", text), name
