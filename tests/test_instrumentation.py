"""Measurement instrumentation of the C ABI: kq_debug_read_floor (the single-launch read floor bench.py reports beside
the decode roofline) and kq_debug_read_floor_shape (the same read at a chosen launch geometry, or an empty kernel of
that grid) reject bad arguments on the host and, on the GPU, read a buffer without writing anything but their sink
(which they touch only when the data XOR to a magic value); kq_debug_mfma_ceiling (the sustained int8 MFMA rate
bench.py reports beside the prefill figure) rejects bad arguments and, on the GPU, runs the MFMAs it is asked for."""

import ctypes

import pytest

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def native():
    from kidi_amd import _native

    _native.load()
    return _native


@pytest.mark.parametrize("bad", ["null", "zero", "ragged", "huge"])
def test_read_floor_rejects_invalid(native, bad):
    lib = native.load()
    data, size, sink = ctypes.c_void_p(256), 4096, ctypes.c_void_p(512)
    if bad == "null":
        data = None
    elif bad == "zero":
        size = 0
    elif bad == "ragged":
        size = 4100
    elif bad == "huge":
        size = (1 << 31) + 16
    assert lib.kq_debug_read_floor(data, size, sink, None) == native.KQ_INVALID_ARGUMENT
    assert lib.kq_last_error()
    assert lib.kq_debug_read_floor_shape(data, size, 256, 8, 0, sink, None) == native.KQ_INVALID_ARGUMENT


@pytest.mark.parametrize("threads,loads", [(32, 8), (96, 8), (2048, 8), (256, 0), (256, 3), (256, 32)])
def test_read_floor_shape_rejects_geometry(native, threads, loads):
    lib = native.load()
    assert lib.kq_debug_read_floor_shape(ctypes.c_void_p(256), 4096, threads, loads, 0, ctypes.c_void_p(512),
                                         None) == native.KQ_INVALID_ARGUMENT
    assert b"threads" in lib.kq_last_error()


@pytest.mark.gpu
def test_read_floor_reads_without_writing():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    lib = _native.load()
    dev = torch.device("cuda:0")
    for size in (16, 4096, 8753152 + 16 * 7, 64 << 20):
        buf = torch.zeros((size,), dtype=torch.uint8, device=dev)
        sink = torch.full((1,), -7, dtype=torch.int32, device=dev)
        assert lib.kq_debug_read_floor(buf.data_ptr(), size, sink.data_ptr(), None) == _native.KQ_OK
        torch.cuda.synchronize()
        assert int(sink.item()) == -7
        assert int(buf.sum().item()) == 0


@pytest.mark.gpu
def test_read_floor_shape_reads_without_writing():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    lib = _native.load()
    dev = torch.device("cuda:0")
    size = 8753152
    buf = torch.zeros((size,), dtype=torch.uint8, device=dev)
    sink = torch.full((1,), -7, dtype=torch.int32, device=dev)
    for threads in (64, 256, 1024):
        for loads in (1, 4, 16):
            for empty in (0, 1):
                assert lib.kq_debug_read_floor_shape(buf.data_ptr(), size, threads, loads, empty, sink.data_ptr(),
                                                     None) == _native.KQ_OK
    torch.cuda.synchronize()
    assert int(sink.item()) == -7
    assert int(buf.sum().item()) == 0


@pytest.mark.parametrize("bad", ["null_cycles", "null_sink", "zero", "negative", "huge"])
def test_mfma_ceiling_rejects_invalid(native, bad):
    lib = native.load()
    cycles, sink, iters = ctypes.c_void_p(256), ctypes.c_void_p(512), 16
    if bad == "null_cycles":
        cycles = None
    elif bad == "null_sink":
        sink = None
    elif bad == "zero":
        iters = 0
    elif bad == "negative":
        iters = -4
    elif bad == "huge":
        iters = (1 << 24) + 1
    assert lib.kq_debug_mfma_ceiling(iters, cycles, sink, None) == native.KQ_INVALID_ARGUMENT
    assert b"mfma ceiling" in lib.kq_last_error()


@pytest.mark.gpu
def test_mfma_ceiling_runs_its_mfmas():
    """Each wave's accumulators grow by the same A x B per round, so the lane-0 sums of n, 2n and 3n rounds are in
    arithmetic progression (mod 2^32) and equal across waves; every wave reports a positive cycle count that grows
    with the rounds."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    lib = _native.load()
    dev = torch.device("cuda:0")
    wgs = int(lib.kq_debug_mfma_ceiling_workgroups())
    assert wgs > 0
    sums, cyc = [], []
    for n in (16, 32, 48):
        cycles = torch.full((wgs * 8,), -1, dtype=torch.int64, device=dev)
        sink = torch.zeros((wgs * 8,), dtype=torch.int32, device=dev)
        assert lib.kq_debug_mfma_ceiling(n, cycles.data_ptr(), sink.data_ptr(), None) == _native.KQ_OK
        torch.cuda.synchronize()
        s = sink.cpu()
        assert bool((s == s[0]).all()), "every wave runs the same MFMAs"
        c = cycles.cpu()
        assert bool((c > 0).all())
        sums.append(int(s[0]) & 0xFFFFFFFF)
        cyc.append(float(c.double().mean()))
    assert (sums[2] - sums[1]) % (1 << 32) == (sums[1] - sums[0]) % (1 << 32)
    assert (sums[1] - sums[0]) % (1 << 32) != 0
    assert cyc[2] > cyc[0]
