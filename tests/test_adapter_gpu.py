"""The compiled C++ adapter on the GPU: a PACKED_LINEAR prepared through the graph::Compiler interceptor or the
OperatorBackend runs (run, with OutputPool reuse), writes caller-owned outputs (run_into), refuses run_ with the
reference's UNSUPPORTED, checks output shapes, and stages a CPU-device graph's host tensors; every result equals
kq_packed_linear's (the same kernels) bit for bit."""

import ctypes

import numpy as np
import pytest

from tests import adapter_lib
from tests.cases import activations, weights

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def desc(values, scales, zp, group, K, on_device):
    from kidi_amd import _native as N

    d = N.PackDesc()
    d.bits, d.group_size, d.rows, d.cols = 4, group, values.shape[0], K
    ptr = (lambda t: t.data_ptr()) if on_device else (lambda a: a.ctypes.data)
    d.values, d.values_dtype = ptr(values), N.KQ_U8
    d.scales, d.scales_dtype = ptr(scales), N.KQ_F16
    d.zeros, d.zeros_dtype = (ptr(zp), N.KQ_ZP_U8) if zp is not None else (None, N.KQ_NONE)
    d.memory = N.KQ_DEVICE if on_device else N.KQ_HOST
    return d


def copy_from_device(dst: torch.Tensor, src_ptr: int):
    """Device-to-device copy of dst.nbytes from a raw device pointer (the HIP runtime torch has loaded)."""
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(dst.data_ptr(), src_ptr, dst.numel() * dst.element_size(), 3) == 0  # hipMemcpyDeviceToDevice


def stats(L, op):
    cnt, byt = ctypes.c_uint64(), ctypes.c_uint64()
    L.kqa_allocations(op, ctypes.byref(cnt), ctypes.byref(byt))
    return cnt.value, byt.value


@pytest.mark.parametrize("via_backend", [0, 1])
@pytest.mark.parametrize("M", [1, 4, 300])
def test_prepare_run_run_into(dev, via_backend, M):
    from kidi_amd import _native as N
    from kidi_amd.ops import DeviceWeight

    L = adapter_lib.load()
    rng = np.random.default_rng(40 + M + via_backend)
    K, Nn = 1024, 512
    values, scales, zp, _ = weights(rng, Nn, K, 4, 128, zero_points=True)
    v, s, z = (torch.from_numpy(a).to(dev) for a in (values, scales, zp))
    x = torch.from_numpy(activations(rng, M, K)).to(dev)
    ref = DeviceWeight(v, s, 4, 128, z).linear(x)
    torch.cuda.synchronize()
    op = ctypes.c_void_p()
    st = torch.cuda.current_stream().cuda_stream
    assert L.kqa_prepare(ctypes.byref(desc(v, s, z, 128, K, True)), 0.0, 0.0, via_backend, st, ctypes.byref(op)) == 0, \
        adapter_lib.error()
    try:
        assert L.kqa_supports_replay(op) == 1
        # run: the result lands in the operator's output pool and equals kq_packed_linear's
        yp = ctypes.c_void_p()
        assert L.kqa_run(op, x.data_ptr(), N.KQ_F32, M, K, 1, 0, ctypes.byref(yp)) == 0, adapter_lib.error()
        assert L.kqa_synchronize(op) == 0
        got = torch.empty((M, Nn), dtype=torch.float32, device=dev)
        copy_from_device(got, yp.value)
        torch.testing.assert_close(got, ref, rtol=0, atol=0)
        assert stats(L, op) == (1, M * Nn * 4)
        # the same shape again: the pool hands the same buffer out (nothing else holds it) ...
        yp2 = ctypes.c_void_p()
        assert L.kqa_run(op, x.data_ptr(), N.KQ_F32, M, K, 1, 1, ctypes.byref(yp2)) == 0
        assert yp2.value == yp.value and stats(L, op)[0] == 1
        # ... but not while a caller still holds it: a second buffer
        yp3 = ctypes.c_void_p()
        assert L.kqa_run(op, x.data_ptr(), N.KQ_F32, M, K, 1, 0, ctypes.byref(yp3)) == 0
        assert yp3.value != yp2.value and stats(L, op)[0] == 2
        L.kqa_release(op)
        # run_into a caller-owned output
        out = torch.full((M, Nn), float("nan"), dtype=torch.float32, device=dev)
        assert L.kqa_run_into(op, x.data_ptr(), N.KQ_F32, M, K, out.data_ptr(), M, Nn, 1) == 0, adapter_lib.error()
        assert L.kqa_synchronize(op) == 0
        torch.testing.assert_close(out, ref, rtol=0, atol=0)
        assert stats(L, op)[0] == 2  # run_into allocates nothing
        # run_: UNSUPPORTED with the reference's message (runtime/ynn/operators.cpp:1256)
        assert L.kqa_run_(op, x.data_ptr(), N.KQ_F32, M, K, out.data_ptr(), Nn, 1) == 4
        assert adapter_lib.error() == "packed linear cannot run in place"
        # an output of the wrong width, an input of the wrong width: INVALID_ARGUMENT
        assert L.kqa_run_into(op, x.data_ptr(), N.KQ_F32, M, K, out.data_ptr(), M, Nn - 32, 1) == 1
        assert L.kqa_run_into(op, x.data_ptr(), N.KQ_F32, M, K // 2, out.data_ptr(), M, Nn, 1) == 1
        # bf16 activations through the same operator
        xb = x.to(torch.bfloat16)
        outb = torch.empty_like(out)
        assert L.kqa_run_into(op, xb.data_ptr(), N.KQ_BF16, M, K, outb.data_ptr(), M, Nn, 1) == 0
        assert L.kqa_synchronize(op) == 0
        torch.testing.assert_close(outb, DeviceWeight(v, s, 4, 128, z).linear(xb), rtol=0, atol=0)
    finally:
        L.kqa_free(op)


def test_cpu_device_graph_is_staged(dev):
    """Host weights and host activations (an unchanged CPU-device graph): the adapter packs the host weight, stages x
    to the GPU and returns a host result before run returns; equal to kq_packed_linear on device copies."""
    from kidi_amd import _native as N
    from kidi_amd.ops import DeviceWeight

    L = adapter_lib.load()
    rng = np.random.default_rng(77)
    M, K, Nn = 3, 512, 256
    values, scales, zp, _ = weights(rng, Nn, K, 4, 128, zero_points=True)
    x = np.ascontiguousarray(activations(rng, M, K))
    op = ctypes.c_void_p()
    assert L.kqa_prepare(ctypes.byref(desc(values, scales, zp, 128, K, False)), 0.0, 0.0, 0, None, ctypes.byref(op)) == 0, \
        adapter_lib.error()
    try:
        y = np.full((M, Nn), np.nan, np.float32)
        assert L.kqa_run_into(op, x.ctypes.data, N.KQ_F32, M, K, y.ctypes.data, M, Nn, 0) == 0, adapter_lib.error()
        yp = ctypes.c_void_p()
        assert L.kqa_run(op, x.ctypes.data, N.KQ_F32, M, K, 0, 0, ctypes.byref(yp)) == 0
        pooled = np.ctypeslib.as_array((ctypes.c_float * (M * Nn)).from_address(yp.value)).reshape(M, Nn).copy()
    finally:
        L.kqa_free(op)
    ref = DeviceWeight(*(torch.from_numpy(a).to(dev) for a in (values, scales)), 4, 128,
                       torch.from_numpy(zp).to(dev)).linear(torch.from_numpy(x).to(dev)).cpu().numpy()
    np.testing.assert_array_equal(y, ref)
    np.testing.assert_array_equal(pooled, ref)
