"""kq_packed_linear_noalloc through the C ABI: the allocation-free entry point (static device scratch) gives exactly
kq_packed_linear's output (with a caller workspace) on two calls in a row, the second with a smaller input, on the
projection kernels that use the workspace (both prefill GEMMs with and without split K, the generic GEMM), on a
decode call, and refuses a call whose workspace exceeds the scratch with a clear error and no launch."""

import ctypes

import numpy as np
import pytest

from tests.cases import activations, weights

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from kidi_amd import _native

    _native.load()
    return torch.device("cuda:0")


def _args(N_, x, y, m, ws=None, ws_bytes=0, input_scale=0.0):
    a = N_.LinearArgs()
    a.x = x.data_ptr()
    a.x_dtype = N_.KQ_BF16 if x.dtype == torch.bfloat16 else N_.KQ_F32
    a.m = m
    a.input_scale = input_scale
    a.output_scale = 0.0
    a.y = y.data_ptr()
    a.workspace = ws.data_ptr() if ws is not None else None
    a.workspace_bytes = ws_bytes
    return a


def _both(N_, lib, dw, x, input_scale=0.0):
    """(y of kq_packed_linear with a caller workspace, y of kq_packed_linear_noalloc) for x [m, K]."""
    m = x.shape[0]
    width = dw.rows
    ws_bytes = lib.kq_linear_workspace_size(dw.handle, m)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    y_ref = torch.full((m, width), float("nan"), dtype=torch.float32, device=x.device)
    y_na = torch.full((m, width), float("nan"), dtype=torch.float32, device=x.device)
    stream = torch.cuda.current_stream().cuda_stream
    N_.check(lib.kq_packed_linear(dw.handle, ctypes.byref(_args(N_, x, y_ref, m, ws, ws_bytes, input_scale)), stream))
    N_.check(lib.kq_packed_linear_noalloc(dw.handle, ctypes.byref(_args(N_, x, y_na, m, None, 0, input_scale)), stream))
    torch.cuda.synchronize()
    return y_ref.cpu().numpy(), y_na.cpu().numpy()


@pytest.mark.parametrize("bits,group,K,N,zp,route,rows", [
    (4, 128, 1024, 400, True, "gemm8_kernel", (300, 40)),       # g = 128 prefill GEMM (codes, transposed scales)
    (4, 128, 8192, 256, True, "gemm8_kernel", (300, 64)),       # split K: partial tiles in the scratch
    (4, 32, 1024, 272, False, "gemm8_kernel", (200, 33)),       # g = 32 prefill GEMM
    (4, 32, 1024, 270, False, "gemm_i4g_kernel", (200, 33)),    # g = 32, N % 4 != 0: the two-stage LDS GEMM
    (8, 32, 512, 200, False, "gemm_kernel", (150, 20)),         # generic quantizer + GEMM
    (4, 128, 2048, 8192, True, "decode_kernel", (4, 1)),        # decode: the scratch is passed, not needed
])
def test_noalloc_equals_workspace_call(dev, bits, group, K, N, zp, route, rows):
    from kidi_amd import _native as N_
    from kidi_amd.ops import DeviceWeight

    lib = N_.load()
    rng = np.random.default_rng(K + N + bits)
    values, scales, zps, _ = weights(rng, N, K, bits, group, zero_points=zp)
    dw = DeviceWeight(torch.from_numpy(values).to(dev), torch.from_numpy(scales).to(dev), bits, group,
                      torch.from_numpy(zps).to(dev) if zps is not None else None)
    for m in rows:  # two calls in a row, the second smaller
        print(f"noalloc case bits={bits} g={group} K={K} N={N} M={m}", flush=True)
        x = torch.from_numpy(activations(rng, m, K, 0.001)).to(dev).to(torch.bfloat16)
        assert dw.route(x) == route
        y_ref, y_na = _both(N_, lib, dw, x)
        assert np.all(np.isfinite(y_ref))
        np.testing.assert_array_equal(y_na, y_ref)


def test_noalloc_refuses_oversized_call(dev):
    """M = 8192 rows of K = 8192 need 64 MiB of activation codes alone: refused before any launch."""
    from kidi_amd import _native as N_
    from kidi_amd.ops import DeviceWeight

    lib = N_.load()
    rng = np.random.default_rng(5)
    values, scales, zps, _ = weights(rng, 256, 8192, 4, 128, zero_points=True)
    dw = DeviceWeight(torch.from_numpy(values).to(dev), torch.from_numpy(scales).to(dev), 4, 128,
                      torch.from_numpy(zps).to(dev))
    m = 8192
    assert lib.kq_linear_workspace_size(dw.handle, m) > (64 << 20)
    x = torch.zeros((m, 8192), dtype=torch.bfloat16, device=dev)
    y = torch.full((m, 256), 7.0, dtype=torch.float32, device=dev)
    st = lib.kq_packed_linear_noalloc(dw.handle, ctypes.byref(_args(N_, x, y, m)), torch.cuda.current_stream().cuda_stream)
    assert st == N_.KQ_INVALID_ARGUMENT
    assert b"scratch" in lib.kq_last_error()
    torch.cuda.synchronize()
    assert bool(torch.all(y == 7.0))  # nothing ran
