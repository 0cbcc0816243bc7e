"""Host-side mirror of Kidi's packed-linear entry points, over the HIP C ABI (include/kq.h).

Kidi's caller-facing interface for this path is ``ops::Context`` (src/kidi/ops/context.h:72-203):
``packed_linear`` (context.cpp:821-939), ``bind_packed_zero`` (:813-815), ``gelu_gate`` (:957-963), and the
dispatcher's prepared-operator cache keyed by parameter storage identity (:148-194, :366-382). This module keeps
those names, argument meanings and error behaviour (``Failure`` carrying the ErrorCode name) for tensors that live
in PyTorch-ROCm device memory. PyTorch is only the allocator and stream here; every projection runs in
``libkq_hip.so``.
"""

from __future__ import annotations

import collections
import ctypes
import math
import struct
import time
from dataclasses import dataclass

import torch

from . import _native as N
from .profiling import Profiler


class Failure(RuntimeError):
    """ops::Failure (src/kidi/ops/context.h:52-59): ``code`` is the kidi::core::ErrorCode name."""

    def __init__(self, code: str, message: str):
        self.code = code
        super().__init__(f"{code}: {message}")


def _raise(status: int) -> None:
    if status != N.KQ_OK:
        raise Failure(N.STATUS_NAMES.get(status, "RUNTIME"), N.load().kq_last_error().decode())


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _meta_dtype(t: torch.Tensor, what: str) -> int:
    if t.dtype == torch.float32:
        return N.KQ_F32
    if t.dtype == torch.float16:
        return N.KQ_F16
    if what == "zeros" and t.dtype == torch.uint8:
        return N.KQ_ZP_U8
    raise Failure("INVALID_ARGUMENT", "packed linear shape or dtype mismatch")


@dataclass
class PackedWeight:
    """ops::PackedWeight (src/kidi/ops/quantization.h:6-11)."""

    values: torch.Tensor
    scales: torch.Tensor
    zeros: torch.Tensor | None
    bits: int
    group_size: int


class DeviceWeight:
    """A packed weight re-laid out for gfx950 and resident in HBM (kq_weight)."""

    _free = None  # kq_weight_free, bound when the first weight is created

    def __init__(self, values, scales, bits: int, group_size: int, zeros=None, concat=None):
        lib = N.load()
        parts = concat if concat is not None else [(values, scales, zeros)]
        descs = (N.PackDesc * len(parts))()
        self._keep = []
        rows = 0
        for i, (v, s, z) in enumerate(parts):
            if v.dim() != 2 or s.dim() != 2:
                raise Failure("INVALID_ARGUMENT", "packed linear shape or dtype mismatch")
            v = v.contiguous()
            s = s.contiguous()
            z = z.contiguous() if z is not None else None
            dev = v.is_cuda
            if s.is_cuda != dev or (z is not None and z.is_cuda != dev):
                raise Failure("INVALID_ARGUMENT", "packed weight parts must share one device")
            self._keep += [v, s, z]
            d = descs[i]
            d.bits = bits
            d.group_size = group_size
            d.rows = v.shape[0]
            d.cols = v.shape[1] * (8 // bits) if bits in (2, 4, 8) else 0
            d.values = v.data_ptr()
            d.values_dtype = N.KQ_I8 if v.dtype == torch.int8 else (N.KQ_U8 if v.dtype == torch.uint8 else 99)
            d.scales = s.data_ptr()
            d.scales_dtype = _meta_dtype(s, "scales")
            d.zeros = z.data_ptr() if z is not None else None
            d.zeros_dtype = _meta_dtype(z, "zeros") if z is not None else N.KQ_NONE
            d.memory = N.KQ_DEVICE if dev else N.KQ_HOST
            if s.shape[0] != v.shape[0] or (group_size > 0 and s.shape[1] * group_size != d.cols):
                raise Failure("INVALID_ARGUMENT", "packed linear shape or dtype mismatch")
            rows += v.shape[0]
        handle = ctypes.c_void_p()
        if concat is None:
            status = lib.kq_weight_pack(descs, _stream() if torch.cuda.is_available() else None, ctypes.byref(handle))
        else:
            status = lib.kq_weight_pack_concat(descs, len(parts), _stream() if torch.cuda.is_available() else None,
                                               ctypes.byref(handle))
        self._keep = None
        _raise(status)
        self.handle = handle
        if DeviceWeight._free is None:
            DeviceWeight._free = N.load().kq_weight_free
        self.bits, self.group_size, self.rows = bits, group_size, rows
        self.cols = descs[0].cols
        self.has_zeros = parts[0][2] is not None

    @classmethod
    def from_handle(cls, handle: ctypes.c_void_p) -> "DeviceWeight":
        """Adopt a kq_weight (e.g. one kq_weight_import made); the object frees it."""
        self = cls.__new__(cls)
        self.handle = handle
        if DeviceWeight._free is None:
            DeviceWeight._free = N.load().kq_weight_free
        b, g, r, c, z = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32()
        _raise(N.load().kq_weight_info(handle, ctypes.byref(b), ctypes.byref(g), ctypes.byref(r), ctypes.byref(c),
                                       ctypes.byref(z), None))
        self.bits, self.group_size, self.rows, self.cols, self.has_zeros = b.value, g.value, r.value, c.value, bool(z.value)
        return self

    def export(self) -> bytes:
        """The packed gfx950 layout as one host blob (kq_weight_export)."""
        L = N.load()
        n = L.kq_weight_export_size(self.handle)
        buf = (ctypes.c_uint8 * n)()
        _raise(L.kq_weight_export(self.handle, buf, n, _stream()))
        return bytes(buf)

    @classmethod
    def import_blob(cls, blob: bytes) -> "DeviceWeight":
        """A weight from a kq_weight_export blob, uploaded to the current device without re-layout."""
        handle = ctypes.c_void_p()
        buf = (ctypes.c_uint8 * len(blob)).from_buffer_copy(blob)
        _raise(N.load().kq_weight_import(buf, len(blob), _stream(), ctypes.byref(handle)))
        return cls.from_handle(handle)

    def __del__(self):
        h = getattr(self, "handle", None)
        if h is not None and h.value:
            # the library's free routine is taken from the class attribute bound at first use, so it stays callable
            # while the interpreter tears modules down
            free = type(self)._free or N.load().kq_weight_free
            free(h)
            self.handle = None

    def path(self, input_scale: float) -> int:
        return N.load().kq_select_path(self.bits, self.group_size, self.cols, self.rows, int(self.has_zeros), input_scale)

    def workspace_size(self, m: int) -> int:
        return N.load().kq_linear_workspace_size(self.handle, m)

    def _args(self, x: torch.Tensor, y: torch.Tensor, m: int, input_scale: float, output_scale: float):
        ws_bytes = self.workspace_size(m)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        a = N.LinearArgs()
        a.x = x.data_ptr()
        a.x_dtype = N.KQ_BF16 if x.dtype == torch.bfloat16 else (N.KQ_F32 if x.dtype == torch.float32 else 99)
        a.m = m
        a.input_scale = input_scale
        a.output_scale = output_scale
        a.y = y.data_ptr()
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws_bytes
        return a, ws

    def linear(self, x: torch.Tensor, input_scale: float = 0.0, output_scale: float = 0.0,
               out: torch.Tensor | None = None, gelu_gate: bool = False) -> torch.Tensor:
        """y [..., N] (or [..., N/2] with GELU gating) for x [..., K] F32/BF16 on the device."""
        if x.dim() < 1 or x.shape[-1] != self.cols:
            raise Failure("INVALID_ARGUMENT", "packed linear shape or dtype mismatch")
        x2 = x.reshape(-1, self.cols).contiguous()
        m = x2.shape[0]
        width = self.rows // 2 if gelu_gate else self.rows
        y = out if out is not None else torch.empty((m, width), dtype=torch.float32, device=x.device)
        a, ws = self._args(x2, y, m, input_scale, output_scale)
        fn = N.load().kq_packed_linear_gelu_gate if gelu_gate else N.load().kq_packed_linear
        _raise(fn(self.handle, ctypes.byref(a), _stream()))
        return y.reshape(*x.shape[:-1], width)

    def linear_greedy(self, x: torch.Tensor, input_scale: float = 0.0, output_scale: float = 0.0,
                      keep_logits: bool = False):
        """(tokens int32 [...], logits [..., N] or None): the projection fused with greedy selection
        (kq_packed_linear_greedy); without keep_logits the decode kernel keeps the logits on chip."""
        if x.dim() < 1 or x.shape[-1] != self.cols:
            raise Failure("INVALID_ARGUMENT", "packed linear shape or dtype mismatch")
        x2 = x.reshape(-1, self.cols).contiguous()
        m = x2.shape[0]
        y = torch.empty((m, self.rows), dtype=torch.float32, device=x.device) if keep_logits else None
        tokens = torch.empty((m,), dtype=torch.int32, device=x.device)
        L = N.load()
        ws_bytes = L.kq_greedy_linear_workspace_size(self.handle, m)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        a = N.LinearArgs()
        a.x = x2.data_ptr()
        a.x_dtype = N.KQ_BF16 if x2.dtype == torch.bfloat16 else (N.KQ_F32 if x2.dtype == torch.float32 else 99)
        a.m = m
        a.input_scale = input_scale
        a.output_scale = output_scale
        a.y = y.data_ptr() if y is not None else None
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws_bytes
        _raise(L.kq_packed_linear_greedy(self.handle, ctypes.byref(a), tokens.data_ptr(), _stream()))
        tokens = tokens.reshape(x.shape[:-1])
        return tokens, (y.reshape(*x.shape[:-1], self.rows) if y is not None else None)

    def linear_rms(self, x: torch.Tensor, norm_weight: torch.Tensor, epsilon: float,
                   residual: torch.Tensor | None = None, residual_weight: torch.Tensor | None = None,
                   residual_scale: torch.Tensor | None = None, residual_epsilon: float | None = None,
                   input_scale: float = 0.0, output_scale: float = 0.0, gelu_gate: bool = False):
        """(y, hidden): the projection of rms_norm(x) (or, with a residual, of rms_norm(hidden) where hidden =
        rms_norm_residual(x, residual_weight, residual, residual_epsilon, residual_scale)), the normalization
        fused into the activation quantization (kq_packed_linear_rms). hidden is None without a residual."""
        if x.dim() < 1 or x.shape[-1] != self.cols:
            raise Failure("INVALID_ARGUMENT", "packed linear shape or dtype mismatch")
        x2 = x.reshape(-1, self.cols).contiguous()
        m = x2.shape[0]
        width = self.rows // 2 if gelu_gate else self.rows
        y = torch.empty((m, width), dtype=torch.float32, device=x.device)
        L = N.load()
        ws_bytes = L.kq_rms_linear_workspace_size(self.handle, m)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
        a = N.LinearArgs()
        a.x = x2.data_ptr()
        a.x_dtype = N.KQ_BF16 if x2.dtype == torch.bfloat16 else (N.KQ_F32 if x2.dtype == torch.float32 else 99)
        a.m = m
        a.input_scale = input_scale
        a.output_scale = output_scale
        a.y = y.data_ptr()
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws_bytes
        d = N.NormDesc()
        w = norm_weight.contiguous()
        d.weight = w.data_ptr()
        d.epsilon = epsilon
        keep = [w]
        hidden = None
        if residual is not None:
            r = residual.reshape(-1, self.cols).contiguous()
            if r.shape != x2.shape or r.dtype != x2.dtype or residual_weight is None:
                raise Failure("INVALID_ARGUMENT", "invalid RMS residual normalization operands")
            rw = residual_weight.contiguous()
            hidden = torch.empty((m, self.cols), dtype=torch.float32, device=x.device)
            d.residual = r.data_ptr()
            d.residual_weight = rw.data_ptr()
            d.residual_scale = residual_scale.data_ptr() if residual_scale is not None else None
            d.residual_epsilon = epsilon if residual_epsilon is None else residual_epsilon
            d.hidden = hidden.data_ptr()
            keep += [r, rw]
        fn = L.kq_packed_linear_rms
        _raise(fn(self.handle, ctypes.byref(a), ctypes.byref(d), int(bool(gelu_gate)), _stream()))
        del keep
        y = y.reshape(*x.shape[:-1], width)
        return y, (hidden.reshape(x.shape) if hidden is not None else None)

    def route(self, x: torch.Tensor, input_scale: float = 0.0, gelu_gate: bool = False) -> str:
        """Name of the projection kernel ``linear`` runs for x (kq_debug_route), without running it."""
        x2 = x.reshape(-1, self.cols)
        m = x2.shape[0]
        a = N.LinearArgs()
        a.x = x2.data_ptr()
        a.x_dtype = N.KQ_BF16 if x2.dtype == torch.bfloat16 else N.KQ_F32
        a.m = m
        a.input_scale = input_scale
        a.y = 1  # any non-null pointer: nothing is written
        r = N.load().kq_debug_route(self.handle, ctypes.byref(a), int(bool(gelu_gate)))
        if r < 0:
            raise Failure("INVALID_ARGUMENT", N.load().kq_last_error().decode())
        return N.ROUTE_NAMES[r]

    def debug_partials(self, x: torch.Tensor, input_scale: float = 0.0, output_scale: float = 0.0):
        """(y, int32 partials [M, N, K/g]) from the same kernel as ``linear`` (for g = 32 in 128 x 160 tiles, its
        256 x 128 form, whose y is bit-identical)."""
        x2 = x.reshape(-1, self.cols).contiguous()
        m = x2.shape[0]
        y = torch.empty((m, self.rows), dtype=torch.float32, device=x.device)
        P = torch.zeros((m, self.rows, self.cols // self.group_size), dtype=torch.int32, device=x.device)
        a, ws = self._args(x2, y, m, input_scale, output_scale)
        _raise(N.load().kq_debug_partials(self.handle, ctypes.byref(a), P.data_ptr(), _stream()))
        return y, P

    def debug_quantize(self, x: torch.Tensor, input_scale: float = 0.0):
        """(codes int8 [M, K], scales f32 [M, B], sums int32 [M, B], zero points int32 [M, B])."""
        x2 = x.reshape(-1, self.cols).contiguous()
        m = x2.shape[0]
        B = self.cols // self.group_size
        codes = torch.zeros((m, self.cols), dtype=torch.int8, device=x.device)
        s = torch.zeros((m, B), dtype=torch.float32, device=x.device)
        q = torch.zeros((m, B), dtype=torch.int32, device=x.device)
        z = torch.zeros((m, B), dtype=torch.int32, device=x.device)
        xt = N.KQ_BF16 if x2.dtype == torch.bfloat16 else N.KQ_F32
        _raise(N.load().kq_debug_quantize(self.handle, x2.data_ptr(), xt, m, input_scale, codes.data_ptr(),
                                          s.data_ptr(), q.data_ptr(), z.data_ptr(), _stream()))
        return codes, s, q, z


def gated_feed_forward(gate_up: DeviceWeight, down: DeviceWeight, x: torch.Tensor, gate_up_input_scale: float,
                       gate_up_output_scale: float, down_input_scale: float, down_output_scale: float,
                       silu: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """y [..., K] = down(act(gate) * up) of packed weights gate_up [2I, K] and down [K, I] (kq_gated_feed_forward)."""
    if x.dim() < 1 or x.shape[-1] != gate_up.cols:
        raise Failure("INVALID_ARGUMENT", "gated feed-forward input shape mismatch")
    x2 = x.reshape(-1, gate_up.cols).contiguous()
    m = x2.shape[0]
    y = out if out is not None else torch.empty((m, down.rows), dtype=torch.float32, device=x.device)
    L = N.load()
    ws_bytes = L.kq_ffn_workspace_size(gate_up.handle, down.handle, m)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    a = N.FfnArgs()
    a.x = x2.data_ptr()
    a.x_dtype = N.KQ_BF16 if x2.dtype == torch.bfloat16 else (N.KQ_F32 if x2.dtype == torch.float32 else 99)
    a.m = m
    a.gate_up_input_scale = gate_up_input_scale
    a.gate_up_output_scale = gate_up_output_scale
    a.down_input_scale = down_input_scale
    a.down_output_scale = down_output_scale
    a.silu = int(bool(silu))
    a.y = y.data_ptr()
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws_bytes
    _raise(L.kq_gated_feed_forward(gate_up.handle, down.handle, ctypes.byref(a), _stream()))
    return y.reshape(*x.shape[:-1], down.rows)


def greedy_token(logits: torch.Tensor) -> torch.Tensor:
    """Greedy token per row of device F32 logits [..., width] (kq_greedy_token): int32 [...]."""
    if logits.dim() < 1 or logits.shape[-1] < 1 or logits.dtype != torch.float32:
        raise Failure("INVALID_ARGUMENT", "greedy selection requires F32 [..., width > 0] logits")
    x = logits.reshape(-1, logits.shape[-1]).contiguous()
    rows, width = x.shape
    tokens = torch.empty((rows,), dtype=torch.int32, device=logits.device)
    L = N.load()
    ws_bytes = L.kq_greedy_workspace_size(rows, width)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=logits.device)
    _raise(L.kq_greedy_token(x.data_ptr(), rows, width, tokens.data_ptr(), ws.data_ptr(), ws_bytes, _stream()))
    return tokens.reshape(logits.shape[:-1])


def gated_multiply(gate: torch.Tensor, value: torch.Tensor, silu: bool = False) -> torch.Tensor:
    """GELU_MULTIPLY / SILU_MULTIPLY on device F32 tensors of one shape (kq_gelu_multiply / kq_silu_multiply)."""
    name = "SiLU" if silu else "GELU"
    if (gate is None or value is None or gate.dtype != torch.float32 or value.dtype != gate.dtype
            or tuple(gate.shape) != tuple(value.shape)):
        raise Failure("INVALID_ARGUMENT", f"{name} multiplication requires matching floating tensors")
    g, v = gate.contiguous(), value.contiguous()
    y = torch.empty_like(g)
    fn = N.load().kq_silu_multiply if silu else N.load().kq_gelu_multiply
    _raise(fn(g.data_ptr(), v.data_ptr(), g.numel(), y.data_ptr(), _stream()))
    return y


def rms_norm(x: torch.Tensor, weight: torch.Tensor, epsilon: float, residual: torch.Tensor | None = None,
             output_scale: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """RMS_NORM / RMS_NORM_RESIDUAL over the last axis of device F32/BF16 x (kq_rms_norm): F32 output."""
    width = x.shape[-1]
    x2 = x.reshape(-1, width).contiguous()
    y = out if out is not None else torch.empty(x2.shape, dtype=torch.float32, device=x.device)
    a = N.RmsArgs()
    a.x = x2.data_ptr()
    a.x_dtype = N.KQ_BF16 if x2.dtype == torch.bfloat16 else (N.KQ_F32 if x2.dtype == torch.float32 else 99)
    a.rows = x2.shape[0]
    a.width = width
    w = weight.contiguous()
    a.weight = w.data_ptr()
    r = residual.reshape(-1, width).contiguous() if residual is not None else None
    a.residual = r.data_ptr() if r is not None else None
    a.output_scale = output_scale.data_ptr() if output_scale is not None else None
    a.epsilon = epsilon
    a.y = y.data_ptr()
    _raise(N.load().kq_rms_norm(ctypes.byref(a), _stream()))
    return y.reshape(x.shape)


def pack_weight(weight: torch.Tensor, bits: int = 4, group_size: int = 128,
                asymmetric_clip: bool = False) -> PackedWeight:
    """ops::pack_weight (src/kidi/ops/quantization.cpp:12-133) on the device (kq_quantize_weight): float weights
    [N, K] (F32, F16 or BF16, device) become Kidi-layout U8 codes, F32 scales and, for the asymmetric 4-bit clip,
    F32 additive zeros. Synchronous; non-finite weights raise INVALID_ARGUMENT."""
    dt = {torch.float32: N.KQ_F32, torch.float16: N.KQ_F16, torch.bfloat16: N.KQ_BF16}.get(weight.dtype, 99)
    if (weight.dim() != 2 or dt == 99 or bits not in (2, 4, 8) or group_size <= 0
            or group_size % (8 // bits) or not weight.shape[0] or not weight.shape[1]
            or weight.shape[1] % group_size):
        raise Failure("INVALID_ARGUMENT", "invalid packed weight dimensions, precision or group size")
    w = weight.contiguous()
    rows, cols = w.shape
    values = torch.empty((rows, cols // (8 // bits)), dtype=torch.uint8, device=w.device)
    scales = torch.empty((rows, cols // group_size), dtype=torch.float32, device=w.device)
    asym = bool(asymmetric_clip) and bits == 4
    zeros = torch.empty_like(scales) if asym else None
    _raise(N.load().kq_quantize_weight(w.data_ptr(), dt, rows, cols, bits, group_size, int(asym),
                                       values.data_ptr(), scales.data_ptr(),
                                       zeros.data_ptr() if zeros is not None else None, _stream()))
    return PackedWeight(values, scales, zeros, bits, group_size)


def _identity(t: torch.Tensor | None):
    if t is None:
        return None
    return (t.device.type, t.untyped_storage().data_ptr(), t.storage_offset(), tuple(t.shape), t.dtype)


# core::InferencePrecision values this library serves (src/kidi/core/precision.h:8-22, names :66-80). CHECKPOINT
# runs PACKED_LINEAR (the operator); LOWBIT_PARITY runs runtime::parity::packed_linear. Kidi's other precisions
# dequantize the weight and run a dense LINEAR on a host device (ops/context.cpp:832-916), outside this library.
CHECKPOINT, LOWBIT_PARITY = "checkpoint", "lowbit-parity"
_PRECISION_NAMES = {"checkpoint": CHECKPOINT, "lowbit-parity": LOWBIT_PARITY, "checkpoint-parity": LOWBIT_PARITY}


def _f32_bits(v: float) -> int:
    """std::bit_cast<std::int32_t>(float) (the output_scale attribute, ops/context.cpp:932)."""
    return struct.unpack("<i", struct.pack("<f", float(v)))[0]


class Context:
    """The packed-linear slice of ops::Context on one HIP device."""

    CAPACITY = 4096  # bounded prepared-operator cache (ops/context.cpp:368-375)

    def __init__(self, device: str | torch.device = "cuda"):
        self.device = torch.device(device)
        self.precision = CHECKPOINT
        self._prepared: collections.OrderedDict = collections.OrderedDict()
        self._zeros: dict = {}
        self._bound: dict = {}  # weight storage -> (source, PackedWeight, packed_prefill, asymmetric_clip)
        self.decode_projections = False  # Context's decode flag: bound weights take the packed path at any M
        self._profiler = Profiler(self.device)  # KIDI_PROFILE_OPS=host|sync (kidi_amd/profiling.py)

    # ---- per-operation profiling (ops/context.cpp:117-133, :406-438, :502-515) ----
    def profile_phase(self, phase: str) -> None:
        """Context::profile_phase: label the following calls; "encoder" / "gemma4_request" count requests for
        KIDI_PROFILE_OPS_SKIP."""
        self._profiler.profile_phase(phase)

    def synchronize(self) -> None:
        """Context::synchronize: wait for the device (timed per phase while profiling)."""
        self._profiler.synchronize()

    def profile_report(self) -> list[str]:
        """The kidi_op / kidi_op_sync lines the context prints when it is closed."""
        return self._profiler.report()

    def close(self) -> None:
        self._profiler.close()

    def __del__(self):
        try:
            self._profiler.close()
        except Exception:
            pass

    def prepare_linear_weights(self, weight: torch.Tensor, bits: int, group_size: int = 128,
                               packed_prefill: bool = False, asymmetric_clip: bool = False) -> None:
        """Context::prepare_linear_weights (ops/context.cpp:783-812): quantize a float weight once
        (``pack_weight``), keep the packed copy on the device and bind it to the source weight, so ``linear``
        on that weight runs the packed projection. Re-binding with another layout is INVALID_ARGUMENT."""
        if (weight is None or weight.dim() != 2 or not weight.is_contiguous()
                or weight.dtype not in (torch.float16, torch.bfloat16, torch.float32) or bits not in (2, 4, 8)
                or group_size <= 0 or group_size % (8 // bits) or weight.shape[1] % group_size
                or not weight.shape[0] or not weight.shape[1]):
            raise Failure("INVALID_ARGUMENT", "invalid packed weight dimensions, precision or group size")
        key = (weight.device.type, weight.untyped_storage().data_ptr() + weight.storage_offset() * weight.element_size())
        found = self._bound.get(key)
        if found is not None:
            src, packed, prefill, asym = found
            if (packed.bits != bits or packed.group_size != group_size or prefill != packed_prefill
                    or asym != asymmetric_clip or tuple(src.shape) != tuple(weight.shape)):
                raise Failure("INVALID_ARGUMENT", "weight already packed with a different layout")
            return
        packed = pack_weight(weight.to(self.device), bits, group_size, asymmetric_clip)
        self._bound[key] = (weight, packed, bool(packed_prefill), bool(asymmetric_clip))

    def linear(self, input: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
               transpose_weight: bool = True) -> torch.Tensor:
        """Context::linear's packed redirect (ops/context.cpp:742-773): a weight bound by
        ``prepare_linear_weights`` runs PACKED_LINEAR with dynamic activations when it was bound with
        packed_prefill, when the context decodes, or for a single input row. The dense LINEAR it otherwise
        falls back to is not part of this library (UNSUPPORTED)."""
        if transpose_weight and bias is None and self._bound:
            key = (weight.device.type,
                   weight.untyped_storage().data_ptr() + weight.storage_offset() * weight.element_size())
            found = self._bound.get(key)
            single_row = input.dim() > 0 and input.numel() == input.shape[-1]
            if (found is not None and found[0].dtype == weight.dtype
                    and tuple(found[0].shape) == tuple(weight.shape)
                    and (found[2] or self.decode_projections or single_row)):
                p = found[1]
                return self.packed_linear(input, p.values, p.scales, p.bits, p.group_size, 0.0, 0.0, p.zeros)
        raise Failure("UNSUPPORTED", "dense LINEAR is outside the packed projection library")

    def set_precision(self, precision: str) -> None:
        """Context::set_precision (ops/context.h): "checkpoint" or "lowbit-parity" (also "checkpoint-parity",
        core::parse_precision, precision.h:74). The dense-dequantized precisions are UNSUPPORTED here."""
        found = _PRECISION_NAMES.get(precision)
        if found is None:
            raise Failure("UNSUPPORTED", "selected precision requires CPU packed weights with compatible group scales")
        self.precision = found

    def bind_packed_zero(self, scales: torch.Tensor, zeros: torch.Tensor) -> None:
        """Context::bind_packed_zero (ops/context.cpp:813-815)."""
        if scales is not None and zeros is not None:
            self._zeros[_identity(scales)] = zeros

    def _prepare(self, weight, scales, bits, group_size, zeros) -> DeviceWeight:
        key = (_identity(weight), _identity(scales), _identity(zeros), bits, group_size)
        found = self._prepared.get(key)
        if found is not None:
            self._prepared.move_to_end(key)
            return found[0]
        started = time.perf_counter_ns()
        dw = DeviceWeight(weight, scales, bits, group_size, zeros)
        self._profiler.prepare_ns += time.perf_counter_ns() - started
        self._prepared[key] = (dw, weight, scales, zeros)
        if len(self._prepared) > self.CAPACITY:
            self._prepared.popitem(last=False)
        return dw

    @staticmethod
    def _validate(input, weight, scales, bits, group_size, input_scale, output_scale):
        # Context::packed_linear (ops/context.cpp:824-825) then Impl::run validation (:207-218)
        if not math.isfinite(input_scale) or input_scale < 0 or not math.isfinite(output_scale) or output_scale < 0:
            raise Failure("INVALID_ARGUMENT", "invalid calibrated projection scales")
        if bits not in (2, 4, 8) or group_size <= 0:
            raise Failure("INVALID_ARGUMENT", "invalid packed linear precision or group")
        per = 8 // bits
        K = input.shape[-1] if input.dim() else 0
        if (input.dtype not in (torch.float32, torch.bfloat16) or input.dim() < 2 or not K or K % group_size
                or group_size % per or weight.dtype != torch.uint8 or weight.dim() != 2 or not weight.shape[0]
                or weight.shape[1] != K // per or scales.dtype not in (torch.float32, torch.float16)
                or scales.dim() != 2 or scales.shape[0] != weight.shape[0] or scales.shape[1] != K // group_size):
            raise Failure("INVALID_ARGUMENT", "packed linear shape or dtype mismatch")

    def packed_linear(self, input: torch.Tensor, weight: torch.Tensor, scales: torch.Tensor, bits: int,
                      group_size: int, input_scale: float = 0.0, output_scale: float = 0.0,
                      zeros: torch.Tensor | None = None) -> torch.Tensor:
        """Context::packed_linear (ops/context.cpp:821-939): PACKED_LINEAR under CHECKPOINT precision, Kidi's
        LOWBIT_PARITY projection under that precision (:917-932). F32 [..., N] output."""
        bound = zeros if zeros is not None else self._zeros.get(_identity(scales))
        operands = [input, weight, scales] + ([bound] if bound is not None and self.precision != LOWBIT_PARITY else [])
        with self._profiler.call("packed_linear", [t.shape for t in operands],
                                 [bits, group_size, _f32_bits(output_scale)]) as rec:
            if self.precision == LOWBIT_PARITY:
                rec["output"] = self._lowbit_parity(input, weight, scales, bits, group_size, input_scale, output_scale)
                return rec["output"]
            self._validate(input, weight, scales, bits, group_size, input_scale, output_scale)
            dw = self._prepare(weight, scales, bits, group_size, bound)
            host = not input.is_cuda
            x = input.to(self.device) if host else input
            y = dw.linear(x, input_scale, output_scale)
            if host:  # a HIP op behind a CPU tensor returns host-visible results (synchronous)
                y = y.cpu()
            rec["output"] = y
            return y

    def _lowbit_parity(self, input, weight, scales, bits, group_size, input_scale, output_scale):
        # Context::packed_linear's scale check (ops/context.cpp:824-825), its LOWBIT_PARITY domain (:919-929), then
        # runtime::parity::packed_linear (kq_lowbit_parity_linear). Bound zeros are not passed in this mode.
        if not math.isfinite(input_scale) or input_scale < 0 or not math.isfinite(output_scale) or output_scale < 0:
            raise Failure("INVALID_ARGUMENT", "invalid calibrated projection scales")
        per = 8 // bits if bits in (2, 4, 8) else 0
        width = weight.shape[1] * per if weight.dim() == 2 else 0
        groups = width // group_size if group_size > 0 else 0
        if (not per or input.dtype != torch.float32 or input.dim() == 0 or input_scale <= 0 or output_scale <= 0
                or group_size <= 0 or width != input.shape[-1] or width % group_size or weight.dim() != 2
                or weight.dtype != torch.uint8 or scales.dtype != torch.float32
                or scales.numel() != weight.shape[0] * groups or input.numel() // max(width, 1) > 2**31 - 1
                or width > 2**31 - 1 or weight.shape[0] > 2**31 - 1):
            raise Failure("UNSUPPORTED", "lowbit-parity requires calibrated CPU packed weights with compatible group scales")
        dw = self._prepare(weight, scales.reshape(weight.shape[0], groups), bits, group_size, None)
        host = not input.is_cuda
        x = (input.to(self.device) if host else input).reshape(-1, width).contiguous()
        y = torch.empty((x.shape[0], weight.shape[0]), dtype=torch.float32, device=x.device)
        a = N.LinearArgs()
        a.x, a.x_dtype, a.m = x.data_ptr(), N.KQ_F32, x.shape[0]
        a.input_scale, a.output_scale, a.y = input_scale, output_scale, y.data_ptr()
        _raise(N.load().kq_lowbit_parity_linear(dw.handle, ctypes.byref(a), _stream()))
        y = y.reshape(*input.shape[:-1], weight.shape[0])
        return y.cpu() if host else y

    def packed_linear_gelu_gate(self, input: torch.Tensor, weight: torch.Tensor, scales: torch.Tensor, bits: int,
                                group_size: int, input_scale: float = 0.0, output_scale: float = 0.0,
                                zeros: torch.Tensor | None = None) -> torch.Tensor:
        """gelu_gate(packed_linear(x, gate_up)) in one pass: Kidi's gate_up_proj followed by Context::gelu_gate
        (ops/context.cpp:957-963, layers/gemma4.cpp:206-210)."""
        self._validate(input, weight, scales, bits, group_size, input_scale, output_scale)
        if weight.shape[0] % 2:
            raise Failure("INVALID_ARGUMENT", "GELU gate requires floating [..., 2 * intermediate] input")
        bound = zeros if zeros is not None else self._zeros.get(_identity(scales))
        operands = [input, weight, scales] + ([bound] if bound is not None else [])
        with self._profiler.call("packed_linear+gelu_gate", [t.shape for t in operands],
                                 [bits, group_size, _f32_bits(output_scale)]) as rec:
            dw = self._prepare(weight, scales, bits, group_size, bound)
            host = not input.is_cuda
            x = input.to(self.device) if host else input
            y = dw.linear(x, input_scale, output_scale, gelu_gate=True)
            rec["output"] = y.cpu() if host else y
            return rec["output"]

    def gated_feed_forward(self, input: torch.Tensor, gate_up_weight: torch.Tensor, gate_up_scales: torch.Tensor,
                           down_weight: torch.Tensor, down_scales: torch.Tensor, bits: int, input_size: int,
                           intermediate_size: int, gate_up_input_scale: float, gate_up_output_scale: float,
                           down_input_scale: float, down_output_scale: float, silu: bool = False) -> torch.Tensor:
        """Context::gated_feed_forward (ops/context.cpp:970-996): per-channel packed gate_up [2I, K] and down [K, I]
        (groups of input_size and intermediate_size columns, as the composed form passes them), GELU-tanh or SiLU
        gating between, F32 [..., K] output."""
        for v in (gate_up_input_scale, gate_up_output_scale, down_input_scale, down_output_scale):
            if not math.isfinite(v) or v < 0:
                raise Failure("INVALID_ARGUMENT", "invalid calibrated projection scales")
        if input_size <= 0 or intermediate_size <= 0 or input.dim() < 2 or input.shape[-1] != input_size:
            raise Failure("INVALID_ARGUMENT", "gated feed-forward shape mismatch")
        if gate_up_weight.dim() != 2 or gate_up_weight.shape[0] != 2 * intermediate_size:
            raise Failure("INVALID_ARGUMENT", "gated feed-forward shape mismatch")
        self._validate(input, gate_up_weight, gate_up_scales, bits, input_size, gate_up_input_scale, gate_up_output_scale)
        hidden = torch.empty((1, intermediate_size), dtype=torch.float32)  # h is F32 (shape check only)
        self._validate(hidden, down_weight, down_scales, bits, intermediate_size, down_input_scale, down_output_scale)
        if down_weight.shape[0] != input_size:
            raise Failure("INVALID_ARGUMENT", "gated feed-forward shape mismatch")
        with self._profiler.call("gated_feed_forward",
                                 [t.shape for t in (input, gate_up_weight, gate_up_scales, down_weight, down_scales)],
                                 [bits, input_size, intermediate_size, int(silu)]) as rec:
            gu = self._prepare(gate_up_weight, gate_up_scales, bits, input_size, None)
            dn = self._prepare(down_weight, down_scales, bits, intermediate_size, None)
            host = not input.is_cuda
            x = input.to(self.device) if host else input
            y = gated_feed_forward(gu, dn, x, gate_up_input_scale, gate_up_output_scale, down_input_scale,
                                   down_output_scale, silu)
            rec["output"] = y.cpu() if host else y
            return rec["output"]

    @staticmethod
    def _validate_norm(input, scale, epsilon, residual=None, output_scale=None):
        # Context::rms_norm_residual (ops/context.cpp:1106-1112) and Impl::run's RMS_NORM checks (:317-330)
        if (input is None or input.dim() == 0 or input.dtype not in (torch.float32, torch.bfloat16) or scale is None
                or scale.dim() != 1 or scale.shape[0] != input.shape[-1] or scale.dtype != torch.float32
                or not math.isfinite(epsilon) or epsilon <= 0):
            raise Failure("INVALID_ARGUMENT", "invalid RMS residual normalization operands")
        if residual is not None and (residual.dtype != input.dtype or tuple(residual.shape) != tuple(input.shape)):
            raise Failure("INVALID_ARGUMENT", "invalid RMS residual normalization operands")
        if output_scale is not None and (output_scale.dtype != torch.float32 or output_scale.numel() != 1):
            raise Failure("INVALID_ARGUMENT", "invalid RMS residual normalization operands")

    def rms_norm(self, input: torch.Tensor, scale: torch.Tensor, epsilon: float) -> torch.Tensor:
        """Context::rms_norm (ops/context.cpp:1043-1049): F32 output; host tensors return host results."""
        self._validate_norm(input, scale, epsilon)
        with self._profiler.call("rms_norm", [input.shape, scale.shape], []) as rec:
            host = not input.is_cuda
            x = input.to(self.device) if host else input
            y = rms_norm(x, scale.to(self.device), epsilon)
            rec["output"] = y.cpu() if host else y
            return rec["output"]

    def rms_norm_residual(self, input: torch.Tensor, scale: torch.Tensor, residual: torch.Tensor, epsilon: float,
                          output_scale: torch.Tensor | None = None) -> torch.Tensor:
        """Context::rms_norm_residual (ops/context.cpp:1103-1122): (residual + rms_norm(input)) [* output_scale]."""
        if residual is None:
            raise Failure("INVALID_ARGUMENT", "invalid RMS residual normalization operands")
        self._validate_norm(input, scale, epsilon, residual, output_scale)
        operands = [input, scale, residual] + ([output_scale] if output_scale is not None else [])
        with self._profiler.call("rms_norm_residual", [t.shape for t in operands], []) as rec:
            host = not input.is_cuda
            x = input.to(self.device) if host else input
            r = residual.to(self.device) if host else residual
            o = output_scale.to(self.device).reshape(1) if output_scale is not None else None
            y = rms_norm(x, scale.to(self.device), epsilon, residual=r, output_scale=o)
            rec["output"] = y.cpu() if host else y
            return rec["output"]

    def gelu_multiply(self, gate: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
        """Context::gelu_multiply (ops/context.cpp:944-950): gelu_tanh(gate) * value over matching F32 tensors, the
        slice form of the gated feed-forward (layers/gemma4.cpp:213-225)."""
        return self._gated_multiply(gate, value, False)

    def silu_multiply(self, gate: torch.Tensor, value: torch.Tensor) -> torch.Tensor:
        """Context::silu_multiply (ops/context.cpp:951-957): silu(gate) * value over matching F32 tensors."""
        return self._gated_multiply(gate, value, True)

    def _gated_multiply(self, gate, value, silu):
        name = "SiLU" if silu else "GELU"
        if (gate is None or value is None or gate.dtype != torch.float32 or value.dtype != gate.dtype
                or tuple(gate.shape) != tuple(value.shape)):
            raise Failure("INVALID_ARGUMENT", f"{name} multiplication requires matching floating tensors")
        with self._profiler.call("silu_multiply" if silu else "gelu_multiply", [gate.shape, value.shape], []) as rec:
            host = not gate.is_cuda
            g = gate.to(self.device) if host else gate
            v = value.to(self.device) if not value.is_cuda else value
            y = gated_multiply(g, v, silu)
            rec["output"] = y.cpu() if host else y
            return rec["output"]

    def greedy_token(self, logits: torch.Tensor) -> torch.Tensor:
        """Context::greedy_token: I32 [...] of F32 logits [..., width]; a scalar is INVALID_ARGUMENT
        (eager_test.cpp:254-260). Host logits return host tokens."""
        if logits.dim() == 0 or logits.shape[-1] == 0:
            raise Failure("INVALID_ARGUMENT", "greedy selection requires [..., width > 0] logits")
        with self._profiler.call("greedy_token", [logits.shape], []) as rec:
            host = not logits.is_cuda
            x = logits.to(self.device, torch.float32) if host else logits.float()
            t = greedy_token(x)
            rec["output"] = t.cpu() if host else t
            return rec["output"]
