"""Packed checkpoint ingestion for the quantized linear layer, and a persisted gfx950 layout cache.

Ingestion follows the part of Gemma4Impl::set_checkpoint (src/kidi/model/gemma4.cpp:328-452) that feeds
PACKED_LINEAR: a projection is a ``<module>.weight`` U8/I8 tensor with ``<module>.weight_scale`` (F32/F16 [N, K/g]),
an optional additive ``<module>.weight_zero`` (bound to the scales, as Context::bind_packed_zero) and optional scalar
``input_activation_scale`` / ``output_activation_scale`` calibration. A QAT checkpoint (``quantization_config``)
takes each module's bit width from its rules (quant_bits, gemma4.cpp:30-43), stores 2/4-bit codes offset by half
the range, and converts them to two's complement with XOR 0xaa / 0x88 unless ``packed_weights_signed``
(:350-370); weight scales must be finite and positive, calibration scales finite and non-negative (:372-386); a
missing ``lm_head`` takes the quantized embedding (:387-397).

The layout cache plays the role of Kidi's packed-operator cache (runtime/ynn/feed_forward_cache.{h,cpp}): one file
per packed weight, a 4096-byte header (magic, format version, source file size and mtime, the weight's spec and a
hash of its source tensors, payload size) then the kq_weight_export blob; a load accepts a file only if every
field matches; writes go to a temporary file renamed into place; ``KQ_LAYOUT_CACHE`` set to "", "0", "off" or
"false" disables it and any other value names the directory."""

from __future__ import annotations

import hashlib
import json
import os
import re
import struct
from dataclasses import dataclass

import numpy as np
import torch
from safetensors import safe_open

from kidi_amd.ops import DeviceWeight, Failure

EMBEDDING = "model.language_model.embed_tokens"


def quant_bits(config: dict, module: str) -> int:
    """Bit width of a module under a QAT ``quantization_config`` (gemma4.cpp:30-43): 0 when unconverted."""
    q = config.get("quantization_config")
    if not q:
        return 0
    if any(item in module for item in q.get("modules_to_not_convert") or []):
        return 0
    bits = int(q["num_bits"])
    for pattern, rule in (q.get("module_quant_configs") or {}).items():
        if re.search(pattern, module):
            bits = int(rule["num_bits"])
            break
    if bits not in (2, 4, 8):
        raise Failure("UNSUPPORTED", "unsupported QAT bit width")
    return bits


def qat_signed(values: np.ndarray, bits: int) -> np.ndarray:
    """Offset-packed QAT codes to two's complement (gemma4.cpp:358-369); 8-bit codes are unchanged."""
    if bits >= 8:
        return values
    return np.bitwise_xor(values, np.uint8(0xAA if bits == 2 else 0x88))


class LayoutCache:
    """Persisted kq_weight_export blobs keyed by weight spec and source-tensor hash (feed_forward_cache.cpp)."""

    MAGIC = b"KQGFX950"
    VERSION = 1
    PAYLOAD_OFFSET = 4096
    HEADER = struct.Struct("<8sIIQqIiqqQQ")  # magic version header_size source_size source_mtime bits group N K hash payload

    def __init__(self, directory: str | os.PathLike | None, source: str | os.PathLike):
        self.readable = self.writable = False
        self.hits = self.stores = 0
        target = directory
        configured = os.environ.get("KQ_LAYOUT_CACHE")
        if configured is not None:
            if configured in ("", "0", "off", "false"):
                return
            target = configured
        if not target or not os.path.isfile(source):
            return
        try:
            os.makedirs(target, exist_ok=True)
        except OSError:
            return
        if not os.path.isdir(target):
            return
        self.directory = os.fspath(target)
        st = os.stat(source)
        self.source_size, self.source_mtime = st.st_size, st.st_mtime_ns
        self.readable = os.access(self.directory, os.R_OK | os.X_OK)
        self.writable = self.readable and os.access(self.directory, os.W_OK | os.X_OK)

    @property
    def enabled(self) -> bool:
        return self.readable or self.writable

    def _path(self, spec) -> str:
        bits, group, rows, cols, digest = spec
        return os.path.join(self.directory, f"kq-{digest:016x}-b{bits}-g{group}-{rows}x{cols}.bin")

    def load(self, spec) -> bytes | None:
        if not self.readable:
            return None
        try:
            with open(self._path(spec), "rb") as f:
                data = f.read()
        except OSError:
            return None
        if len(data) < self.PAYLOAD_OFFSET:
            return None
        h = self.HEADER.unpack_from(data)
        magic, version, header_size, size, mtime, bits, group, rows, cols, digest, payload = h
        if (magic != self.MAGIC or version != self.VERSION or header_size != self.PAYLOAD_OFFSET
                or size != self.source_size or mtime != self.source_mtime or (bits, group, rows, cols, digest) != tuple(spec)
                or len(data) != self.PAYLOAD_OFFSET + payload):
            return None
        self.hits += 1
        return data[self.PAYLOAD_OFFSET:]

    def store(self, spec, payload: bytes) -> None:
        if not self.writable or not payload:
            return
        dest = self._path(spec)
        tmp = f"{dest}.tmp.{os.getpid()}.{id(payload)}"
        header = self.HEADER.pack(self.MAGIC, self.VERSION, self.PAYLOAD_OFFSET, self.source_size, self.source_mtime,
                                  *spec, len(payload))
        try:
            with open(tmp, "xb") as f:
                f.write(header.ljust(self.PAYLOAD_OFFSET, b"\0"))
                f.write(payload)
            os.replace(tmp, dest)
            self.stores += 1
        except OSError:
            try:
                os.remove(tmp)
            except OSError:
                pass


@dataclass
class PackedLinear:
    """One ingested projection: the gfx950 weight and its calibration (Linear::forward, layers/linear.cpp:181-190)."""

    weight: DeviceWeight
    bits: int
    group_size: int
    input_scale: float = 0.0
    output_scale: float = 0.0

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        return self.weight.linear(x, self.input_scale, self.output_scale)


def _scalar(f, name: str) -> float:
    if name not in f.keys():
        return 0.0
    v = np.asarray(f.get_tensor(name), dtype=np.float32).reshape(-1)
    if v.size != 1 or not np.isfinite(v[0]) or v[0] < 0:
        raise Failure("INVALID_ARGUMENT", f"invalid trained quantization scale: {name}")
    return float(v[0])


def _digest(*arrays) -> int:
    h = hashlib.blake2b(digest_size=8)
    for a in arrays:
        if a is None:
            h.update(b"-")
            continue
        a = np.ascontiguousarray(a)
        h.update(str((a.dtype.str, a.shape)).encode())
        h.update(a.tobytes())
    return int.from_bytes(h.digest(), "little")


def load_packed_linears(path: str | os.PathLike, config: dict | None = None, signed: bool | None = None,
                        cache_dir: str | os.PathLike | None = None, device: str | torch.device = "cuda",
                        bits: int | None = None) -> dict[str, PackedLinear]:
    """Every packed projection of a safetensors checkpoint, re-laid out for gfx950 on ``device``.

    ``config`` defaults to the ``config.json`` beside the file; a checkpoint without ``quantization_config`` needs
    ``bits``. With ``cache_dir`` (or ``KQ_LAYOUT_CACHE``) the packed layouts persist across loads."""
    path = os.fspath(path)
    if config is None:
        cfg_path = os.path.join(os.path.dirname(path), "config.json")
        config = json.load(open(cfg_path)) if os.path.isfile(cfg_path) else {}
    if signed is None:
        signed = bool(config.get("packed_weights_signed", False))
    qat = bool(config.get("quantization_config"))
    cache = LayoutCache(cache_dir, path)
    dev = torch.device(device)
    out: dict[str, PackedLinear] = {}
    with safe_open(path, framework="np") as f:
        keys = set(f.keys())
        modules = []
        for k in sorted(keys):
            if k.endswith(".weight") and k[:-len(".weight")] + ".weight_scale" in keys:
                modules.append((k[:-len(".weight")], k, k[:-len(".weight")] + ".weight_scale", k[:-len(".weight")] + ".weight_zero"))
        if qat and "lm_head.weight" not in keys and EMBEDDING + ".embedding_quantized" in keys:
            modules.append(("lm_head", EMBEDDING + ".embedding_quantized", EMBEDDING + ".embedding_scale", EMBEDDING + ".embedding_zero"))
        for module, wname, sname, zname in modules:
            values = f.get_tensor(wname)
            if values.ndim != 2 or values.dtype not in (np.uint8, np.int8):
                continue
            # (a tied head is stored as the embedding: its bit width is the embedding's)
            b = (quant_bits(config, EMBEDDING if wname.startswith(EMBEDDING) else module) if qat else bits)
            if not b:
                raise Failure("INVALID_ARGUMENT", "QAT weight storage does not match configured precision")
            if values.dtype == np.int8:
                if b != 8:
                    raise Failure("INVALID_ARGUMENT", "QAT weight storage does not match configured precision")
                values = values.view(np.uint8)
            elif qat and not signed:
                values = qat_signed(values, b)
            scales = f.get_tensor(sname)
            sf = scales.astype(np.float32)
            if scales.ndim != 2 or scales.dtype not in (np.float32, np.float16) or not np.all(np.isfinite(sf)) or np.any(sf <= 0):
                raise Failure("INVALID_ARGUMENT", f"invalid trained quantization scale: {sname}")
            K = values.shape[1] * (8 // b)
            if scales.shape[0] != values.shape[0] or K % scales.shape[1]:
                raise Failure("INVALID_ARGUMENT", f"packed linear shape or dtype mismatch: {module}")
            group = K // scales.shape[1]
            zeros = f.get_tensor(zname) if zname in keys else None
            in_s = 0.0 if module == "lm_head" and "lm_head.input_activation_scale" not in keys else _scalar(f, module + ".input_activation_scale")
            out_s = 0.0 if module == "lm_head" and "lm_head.output_activation_scale" not in keys else _scalar(f, module + ".output_activation_scale")
            spec = (b, group, values.shape[0], K, _digest(values, scales, zeros))
            blob = cache.load(spec) if cache.enabled else None
            if blob is not None:
                dw = DeviceWeight.import_blob(blob)
            else:
                t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
                dw = DeviceWeight(t(values), t(scales), b, group, t(zeros) if zeros is not None else None)
                if cache.writable:
                    cache.store(spec, dw.export())
            out[module] = PackedLinear(dw, b, group, in_s, out_s)
    load_packed_linears.last_cache = cache
    return out


def prepare_runtime_packing(context, state: dict, weight_bits: int, group_size: int = 128,
                            packed_prefill: bool = False, asymmetric_clip: bool = False) -> list[tuple[str, int, int]]:
    """Runtime quantization of a float checkpoint (Gemma4Impl::set_checkpoint, src/kidi/model/gemma4.cpp:435-447):
    every 2-D weight except the token embeddings is bound with ``context.prepare_linear_weights``, 4-bit groups of
    ``group_size`` when ``weight_bits == 4`` and the width divides into them (the asymmetric clip only there), else
    8-bit with one group per row. Returns the (name, bits, group) choices in ``state`` order."""
    chosen = []
    if not weight_bits:
        return chosen
    for name, weight in state.items():
        if weight.dim() != 2 or name in ("embed_tokens.weight", "embed_tokens_per_layer.weight"):
            continue
        grouped = weight_bits == 4 and weight.shape[1] % group_size == 0
        bits, group = (4, group_size) if grouped else (8, int(weight.shape[1]))
        context.prepare_linear_weights(weight, bits, group, packed_prefill, grouped and asymmetric_clip)
        chosen.append((name, bits, group))
    return chosen
