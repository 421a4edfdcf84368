"""4-bit group storage for frozen base weights, decoded on the GPU.

Mirrors quantization/codecs.py of the reference (paths relative to
/root/reference/src/ram_vram_finetune) for the 4-bit formats:

* ``int4-sym-g128`` -- the reference's in-repo format (codecs.py:1-6,55-116):
  codes 1..15 -> -7..7 (code 0 reserved), low nibble first, one fp32 scale per
  flattened 128-group, scale = absmax/7 (0 -> 1), round-half-even.
* ``nf4-g128`` -- this build's name for the north-star format: the same
  container (``payload`` uint8[ceil(n/128)*64], ``scales`` fp32[ceil(n/128)],
  low nibble first) with the published NF4 codebook (QLoRA, arXiv:2305.14314,
  appendix E), scale = group absmax (0 -> 1), code = nearest codebook entry
  (ties to the lower code).  The reference's ``TrainConfig`` rejects the bare
  name ``nf4`` (config.py:56-58 -> codecs.py:29-31); this distinct name keeps
  that behaviour.

``Record``/``encode``/``validate_spec``/``decode_into``/``materialize`` keep the
reference's names and argument meaning; ``decode_into``/``materialize`` run on
the device through ``st_dequant4`` (no CPU decode path).  Encoding is an
offline host step, as in the reference (storage.py:138).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib

GROUP = 128
CHUNK_GROUPS = 8192  # host encode chunk, as codecs.py:19
VALIDATION_CHUNK_GROUPS = 2048  # groups decoded at once by validate_spec, as codecs.py:20
FORMATS = ("int4-sym-g128", "nf4-g128")
STRIDE = 64  # payload bytes per group

NF4_CODEBOOK = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
    0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0)
INT4_CODEBOOK = tuple(float(i - 8) for i in range(16))
CODEBOOKS = {"int4-sym-g128": INT4_CODEBOOK, "nf4-g128": NF4_CODEBOOK}


def check_format(name: str) -> None:
    if name not in FORMATS:
        raise ValueError(f"unsupported_quantization: explicit format required; supported={FORMATS}")


@dataclass
class Record:
    spec: dict
    parts: dict

    @property
    def shape(self):
        return tuple(self.spec["shape"])


def codebook(mode: str) -> tuple:
    check_format(mode)
    return CODEBOOKS[mode]


def _nf4_midpoints() -> torch.Tensor:
    cb = torch.tensor(NF4_CODEBOOK, dtype=torch.float32)
    return (cb[:-1] + cb[1:]) * 0.5


def encode(tensor: torch.Tensor, mode: str) -> Record:
    """Offline host encode of a frozen fp32/bf16 matrix (codecs.py:66-116)."""
    if tensor.device.type != "cpu" or tensor.requires_grad or not tensor.is_contiguous():
        raise ValueError("encoder requires frozen contiguous CPU weights")
    if tensor.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("unsupported_quantization: source dtype")
    check_format(mode)
    count = tensor.numel()
    groups = (count + GROUP - 1) // GROUP
    payload = torch.empty(groups * STRIDE, dtype=torch.uint8)
    scales = torch.empty(groups, dtype=torch.float32)
    flat = tensor.reshape(-1)
    mids = _nf4_midpoints()
    for g in range(0, groups, CHUNK_GROUPS):
        end = min(g + CHUNK_GROUPS, groups)
        valid = min(end * GROUP, count) - g * GROUP
        chunk = torch.zeros((end - g) * GROUP, dtype=torch.float32)
        chunk[:valid].copy_(flat[g * GROUP:g * GROUP + valid])
        chunk = chunk.view(-1, GROUP)
        if not torch.isfinite(chunk).all():
            raise ValueError("nonfinite quantization input")
        amax = chunk.abs().amax(1)
        if mode == "int4-sym-g128":
            scale = amax / 7
            scale = torch.where(scale == 0, torch.ones_like(scale), scale)
            codes = ((chunk / scale[:, None]).clamp(-7, 7).round() + 8).to(torch.uint8)
        else:
            scale = torch.where(amax == 0, torch.ones_like(amax), amax)
            norm = chunk / scale[:, None]
            codes = torch.searchsorted(mids, norm.contiguous(), side="left").to(torch.uint8)
        scales[g:end].copy_(scale)
        q = codes.flatten().view(-1, 2)
        payload[g * STRIDE:end * STRIDE].copy_((q[:, 0] | (q[:, 1] << 4)).flatten())
    spec = {"version": 1, "shape": list(tensor.shape), "dtype": "bfloat16", "codec": mode,
            "group_size": GROUP, "numel": count}
    return Record(spec, {"payload": payload, "scales": scales})


def validate_spec(spec: dict, parts: dict) -> None:
    """Schema/inventory checks of codecs.py:119-155 for the 4-bit formats."""
    if spec.get("version") != 1 or not isinstance(spec.get("shape"), list) or not spec["shape"] \
            or any(type(n) is not int or n < 1 for n in spec["shape"]):
        raise ValueError("invalid stored weight shape/version")
    check_format(spec.get("codec"))
    count = math.prod(spec["shape"])
    if set(spec) != {"version", "shape", "dtype", "codec", "group_size", "numel"} \
            or spec["group_size"] != GROUP or spec["numel"] != count or spec["dtype"] != "bfloat16":
        raise ValueError("invalid quantized storage schema")
    groups = (count + GROUP - 1) // GROUP
    if set(parts) != {"payload", "scales"} or parts["payload"].dtype != torch.uint8 \
            or tuple(parts["payload"].shape) != (groups * STRIDE,) \
            or parts["scales"].dtype != torch.float32 or tuple(parts["scales"].shape) != (groups,):
        raise ValueError("invalid quantized part inventory/shape/dtype")
    scales = parts["scales"]
    if not torch.isfinite(scales).all() or (scales <= 0).any():
        raise ValueError("invalid stored scales")
    payload = parts["payload"]
    cb = torch.tensor(codebook(spec["codec"]), dtype=torch.float32)
    # bounded chunks of decoded values, as codecs.py:135-154: reserved codes,
    # zero tail padding, and every decoded fp32 product finite as bf16 (a
    # group's largest |value| decides it: the conversion is monotonic)
    for g0 in range(0, groups, VALIDATION_CHUNK_GROUPS):
        g1 = min(g0 + VALIDATION_CHUNK_GROUPS, groups)
        raw = payload[g0 * STRIDE:g1 * STRIDE]
        codes = torch.stack((raw & 15, raw >> 4), 1).flatten().long()
        if spec["codec"] == "int4-sym-g128" and (codes == 0).any():
            raise ValueError("reserved int4 -8 code")
        values = cb[codes]
        valid = max(0, min(values.numel(), count - g0 * GROUP))
        if (values[valid:] != 0).any():
            raise ValueError("nonzero quantized tail padding")
        peak = values.abs().view(-1, GROUP).amax(1) * scales[g0:g1]
        if not torch.isfinite(peak.to(torch.bfloat16)).all():
            raise ValueError("quantized value overflows BF16 compute range")
    if any(t.requires_grad or not t.is_contiguous() for t in parts.values()):
        raise ValueError("invalid trainable/noncontiguous frozen storage")


def decode_into(destination: torch.Tensor, spec: dict, parts: dict) -> None:
    """Decode into a caller-owned bf16 device view with ``st_dequant4``
    (replaces codecs.py:158-170; bit-identical output)."""
    check_format(spec["codec"])
    payload, scales = parts["payload"], parts["scales"]
    if destination.device.type != "cuda" or payload.device != destination.device \
            or scales.device != destination.device:
        raise ValueError("unsupported_capability: decode_into runs on the GPU only")
    if destination.dtype != torch.bfloat16 or not destination.is_contiguous() \
            or destination.numel() != spec["numel"]:
        raise ValueError("decode destination must be a contiguous bf16 view of numel elements")
    lut = _lib.lut_array(codebook(spec["codec"]))
    _lib.call("st_dequant4", _lib.ptr(payload), _lib.ptr(scales), spec["numel"], GROUP, lut, 0,
              _lib.ptr(destination), _lib.stream_handle(destination.device))


def materialize(record: Record, device) -> torch.Tensor:
    value = torch.empty(record.shape, dtype=torch.bfloat16, device=device)
    decode_into(value, record.spec, {k: t.to(device) for k, t in record.parts.items()})
    return value
