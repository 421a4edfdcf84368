"""bitsandbytes NF4 + double-quantisation state on the fused 4-bit GEMMs.

The reference's NF4 path (paths relative to /root/reference/src/ram_vram_finetune)
keeps each frozen matrix as bitsandbytes 0.50.2 state:
``quantize_4bit(blocksize=64, compress_statistics=True, quant_type="nf4")``
(quantization/nf4_backend.py:292-298), exported as a packed uint8 ``[bytes, 1]``
tensor plus five parts -- ``absmax`` (uint8 codes, one per 64 flat elements),
``quant_map`` (the NF4 codebook), ``nested_absmax`` (fp32, one per 256
blocks), ``nested_quant_map`` (256 fp32 entries) and the JSON metadata tensor
``quant_state.bitsandbytes__nf4`` (nf4_backend.py:17-24,184-240).  Its CUDA
path pins those six parts, stages them on a copy stream and runs
``matmul_4bit`` (nf4_backend_cuda.py:300-519,748-837,888-917).

This module takes the same parts:

* :func:`validate_parts` -- the shape and metadata rules of
  nf4_backend.py:184-240 and nf4_backend_cuda.py:314-380 (same error texts),
  except the comparison of the 256-entry nested map with bitsandbytes' own
  generated table, which needs the library (absent here); the map is taken as
  data and must be 256 finite fp32 values in [-1, 1].
* :func:`dq_scales_host` -- the block scales the state encodes, on the host:
  ``absmax_j = fp32(fp32(map[q_j] * nested[j // 256]) + offset)``.
* :class:`PinnedNF4State` / :meth:`PinnedNF4State.stage` -- pinned host
  copies, staged with ``non_blocking`` copies on a caller's stream and
  converted on the device by ``st_nf4_dq_scales`` into a :class:`ops.Q4Weight`
  whose GEMMs read the packed bytes as they lie (high nibble first,
  ``ST_FLAG_GROUP64``): W is never written to HBM as bf16.
* :func:`linear_cuda` -- the base linear of nf4_backend_cuda.py:888-917 on
  the fused GEMM (autograd: the input gradient on the fused dgrad GEMM).

bitsandbytes' own bytes (its quantiser's choices, its generated nested map)
are not reproduced here and no reference test holds them; decoding a given
state is exact.
"""
from __future__ import annotations

import json
import math
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib, ops
from .codecs import NF4_CODEBOOK

PRIMARY_BLOCKSIZE = 64        # nf4_backend.py:16
SECONDARY_BLOCKSIZE = 256     # nf4_backend.py:17
PACKED_STATE_KEY = "quant_state.bitsandbytes__nf4"   # nf4_backend.py:18
EXPECTED_KEYS = frozenset({"absmax", "nested_absmax", "nested_quant_map", "quant_map",
                           PACKED_STATE_KEY})
EXPECTED_META_KEYS = frozenset({"quant_type", "blocksize", "dtype", "shape", "nested_blocksize",
                                "nested_dtype", "nested_offset"})
CODEC = "nf4-g128"            # codebook name of Q4Weight (the NF4 table)
FLAGS = _lib.ST_FLAG_HI_NIBBLE_FIRST | _lib.ST_FLAG_GROUP64


def pack_metadata(meta: dict) -> torch.Tensor:
    """The metadata part: UTF-8 JSON bytes in a uint8 tensor (bitsandbytes'
    tensor form of a dict)."""
    return torch.tensor(list(json.dumps(meta).encode("utf-8")), dtype=torch.uint8)


def unpack_metadata(t: torch.Tensor) -> dict:
    if not torch.is_tensor(t) or t.dtype != torch.uint8:
        raise ValueError("packed quant-state metadata must use uint8 storage")
    if t.ndim != 1 or t.numel() == 0:
        raise ValueError("packed quant-state metadata must be a nonempty one-dimensional tensor")
    try:
        meta = json.loads(bytes(t.cpu().numpy().tobytes()).decode("utf-8"))
    except Exception as exc:
        raise ValueError("packed quant-state metadata is malformed") from exc
    if not isinstance(meta, dict):
        raise ValueError("packed quant-state metadata must decode to a dictionary")
    return meta


@dataclass(frozen=True)
class NF4StateInfo:
    shape: tuple
    elements: int
    blocks: int
    nested_blocks: int
    offset: float


def _cpu_tensor(value, name):
    if not torch.is_tensor(value):
        raise TypeError(f"{name} must be a torch.Tensor")
    if value.device.type != "cpu":
        raise ValueError(f"{name} must be on CPU, got {value.device}")
    return value


def validate_parts(packed: torch.Tensor, parts) -> NF4StateInfo:
    """The reference's state rules (nf4_backend.py:184-240), raising its
    ValueError texts; returns the logical shape, block counts and offset."""
    _cpu_tensor(packed, "packed")
    if packed.dtype != torch.uint8:
        raise TypeError(f"packed must have dtype {torch.uint8}, got {packed.dtype}")
    if packed.ndim != 2 or packed.shape[1] != 1:
        raise ValueError("packed must use the official uint8 [bytes, 1] layout")
    if not hasattr(parts, "keys"):
        raise TypeError("quant_state_parts must be a mapping")
    keys = set(parts.keys())
    if keys != EXPECTED_KEYS:
        missing = sorted(EXPECTED_KEYS.difference(keys))
        extra = sorted(repr(k) for k in keys.difference(EXPECTED_KEYS))
        raise ValueError(f"malformed quant_state_parts keys (missing={missing}, extra={extra})")
    for key, value in parts.items():
        _cpu_tensor(value, f"quant_state_parts[{key!r}]")
    meta = unpack_metadata(parts[PACKED_STATE_KEY])
    if set(meta) != EXPECTED_META_KEYS:
        raise ValueError("packed quant-state metadata has missing or unknown fields")
    if meta["quant_type"] != "nf4":
        raise ValueError("only official NF4 quantization state is supported")
    if type(meta["blocksize"]) is not int or meta["blocksize"] != PRIMARY_BLOCKSIZE:
        raise ValueError("NF4 state must use blocksize 64")
    if type(meta["nested_blocksize"]) is not int or meta["nested_blocksize"] != SECONDARY_BLOCKSIZE:
        raise ValueError("double-quantization state must use secondary blocksize 256")
    if meta["dtype"] != "bfloat16" or meta["nested_dtype"] != "float32":
        raise ValueError("NF4/DQ state has an unsupported compute or nested dtype")
    shape = meta["shape"]
    if (not isinstance(shape, list) or len(shape) != 2
            or any(type(e) is not int or e <= 0 for e in shape)):
        raise ValueError("NF4 state shape must contain two positive integer dimensions")
    elements = shape[0] * shape[1]
    if packed.numel() != (elements + 1) // 2:
        raise ValueError("packed byte count does not match the NF4 state shape")
    blocks = (elements + PRIMARY_BLOCKSIZE - 1) // PRIMARY_BLOCKSIZE
    nested_blocks = (blocks + SECONDARY_BLOCKSIZE - 1) // SECONDARY_BLOCKSIZE
    absmax, nested = parts["absmax"], parts["nested_absmax"]
    nested_map, nf4_map = parts["nested_quant_map"], parts["quant_map"]
    if absmax.dtype != torch.uint8 or absmax.ndim != 1 or absmax.numel() != blocks:
        raise ValueError("primary NF4 absmax state has an invalid dtype or shape")
    if nested.dtype != torch.float32 or nested.ndim != 1 or nested.numel() != nested_blocks:
        raise ValueError("secondary DQ absmax state has an invalid dtype or shape")
    if nested_map.dtype != torch.float32 or nested_map.ndim != 1 or nested_map.numel() != 256:
        raise ValueError("secondary DQ codebook must be a 256-entry float32 vector")
    if nf4_map.dtype != torch.float32 or nf4_map.ndim != 1 or nf4_map.numel() != 16:
        raise ValueError("NF4 codebook must be a 16-entry float32 vector")
    offset = meta["nested_offset"]
    if type(offset) not in (int, float) or not math.isfinite(offset) or offset < 0:
        raise ValueError("secondary DQ offset must be finite and non-negative")
    if float(np.float32(offset)) != float(offset):
        # the library rebuilds the offset as an fp32 tensor and the reference
        # requires it to equal the metadata value (nf4_backend_cuda.py:372-375)
        raise ValueError("decoded official QuantState does not match the canonical record")
    if not bool(torch.isfinite(nested).all()):
        raise ValueError("secondary DQ absmax state contains a non-finite value")
    if not bool((nested >= 0).all()):
        raise ValueError("secondary DQ absmax values must be non-negative")
    if not torch.equal(nf4_map, torch.tensor(NF4_CODEBOOK, dtype=torch.float32)):
        raise ValueError("NF4 state codebook does not match the official NF4 codebook")
    if not bool(torch.isfinite(nested_map).all()) or not bool((nested_map.abs() <= 1).all()):
        raise ValueError("secondary DQ codebook does not match the official dynamic map")
    return NF4StateInfo(tuple(shape), elements, blocks, nested_blocks, float(offset))


def dq_scales_host(absmax_q, nested_absmax, nested_map, offset: float) -> np.ndarray:
    """Per-64 fp32 block scales of the state, on the host:
    fp32(fp32(map[q_j] * nested[j // 256]) + offset) (bitsandbytes' blockwise
    dequantize of the statistics, then ``absmax += offset``)."""
    q = np.asarray(absmax_q, dtype=np.uint8).reshape(-1)
    nested = np.asarray(nested_absmax, dtype=np.float32).reshape(-1)
    m = np.asarray(nested_map, dtype=np.float32).reshape(-1)
    idx = np.arange(q.size, dtype=np.int64) // SECONDARY_BLOCKSIZE
    prod = (m[q] * nested[idx]).astype(np.float32)          # fp32 product
    return (prod + np.float32(offset)).astype(np.float32)   # fp32 sum


def dq_scales_device(absmax_q: torch.Tensor, nested_absmax: torch.Tensor,
                     nested_map: torch.Tensor, offset: float, out: torch.Tensor | None = None,
                     stream=None) -> torch.Tensor:
    """The same scales on the device (``st_nf4_dq_scales``)."""
    blocks = absmax_q.numel()
    if out is None:
        out = torch.empty(blocks, dtype=torch.float32, device=absmax_q.device)
    for t in (absmax_q, nested_absmax, nested_map, out):
        if not t.is_cuda or not t.is_contiguous():
            raise ValueError("unsupported_capability: dq_scales_device takes contiguous device tensors")
    _lib.call("st_nf4_dq_scales", _lib.ptr(absmax_q), _lib.ptr(nested_absmax), _lib.ptr(nested_map),
              float(offset), blocks, SECONDARY_BLOCKSIZE, _lib.ptr(out),
              stream if stream is not None else _lib.stream_handle(absmax_q.device))
    return out


class PinnedNF4State:
    """Pinned host copies of one validated state (the six parts
    nf4_backend_cuda.py:383-402 pins), staged on demand."""

    def __init__(self, packed: torch.Tensor, parts) -> None:
        info = validate_parts(packed, parts)
        self.info = info
        self.shape = info.shape
        self.offset = info.offset

        def pin(t):
            return t.detach().contiguous().reshape(-1).pin_memory()
        self.packed = pin(packed)
        self.absmax = pin(parts["absmax"])
        self.nested_absmax = pin(parts["nested_absmax"])
        self.nested_quant_map = pin(parts["nested_quant_map"])
        self.metadata = unpack_metadata(parts[PACKED_STATE_KEY])
        self.nbytes = sum(t.numel() * t.element_size() for t in
                          (self.packed, self.absmax, self.nested_absmax, self.nested_quant_map))

    def stage(self, device, stream: torch.cuda.Stream | None = None) -> "StagedNF4":
        """Copy the parts to ``device`` with ``non_blocking`` copies on
        ``stream`` (default: the current stream), convert the block scales
        there, and record a ready event on it (nf4_backend_cuda.py:748-837)."""
        device = torch.device(device)
        stream = stream if stream is not None else torch.cuda.current_stream(device)
        with torch.cuda.stream(stream):
            payload = self.packed.to(device, non_blocking=True)
            absmax = self.absmax.to(device, non_blocking=True)
            nested = self.nested_absmax.to(device, non_blocking=True)
            nmap = self.nested_quant_map.to(device, non_blocking=True)
            scales = dq_scales_device(absmax, nested, nmap, self.offset, stream=stream.cuda_stream)
            ready = torch.cuda.Event()
            ready.record(stream)
        # absmax/nested/nmap are read only by the conversion on `stream`,
        # where they were allocated; consumers record their own streams
        weight = ops.Q4Weight(payload, scales, self.shape, CODEC, flags=FLAGS)
        return StagedNF4(weight, ready, stream)


@dataclass
class StagedNF4:
    """A staged state: the fused GEMMs' weight and the event its copies and
    scale conversion recorded."""
    weight: ops.Q4Weight
    ready: torch.cuda.Event
    stream: torch.cuda.Stream

    @property
    def shape(self):
        return self.weight.shape

    def wait_on(self, consumer: torch.cuda.Stream) -> None:
        """Order ``consumer`` after the staging and keep the weight's memory
        from being reused before ``consumer``'s work on it completes."""
        consumer.wait_event(self.ready)
        if consumer != self.stream:
            self.weight.payload.record_stream(consumer)
            self.weight.scales.record_stream(consumer)

    def synchronize_ready(self) -> None:
        self.ready.synchronize()


def linear_cuda(inputs: torch.Tensor, state) -> torch.Tensor:
    """Base linear of a staged state (nf4_backend_cuda.py:888-917): y = x W^T
    in bf16 with fp32 accumulation, W decoded inside the GEMM; differentiable
    in ``inputs`` (the fused dgrad GEMM)."""
    weight = state.weight if isinstance(state, StagedNF4) else state
    if not isinstance(weight, ops.Q4Weight):
        raise TypeError("exact owned CUDA record required")
    if not isinstance(inputs, torch.Tensor):
        raise TypeError("inputs must be a torch.Tensor")
    if inputs.device.type != "cuda":
        raise ValueError("inputs must be on a CUDA device")
    if inputs.dtype is not torch.bfloat16:
        raise TypeError("inputs must have dtype torch.bfloat16")
    if inputs.ndim < 1:
        raise ValueError("inputs must have at least one dimension")
    if inputs.shape[-1] != weight.shape[1]:
        raise ValueError(f"input feature size {inputs.shape[-1]} does not match NF4 weight size "
                         f"{weight.shape[1]}")
    if isinstance(state, StagedNF4):
        state.wait_on(torch.cuda.current_stream(inputs.device))
    y = ops.q4_lora_linear(inputs.reshape(-1, weight.shape[1]), weight, None)
    return y.view(*inputs.shape[:-1], weight.shape[0])
