"""ctypes binding of the C codec oracle (``oracle/codec.c``).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Pinning:
* ``decode4`` with the int4-sym-g128 codebook: the reference's known-answer
  vector (tests/test_quantization.py:73-81: values [-7,-1.5,-.5,.5,1.5,7] ->
  bytes [0x61,0x88,0xfa] -> [-7,-2,0,0,2,7]), its zero-group scale rule
  (test_quantization.py:63,70), its payload size rule (:69) and a
  pure-Python scalar decoder written from the closed form (test_quantization.py
  :43-56 restated) on tails 128/129/257 and a chunk-boundary length.
* ``decode4`` with the NF4 codebook: brute force of all 16 codes x edge
  scales against Python float arithmetic, the invariants |w| <= absmax,
  code 7 -> +0, codes 0/15 -> -/+absmax.
* ``dq_absmax`` (bitsandbytes' double-quantised NF4 statistics; the library,
  bitsandbytes==0.50.2, is absent and no reference test holds its bytes):
  closed forms a plausible mistake fails -- a zero map gives the offset
  exactly; nested scales that change every 256 blocks (j // 256 against
  j // 64); an offset added after the rounded product (not folded into the
  scale); power-of-two operands where every step is exact against Python
  float arithmetic; ragged block counts.
* ``dynamic_map`` / ``encode_nf4_dq``: test inputs only (a restatement of
  bitsandbytes' ``create_dynamic_map`` from its published description and a
  nearest-entry quantiser).  Parity unpinned: bitsandbytes' own tables and
  quantiser choices are not reproduced bit for bit; nothing checked against
  the GPU depends on them (the decode takes the map and codes as data).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle_codec.so"

NF4_LUT = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
    0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0], dtype=np.float32)

INT4_LUT = (np.arange(16, dtype=np.float32) - 8.0).astype(np.float32)

_lib = None


def build() -> Path:
    """Compile the C oracle with gcc (no reference build is involved)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.st_oracle_decode4.argtypes = [P, P, I64, ctypes.c_int, P, ctypes.c_int, P]
        L.st_oracle_decode4.restype = None
        L.st_oracle_encode_int4.argtypes = [P, I64, P, P]
        L.st_oracle_encode_int4.restype = ctypes.c_int
        L.st_oracle_encode_nf4.argtypes = [P, I64, ctypes.c_int, P, P]
        L.st_oracle_encode_nf4.restype = ctypes.c_int
        L.st_oracle_dq_absmax.argtypes = [P, P, I64, ctypes.c_int, P, ctypes.c_float, P]
        L.st_oracle_dq_absmax.restype = None
        L.st_oracle_bf16_rne.argtypes = [ctypes.c_float]
        L.st_oracle_bf16_rne.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


def groups_of(numel: int, group: int = 128) -> int:
    return (numel + group - 1) // group


def decode4(payload: np.ndarray, scales: np.ndarray, numel: int, *, lut: np.ndarray,
            group: int = 128, hi_first: bool = False) -> np.ndarray:
    """bf16 bit patterns (uint16) of bf16(lut[code_i] * scales[i // group])."""
    payload = np.ascontiguousarray(payload, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    lut = np.ascontiguousarray(lut, dtype=np.float32)
    if payload.size * 2 < numel or scales.size < groups_of(numel, group):
        raise ValueError("payload/scales too small for numel")
    out = np.empty(numel, dtype=np.uint16)
    lib().st_oracle_decode4(_ptr(payload), _ptr(scales), numel, group, _ptr(lut),
                            int(hi_first), _ptr(out))
    return out


def encode_int4(x: np.ndarray):
    """int4-sym-g128 encode (codecs.py:81-116) -> (payload uint8, scales fp32)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    g = groups_of(x.size)
    payload = np.empty(g * 64, dtype=np.uint8)
    scales = np.empty(g, dtype=np.float32)
    if lib().st_oracle_encode_int4(_ptr(x), x.size, _ptr(payload), _ptr(scales)) != 0:
        raise ValueError("nonfinite quantization input")
    return payload, scales


def encode_nf4(x: np.ndarray, *, hi_first: bool = False):
    """nf4-g128 encode (nearest codebook entry, ties to the lower code)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    g = groups_of(x.size)
    payload = np.empty(g * 64, dtype=np.uint8)
    scales = np.empty(g, dtype=np.float32)
    if lib().st_oracle_encode_nf4(_ptr(x), x.size, int(hi_first), _ptr(payload), _ptr(scales)) != 0:
        raise ValueError("nonfinite quantization input")
    return payload, scales


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Vectorised RNE fp32 -> bf16 bits (finite inputs), same rule as codec.c."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def dq_absmax(q: np.ndarray, nested: np.ndarray, nested_map: np.ndarray, offset: float,
              nested_block: int = 256) -> np.ndarray:
    """fp32 block absmax of a double-quantised NF4 state:
    fp32(fp32(map[q_j] * nested[j // nested_block]) + offset)."""
    q = np.ascontiguousarray(q, dtype=np.uint8).reshape(-1)
    nested = np.ascontiguousarray(nested, dtype=np.float32).reshape(-1)
    m = np.ascontiguousarray(nested_map, dtype=np.float32).reshape(-1)
    if m.size != 256 or nested.size < (q.size + nested_block - 1) // nested_block:
        raise ValueError("nested map must have 256 entries and one scale per nested block")
    out = np.empty(q.size, dtype=np.float32)
    lib().st_oracle_dq_absmax(_ptr(q), _ptr(nested), q.size, nested_block, _ptr(m),
                              float(np.float32(offset)), _ptr(out))
    return out


def dynamic_map() -> np.ndarray:
    """256-entry signed map of dynamic (tree) quantisation, the nested map
    bitsandbytes' double quantisation uses (create_dynamic_map(signed=True,
    max_exponent_bits=7, total_bits=8)): for exponents i = 0..6, the 2**i
    midpoints of a uniform split of [0.1, 1] scaled by 10**(i - 6), both
    signs, plus 0 and 1, sorted.  Test input only (see the module header)."""
    vals = [0.0, 1.0]
    for i in range(7):
        b = np.linspace(0.1, 1.0, 2 ** i + 1, dtype=np.float32)
        mid = ((b[:-1] + b[1:]) / np.float32(2.0)).astype(np.float32)
        scaled = (mid * np.float32(10.0 ** (i - 6))).astype(np.float32)
        vals += scaled.tolist() + (-scaled).tolist()
    assert len(vals) == 256
    return np.array(sorted(vals), dtype=np.float32)


def encode_nf4_dq(w: np.ndarray, nested_map: np.ndarray | None = None):
    """A double-quantised NF4 state for tests: per 64 flat elements absmax
    (0 -> every code 7), codes = nearest NF4 entry (ties to the lower code),
    packed HIGH nibble first into (n+1)//2 bytes; offset = mean absmax; per
    256 blocks nested = max |absmax - offset| (0 -> 1), code = nearest map
    entry to (absmax - offset) / nested.  Returns (packed uint8, absmax_q
    uint8, nested fp32, offset float, nested_map fp32)."""
    x = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    n = x.size
    m = dynamic_map() if nested_map is None else np.asarray(nested_map, dtype=np.float32)
    blocks = (n + 63) // 64
    xp = np.zeros(blocks * 64, dtype=np.float32)
    xp[:n] = x
    xb = xp.reshape(blocks, 64)
    absmax = np.abs(xb).max(1).astype(np.float32)
    safe = np.where(absmax > 0, absmax, np.float32(1.0)).astype(np.float32)
    v = (xb / safe[:, None]).astype(np.float32)
    codes = np.abs(v[..., None] - NF4_LUT[None, None, :]).argmin(-1).astype(np.uint8)
    codes[absmax == 0] = 7
    flat = codes.reshape(-1)[:n]
    if n % 2:
        flat = np.concatenate([flat, np.zeros(1, np.uint8)])
    packed = ((flat[0::2] << 4) | flat[1::2]).astype(np.uint8)
    offset = np.float32(absmax.mean(dtype=np.float32))
    centred = (absmax - offset).astype(np.float32)
    nb = (blocks + 255) // 256
    cp = np.zeros(nb * 256, dtype=np.float32)
    cp[:blocks] = centred
    nested = np.abs(cp.reshape(nb, 256)).max(1).astype(np.float32)
    nested = np.where(nested > 0, nested, np.float32(1.0)).astype(np.float32)
    ratio = (cp.reshape(nb, 256) / nested[:, None]).reshape(-1)[:blocks]
    q = np.abs(ratio[:, None] - m[None, :]).argmin(-1).astype(np.uint8)
    return packed, q, nested, float(offset), m
