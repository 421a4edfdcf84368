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
