"""ctypes binding of ``libspilltune_hip.so`` (the C ABI in include/spilltune_hip.h).

The library is the only compute path: if it is missing or fails to load, every
op raises instead of falling back (the reference itself forbids implicit
fallback, docs/public/architecture.md:32).  Status codes map to the
reference's exception categories: ``ValueError('unsupported_capability: ..')``
for argument/capability errors, ``RuntimeError`` for device failures.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libspilltune_hip.so"

ST_OK, ST_EINVAL, ST_EUNSUPPORTED, ST_EDEVICE, ST_EWORKSPACE = range(5)
ST_FLAG_HI_NIBBLE_FIRST = 1
ST_FLAG_GROUP64 = 2
ST_DTYPE_BF16, ST_DTYPE_F32 = 0, 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float

# name -> (restype, argtypes)
_SIGNATURES = {
    "st_abi_version": (_I32, []),
    "st_last_error": (ctypes.c_char_p, []),
    "st_dequant4": (_I32, [_P, _P, _I64, _I32, _P, _I32, _P, _P]),
    "st_nf4_dq_scales": (_I32, [_P, _P, _P, _F, _I64, _I32, _P, _P]),
    "st_q4_linear_fwd_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "st_q4_linear_fwd": (_I32, [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I32, _P, _I64, _P, _I32,
                                _F, _I32, _P, _P, _I64, _P, _I64, _P, _I64, _P]),
    "st_q4_linear_dgrad_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "st_q4_linear_dgrad": (_I32, [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I32, _P, _I64, _P,
                                  _I32, _P, _I64, _P, _I64, _P]),
    "st_q4_linear_dgrad_swiglu": (_I32, [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I32, _P, _I64,
                                         _P, _I32, _P, _I64, _P, _I64, _P, _I64, _P]),
    "st_lora_gemm_workspace_bytes": (_I64, [_I64, _I64, _I64]),
    "st_lora_gemm": (_I32, [_I64, _I64, _I64, _P, _I32, _I64, _I64, _P, _I32, _I64, _I64, _F, _P,
                            _I64, _I32, _P, _I64, _P]),
    "st_lora_gemm_noalloc": (_I32, [_I64, _I64, _I64, _P, _I32, _I64, _I64, _P, _I32, _I64, _I64,
                                    _F, _P, _I64, _I32, _P]),
    "st_lora_bwd_dy_workspace_bytes": (_I64, [_I64, _I64, _I32, _I32, _P]),
    "st_lora_bwd_dy": (_I32, [_P, _I64, _I64, _I64, _P, _P, _I64, _I32, _I32, _P, _F, _P, _I64,
                              _P, _P, _I64, _P]),
    "st_rmsnorm_fwd": (_I32, [_P, _P, _I64, _I64, _F, _P, _P, _P]),
    "st_rmsnorm_bwd": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _P, _P]),
    "st_rope_fwd": (_I32, [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I32, _P, _P]),
    "st_rope_bwd": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _I32, _P, _I64, _P]),
    "st_rope_qkv_fwd": (_I32, [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _P]),
    "st_rope_qkv_bwd": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P]),
    "st_rk_batch_workspace_bytes": (_I64, [_I32, _P]),
    "st_rk_batch": (_I32, [_I32, _P, _P, _I64, _P]),
    "st_rope_qkv_norm_fwd": (_I32, [_P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P, _F,
                                    _P, _P, _P, _P, _P]),
    "st_rope_qkv_norm_bwd": (_I32, [_P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64,
                                    _I64, _I64, _P, _I64, _P]),
    "st_heads_to_tokens": (_I32, [_P, _I64, _I64, _I64, _I64, _P, _P]),
    "st_tokens_to_heads": (_I32, [_P, _I64, _I64, _I64, _I64, _P, _P]),
    "st_swiglu_fwd": (_I32, [_P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P]),
    "st_swiglu_bwd": (_I32, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P]),
    "st_linear_bf16_fwd": (_I32, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "st_linear_bf16_dgrad": (_I32, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "st_moe_route_softmax": (_I32, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P]),
    "st_moe_route_softmax_bwd": (_I32, [_P, _P, _P, _I64, _I32, _I32, _I32, _P, _P]),
    "st_moe_route_sigmoid": (_I32, [_P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _F, _P, _P,
                                    _P]),
    "st_moe_route_sigmoid_bwd": (_I32, [_P, _P, _P, _I64, _I32, _I32, _I32, _F, _P, _P]),
    "st_moe_permute": (_I32, [_P, _I64, _I32, _I32, _P, _P, _P, _P]),
    "st_moe_combine": (_I32, [_P, _I64, _P, _P, _P, _I64, _I32, _I64, _P, _P]),
    "st_moe_combine_bwd": (_I32, [_P, _P, _I64, _P, _P, _I64, _I32, _I64, _I32, _P, _P, _P]),
    "st_moe_gather_sum": (_I32, [_P, _I64, _P, _I64, _I32, _I64, _P, _I32, _P, _P]),
    "st_q4_grouped_fwd": (_I32, [_P, _I64, _I64, _P, _I64, _I64, _P, _I32, _P, _P, _I64, _P,
                                 _I32, _P, _I64, _P, _I32, _F, _I32, _P, _P, _I64, _P]),
    "st_q4_grouped_dgrad": (_I32, [_P, _I64, _I64, _I64, _P, _I32, _P, _P, _I64, _P, _I32, _P,
                                   _I64, _P, _I32, _P, _I64, _P]),
    "st_q4_grouped_dgrad_swiglu": (_I32, [_P, _I64, _I64, _I64, _P, _I32, _P, _P, _I64, _P, _I32,
                                          _P, _I64, _P, _I32, _P, _I64, _P, _I64, _P]),
    "st_moe_lora_rows": (_I32, [_I64, _I32, _I64, _I32, _P, _I64, _I64, _P, _P, _I64, _I64, _I64,
                                _P, _I32, _F, _P, _I64, _P]),
    "st_flash_attn_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64, _I32]),
    "st_flash_attn_fwd": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P, _P,
                                 _I64, _P]),
    "st_flash_attn_bwd": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P, _P,
                                 _P, _P, _P, _I64, _P]),
    "st_mla_rope_fwd": (_I32, [_P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64,
                               _I64, _I32, _P, _P, _P, _P]),
    "st_mla_rope_bwd": (_I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P,
                               _I64, _P, _I64, _P, _I64, _P]),
    "st_mla_attn_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64, _I64, _I32]),
    "st_mla_attn_fwd": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P, _P, _I64,
                               _P]),
    "st_mla_attn_bwd": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _P, _P,
                               _P, _P, _P, _I64, _P]),
    "st_cross_entropy_rows": (_I32, [_P, _I64, _I64, _I64, _P, _I64, _F, _P, _P]),
    "st_moe_lora_grads": (_I32, [_I64, _I32, _I64, _I32, _P, _I64, _I64, _P, _P, _I64, _I64, _P,
                                 _I32, _F, _P, _I64, _I64, _I64, _I32, _P]),
}

EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


class KernelError(RuntimeError):
    """A device/runtime failure reported by the kernel library."""


def load():
    """Load and bind the library once; raise loudly when it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"dependency: {LIB_PATH.name} is not built; run "
                    "`python __graft_entry__.py build` (make -C spilltune_amd/csrc)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.st_abi_version() != 1:
                raise RuntimeError("dependency: libspilltune_hip.so ABI version mismatch")
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc == ST_OK:
        return
    msg = _lib.st_last_error().decode(errors="replace")
    if rc in (ST_EINVAL, ST_EUNSUPPORTED, ST_EWORKSPACE):
        raise ValueError(f"unsupported_capability: {what}: {msg}")
    raise KernelError(f"{what}: {msg}")


def call(name: str, *args) -> None:
    lib = load()
    check(getattr(lib, name)(*args), name)


def query(name: str, *args) -> int:
    return int(getattr(load(), name)(*args))


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_handle(device: torch.device | None = None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class RkProduct(ctypes.Structure):
    """``st_rk_product`` (include/spilltune_hip.h): one product of st_rk_batch."""
    _fields_ = [("G", ctypes.c_void_p), ("ldg", ctypes.c_int64), ("col", ctypes.c_int32),
                ("S", ctypes.c_void_p), ("ssk", ctypes.c_int64), ("ssj", ctypes.c_int64),
                ("big", ctypes.c_int64), ("r", ctypes.c_int64), ("Kc", ctypes.c_int64),
                ("alpha", ctypes.c_float), ("out", ctypes.c_void_p), ("so_m", ctypes.c_int64),
                ("so_j", ctypes.c_int64), ("accumulate", ctypes.c_int32)]


def lut_array(values) -> ctypes.Array:
    arr = (ctypes.c_float * 16)(*[float(v) for v in values])
    return arr


def i64_array(values) -> ctypes.Array:
    return (ctypes.c_int64 * max(1, len(values)))(*[int(v) for v in values])
