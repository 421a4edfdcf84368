"""The C ABI library loads, exports exactly what include/spilltune_hip.h
declares, and rejects bad arguments before touching the device (CPU only)."""
import ctypes
import re
from pathlib import Path

import pytest

from spilltune_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "spilltune_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(st_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(_lib.EXPORTED) == names


def test_abi_version_and_error_mapping():
    lib = _lib.load()
    assert lib.st_abi_version() == 1
    lut = _lib.lut_array(range(16))
    with pytest.raises(ValueError, match="group must be 64 or 128"):
        _lib.call("st_dequant4", None, None, 10, 96, lut, 0, None, None)
    with pytest.raises(ValueError, match="NULL"):
        _lib.call("st_dequant4", None, None, 10, 128, lut, 0, None, None)
    # zero-size work is a no-op that succeeds without a device
    _lib.call("st_dequant4", None, None, 0, 128, lut, 0, None, None)
    with pytest.raises(ValueError, match="multiple of 8"):
        _lib.call("st_q4_linear_dgrad", ctypes.c_void_p(16), 4, 100, 100, ctypes.c_void_p(16),
                  ctypes.c_void_p(16), 128, lut, 0, None, 0, None, 0, ctypes.c_void_p(16), 128,
                  None, 0, None)
    with pytest.raises(ValueError, match="dtype codes"):
        _lib.call("st_lora_gemm", 4, 4, 4, ctypes.c_void_p(16), 7, 1, 1, ctypes.c_void_p(16), 0,
                  1, 1, 1.0, ctypes.c_void_p(16), 4, 0, None, 0, None)


def test_lora_rank_limits_rejected_before_any_launch():
    """Rank bounds of the LoRA entry points: checked on the host, before any
    device work (fake pointers never reach a kernel)."""
    lut = _lib.lut_array(range(16))
    p = ctypes.c_void_p(16)
    ends = _lib.i64_array([256])

    def fwd(rank):
        _lib.call("st_q4_linear_fwd", p, 4, 256, 256, p, p, 256, lut, 0, p, 256, p, rank, 1.0, 1,
                  ends, None, 0, p, 256, None, 0, None)
    for rank in (0, -3, 70000):
        with pytest.raises(ValueError, match="out of range"):
            fwd(rank)
    # the batched dY-side products take r <= 64: the query says so with 0
    assert _lib.query("st_lora_bwd_dy_workspace_bytes", 2048, 4096, 16, 1, _lib.i64_array([4096])) > 0
    assert _lib.query("st_lora_bwd_dy_workspace_bytes", 2048, 4096, 65, 1, _lib.i64_array([4096])) == 0
    with pytest.raises(ValueError, match="rank must be 1..64"):
        _lib.call("st_lora_bwd_dy", p, 4, 256, 256, p, p, 65, 65, 1, ends, 1.0, p, 65, None, p,
                  1 << 20, None)
    with pytest.raises(ValueError, match="0 < R"):
        _lib.call("st_moe_lora_rows", 4, 0, 256, 1, p, 256, 4, None, p, 1, 256, 0, p, 1, 1.0, p,
                  1, None)


def test_workspace_queries():
    assert _lib.query("st_q4_linear_fwd_workspace_bytes", 16, 256, 4096) == 0
    # K % 128 != 0 runs on the flat-group kernels from the packed weight
    assert _lib.query("st_q4_linear_fwd_workspace_bytes", 16, 256, 688) == 0
    assert _lib.query("st_q4_linear_dgrad_workspace_bytes", 16, 256, 688) == 0
    ws = _lib.query("st_lora_gemm_workspace_bytes", 2048, 16, 4096)
    assert ws > 0 and ws % (2048 * 16 * 4) == 0


def test_product_does_not_import_the_oracle():
    root = Path(__file__).resolve().parents[1] / "spilltune_amd"
    for path in root.rglob("*.py"):
        src = path.read_text()
        assert "import oracle" not in src and "from oracle" not in src, path
