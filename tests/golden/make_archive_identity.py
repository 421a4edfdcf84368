"""Golden identities of a quantized archive, written by the reference's loader.

`checkpoint(root)` writes a small synthetic checkpoint (seeded tensors: bf16
matrices with and without a 128-element group tail, a bf16 norm, an fp32
raw tensor) and returns the adapter report that drives an export.  Run with
the reference's source tree as argument, this script feeds that checkpoint
through the reference's `WeightLoader` (quantization/storage.py:89-165:
`read` of every required key, then `finish`) in int4-sym-g128, the one
quantized format both builds share, and writes `archive_identity.json`: the
source, storage and base identities and the stored byte count.  The fixture
is data only; tests rebuild the checkpoint with `checkpoint` and compare
`archive.export_quantized`'s identities with it.

    python tests/golden/make_archive_identity.py /root/reference/src
"""
from __future__ import annotations

import json
import sys
import tempfile
from pathlib import Path

import torch
from safetensors.torch import save_file

MODE = "int4-sym-g128"
FIXTURE = Path(__file__).resolve().parent / "archive_identity.json"


def checkpoint(root: Path) -> dict:
    """Write model.safetensors under ``root``; return the export report."""
    g = torch.Generator().manual_seed(20240611)
    tensors = {
        "model.layers.0.self_attn.q_proj.weight": (torch.randn(64, 200, generator=g) * 0.02).to(torch.bfloat16),
        "model.layers.0.mlp.down_proj.weight": (torch.randn(33, 7, generator=g) * 0.05).to(torch.bfloat16),
        "model.layers.0.input_layernorm.weight": (1.0 + torch.randn(200, generator=g) * 0.1).to(torch.bfloat16),
        "model.layers.0.router.bias": torch.randn(9, generator=g),
    }
    root.mkdir(parents=True, exist_ok=True)
    file = root / "model.safetensors"
    save_file(tensors, str(file))
    keys = sorted(tensors)
    entries = {k: {"file": str(file), "shape": list(t.shape),
                   "dtype": "F32" if t.dtype == torch.float32 else "BF16"} for k, t in tensors.items()}
    return {
        "text_config": {"hidden_size": 200, "num_hidden_layers": 1, "model_type": "llama",
                        "rms_norm_eps": 1e-5},
        "entries": entries,
        "required": keys,
        "quantization_matrix_keys": ["model.layers.0.mlp.down_proj.weight",
                                     "model.layers.0.self_attn.q_proj.weight"],
        "quantization_fp32_keys": ["model.layers.0.router.bias"],
        "quantized_export": {"version": 1, "formats": [MODE], "rejection_reason": ""},
    }


def main(reference_src: str) -> None:
    sys.path.insert(0, reference_src)
    from ram_vram_finetune.quantization.storage import WeightLoader

    with tempfile.TemporaryDirectory() as tmp:
        report = checkpoint(Path(tmp) / "src")
        loader = WeightLoader(Path(tmp) / "src", report, MODE)
        for key in report["required"]:
            loader.read(key)
        identity = loader.finish()
        out = {"mode": MODE, "source_identity": loader.source_identity,
               "storage_identity": loader.storage_identity, "identity": identity,
               "stored_bytes": loader.stored_bytes, "quantized_tensors": loader.quantized_tensors}
    FIXTURE.write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")
    print(json.dumps(out, indent=1, sort_keys=True))


if __name__ == "__main__":
    main(sys.argv[1])
