"""Model adapters with the reference's factory signature, built from a
4-bit ``rvft.quantized_base.v1`` archive (paths relative to
/root/reference/src/ram_vram_finetune).

The reference's engine builds its model as

    adapter = factory(config.model, rank=, alpha=, device=, host_budget_bytes=,
                      device_budget_bytes=, quantization=, quantized_compute=)

(training/engine.py:127-130) from a name registered with
``register(name, factory, inspector=...)`` (adapters/registry.py:6-15), and
uses the result through the ``ModelAdapter`` protocol: ``blocks``,
``embedding``, ``head``, ``identity``, ``device``, ``positions_and_masks``,
``terminal_norm``, ``artifact_key``, ``runtime_metadata``, ``close``
(adapters/protocol.py:23-34).  :class:`ArchiveDenseAdapter` is that object
for the Llama family (and Qwen3, with its per-head q/k norm) over an archive
that ``archive.export_quantized`` wrote in ``nf4-g128`` or ``int4-sym-g128``
-- the counterpart of DenseDecoderAdapter (adapters/dense.py:178-263):

* every decoder layer is a ``slots.BlockPlan`` whose functional is
  ``dense.dense_block``; its packed image is read from the archive files
  straight into pinned host memory at construction (each file digest-checked
  as it is read) and adopted by ``slots.Q4SlotSession``, so the one change
  in the engine is the session line;
* the embedding stays on the host, the final norm and the head go to the
  device (bf16), as the reference places them;
* ``identity`` is the archive's base identity, recomputed over the buffers
  the records were read into (storage.py:155-163);
* LoRA targets default to the reference's (q, v, o: adapters/targets.py:3-9).

:func:`register_all` registers the factories with a reference-style
``register`` callable.
"""
from __future__ import annotations

import functools
import json
import math
from pathlib import Path

import torch

from . import ops, slots
from .archive import MARKER, ArchiveReader
from .codecs import FORMATS
from .dense import positions_and_masks

# adapters/targets.py:3-9 (checkpoint-stable order)
REFERENCE_TARGETS = ("self_attn.q_proj", "self_attn.v_proj", "self_attn.o_proj")
ALL_TARGETS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
               "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")
_BOUNDARY = ("model.embed_tokens.weight", "model.norm.weight", "lm_head.weight")


def _text_config(raw: dict, family: str) -> dict:
    """The config fields the layer functional needs, with the reference's
    capability checks (adapters/dense.py:40-112) for what this path covers."""
    if raw.get("model_type") != family:
        raise ValueError(f"unsupported_architecture: expected {family}")
    if raw.get("hidden_act", "silu") != "silu" or raw.get("attention_dropout", 0.0) != 0:
        raise ValueError("unsupported_capability: dropout/activation")
    if raw.get("attention_bias", False) or raw.get("mlp_bias", False):
        raise ValueError("unsupported_capability: projection biases")
    if raw.get("pretraining_tp", 1) != 1:
        raise ValueError("unsupported_capability: pretraining_tp")
    rope = dict(raw.get("rope_parameters") or {})
    if not rope:
        rope = {"rope_type": "default", "rope_theta": raw.get("rope_theta", 10000.0)}
    if rope.get("rope_type", "default") != "default" or set(rope) - {"rope_type", "rope_theta"}:
        raise ValueError("unsupported_capability: only default full rotary embeddings")
    theta = float(rope["rope_theta"])
    if not math.isfinite(theta) or theta <= 0:
        raise ValueError("invalid rotary base")
    if raw.get("sliding_window") is not None or raw.get("use_sliding_window", False):
        raise ValueError("unsupported_capability: active or unresolved sliding window")
    heads, hidden = int(raw["num_attention_heads"]), int(raw["hidden_size"])
    head_dim = int(raw.get("head_dim") or hidden // heads)
    eps = float(raw["rms_norm_eps"])
    if not math.isfinite(eps) or eps <= 0:
        raise ValueError("invalid rms_norm_eps")
    tied = bool(raw.get("tie_word_embeddings", False))
    if tied and family != "qwen3":
        raise ValueError("unsupported_capability: tied embeddings")
    return {"layers": int(raw["num_hidden_layers"]), "heads": heads,
            "kv_heads": int(raw.get("num_key_value_heads") or heads), "head_dim": head_dim,
            "eps": eps, "theta": theta, "tied": tied,
            "max_positions": int(raw.get("max_position_embeddings") or 1 << 30)}


class ArchiveDenseAdapter:
    """ModelAdapter of a dense decoder stored as a 4-bit archive (see the
    module docstring).  Constructed by the reference's factory call."""

    family: str | None = None

    def __init__(self, path, *, rank=2, alpha=4.0, device="cpu", host_budget_bytes=1024 ** 3,
                 device_budget_bytes=2 * 1024 ** 3, quantization="none", quantized_compute="bf16",
                 targets=REFERENCE_TARGETS, generator=None):
        if quantized_compute != "bf16":
            raise ValueError("unsupported_quantization: only storage plus BF16 compute")
        if quantization not in FORMATS:
            raise ValueError(f"unsupported_quantization: explicit format required; supported={FORMATS}")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("unsupported_capability: the 4-bit HIP path runs on a GPU device")
        if not torch.cuda.is_available():
            raise RuntimeError("dependency: explicit CUDA requested but unavailable")
        root = Path(path)
        if not (root / MARKER).is_file():
            raise ValueError("unsupported_quantization: not a quantized archive")
        self.reader = reader = ArchiveReader(root, self.family, quantization)
        raw = json.loads((root / "config.json").read_text(encoding="utf-8"))
        cfg = self.config = _text_config(raw, self.family)
        self.quantization = quantization
        self.targets = tuple(targets)
        # metadata-only budget gates before anything is read (dense.py:155-176)
        blocks = [slots.make_archive_block(reader, i, heads=cfg["heads"], kv_heads=cfg["kv_heads"],
                                           head_dim=cfg["head_dim"], eps=cfg["eps"], rank=rank,
                                           alpha=alpha, targets=self.targets, device=self.device,
                                           generator=generator, qk_norm=self.family == "qwen3")
                  for i in range(cfg["layers"])]
        layouts = [slots.plan_layout(b) for b in blocks]
        boundary = {k: reader.entries[k] for k in _BOUNDARY if k in reader.entries}
        if "lm_head.weight" not in boundary and not cfg["tied"]:
            raise ValueError("unsupported_capability: untied checkpoint without lm_head.weight")

        def nbytes(entry):
            spec = entry["spec"]
            return math.prod(spec["shape"]) * (4 if spec.get("dtype") == "float32" else 2)
        host_bytes = sum(l.nbytes for l in layouts) + nbytes(boundary["model.embed_tokens.weight"])
        if host_bytes > host_budget_bytes:
            raise MemoryError("resource_budget: host weights exceed allowance before loading")
        head_key = "lm_head.weight" if "lm_head.weight" in boundary else "model.embed_tokens.weight"
        if nbytes(boundary[head_key]) > device_budget_bytes:
            raise MemoryError("resource_budget: model exceeds host/head allowance before loading")
        # layer images: archive files -> pinned host buffers, adopted by the session
        for b, layout in zip(blocks, layouts):
            img = torch.empty(layout.nbytes, dtype=torch.uint8, pin_memory=True)
            reader.image_loader(f"model.layers.{b.index}.")(b, layout, img)
            b.host_image = img
        records = {k: reader.read(k) for k in boundary}
        self.identity = reader.finish()
        bf = torch.bfloat16
        self.embedding = records["model.embed_tokens.weight"].parts["value"].to(bf).contiguous()
        self.norm = records["model.norm.weight"].parts["value"].to(bf).to(self.device)
        if "lm_head.weight" in records:
            self.head = records["lm_head.weight"].parts["value"].to(bf).to(self.device)
        else:
            self.head = self.embedding.to(self.device)
        self.blocks = blocks
        self.storage_metadata = {
            "format": quantization, "compute": "bf16",
            "storage_identity": reader.meta["storage_identity"],
            "source_identity": reader.meta["source_identity"],
            "total_stored_bytes": reader.stored_bytes, "full_bf16_decoder_retained": False,
            "host_loading": "archive_files_into_pinned_layer_images",
            "decoder_stored_bytes": sum(l.nbytes for l in layouts)}

    # -- ModelAdapter protocol (adapters/protocol.py:23-34) -------------------
    def positions_and_masks(self, valid):
        if valid.dtype != torch.bool or valid.ndim != 2 or valid.shape[1] < 1:
            raise ValueError("unsupported_capability: mask must be 2D bool")
        if valid.shape[1] > self.config["max_positions"]:
            raise ValueError("unsupported_capability: sequence beyond configured context")
        rot, mask = positions_and_masks(valid, head_dim=self.config["head_dim"],
                                        theta=self.config["theta"], device=self.device)
        return rot, {"full_attention": mask}

    def terminal_norm(self, hidden):
        B, S, H = hidden.shape
        return ops.rms_norm(hidden.reshape(B * S, H), self.norm, self.config["eps"]).view(B, S, H)

    def artifact_key(self, layer, target, parameter):
        return f"base_model.model.model.layers.{layer}.{target}.lora_{parameter}.weight"

    def runtime_metadata(self):
        return {"architecture": self.family, "layer_count": len(self.blocks),
                "shared_weights": "frozen_embedding_head_source_alias" if self.config["tied"]
                else "untied",
                "boundary_storage": "CPU embedding plus device head replica",
                "cpu_embedding_bytes": self.embedding.numel() * self.embedding.element_size(),
                "device_head_bytes": self.head.numel() * self.head.element_size(),
                "asynchronous_transfers": "two device slots, one-layer prefetch",
                "kv_cache": "disabled", "rope": "default_full",
                "attention": "flash_GQA_hip", "positions": "absolute_zero_start",
                "resolved_head_dim": self.config["head_dim"], "lora_targets": list(self.targets),
                "storage": dict(self.storage_metadata)}

    def close(self):
        for b in self.blocks:
            b.host_image = None
        self.blocks.clear()
        self.embedding = self.head = self.norm = None


class LlamaArchiveAdapter(ArchiveDenseAdapter):
    family = "llama"


class Qwen3ArchiveAdapter(ArchiveDenseAdapter):
    family = "qwen3"


def inspect_archive(path) -> dict:
    """Inspector for the registry (adapters/registry.py:6-15): the archive's
    marker fields and its layer count, without reading tensor data."""
    root = Path(path)
    meta = json.loads((root / MARKER).read_text(encoding="utf-8"))
    raw = json.loads((root / "config.json").read_text(encoding="utf-8"))
    return {"format": meta.get("format"), "quantization": meta.get("quantization"),
            "family": meta.get("family", raw.get("model_type")),
            "layers": raw.get("num_hidden_layers"), "source_identity": meta.get("source_identity"),
            "storage_identity": meta.get("storage_identity")}


FACTORIES = {"llama_q4_hip": LlamaArchiveAdapter, "qwen3_q4_hip": Qwen3ArchiveAdapter,
             "llama_q4_hip_all_targets": functools.partial(LlamaArchiveAdapter,
                                                           targets=ALL_TARGETS),
             "qwen3_q4_hip_all_targets": functools.partial(Qwen3ArchiveAdapter,
                                                           targets=ALL_TARGETS)}


def register_all(register) -> list:
    """``register(name, factory, inspector=...)`` for every factory above
    (names distinct from the reference's built-in ones, which its registry
    refuses); returns the names."""
    for name, factory in FACTORIES.items():
        register(name, factory, inspector=inspect_archive)
    return list(FACTORIES)


__all__ = ["ArchiveDenseAdapter", "LlamaArchiveAdapter", "Qwen3ArchiveAdapter", "FACTORIES",
           "REFERENCE_TARGETS", "ALL_TARGETS", "inspect_archive", "register_all"]
