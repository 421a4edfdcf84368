"""Projection-level LoRA state (mirror of finetune/lora.py:97-228,319-388 in
/root/reference/src/ram_vram_finetune).

A projection owns fp32 master tensors ``A [rank, in]`` and ``B [out, rank]``
(trainable), fp32 gradient buffers ``grad_A``/``grad_B`` and AdamW moments; the
forward is ``y = bf16(fp32(x W^T) + (alpha/rank) * (x_f32 A^T) B^T)``, executed
by :func:`spilltune_amd.ops.q4_lora_linear` when ``W`` is a 4-bit slot view.
Same field names, shapes, validation messages' meaning and init rule
(``A = randn * 0.02``, ``B = 0``) as the reference, so checkpoints keyed
``{layer}:{target}/{A,B,grad_A,...}`` keep their layout.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

# Llama/Qwen dense decoder projections, in checkpoint-stable order.  The
# reference trains q/v/o by default (adapters/targets.py:2-9); the build's
# headline configuration adapts all seven through the explicit-targets API.
ALL_DENSE_TARGETS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                     "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")
DEFAULT_DENSE_TARGETS = ("self_attn.q_proj", "self_attn.v_proj", "self_attn.o_proj")


def _check_fp32(t, name, shape, device, trainable):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must be FP32, got {t.dtype}")
    if tuple(t.shape) != shape:
        raise ValueError(f"{name} shape mismatch: expected {shape}, got {tuple(t.shape)}")
    if t.device != device:
        raise ValueError(f"{name} must be on {device}, got {t.device}")
    if not trainable and t.requires_grad:
        raise ValueError(f"{name} is an optimizer/gradient buffer and must not require gradients")


@dataclass
class LoRAProjection:
    name: str
    rank: int
    alpha: float
    in_features: int
    out_features: int
    A: torch.Tensor
    B: torch.Tensor
    grad_A: torch.Tensor
    grad_B: torch.Tensor
    m_A: torch.Tensor
    v_A: torch.Tensor
    m_B: torch.Tensor
    v_B: torch.Tensor
    target_path: Optional[str] = None
    layer: Optional[int] = None
    block_type: Optional[str] = None
    architecture: Optional[str] = None

    def __post_init__(self):
        if isinstance(self.rank, bool) or not isinstance(self.rank, int) or self.rank <= 0:
            raise ValueError(f"rank must be a positive integer, got {self.rank!r}")
        self.alpha = float(self.alpha)
        if not math.isfinite(self.alpha):
            raise ValueError(f"alpha must be finite, got {self.alpha!r}")
        if not self.name:
            raise ValueError("LoRA projection name must not be empty")
        self.target_path = self.target_path or self.name
        dev = self.A.device
        r, i, o = self.rank, self.in_features, self.out_features
        _check_fp32(self.A, f"{self.target_path}.A", (r, i), dev, True)
        _check_fp32(self.B, f"{self.target_path}.B", (o, r), dev, True)
        for suffix, shape in (("grad_A", (r, i)), ("grad_B", (o, r)), ("m_A", (r, i)),
                              ("v_A", (r, i)), ("m_B", (o, r)), ("v_B", (o, r))):
            _check_fp32(getattr(self, suffix), f"{self.target_path}.{suffix}", shape, dev, False)
        # private copies, as the reference does, so no two projections share state
        self.A = self.A.detach().clone().requires_grad_(True)
        self.B = self.B.detach().clone().requires_grad_(True)
        for suffix in ("grad_A", "grad_B", "m_A", "v_A", "m_B", "v_B"):
            setattr(self, suffix, getattr(self, suffix).detach().clone())

    @property
    def scale(self) -> float:
        return self.alpha / self.rank

    @property
    def base_weight_shape(self):
        return (self.out_features, self.in_features)

    def zero_grad(self) -> None:
        self.grad_A.zero_()
        self.grad_B.zero_()
        if self.A.grad is not None:
            self.A.grad.zero_()
        if self.B.grad is not None:
            self.B.grad.zero_()


def create_lora_for_block(block_idx: int, block_type: str, weight_shapes: dict, rank: int = 4,
                          alpha: float = 8.0, device=None, *, targets=DEFAULT_DENSE_TARGETS,
                          architecture: Optional[str] = None, generator=None) -> dict:
    """One adapter per target, ``A = randn*0.02``, ``B = 0`` (lora.py:319-388).
    ``weight_shapes`` maps ``<target>.weight`` (or ``<target>``) to ``(out, in)``."""
    if isinstance(block_idx, bool) or not isinstance(block_idx, int) or block_idx < 0:
        raise ValueError(f"block_idx must be a non-negative integer, got {block_idx!r}")
    if isinstance(rank, bool) or not isinstance(rank, int) or rank <= 0:
        raise ValueError(f"rank must be a positive integer, got {rank!r}")
    if not targets or len(set(targets)) != len(targets):
        raise ValueError("LoRA requires an explicit nonempty ordered target mapping")
    device = torch.device("cpu" if device is None else device)
    adapters = {}
    for target in targets:
        shape = weight_shapes.get(target + ".weight", weight_shapes.get(target))
        if shape is None:
            raise ValueError(f"Missing required LoRA target {target!r} in block {block_idx}")
        out_f, in_f = (int(s) for s in shape)
        A = torch.randn(rank, in_f, dtype=torch.float32, generator=generator).mul_(0.02).to(device)
        B = torch.zeros(out_f, rank, dtype=torch.float32, device=device)
        adapters[target] = LoRAProjection(
            name=target, target_path=target, layer=block_idx, block_type=block_type,
            architecture=architecture, rank=rank, alpha=alpha, in_features=in_f,
            out_features=out_f, A=A, B=B, grad_A=torch.zeros_like(A), grad_B=torch.zeros_like(B),
            m_A=torch.zeros_like(A), v_A=torch.zeros_like(A), m_B=torch.zeros_like(B),
            v_B=torch.zeros_like(B))
    share_fused_storage(adapters)
    return adapters


# projections the dense functional runs as one N-concatenated GEMM
FUSED_GROUPS = (("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj"),
                ("mlp.gate_proj", "mlp.up_proj"),
                ("self_attn.q_a_proj", "self_attn.kv_a_proj_with_mqa"),
                ("mlp.shared_experts.gate_proj", "mlp.shared_experts.up_proj"))


def share_fused_storage(adapters: dict, groups=FUSED_GROUPS) -> None:
    """Place the ``A`` (and ``B``) tensors of each fused group in one
    contiguous buffer, in segment order, so the fused GEMM reads
    ``A_cat [sum r, K]`` and ``B_cat [sum N, r]`` as views instead of
    concatenating them on every call.  Each ``A``/``B`` stays a leaf tensor
    of its own (a view of the shared buffer) with the same values; optimizer
    updates in place land in the shared buffer.  Groups whose members differ
    in rank, width, device or are missing are left alone."""
    for group in groups:
        projs = [adapters.get(n) for n in group]
        if any(p is None for p in projs):
            continue
        p0 = projs[0]
        if any(p.rank != p0.rank or p.in_features != p0.in_features or p.A.device != p0.A.device
               for p in projs):
            continue
        A_all = torch.cat([p.A.detach() for p in projs], 0)
        B_all = torch.cat([p.B.detach() for p in projs], 0)
        ra = rb = 0
        for p in projs:
            p.A = A_all[ra:ra + p.rank].requires_grad_(True)
            p.B = B_all[rb:rb + p.out_features].requires_grad_(True)
            ra += p.rank
            rb += p.out_features
