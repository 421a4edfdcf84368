"""Llama/Qwen2/Qwen3 dense decoder block on 4-bit slot weights (HIP path).

``dense_block`` keeps the functional contract of adapters/dense.py:120-153
(/root/reference/src/ram_vram_finetune): called as
``functional(hidden_states, position_embeddings, attention_mask, **weights,
**kwargs)`` by the recompute driver, returns new bf16 hidden states and keeps
no reference to slot memory.  Differences in *how*, not *what*:

* ``weights['<proj>.weight']`` are :class:`~spilltune_amd.ops.Q4Weight` slot
  views (packed 4-bit + fp32 scales), dequantised inside the GEMM;
* LoRA may sit on any of the seven projections (``lora_q`` .. ``lora_down``);
* when q|k|v (and gate|up) are adjacent in the slot they run as one GEMM over
  the concatenated rows, and the residual adds run in the o/down epilogues;
* ``qk_norm`` (Qwen3): each head of q and k is RMS-normalised over head_dim
  by the HIP RMSNorm kernel before RoPE;
* ``attention_mask`` is a :class:`CausalMask` marker: causal attention with
  each row's keys past its valid prefix masked (right padding; none for the
  all-valid rows the engine builds) -- applied structurally by the softmax
  kernel, exactly as adding ``finfo(bf16).min`` does (exp underflows to 0).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import ops


@dataclass(frozen=True)
class CausalMask:
    """The additive mask of dense.py:246-247, [batch, 1, S, S]: causal, and
    with right padding the keys past each row's valid prefix blocked.
    ``lengths`` is None when every row is all valid, else the device int32
    [batch] prefix lengths."""
    batch: int
    length: int
    lengths: torch.Tensor | None = field(default=None, compare=False)


def key_lengths(valid: torch.Tensor, device, what: str = "unsupported_capability: only "
                "all-valid or right-padding masks"):
    """None for all-valid rows, else each row's valid prefix length (device
    int32 [batch]); rows must start valid and never turn valid again after a
    padded position (dense.py:236-237)."""
    if not bool(valid[:, 0].all()) or bool(((~valid[:, :-1]) & valid[:, 1:]).any()):
        raise ValueError(what)
    if bool(valid.all()):
        return None
    return valid.sum(1).to(device=device, dtype=torch.int32)


def positions_and_masks(valid: torch.Tensor, *, head_dim: int, theta: float, device,
                        dtype=torch.bfloat16):
    """Rotary tables (bf16 cos/sin [B,S,D]) and the causal mask marker
    (dense.py:232-248), with the valid prefix lengths of right-padded rows."""
    if valid.dtype != torch.bool or valid.ndim != 2 or valid.shape[1] < 1:
        raise ValueError("unsupported_capability: mask must be 2D bool")
    lengths = key_lengths(valid, device)
    batch, length = valid.shape
    positions = torch.arange(length, device=device).expand(batch, -1)
    inv = 1.0 / theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim)
    freq = (inv[None, :, None].expand(batch, -1, 1) @ positions[:, None].float()).transpose(1, 2)
    phase = torch.cat((freq, freq), -1)
    return (phase.cos().to(dtype), phase.sin().to(dtype)), CausalMask(batch, length, lengths)


def _weight(weights, name):
    w = weights[name + ".weight"]
    if not isinstance(w, ops.Q4Weight):
        raise TypeError(f"{name}.weight must be a 4-bit slot view (Q4Weight), got {type(w).__name__}")
    return w


def dense_block(hidden_states, position_embeddings, attention_mask, *, heads, kv_heads, head_dim,
                eps, lora_q=None, lora_k=None, lora_v=None, lora_o=None, lora_gate=None,
                lora_up=None, lora_down=None, qk_norm=False, feed_forward=None, moe=None,
                lora_experts_gate_up=None, lora_experts_down=None, **weights):
    """``moe`` (``num_experts``, ``top_k``, ``norm_topk_prob``) makes the
    feed-forward the Qwen3-MoE block of qwen3_moe.py:95-113 over the slot's
    ``mlp.experts.*`` stacks, with the optional per-expert LoRA objects
    ``lora_experts_gate_up`` / ``lora_experts_down``."""
    if attention_mask is not None and not isinstance(attention_mask, CausalMask):
        raise ValueError("unsupported_capability: only the causal mask marker is supported")
    if moe is not None and feed_forward is None:
        from . import moe as moe_ops

        def feed_forward(x, w):
            return moe_ops.moe_feed_forward(x, w, lora_gate_up=lora_experts_gate_up,
                                            lora_down=lora_experts_down, **moe)
    B, S, Hd = hidden_states.shape
    cos, sin = position_embeddings
    x2d = hidden_states.reshape(B * S, Hd)
    residual, xn = ops.rms_norm_residual(x2d, weights["input_layernorm.weight"], eps)

    def head_norm(t, name):  # Qwen3: RMSNorm of every head over head_dim (dense.py:128-133)
        if not qk_norm:
            return t
        rows = t.shape[0]
        return ops.rms_norm(t.reshape(-1, head_dim), weights[name], eps).reshape(rows, -1)

    wq, wk, wv = (_weight(weights, f"self_attn.{p}_proj") for p in "qkv")
    qkv = ops.concat_rows([wq, wk, wv])
    loras_qkv = [lora_q, lora_k, lora_v]
    if qkv is not None and ops.lora_fusable(loras_qkv):
        y = ops.q4_lora_linear(xn, qkv, loras_qkv)
        if qk_norm:
            # per-head q/k RMSNorm and the rotation in one kernel each way
            q, k, v = ops.rope_qkv_norm(y, B, S, heads, kv_heads, head_dim, cos, sin,
                                        weights["self_attn.q_norm.weight"],
                                        weights["self_attn.k_norm.weight"], eps)
        else:
            q, k, v = ops.rope_qkv(y, B, S, heads, kv_heads, head_dim, cos, sin)
    else:
        q = ops.rope_heads(head_norm(ops.q4_lora_linear(xn, wq, [lora_q]), "self_attn.q_norm.weight"),
                           0, B, S, heads, head_dim, cos, sin)
        k = ops.rope_heads(head_norm(ops.q4_lora_linear(xn, wk, [lora_k]), "self_attn.k_norm.weight"),
                           0, B, S, kv_heads, head_dim, cos, sin)
        v = ops.rope_heads(ops.q4_lora_linear(xn, wv, [lora_v]), 0, B, S, kv_heads, head_dim, cos,
                           sin, rotate=False)

    kv_len = attention_mask.lengths if attention_mask is not None else None
    attended = ops.causal_attention(q, k, v, ops.attention_scale(head_dim),
                                    kv_len).reshape(B * S, heads * head_dim)
    h1 = ops.q4_lora_linear(attended, _weight(weights, "self_attn.o_proj"), [lora_o], residual=residual)

    h1, xn2 = ops.rms_norm_residual(h1, weights["post_attention_layernorm.weight"], eps)
    if feed_forward is not None:  # e.g. the MoE block (dense.py:152)
        return (h1 + feed_forward(xn2.view(B, S, Hd), weights).reshape(B * S, Hd)).view(B, S, Hd)
    wg, wu = _weight(weights, "mlp.gate_proj"), _weight(weights, "mlp.up_proj")
    gu = ops.concat_rows([wg, wu])
    loras_gu = [lora_gate, lora_up]
    inter = wg.out_features
    wd = _weight(weights, "mlp.down_proj")
    if gu is not None and ops.lora_fusable(loras_gu):
        # down reads silu(gate) * up of the fused gate|up output; its input-
        # gradient GEMM applies the SwiGLU VJP in the epilogue
        out = ops.q4_lora_linear(ops.q4_lora_linear(xn2, gu, loras_gu), wd, [lora_down],
                                 residual=h1, swiglu=True)
    else:
        act = ops.swiglu_pair(ops.q4_lora_linear(xn2, wg, [lora_gate]),
                              ops.q4_lora_linear(xn2, wu, [lora_up]))
        out = ops.q4_lora_linear(act, wd, [lora_down], residual=h1)
    return out.view(B, S, Hd)


def lora_kwargs(adapters: dict) -> dict:
    """Map target paths to the functional's ``lora_*`` keyword arguments."""
    names = {"self_attn.q_proj": "lora_q", "self_attn.k_proj": "lora_k",
             "self_attn.v_proj": "lora_v", "self_attn.o_proj": "lora_o",
             "mlp.gate_proj": "lora_gate", "mlp.up_proj": "lora_up", "mlp.down_proj": "lora_down",
             "mlp.experts.gate_up_proj": "lora_experts_gate_up",
             "mlp.experts.down_proj": "lora_experts_down"}
    return {names[t]: p for t, p in adapters.items()}
