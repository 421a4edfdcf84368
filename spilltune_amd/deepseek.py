"""DeepSeek-V3 decoder block -- multi-head latent attention plus the routed /
shared-expert MoE (or a dense MLP) -- on 4-bit slot weights (HIP path).

``deepseek_block`` keeps the functional contract of adapters/deepseek.py:
129-176 (/root/reference/src/ram_vram_finetune): called as
``functional(hidden_states, position_embeddings, attention_mask, **weights,
parameters=..., lora_*=...)`` by the recompute driver, with the reference's
``parameters`` keys, and returns the new bf16 hidden states.  How it runs:

* q_a_proj and kv_a_proj_with_mqa (both read the normalised input) run as one
  fused 4-bit GEMM when their storage is adjacent in the slot;
* the latent RMSNorms (eps 1e-6) are the HIP RMSNorm kernels;
* ``st_mla_rope_fwd`` assembles the per-head query (q_nope | rotated q_rope)
  and key (k_nope | the shared rotated rope key) and the value head-major,
  default or interleaved rotation; ``st_mla_attn_fwd`` is flash attention
  with query/key heads of nope+rope against value heads of v;
* o_proj adds the residual in its epilogue; the MoE part is
  :func:`spilltune_amd.moe.deepseek_moe_feed_forward` (fp32 router, routed
  experts as :class:`~spilltune_amd.moe.Q4Experts`, shared expert), a dense
  layer runs the SwiGLU MLP with the residual in the down epilogue.

LoRA sits on the reference's targets (deepseek.py:207-208: q_proj or
q_a_proj/q_b_proj, kv_a_proj_with_mqa, kv_b_proj, o_proj) and optionally, as
this build's extension, on the shared expert's gate/up/down.
"""
from __future__ import annotations

import math

import torch

from . import moe, ops
from .dense import CausalMask, key_lengths

ATTENTION_TARGETS_Q_LORA = ("self_attn.q_a_proj", "self_attn.q_b_proj",
                            "self_attn.kv_a_proj_with_mqa", "self_attn.kv_b_proj",
                            "self_attn.o_proj")
ATTENTION_TARGETS_Q = ("self_attn.q_proj", "self_attn.kv_a_proj_with_mqa",
                       "self_attn.kv_b_proj", "self_attn.o_proj")
SHARED_EXPERT_TARGETS = ("mlp.shared_experts.gate_proj", "mlp.shared_experts.up_proj",
                         "mlp.shared_experts.down_proj")
LORA_KWARGS = {"self_attn.q_proj": "lora_q", "self_attn.q_a_proj": "lora_qa",
               "self_attn.q_b_proj": "lora_qb", "self_attn.kv_a_proj_with_mqa": "lora_kva",
               "self_attn.kv_b_proj": "lora_kvb", "self_attn.o_proj": "lora_o",
               "mlp.shared_experts.gate_proj": "lora_shared_gate",
               "mlp.shared_experts.up_proj": "lora_shared_up",
               "mlp.shared_experts.down_proj": "lora_shared_down"}


def mscale(factor, scale=1.0):
    return 1.0 if factor <= 1 else 1.0 + 0.1 * scale * math.log(factor)


def rope_parameters(rope: dict, dim: int, device=None):
    """Inverse frequencies [dim/2] (fp32) and amplitude of the default or YaRN
    rotary embedding (deepseek.py:94-112); host-side table construction."""
    base = rope["rope_theta"]
    freq = base ** (torch.arange(0, dim, 2, device=device, dtype=torch.float32) / dim)
    kind = rope.get("rope_type", "default")
    if kind == "default":
        return 1.0 / freq, 1.0
    if kind != "yarn":
        raise ValueError("unsupported_capability: only default/YaRN rotary embeddings")
    factor, original = rope["factor"], rope["original_max_position_embeddings"]

    def correction(rot):
        return dim * math.log(original / (rot * 2 * math.pi)) / (2 * math.log(base))

    lo = correction(rope.get("beta_fast", 32) or 32)
    hi = correction(rope.get("beta_slow", 1) or 1)
    if rope.get("truncate", True):
        lo, hi = math.floor(lo), math.ceil(hi)
    lo, hi = max(lo, 0), min(hi, dim - 1)
    if lo == hi:
        hi += 0.001
    ramp = ((torch.arange(dim // 2, device=device, dtype=torch.float32) - lo) / (hi - lo)).clamp(0, 1)
    keep = 1 - ramp  # two subtractions, as the reference keeps them (fp32 rounding)
    inverse = (1.0 / (factor * freq)) * (1 - keep) + (1.0 / freq) * keep
    amplitude = rope.get("attention_factor")
    if amplitude is None:
        if rope.get("mscale") and rope.get("mscale_all_dim"):
            amplitude = mscale(factor, rope["mscale"]) / mscale(factor, rope["mscale_all_dim"])
        else:
            amplitude = mscale(factor)
    return inverse, amplitude


def attention_scale(nope: int, rope_dim: int, rope: dict) -> float:
    """Softmax scale of deepseek.py:205-206."""
    scale = (nope + rope_dim) ** -0.5
    if rope.get("rope_type") == "yarn" and rope.get("mscale_all_dim", 0):
        scale *= mscale(rope["factor"], rope["mscale_all_dim"]) ** 2
    return scale


def positions_and_masks(valid: torch.Tensor, *, rope: dict, rope_dim: int, device,
                        dtype=torch.bfloat16):
    """bf16 (cos, sin) [B, S, rope_dim] scaled by the YaRN amplitude and the
    causal mask marker with the valid prefix lengths of right-padded rows
    (deepseek.py:234-243)."""
    if valid.dtype != torch.bool or valid.ndim != 2 or valid.shape[1] < 1:
        raise ValueError("unsupported_deepseek: invalid mask/context")
    lengths = key_lengths(valid, device, "unsupported_deepseek: all-valid/right padding only")
    batch, length = valid.shape
    inverse, amplitude = rope_parameters(rope, rope_dim, device)
    pos = torch.arange(length, device=device).expand(batch, -1)
    phase = (inverse[None, :, None].expand(batch, -1, 1) @ pos[:, None].float()).transpose(1, 2)
    phase = torch.cat((phase, phase), -1)
    return ((phase.cos() * amplitude).to(dtype), (phase.sin() * amplitude).to(dtype)), \
        CausalMask(batch, length, lengths)


def _weight(weights, name):
    w = weights[name + ".weight"]
    if not isinstance(w, ops.Q4Weight):
        raise TypeError(f"{name}.weight must be a 4-bit slot view (Q4Weight), got {type(w).__name__}")
    return w


def _pair(weights, a, b, la, lb):
    """Fused N-concatenation of two projections that read the same input when
    their storage is adjacent and their adapters fit one fused GEMM."""
    wa, wb = _weight(weights, a), _weight(weights, b)
    fused = ops.concat_rows([wa, wb])
    if fused is not None and ops.lora_fusable([la, lb]):
        return fused
    return None


def deepseek_block(hidden_states, position_embeddings, attention_mask, *, parameters,
                   lora_q=None, lora_qa=None, lora_qb=None, lora_kva=None, lora_kvb=None,
                   lora_o=None, lora_shared_gate=None, lora_shared_up=None,
                   lora_shared_down=None, **w):
    if attention_mask is not None and not isinstance(attention_mask, CausalMask):
        raise ValueError("unsupported_capability: only the causal mask marker is supported")
    c = parameters
    B, S, Hd = hidden_states.shape
    cos, sin = position_embeddings
    heads, nope, rope, vdim, kv_rank = c["heads"], c["nope"], c["rope"], c["value"], c["kv_rank"]
    residual, xn = ops.rms_norm_residual(hidden_states.reshape(B * S, Hd),
                                         w["input_layernorm.weight"], c["eps"])
    # q (direct, or q_a -> RMSNorm -> q_b) and the compressed kv with the rope key
    if c["q_rank"] is None:
        q = ops.q4_lora_linear(xn, _weight(w, "self_attn.q_proj"), [lora_q])
        comp = ops.q4_lora_linear(xn, _weight(w, "self_attn.kv_a_proj_with_mqa"), [lora_kva])
    else:
        fused = _pair(w, "self_attn.q_a_proj", "self_attn.kv_a_proj_with_mqa", lora_qa, lora_kva)
        if fused is not None:
            y = ops.q4_lora_linear(xn, fused, [lora_qa, lora_kva])
            qa, comp = y[:, :c["q_rank"]], y[:, c["q_rank"]:]
        else:
            qa = ops.q4_lora_linear(xn, _weight(w, "self_attn.q_a_proj"), [lora_qa])
            comp = ops.q4_lora_linear(xn, _weight(w, "self_attn.kv_a_proj_with_mqa"), [lora_kva])
        qn = ops.rms_norm(qa, w["self_attn.q_a_layernorm.weight"], 1e-6)
        q = ops.q4_lora_linear(qn, _weight(w, "self_attn.q_b_proj"), [lora_qb])
    kvn = ops.rms_norm(comp[:, :kv_rank], w["self_attn.kv_a_layernorm.weight"], 1e-6)
    kv = ops.q4_lora_linear(kvn, _weight(w, "self_attn.kv_b_proj"), [lora_kvb])
    Q, K, V = ops.mla_rope(q, kv, comp, cos, sin, batch=B, seq=S, heads=heads, nope=nope,
                           rope=rope, v_dim=vdim, kv_rank=kv_rank, interleave=c["interleave"])
    kv_len = attention_mask.lengths if attention_mask is not None else None
    attended = ops.mla_attention(Q, K, V, c["attention_scale"], kv_len).reshape(B * S, heads * vdim)
    h1 = ops.q4_lora_linear(attended, _weight(w, "self_attn.o_proj"), [lora_o], residual=residual)
    h1, xn2 = ops.rms_norm_residual(h1, w["post_attention_layernorm.weight"], c["eps"])
    if not c["moe"]:  # dense layer: residual + down(silu(gate) * up)
        gu = _pair(w, "mlp.gate_proj", "mlp.up_proj", None, None)
        wd = _weight(w, "mlp.down_proj")
        if gu is not None:
            out = ops.q4_lora_linear(ops.q4_lora_linear(xn2, gu), wd, residual=h1, swiglu=True)
        else:
            act = ops.swiglu_pair(ops.q4_lora_linear(xn2, _weight(w, "mlp.gate_proj")),
                                  ops.q4_lora_linear(xn2, _weight(w, "mlp.up_proj")))
            out = ops.q4_lora_linear(act, wd, residual=h1)
        return out.view(B, S, Hd)
    shared = {k: v for k, v in (("gate", lora_shared_gate), ("up", lora_shared_up),
                                ("down", lora_shared_down)) if v is not None}
    routed_shared = moe.deepseek_moe_feed_forward(
        xn2, w, num_experts=c["experts"], top_k=c["top_k"], groups=c["groups"],
        group_k=c["group_k"], normalize=c["normalize"], scale=c["router_scale"],
        lora_shared=shared or None)
    return (h1 + routed_shared).view(B, S, Hd)


def make_deepseek_block(index: int, weights: dict, *, codec: str, parameters: dict, rank: int,
                        alpha: float, device, shared_lora: bool = False, functional=None,
                        generator=None):
    """Encode one DeepSeek-V3 decoder layer into a BlockPlan (the adapter
    factory of deepseek.py:209-226 for one layer).  ``weights`` maps HF names
    (without ``model.layers.{i}.``) to CPU tensors or to ready
    ``codecs.Record`` values; every 2-D or packed 3-D matrix except the router
    is stored 4-bit (deepseek.py:87), the router weight and bias stay fp32
    (quantization_fp32_keys, deepseek.py:81-88), norm vectors bf16.  LoRA:
    the reference's attention targets (A = randn * 0.02, B = 0, deepseek.py:
    213-217), plus the shared expert when ``shared_lora``."""
    from .codecs import Record, encode
    from .lora import create_lora_for_block
    from .slots import BlockPlan
    host, specs, shapes = {}, {}, {}
    router = ("mlp.gate.weight", "mlp.gate.e_score_correction_bias")
    for name, t in weights.items():
        if isinstance(t, Record) or (name not in router and t.dim() in (2, 3)
                                     and t.numel() >= 128):
            rec = t if isinstance(t, Record) else encode(t.reshape(-1, t.shape[-1]).contiguous(),
                                                         codec)
            shape = list(t.shape) if not isinstance(t, Record) else list(rec.spec["shape"])
            spec = dict(rec.spec, shape=shape)
            specs[name] = {"spec": spec, "parts": {}}
            for part, tensor in rec.parts.items():
                key = f"@{name}/{part}"
                host[key] = tensor
                specs[name]["parts"][part] = key
            if len(shape) == 2:
                shapes[name] = tuple(shape)
        elif name in router:
            host[name] = t.float().contiguous()
        else:
            host[name] = t.to(torch.bfloat16).contiguous()
    targets = ATTENTION_TARGETS_Q if parameters["q_rank"] is None else ATTENTION_TARGETS_Q_LORA
    if shared_lora and parameters["moe"]:
        targets = targets + SHARED_EXPERT_TARGETS
    adapters = create_lora_for_block(index, "mla_moe", shapes, rank=rank, alpha=alpha,
                                     device=device, targets=targets, architecture="deepseek_v3",
                                     generator=generator)
    kwargs = {"parameters": dict(parameters), **lora_kwargs(adapters)}
    return BlockPlan(index, "mla_moe", functional or deepseek_block, kwargs, host, adapters,
                     specs)


def lora_kwargs(adapters: dict) -> dict:
    """Map target paths to the functional's ``lora_*`` keyword arguments."""
    return {LORA_KWARGS[t]: p for t, p in adapters.items()}


__all__ = ["deepseek_block", "rope_parameters", "attention_scale", "positions_and_masks",
           "lora_kwargs", "make_deepseek_block", "ATTENTION_TARGETS_Q_LORA", "ATTENTION_TARGETS_Q",
           "SHARED_EXPERT_TARGETS"]
