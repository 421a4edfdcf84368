"""PyTorch-CPU restatement of DeepSeek-V3's decoder block: multi-head latent
attention plus the routed/shared-expert MoE (or a dense MLP).

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker of the HIP
``spilltune_amd.deepseek.deepseek_block``, never the thing measured or
shipped.

Follows /root/reference/src/ram_vram_finetune/adapters/deepseek.py:

* ``mscale`` / ``rope_parameters`` -- deepseek.py:91-112 (default and YaRN
  inverse frequencies, amplitude);
* ``rotary`` -- deepseek.py:237-240 (bf16 ``cos * amplitude``,
  ``sin * amplitude`` of ``cat(freqs, freqs)``);
* ``attention_scale`` -- deepseek.py:205-206;
* ``deepseek_block`` -- deepseek.py:129-176: q (direct or q_a -> RMSNorm(1e-6)
  -> q_b), kv_a_proj_with_mqa split into the latent and the shared rope key,
  RMSNorm(1e-6) -> kv_b, nope/rope split, rotation (default or interleaved),
  eager scores with the additive mask, fp32 softmax, probabilities @ value,
  o_proj + residual, then the MoE (``oracle.moe`` router and expert loop,
  shared expert) or the dense MLP.  LoRA (``oracle.layer.lora_linear``) may
  sit on any projection: the reference's attention targets
  (deepseek.py:207-208) and, as this build's extension, the shared expert.

Pinning (tests/test_oracle_mla.py): against transformers' DeepseekV3
``DeepseekV3DecoderLayer`` (eager attention and experts) with LoRA-wrapped
attention projections, default and interleaved rotary, with and without
q_lora_rank, YaRN rotary tables against ``DeepseekV3RotaryEmbedding``,
forward and input/LoRA gradients in fp32 and bf16.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import layer as OL
from . import moe as OM


def mscale(factor, scale=1.0):
    return 1.0 if factor <= 1 else 1.0 + 0.1 * scale * math.log(factor)


def rope_parameters(rope: dict, dim: int):
    """(inverse frequencies [dim/2] fp32, amplitude) of deepseek.py:94-112."""
    base = rope["rope_theta"]
    freq = base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim)
    if rope.get("rope_type", "default") == "default":
        return 1.0 / freq, 1.0
    factor = rope["factor"]
    original = rope["original_max_position_embeddings"]

    def correction(rot):
        return dim * math.log(original / (rot * 2 * math.pi)) / (2 * math.log(base))

    lo, hi = correction(rope.get("beta_fast", 32) or 32), correction(rope.get("beta_slow", 1) or 1)
    if rope.get("truncate", True):
        lo, hi = math.floor(lo), math.ceil(hi)
    lo, hi = max(lo, 0), min(hi, dim - 1)
    if lo == hi:
        hi += 0.001
    ramp = ((torch.arange(dim // 2, dtype=torch.float32) - lo) / (hi - lo)).clamp(0, 1)
    extrapolation = 1 - ramp
    inverse = (1.0 / (factor * freq)) * (1 - extrapolation) + (1.0 / freq) * extrapolation
    amplitude = rope.get("attention_factor")
    if amplitude is None:
        if rope.get("mscale") and rope.get("mscale_all_dim"):
            amplitude = mscale(factor, rope["mscale"]) / mscale(factor, rope["mscale_all_dim"])
        else:
            amplitude = mscale(factor)
    return inverse, amplitude


def rotary(batch, length, rope: dict, dim: int, dtype):
    """bf16 (cos, sin) [B, S, dim] (deepseek.py:237-240)."""
    inverse, amplitude = rope_parameters(rope, dim)
    pos = torch.arange(length).expand(batch, -1)
    phase = (inverse[None, :, None].expand(batch, -1, 1) @ pos[:, None].float()).transpose(1, 2)
    phase = torch.cat((phase, phase), -1)
    return (phase.cos() * amplitude).to(dtype), (phase.sin() * amplitude).to(dtype)


def attention_scale(nope: int, rope_dim: int, rope: dict) -> float:
    """deepseek.py:205-206: (nope + rope)^-0.5, times mscale(factor,
    mscale_all_dim)^2 for YaRN with mscale_all_dim."""
    scale = (nope + rope_dim) ** -0.5
    if rope.get("rope_type") == "yarn" and rope.get("mscale_all_dim", 0):
        scale *= mscale(rope["factor"], rope["mscale_all_dim"]) ** 2
    return scale


def deepseek_block(hidden, rotary_tables, mask, *, parameters, weights, loras=None,
                   indices=None):
    """One DeepSeek-V3 decoder block (deepseek.py:129-176).  ``parameters``
    has the reference's keys (heads, nope, rope, value, kv_rank, q_rank, eps,
    attention_scale, interleave, moe, experts, groups, group_k, top_k,
    normalize, router_scale); ``weights`` the block's tensors by their HF
    names (routed experts packed: ``mlp.experts.gate_up_proj [E, 2I, H]``,
    ``mlp.experts.down_proj [E, H, I]``); ``loras`` maps projection names
    (``self_attn.q_a_proj`` .. ``mlp.shared_experts.down_proj``) to
    :class:`oracle.layer.Lora`.  ``indices`` (token-major picks [T, top_k])
    replaces the router's selection -- for checking a device path on its own
    picks where fp32 summation order decides near-ties; the weights are then
    the router's for those picks (``oracle.moe.deepseek_weights_given``)."""
    c = parameters
    loras = loras or {}

    def linear(x, name):
        return OL.lora_linear(x, weights[name + ".weight"], loras.get(name))

    residual, x = _attention(hidden, rotary_tables, mask, c, weights, linear)

    def mlp(t, prefix):
        return linear(F.silu(linear(t, prefix + "gate_proj")) * linear(t, prefix + "up_proj"),
                      prefix + "down_proj")

    if not c["moe"]:
        return residual + mlp(x, "mlp.")
    flat = x.reshape(-1, x.shape[-1])
    if indices is None:
        _, routing, indices = OM.deepseek_route(flat, weights["mlp.gate.weight"],
                                                weights["mlp.gate.e_score_correction_bias"],
                                                groups=c["groups"], group_k=c["group_k"],
                                                top_k=c["top_k"], normalize=c["normalize"],
                                                scale=c["router_scale"])
    else:
        logits = F.linear(flat.float(), weights["mlp.gate.weight"].float())
        routing = OM.deepseek_weights_given(logits, indices, normalize=c["normalize"],
                                            scale=c["router_scale"])
    routed = OM.expert_loop(flat, routing, indices, weights["mlp.experts.gate_up_proj"],
                            weights["mlp.experts.down_proj"], num_experts=c["experts"])
    return residual + (routed.view_as(x) + mlp(x, "mlp.shared_experts."))


def deepseek_block_rows(hidden, rotary_tables, mask, *, parameters, weights, loras, rows,
                        indices, experts):
    """``deepseek_block``'s output on the token rows ``rows`` only (flat
    indices into [B*S]), with the MoE evaluated on those rows alone: the
    attention runs over every token (each row's attention reads all earlier
    tokens), while a row's routed and shared experts read only that row.  So
    with an upstream gradient that is zero off ``rows``, autograd of this
    output gives every gradient of the whole block (the other rows' MoE terms
    get zero gradient).  ``indices`` [len(rows), top_k] are global expert ids
    and ``weights["mlp.experts.*"]`` hold only the experts ``experts``
    (ascending ids, stacked in that order), so only the experts these rows
    hit need decoding.  Returns [len(rows), hidden]."""
    c = parameters
    loras = loras or {}

    def linear(x, name):
        return OL.lora_linear(x, weights[name + ".weight"], loras.get(name))

    residual, x = _attention(hidden, rotary_tables, mask, c, weights, linear)
    flat = x.reshape(-1, x.shape[-1])[rows]
    res = residual.reshape(-1, residual.shape[-1])[rows]
    remap = torch.full((c["experts"],), -1, dtype=torch.long)
    remap[torch.as_tensor(experts)] = torch.arange(len(experts))
    local = remap[indices]
    if bool((local < 0).any()):
        raise ValueError("a pick outside the decoded experts")
    logits = F.linear(flat.float(), weights["mlp.gate.weight"].float())
    routing = OM.deepseek_weights_given(logits, indices, normalize=c["normalize"],
                                        scale=c["router_scale"])
    routed = OM.expert_loop(flat, routing, local, weights["mlp.experts.gate_up_proj"],
                            weights["mlp.experts.down_proj"], num_experts=len(experts))
    shared = linear(F.silu(linear(flat, "mlp.shared_experts.gate_proj"))
                    * linear(flat, "mlp.shared_experts.up_proj"), "mlp.shared_experts.down_proj")
    return res + (routed + shared)


def pre_moe_hidden(hidden, rotary_tables, mask, *, parameters, weights, loras=None):
    """The normalised hidden state the MoE router reads ([tokens, hidden])."""
    loras = loras or {}

    def linear(x, name):
        return OL.lora_linear(x, weights[name + ".weight"], loras.get(name))

    _, x = _attention(hidden, rotary_tables, mask, parameters, weights, linear)
    return x.reshape(-1, x.shape[-1])


def _attention(hidden, rotary_tables, mask, c, weights, linear):
    """deepseek.py:134-155: returns (residual after o_proj, post-attention RMSNorm)."""
    residual = hidden
    x = OL.rms(hidden, weights["input_layernorm.weight"], c["eps"])
    if c["q_rank"] is None:
        q = linear(x, "self_attn.q_proj")
    else:
        q = linear(OL.rms(linear(x, "self_attn.q_a_proj"), weights["self_attn.q_a_layernorm.weight"],
                          1e-6), "self_attn.q_b_proj")
    q = q.view(*x.shape[:-1], c["heads"], c["nope"] + c["rope"]).transpose(1, 2)
    q_pass, q_rot = q.split([c["nope"], c["rope"]], -1)
    compressed = linear(x, "self_attn.kv_a_proj_with_mqa")
    kv, k_rot = compressed.split([c["kv_rank"], c["rope"]], -1)
    kv = linear(OL.rms(kv, weights["self_attn.kv_a_layernorm.weight"], 1e-6), "self_attn.kv_b_proj")
    kv = kv.view(*x.shape[:-1], c["heads"], c["nope"] + c["value"]).transpose(1, 2)
    k_pass, value = kv.split([c["nope"], c["value"]], -1)
    k_rot = k_rot.view(x.shape[0], 1, x.shape[1], c["rope"])
    cos, sin = (t.unsqueeze(1) for t in rotary_tables)

    def rotate(t):
        if c["interleave"]:
            a, b = t[..., 0::2], t[..., 1::2]
            co, si = cos[..., :c["rope"] // 2], sin[..., :c["rope"] // 2]
            return torch.cat((a * co - b * si, b * co + a * si), -1)
        first, second = t.chunk(2, -1)
        return t * cos + torch.cat((-second, first), -1) * sin

    query = torch.cat((q_pass, rotate(q_rot)), -1)
    key = torch.cat((k_pass, rotate(k_rot).expand_as(q_rot)), -1)
    scores = (query @ key.transpose(-2, -1)) * c["attention_scale"]
    probs = torch.softmax(scores + mask, -1, dtype=torch.float32).to(query.dtype)
    attended = (probs @ value).transpose(1, 2).contiguous().reshape(*x.shape[:-1],
                                                                    c["heads"] * c["value"])
    x = residual + linear(attended, "self_attn.o_proj")
    return x, OL.rms(x, weights["post_attention_layernorm.weight"], c["eps"])


def streaming_step(hidden, rotary_tables, mask, grad_output, *, parameters, weights, loras,
                   indices=None):
    """Forward (no grad), then recompute + ``autograd.grad`` over
    ``[hidden, A0, B0, ...]`` (training/recompute.py:26-133) for the DeepSeek
    block; fills each Lora's grad buffers.  Returns ``(output, grad_hidden)``."""
    with torch.no_grad():
        output = deepseek_block(hidden, rotary_tables, mask, parameters=parameters,
                                weights=weights, loras=loras, indices=indices)
    saved = hidden.detach().clone().requires_grad_(True)
    ordered = sorted(loras.values(), key=lambda p: p.name)
    inputs = [saved] + [t for p in ordered for t in (p.A, p.B)]
    with torch.enable_grad():
        recomputed = deepseek_block(saved, rotary_tables, mask, parameters=parameters,
                                    weights=weights, loras=loras, indices=indices)
    grads = torch.autograd.grad(recomputed, inputs, grad_output, allow_unused=True)
    for i, p in enumerate(ordered):
        p.grad_A.zero_()
        p.grad_B.zero_()
        p.grad_A.add_(grads[1 + 2 * i].detach().float())
        p.grad_B.add_(grads[2 + 2 * i].detach().float())
    return output, grads[0]
