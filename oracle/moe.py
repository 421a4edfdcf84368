"""PyTorch-CPU restatement of SpillTune's MoE feed-forward and routers.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``): the checker of the
grouped HIP path, never the thing measured or shipped.

Follows /root/reference/src/ram_vram_finetune:

* ``qwen3_moe_ffn``  -- adapters/qwen3_moe.py:95-113 (``moe_feed_forward``):
  bf16 router logits, fp32 softmax, ``topk``, optional renormalisation, bf16
  routing weights; per hit expert (ascending) ``gate, up = chunk(x_e W_gu^T)``,
  ``y = (silu(gate) up) W_d^T``, ``y * w`` in bf16, ``index_add_`` into a bf16
  output.  Optional per-expert LoRA on gate/up/down with the projection rule
  of finetune/lora.py:205-220 (``bf16(fp32(bf16(x W^T)) + s (x A^T) B^T)``);
  the reference keeps experts frozen, the LoRA is the benchmark's extension
  and reduces to the reference when absent.
* ``deepseek_route`` -- adapters/deepseek.py:115-126: fp32 sigmoid scores,
  selection bias, group top-2 sum, top-``group_k`` groups, top-``k`` experts,
  weights from the unbiased scores (renormalised + 1e-20) times ``scale``.
* ``deepseek_moe_ffn`` -- the expert loop of adapters/deepseek.py:161-174
  (fp32 weights: ``bf16(y * w)`` before the bf16 ``index_add_``).

Pinning (tests/test_oracle_moe.py): ``qwen3_moe_ffn`` without LoRA against
transformers' ``Qwen3MoeSparseMoeBlock`` (forward and input VJP, fp32 and
bf16); ``deepseek_route`` against transformers' ``DeepseekV3TopkRouter``;
the LoRA terms against a float64 closed form; the combine order against a
brute-force per-token sum; the given-pick routers against the ``topk``
routers (value and VJP); ``topk_lowest_index`` against a brute-force scan.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def expert_lora_linear(x, weight, lora, expert):
    """One expert projection with optional LoRA ``(A [E,r,K], B [E,N,r], scale)``."""
    base = F.linear(x, weight)
    if lora is None:
        return base
    A, B, scale = lora
    update = F.linear(F.linear(x.float(), A[expert]), B[expert])
    return (base.float() + update * scale).to(base.dtype)


def qwen3_route(flat, router_weight, *, top_k, norm_topk_prob):
    """Router of qwen3_moe.py:97-100: returns ``(logits, bf16 weights, indices)``."""
    logits = F.linear(flat, router_weight)
    probs = F.softmax(logits, dtype=torch.float32, dim=-1)
    routing, indices = torch.topk(probs, top_k, dim=-1)
    if norm_topk_prob:
        routing = routing / routing.sum(dim=-1, keepdim=True)
    return logits, routing.to(logits.dtype), indices


def qwen3_route_given(flat, router_weight, indices, *, norm_topk_prob):
    """The router of :func:`qwen3_route` for given picks: ``topk`` values are the
    probabilities at ``indices`` and its VJP scatters into them, so with the
    indices ``topk`` returns both routers agree in value and gradient.  Used
    where ``topk`` ties (equal bf16 logits) leave the pick order open."""
    logits = F.linear(flat, router_weight)
    probs = F.softmax(logits, dtype=torch.float32, dim=-1)
    routing = probs.gather(1, indices)
    if norm_topk_prob:
        routing = routing / routing.sum(dim=-1, keepdim=True)
    return logits, routing.to(logits.dtype)


def topk_lowest_index(values, k):
    """Top-k by value with equal values ordered by the lower index (the rule
    of the HIP routers; ``torch.topk`` leaves the order of ties open)."""
    srt = torch.sort(values, dim=-1, descending=True, stable=True)
    return srt.values[..., :k], srt.indices[..., :k]


def expert_loop(flat, routing, indices, gate_up, down, *, num_experts, loras=None):
    """The per-expert loop of qwen3_moe.py:101-112 / deepseek.py:161-174.

    ``gate_up`` [E, 2I, H], ``down`` [E, H, I]; ``loras`` optionally maps
    ``"gate"``, ``"up"``, ``"down"`` to ``(A, B, scale)``.  ``routing`` keeps
    its dtype in the product (bf16 for Qwen3, fp32 for DeepSeek)."""
    loras = loras or {}
    output = torch.zeros_like(flat)
    with torch.no_grad():
        mask = F.one_hot(indices, num_classes=num_experts).permute(2, 1, 0)
        hit = (mask.sum(dim=(-1, -2)) > 0).nonzero()
    inter = gate_up.shape[1] // 2
    for expert in hit:
        expert = expert[0]
        position, tokens = torch.where(mask[expert])
        current = flat[tokens]
        w = gate_up[expert]
        if "gate" in loras or "up" in loras:
            gate = expert_lora_linear(current, w[:inter], loras.get("gate"), expert)
            up = expert_lora_linear(current, w[inter:], loras.get("up"), expert)
        else:
            gate, up = F.linear(current, w).chunk(2, dim=-1)
        value = expert_lora_linear(F.silu(gate) * up, down[expert], loras.get("down"), expert)
        value = value * routing[tokens, position, None]
        output.index_add_(0, tokens, value.to(output.dtype))
    return output


def qwen3_moe_ffn(hidden, router_weight, gate_up, down, *, top_k, norm_topk_prob, loras=None):
    """``moe_feed_forward`` (qwen3_moe.py:95-113) with optional per-expert LoRA."""
    shape = hidden.shape
    flat = hidden.reshape(-1, shape[-1])
    _, routing, indices = qwen3_route(flat, router_weight, top_k=top_k,
                                      norm_topk_prob=norm_topk_prob)
    out = expert_loop(flat, routing, indices, gate_up, down, num_experts=gate_up.shape[0],
                      loras=loras)
    return out.reshape(shape)


def deepseek_route(hidden, weight, bias, *, groups, group_k, top_k, normalize, scale):
    """fp32 sigmoid group-limited router (deepseek.py:115-126)."""
    logits = F.linear(hidden.reshape(-1, hidden.shape[-1]).float(), weight.float())
    return deepseek_select(logits, bias, groups=groups, group_k=group_k, top_k=top_k,
                           normalize=normalize, scale=scale)


def deepseek_select(logits, bias, *, groups, group_k, top_k, normalize, scale):
    """The selection and weights of :func:`deepseek_route` (deepseek.py:118-126)
    from given fp32 logits; returns ``(logits, weights, indices)``."""
    scores = logits.sigmoid()
    choice = scores + bias.float()
    group_scores = choice.view(-1, groups, choice.shape[-1] // groups).topk(2, dim=-1)[0].sum(-1)
    selected = group_scores.topk(group_k, dim=-1, sorted=False)[1]
    mask = torch.zeros_like(group_scores).scatter_(1, selected, 1).bool()
    mask = mask[:, :, None].expand(-1, groups, choice.shape[-1] // groups).reshape_as(choice)
    indices = choice.masked_fill(~mask, float("-inf")).topk(top_k, dim=-1, sorted=False)[1]
    weights = scores.gather(1, indices)
    if normalize:
        weights = weights / (weights.sum(-1, keepdim=True) + 1e-20)
    return logits, weights * scale, indices


def deepseek_weights_given(logits, indices, *, normalize, scale):
    """The weights of :func:`deepseek_route` for given picks (selection carries
    no gradient, so value and VJP equal the router's for its own picks)."""
    weights = logits.sigmoid().gather(1, indices)
    if normalize:
        weights = weights / (weights.sum(-1, keepdim=True) + 1e-20)
    return weights * scale


def deepseek_moe_ffn(hidden, router_weight, bias, gate_up, down, *, groups, group_k, top_k,
                     normalize, scale, loras=None):
    """Routed-expert part of deepseek.py:160-174 (shared expert excluded)."""
    flat = hidden.reshape(-1, hidden.shape[-1])
    _, weights, indices = deepseek_route(flat, router_weight, bias, groups=groups,
                                         group_k=group_k, top_k=top_k, normalize=normalize,
                                         scale=scale)
    out = expert_loop(flat, weights, indices, gate_up, down, num_experts=gate_up.shape[0],
                      loras=loras)
    return out.reshape(hidden.shape)
