"""PyTorch-CPU restatement of SpillTune's per-layer LoRA training compute.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).  Used by ``tests/`` as
the checker for the HIP path, by ``__graft_entry__.smoke()`` and by the
``cpu_baseline`` leg of ``bench.py`` (the reference's CPU training path).

Each function follows a reference file:line (relative to
/root/reference/src/ram_vram_finetune) and keeps its dtype policy:

* ``lora_linear``  -- finetune/lora.py:205-220:
  ``bf16( fp32(bf16(x W^T)) + s * ((x_f32 A^T) B^T) )``.
* ``rms``          -- adapters/dense.py:115-117.
* ``rotary``/``causal_mask`` -- adapters/dense.py:241-247 (bf16 cos/sin,
  additive mask filled with the bf16 minimum).
* ``dense_block``  -- adapters/dense.py:120-153 (Llama: GQA, default full RoPE,
  eager fp32 softmax), generalised to LoRA on any of the seven projections
  (the reference's explicit-targets API, finetune/lora.py:319-388).
* ``streaming_step`` -- training/recompute.py:26-133: forward under no_grad,
  backward = recompute with grad + ``autograd.grad`` over ``[hidden, A0, B0..]``
  in name order, fp32 accumulation into grad buffers.
* ``causal_lm_terminal`` -- training/engine.py:58-79 and
  quantization/native_terminal.py:11-37 (token-chunked summed CE / normaliser).
* ``adamw_step``   -- finetune/optimizer.py:324-342 (the torch.optim.AdamW
  non-foreach order).

Pinning (tests/test_oracle_layer.py): ``dense_block`` in fp32 against
transformers' ``LlamaDecoderLayer`` (eager attention) with LoRA-wrapped
projections, forward and VJP; ``lora_linear`` gradients against a float64
closed form; ``causal_lm_terminal`` against full-sequence ``F.cross_entropy``;
``adamw_step`` against ``torch.optim.AdamW(foreach=False)``.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

PROJECTIONS = ("self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
               "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")


@dataclass
class Lora:
    """fp32 LoRA master state of one projection (finetune/lora.py:97-228)."""
    name: str
    A: torch.Tensor          # [r, in]
    B: torch.Tensor          # [out, r]
    alpha: float
    grad_A: torch.Tensor = field(default=None)
    grad_B: torch.Tensor = field(default=None)

    def __post_init__(self):
        self.A = self.A.detach().clone().float().requires_grad_(True)
        self.B = self.B.detach().clone().float().requires_grad_(True)
        self.grad_A = torch.zeros_like(self.A, requires_grad=False)
        self.grad_B = torch.zeros_like(self.B, requires_grad=False)

    @property
    def rank(self) -> int:
        return self.A.shape[0]

    @property
    def scale(self) -> float:
        return self.alpha / self.rank


def lora_linear(x, weight, lora: Lora | None):
    """Base bf16 linear plus fp32 LoRA, rounded once to bf16 (lora.py:218-220)."""
    base = F.linear(x, weight.detach())
    if lora is None:
        return base
    update = F.linear(F.linear(x.float(), lora.A), lora.B)
    return (base.float() + update * lora.scale).to(base.dtype)


def rms(hidden, weight, eps):
    """``w * bf16(x * rsqrt(mean(x^2) + eps))`` with fp32 statistics (dense.py:115-117)."""
    value = hidden.float()
    normed = value * torch.rsqrt(value.square().mean(-1, keepdim=True) + eps)
    return weight * normed.to(hidden.dtype)


def rotary(batch, length, head_dim, theta, dtype):
    """Default full rotary tables in the compute dtype (dense.py:241-245)."""
    positions = torch.arange(length).expand(batch, -1)
    inv = 1.0 / theta ** (torch.arange(0, head_dim, 2).float() / head_dim)
    freq = (inv[None, :, None].expand(batch, -1, 1) @ positions[:, None].float()).transpose(1, 2)
    phase = torch.cat((freq, freq), -1)
    return phase.cos().to(dtype), phase.sin().to(dtype)


def causal_mask(batch, length, dtype, valid=None):
    """Additive causal (+ right padding) mask, ``finfo(dtype).min`` when blocked (dense.py:246-247)."""
    blocked = torch.ones(length, length, dtype=torch.bool).triu(1)[None, None]
    if valid is not None:
        blocked = blocked | ~valid[:, None, None, :]
    else:
        blocked = blocked.expand(batch, 1, length, length)
    return torch.zeros(blocked.shape, dtype=dtype).masked_fill(blocked, torch.finfo(dtype).min)


def _rotate(x, cos, sin):
    left, right = x.chunk(2, dim=-1)
    return x * cos + torch.cat((-right, left), dim=-1) * sin


def dense_block(hidden, rotary_tables, mask, *, heads, kv_heads, head_dim, eps,
                weights: dict, loras: dict, feed_forward=None, qk_norm=False):
    """One Llama/Qwen3 decoder block (dense.py:120-153); ``weights`` holds bf16
    matrices keyed ``<proj>.weight`` plus the norm vectors, ``loras`` maps
    projection names to :class:`Lora` (absent projections have no adapter).
    ``qk_norm`` (Qwen3) normalises each head of q and k over head_dim with
    ``self_attn.q_norm.weight`` / ``k_norm.weight`` before RoPE, on the
    [B, S, heads, D] view (dense.py:128-133).  A ``feed_forward(x, weights)``
    replaces the SwiGLU MLP (dense.py:152)."""
    def linear(x, name):
        return lora_linear(x, weights[name + ".weight"], loras.get(name))

    residual = hidden
    x = rms(hidden, weights["input_layernorm.weight"], eps)
    shape = (*x.shape[:-1], -1, head_dim)
    q = linear(x, "self_attn.q_proj").view(shape)
    k = linear(x, "self_attn.k_proj").view(shape)
    v = linear(x, "self_attn.v_proj").view(shape).transpose(1, 2)
    if qk_norm:
        q = rms(q, weights["self_attn.q_norm.weight"], eps)
        k = rms(k, weights["self_attn.k_norm.weight"], eps)
    q, k = q.transpose(1, 2), k.transpose(1, 2)
    cos, sin = (t.unsqueeze(1) for t in rotary_tables)
    q, k = _rotate(q, cos, sin), _rotate(k, cos, sin)
    group = heads // kv_heads

    def repeat(t):
        b, h, s, d = t.shape
        return t[:, :, None].expand(b, h, group, s, d).reshape(b, heads, s, d)

    k, v = repeat(k), repeat(v)
    scores = (q @ k.transpose(-2, -1)) * head_dim ** -0.5
    probs = torch.softmax(scores + mask, dim=-1, dtype=torch.float32).to(q.dtype)
    attended = (probs @ v).transpose(1, 2).contiguous().reshape(*x.shape[:-1], heads * head_dim)
    x = residual + linear(attended, "self_attn.o_proj")
    residual = x
    x = rms(x, weights["post_attention_layernorm.weight"], eps)
    if feed_forward is not None:
        return residual + feed_forward(x, weights)
    act = F.silu(linear(x, "mlp.gate_proj")) * linear(x, "mlp.up_proj")
    return residual + linear(act, "mlp.down_proj")


def streaming_step(hidden, rotary_tables, mask, grad_output, *, weights, loras, cfg,
                   accumulate=False):
    """Forward (no grad) then backward by recompute + ``autograd.grad``
    (recompute.py:26-133).  Returns ``(output, grad_hidden)`` and fills each
    ``Lora.grad_A/grad_B`` (replace unless ``accumulate``)."""
    with torch.no_grad():
        output = dense_block(hidden, rotary_tables, mask, weights=weights, loras=loras, **cfg)
    saved = hidden.detach().clone().requires_grad_(True)
    ordered = sorted(loras.values(), key=lambda p: p.name)
    inputs = [saved] + [t for p in ordered for t in (p.A, p.B)]
    with torch.enable_grad():
        recomputed = dense_block(saved, rotary_tables, mask, weights=weights, loras=loras, **cfg)
    grads = torch.autograd.grad(recomputed, inputs, grad_output, allow_unused=True)
    if grads[0] is None:
        raise RuntimeError("block lost its input gradient")
    for i, p in enumerate(ordered):
        ga, gb = grads[1 + 2 * i], grads[2 + 2 * i]
        if ga is None or gb is None:
            raise RuntimeError(f"adapter {p.name} is disconnected")
        if not accumulate:
            p.grad_A.zero_()
            p.grad_B.zero_()
        p.grad_A.add_(ga.detach().float())
        p.grad_B.add_(gb.detach().float())
    return output, grads[0]


def causal_lm_terminal(hidden, norm_weight, head, labels, *, eps, normalization, token_chunk):
    """Full-sequence terminal norm, token-chunked head + summed CE / normaliser
    and the norm VJP (engine.py:58-79).  Returns ``(loss, grad_hidden)``."""
    terminal = hidden.detach().requires_grad_(True)
    normalized = rms(terminal, norm_weight, eps)
    vjp = torch.zeros_like(normalized)
    total = torch.zeros(())
    length = hidden.shape[1]
    for start in range(0, length - 1, token_chunk):
        end = min(start + token_chunk, length - 1)
        target = labels[:, start + 1:end + 1]
        if not (target != -100).any():
            continue
        h = normalized[:, start:end].detach().requires_grad_(True)
        logits = F.linear(h, head)
        value = F.cross_entropy(logits.float().reshape(-1, logits.shape[-1]), target.reshape(-1),
                                ignore_index=-100, reduction="sum")
        (g,) = torch.autograd.grad(value / normalization, h)
        vjp[:, start:end].copy_(g.detach())
        total += value.detach()
    (grad,) = torch.autograd.grad(normalized, terminal, vjp)
    return float(total / normalization), grad


def adamw_step(params_grads_states, *, step, lr, beta1=0.9, beta2=0.999, eps=1e-8,
               weight_decay=0.0):
    """One fp32 AdamW update per (param, grad, exp_avg, exp_avg_sq) tuple, in
    the torch.optim.AdamW non-foreach operation order (optimizer.py:324-342)."""
    bc1 = 1.0 - beta1 ** step
    bc2_sqrt = (1.0 - beta2 ** step) ** 0.5
    step_size = lr / bc1
    with torch.no_grad():
        for param, grad, m, v in params_grads_states:
            if weight_decay != 0.0:
                param.mul_(1.0 - lr * weight_decay)
            m.lerp_(grad, 1.0 - beta1)
            v.mul_(beta2).addcmul_(grad, grad, value=1.0 - beta2)
            denom = (v.sqrt() / bc2_sqrt).add_(eps)
            param.addcdiv_(m, denom, value=-step_size)


def train_reference(embedding, norm_weight, head, layers, loras, rows, *, cfg, theta, steps,
                    lr, weight_decay=0.0, token_chunk=64, accumulation=1):
    """The reference's optimizer-step loop (engine.py:162-182 with microbatch,
    engine.py:48-79) on the CPU: bf16 layer math through autograd (the
    per-layer recompute computes the same graph), token-chunked CE, fp32
    AdamW.  ``layers``: per-layer bf16 weight dicts; ``loras``: per-layer
    ``{name: Lora}``.  Returns the per-step losses."""
    import torch.nn.functional as F  # noqa: F811
    tensors = [(p.A, p) for lo in loras for p in lo.values()] + \
              [(p.B, p) for lo in loras for p in lo.values()]
    states = {id(t): (torch.zeros_like(t), torch.zeros_like(t)) for t, _ in tensors}
    cursor, losses = 0, []
    for step in range(1, steps + 1):
        items = [rows[(cursor + i) % len(rows)] for i in range(accumulation)]
        normalization = sum(int((labels[:, 1:] != -100).sum()) for _, labels in items)
        for t, _ in tensors:
            t.grad = None
        loss = 0.0
        for ids, labels in items:
            B, S = ids.shape
            rot = rotary(B, S, cfg["head_dim"], theta, torch.bfloat16)
            mask = causal_mask(B, S, torch.bfloat16)
            hidden = F.embedding(ids, embedding).detach()
            for w, lo in zip(layers, loras):
                hidden = dense_block(hidden, rot, mask, weights=w, loras=lo, **cfg)
            value, grad = causal_lm_terminal(hidden, norm_weight, head, labels, eps=cfg["eps"],
                                             normalization=normalization, token_chunk=token_chunk)
            hidden.backward(grad)
            loss += value
        adamw_step([(t, t.grad.float(), *states[id(t)]) for t, _ in tensors], step=step, lr=lr,
                   weight_decay=weight_decay)
        cursor += accumulation
        losses.append(loss)
    return losses
