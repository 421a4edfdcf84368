"""Causal-LM training step over 4-bit streamed blocks (mirror of
training/engine.py:21-195 and finetune/optimizer.py:227-342 in
/root/reference/src/ram_vram_finetune, without the config/dataset/checkpoint
I/O around it).

* :func:`forward` -- the per-layer loop through the streaming recompute driver
  (engine.py:36-45).
* :func:`microbatch` -- embedding, layers, full-sequence terminal norm,
  token-chunked head + summed cross-entropy / normaliser, norm VJP, one
  decoder backward (engine.py:48-79).  The terminal runs on the HIP path:
  RMSNorm kernels for the norm and its VJP, and ``ops.chunked_causal_loss``
  (native_terminal.py:11-47) -- per token chunk a bf16 head GEMM, one
  in-place cross-entropy/gradient pass over the bf16 logits and a bf16 GEMM
  back to the hidden size.
* :class:`AdamW` -- the fp32 update in torch.optim.AdamW's non-foreach order
  (optimizer.py:324-342), on the device.
* :func:`train` -- the optimizer-step loop with gradient accumulation over
  cyclic rows (engine.py:162-182), microbatch-major as the reference or
  layer-major (:func:`window_layer_major`: one layer load per phase per
  accumulation window instead of one per microbatch, same results).
* :class:`DenseModel` -- the adapter surface the engine uses
  (adapters/protocol.py:23-34) for a Llama-family model whose decoder
  matrices are stored 4-bit.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from . import ops, slots
from .dense import positions_and_masks
from .recompute import (_borrow_weights, _call_functional_block, block_adapter_backward,
                        streaming_block)


def flatten(model) -> dict:
    """``{"{layer}:{target}": projection}`` (engine.py:21-33)."""
    result, seen = {}, set()
    for block in model.blocks:
        for name, proj in block.adapters.items():
            key = f"{block.index}:{name}"
            if key in result or id(proj) in seen:
                raise ValueError("unsupported_capability: duplicate/shared trainable parameter")
            result[key] = proj
            seen.add(id(proj))
    if not result:
        raise ValueError("training plan has no trainable projections")
    return result


def forward(model, session, hidden, positions, masks, *, accumulate=False):
    for block in model.blocks:
        hidden = streaming_block(hidden, positions, masks[block.kind], block.functional, block.kwargs,
                                 session.reloader(block), block.adapters, block.index,
                                 accumulate_adapter_grads=accumulate)
    return hidden


def microbatch(model, session, input_ids, labels, *, normalization, token_chunk, accumulate=False):
    """Exact shifted summed CE / window token count; one decoder backward."""
    device = model.device
    valid = torch.ones_like(input_ids, dtype=torch.bool)
    positions, masks = model.positions_and_masks(valid)
    embedded = F.embedding(input_ids.cpu(), model.embedding).to(device).detach().requires_grad_(True)
    hidden = forward(model, session, embedded, positions, masks, accumulate=accumulate)
    terminal_input = hidden.detach().requires_grad_(True)
    normalized = model.terminal_norm(terminal_input)
    chunks = ops.supervised_chunk_intervals(labels, token_chunk)
    loss = ops.chunked_causal_loss(normalized, model.head, labels,
                                   normalization=normalization, token_chunk=token_chunk,
                                   supervised_chunks=chunks)
    (gradient,) = torch.autograd.grad(loss, terminal_input)
    if not torch.isfinite(loss) or not torch.isfinite(gradient).all():
        raise FloatingPointError("non-finite causal loss/gradient")
    hidden.backward(gradient)
    return float(loss.detach()), embedded.grad.detach().clone()


def window_layer_major(model, session, items, *, normalization, token_chunk):
    """One gradient-accumulation window processed layer by layer, so each
    layer's 4-bit image crosses PCIe once per phase instead of once per
    microbatch (the reference streams every layer for every microbatch,
    engine.py:168-178):

    * forward: every microbatch through layer i (no grad) before layer i+1,
      keeping each microbatch's layer inputs (one bf16 [B,S,H] per layer and
      microbatch, as the recompute driver saves);
    * terminal per microbatch, in order (as ``microbatch``);
    * backward: per layer in reverse, the recompute + VJP of every microbatch
      in order, adding adapter gradients (the first microbatch replaces).

    For each layer the fp32 adapter-gradient sums take the microbatches in the
    same order as the microbatch-major loop, so the gradients and losses are
    the same bits.  Returns the per-microbatch losses."""
    device = model.device
    mbs = []
    for ids, labels in items:
        valid = torch.ones_like(ids, dtype=torch.bool)
        positions, masks = model.positions_and_masks(valid)
        embedded = F.embedding(ids.cpu(), model.embedding).to(device)
        mbs.append({"pos": positions, "masks": masks, "h": [embedded], "labels": labels})
    for block in model.blocks:
        with _borrow_weights(session.reloader(block), "forward") as weights, torch.no_grad():
            for mb in mbs:
                mb["h"].append(_call_functional_block(block.functional, mb["h"][-1], mb["pos"],
                                                      mb["masks"][block.kind], weights,
                                                      block.kwargs))
    losses = []
    for mb in mbs:
        terminal_input = mb["h"].pop().detach().requires_grad_(True)
        normalized = model.terminal_norm(terminal_input)
        loss = ops.chunked_causal_loss(
            normalized, model.head, mb["labels"], normalization=normalization,
            token_chunk=token_chunk,
            supervised_chunks=ops.supervised_chunk_intervals(mb["labels"], token_chunk))
        (mb["g"],) = torch.autograd.grad(loss, terminal_input)
        if not torch.isfinite(loss) or not torch.isfinite(mb["g"]).all():
            raise FloatingPointError("non-finite causal loss/gradient")
        losses.append(float(loss.detach()))
    for block in reversed(model.blocks):
        ordered = sorted(block.adapters.values(), key=lambda p: p.name)
        with _borrow_weights(session.reloader(block), "backward") as weights:
            for k, mb in enumerate(mbs):
                hidden = mb["h"].pop().detach().requires_grad_(True)
                with torch.enable_grad():
                    out = _call_functional_block(block.functional, hidden, mb["pos"],
                                                 mb["masks"][block.kind], weights, block.kwargs)
                # the first microbatch replaces (zero + add), later ones accumulate
                mb["g"] = block_adapter_backward(out, hidden, ordered, mb["g"], k > 0, block.index)
    return losses


class AdamW:
    """Bias-corrected fp32 AdamW over LoRA projections (optimizer.py:227-342)."""

    def __init__(self, lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0):
        self.lr, self.beta1, self.beta2, self.eps = lr, beta1, beta2, eps
        self.weight_decay = weight_decay
        self.step_count = 0

    def zero_grad(self, projections):
        for p in projections.values():
            p.grad_A.zero_()
            p.grad_B.zero_()
            p.A.grad = None
            p.B.grad = None

    def step(self, projections):
        n = self.step_count + 1
        step_size = self.lr / (1.0 - self.beta1 ** n)
        bc2_sqrt = math.sqrt(1.0 - self.beta2 ** n)
        with torch.no_grad():
            for p in projections.values():
                for param, grad, m, v in ((p.A, p.grad_A, p.m_A, p.v_A), (p.B, p.grad_B, p.m_B, p.v_B)):
                    if self.weight_decay != 0.0:
                        param.mul_(1.0 - self.lr * self.weight_decay)
                    m.lerp_(grad, 1.0 - self.beta1)
                    v.mul_(self.beta2).addcmul_(grad, grad, value=1.0 - self.beta2)
                    denom = (v.sqrt() / bc2_sqrt).add_(self.eps)
                    param.addcdiv_(m, denom, value=-step_size)
        self.step_count = n


def train(model, session, rows, *, steps, accumulation=1, lr=1e-4, weight_decay=0.0,
          token_chunk=64, layer_major=False):
    """Optimizer-step loop with cyclic rows (engine.py:162-182); returns losses.
    ``layer_major`` runs each accumulation window with ``window_layer_major``
    (same results, one layer load per phase per window)."""
    projections = flatten(model)
    optimizer = AdamW(lr=lr, weight_decay=weight_decay)
    cursor, losses = 0, []
    for _ in range(steps):
        items = [rows[(cursor + i) % len(rows)] for i in range(accumulation)]
        normalization = sum(int((labels[:, 1:] != -100).sum()) for _, labels in items)
        optimizer.zero_grad(projections)
        loss = 0.0
        with session.run():
            if layer_major:
                for micro in window_layer_major(model, session, items,
                                                normalization=normalization,
                                                token_chunk=token_chunk):
                    loss += micro
            else:
                for i, (ids, labels) in enumerate(items):
                    micro, _ = microbatch(model, session, ids, labels,
                                          normalization=normalization, token_chunk=token_chunk,
                                          accumulate=i > 0)
                    loss += micro
            optimizer.step(projections)
        cursor += accumulation
        losses.append(loss)
    return losses


class DenseModel:
    """Llama-family model with 4-bit decoder matrices in slot images: the
    runtime surface of adapters/dense.py:178-263 the engine needs."""

    def __init__(self, *, embedding, norm, head, layers=None, heads, kv_heads, head_dim, eps,
                 theta, rank, alpha, targets, device, codec="nf4-g128", generator=None,
                 blocks=None, qk_norm=False):
        """``layers``: per-layer weight dicts, encoded here; or ``blocks``:
        prebuilt BlockPlans (e.g. ``slots.make_archive_block``)."""
        self.device = torch.device(device)
        self.embedding = embedding.to(torch.bfloat16).contiguous()      # stays on the host
        self.norm = norm.to(torch.bfloat16).to(self.device)
        self.head = head.to(torch.bfloat16).to(self.device)
        self.eps, self.theta, self.head_dim = eps, theta, head_dim
        if (layers is None) == (blocks is None):
            raise ValueError("DenseModel needs exactly one of layers / blocks")
        self.blocks = list(blocks) if blocks is not None else [
            slots.make_dense_block(i, w, codec=codec, heads=heads, kv_heads=kv_heads,
                                   head_dim=head_dim, eps=eps, rank=rank, alpha=alpha,
                                   targets=targets, device=self.device, generator=generator,
                                   qk_norm=qk_norm)
            for i, w in enumerate(layers)]

    def positions_and_masks(self, valid):
        rot, mask = positions_and_masks(valid, head_dim=self.head_dim, theta=self.theta,
                                        device=self.device)
        return rot, {"full_attention": mask}

    def terminal_norm(self, hidden):
        B, S, H = hidden.shape
        return ops.rms_norm(hidden.reshape(B * S, H), self.norm, self.eps).view(B, S, H)

    def close(self):
        self.blocks.clear()
