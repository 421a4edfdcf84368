"""Streaming recompute driver (mirror of training/recompute.py:16-227 in
/root/reference/src/ram_vram_finetune).

Forward: borrow the block's weights, run the functional without grad, keep a
clone of the input.  Backward: borrow again, recompute with grad, call
``torch.autograd.grad(output, [hidden, A0, B0, ...])`` (adapters in name
order) and add the adapter gradients into the fp32 ``grad_A``/``grad_B``
buffers (replace unless accumulating).  Same signature, argument meaning and
errors as the reference, so an engine can switch implementations freely;
the weight views it borrows are 4-bit slot views for the HIP functional.
"""
from __future__ import annotations

from contextlib import contextmanager
from typing import Callable, Optional

import torch

from . import ops


class StreamingBlockFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden_states, position_embeddings, attention_mask, func_block, func_kwargs,
                weight_reloader, lora_dict, block_idx, accumulate_adapter_grads=False):
        _validate_lora_bindings(func_kwargs, lora_dict)
        ctx.func_block = func_block
        ctx.func_kwargs = func_kwargs
        ctx.weight_reloader = weight_reloader
        ctx.lora_dict = lora_dict
        ctx.block_idx = block_idx
        ctx.accumulate_adapter_grads = accumulate_adapter_grads
        ctx.position_embeddings = position_embeddings
        ctx.attention_mask = attention_mask
        ctx.save_for_backward(hidden_states.detach().clone())
        with _borrow_weights(weight_reloader, "forward") as weights:
            return _call_functional_block(func_block, hidden_states, position_embeddings,
                                          attention_mask, weights, func_kwargs)

    @staticmethod
    def backward(ctx, grad_output):
        hidden = ctx.saved_tensors[0].detach().requires_grad_(True)
        ordered = sorted(ctx.lora_dict.values(), key=lambda p: p.name)
        with _borrow_weights(ctx.weight_reloader, "backward") as weights:
            with torch.enable_grad():
                output = _call_functional_block(ctx.func_block, hidden, ctx.position_embeddings,
                                                ctx.attention_mask, weights, ctx.func_kwargs)
            dx = block_adapter_backward(output, hidden, ordered, grad_output,
                                        ctx.accumulate_adapter_grads, ctx.block_idx)
        return (dx,) + (None,) * 8


def block_adapter_backward(output, hidden, ordered, grad_output, accumulate, block_idx):
    """Backward of one recomputed block: returns d hidden and replaces (or,
    with ``accumulate``, adds to) every projection's ``grad_A``/``grad_B``
    (training/recompute.py:102-133).

    The q4 projections hand their adapter products to a gradient sink that
    writes the buffers directly after autograd returns (one batched launch per
    16 products); the gradients autograd still returns (adapters outside those
    projections) go through one multi-tensor copy or add."""
    inputs = [hidden] + [t for p in ordered for t in (p.A, p.B)]
    with ops.lora_grad_sink(hidden.device, accumulate) as sink:
        grads = torch.autograd.grad(output, inputs, grad_output, allow_unused=True)
        sink.flush()
    if grads[0] is None:
        raise RuntimeError(f"block {block_idx} lost its input gradient")
    dst, src, dst_add, src_add = [], [], [], []
    for i, proj in enumerate(ordered):
        if not accumulate:
            for t in (proj.A.grad, proj.B.grad):
                if t is not None:
                    t.zero_()
        ga, gb = grads[1 + 2 * i], grads[2 + 2 * i]
        if id(proj) in sink.written:
            # the sink wrote (or added) this adapter's products; a further use
            # of it in the block came back through autograd and is added
            for buf, g in ((proj.grad_A, ga), (proj.grad_B, gb)):
                if g is not None:
                    dst_add.append(buf)
                    src_add.append(g.detach().to(buf))
            continue
        if ga is None or gb is None:
            missing = [n for n, g in (("A", ga), ("B", gb)) if g is None]
            raise RuntimeError(f"block {block_idx} adapter {proj.name} is disconnected; "
                               f"missing gradients for {missing}")
        if accumulate:
            dst_add += [proj.grad_A, proj.grad_B]
            src_add += [ga.detach().to(proj.grad_A), gb.detach().to(proj.grad_B)]
        else:
            dst += [proj.grad_A, proj.grad_B]
            src += [ga.detach().to(proj.grad_A), gb.detach().to(proj.grad_B)]
    # one multi-tensor launch each: replace (zero + add in the reference) or
    # accumulate
    if dst:
        torch._foreach_copy_(dst, src)
    if dst_add:
        torch._foreach_add_(dst_add, src_add)
    return grads[0]


@contextmanager
def _borrow_weights(reloader, phase):
    borrow = getattr(reloader, "borrow", None)
    if borrow is None:
        yield reloader()
    else:
        with borrow(phase) as weights:
            yield weights


def _call_functional_block(func_block, hidden_states, position_embeddings, attention_mask,
                           weights, func_kwargs):
    reserved = {"hidden_states", "position_embeddings", "attention_mask"}
    dup = reserved.intersection(func_kwargs)
    if dup:
        raise TypeError(f"func_kwargs duplicates StreamingBlockFunction arguments: {sorted(dup)}")
    overlap = set(weights).intersection(func_kwargs)
    if overlap:
        raise TypeError(f"weight/functional kwargs overlap: {sorted(overlap)}")
    for name, weight in weights.items():
        if getattr(weight, "requires_grad", False):
            raise ValueError(f"base weight {name!r} must remain frozen")
    return func_block(hidden_states=hidden_states, position_embeddings=position_embeddings,
                      attention_mask=attention_mask, **weights, **func_kwargs)


def _validate_lora_bindings(func_kwargs, lora_dict):
    if not isinstance(lora_dict, dict):
        raise TypeError("lora_dict must be a dict of LoRA projections")
    expected = [id(v) for v in lora_dict.values()]
    bound = [id(v) for v in func_kwargs.values() if hasattr(v, "A") and hasattr(v, "grad_A")]
    if len(expected) != len(set(expected)):
        raise ValueError("lora_dict contains the same projection more than once")
    if len(bound) != len(set(bound)):
        raise ValueError("functional kwargs bind the same LoRA projection more than once")
    if set(expected) != set(bound):
        raise ValueError("functional LoRA bindings must be the exact projections exposed "
                         "to the optimizer/gradient buffers")


def streaming_block(hidden_states, position_embeddings, attention_mask, func_block: Callable,
                    func_kwargs: dict, weight_reloader, lora_dict: dict, block_idx: int, *,
                    accumulate_adapter_grads: bool = False) -> torch.Tensor:
    return StreamingBlockFunction.apply(hidden_states, position_embeddings, attention_mask,
                                        func_block, func_kwargs, weight_reloader, lora_dict,
                                        block_idx, accumulate_adapter_grads)
