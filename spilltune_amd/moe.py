"""Mixture-of-experts feed-forward over 4-bit experts (mirror of
adapters/qwen3_moe.py:95-113 and the routed-expert loop of
adapters/deepseek.py:115-176 in /root/reference/src/ram_vram_finetune).

The reference loops over hit experts in Python, gathering each expert's
tokens, running two small ``F.linear`` calls and ``index_add_``-ing the
weighted result.  Here one forward is a fixed sequence of launches,
independent of the routing:

1. router logits (bf16 GEMM) and softmax top-k (``st_moe_route_softmax``);
2. token permutation by expert (``st_moe_permute``);
3. grouped gate|up 4-bit GEMM over the permuted rows, gathering token rows
   on the fly, with the per-expert LoRA of gate and up in its epilogue;
4. SwiGLU; grouped down GEMM (+ per-expert LoRA);
5. weighted combine in the reference's bf16 ``index_add_`` order.

The backward is the VJP autograd derives for the reference expression:
combine VJP (value and routing-weight gradients), grouped dgrad GEMMs with
the LoRA terms in their epilogues, per-expert LoRA gradients, router VJP,
and the gather-sum of the permuted input gradients.

The experts stay frozen as in the reference; the per-expert LoRA on
gate/up/down (``ExpertLoRA``) is this build's extension for the MoE
benchmark configuration and is optional.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

from . import _lib
from .codecs import GROUP, codebook, encode
from .ops import _launch, lora_gemm

_BF16 = torch.bfloat16
_F32 = torch.float32
_I32 = torch.int32


@dataclass
class Q4Experts:
    """``E`` frozen ``[N, K]`` 4-bit matrices stored back to back (expert e's
    payload is bytes ``[e N K/2, (e+1) N K/2)``, its scales the matching
    ``N K / 128`` floats), the packed-3D layout of qwen3_moe.py:107-108."""
    payload: torch.Tensor
    scales: torch.Tensor
    experts: int
    out_features: int
    in_features: int
    codec: str
    flags: int = 0

    def __post_init__(self):
        E, N, K = self.experts, self.out_features, self.in_features
        if K % GROUP:
            raise ValueError(f"unsupported_capability: expert in_features {K} must be a multiple "
                             f"of {GROUP}")
        if self.payload.numel() != E * N * K // 2 or self.scales.numel() != E * N * K // GROUP:
            raise ValueError("Q4Experts payload/scales sizes do not match the expert shape")

    def lut(self):
        return _lib.lut_array(codebook(self.codec))

    @property
    def device(self):
        return self.payload.device

    def dequantize(self) -> torch.Tensor:
        """bf16 ``[E, N, K]`` copy (for checks only)."""
        E, N, K = self.experts, self.out_features, self.in_features
        out = torch.empty((E, N, K), dtype=_BF16, device=self.device)
        _lib.call("st_dequant4", _lib.ptr(self.payload), _lib.ptr(self.scales), E * N * K, GROUP,
                  self.lut(), self.flags, _lib.ptr(out), _lib.stream_handle(self.device))
        return out


def quantize_experts(weights: torch.Tensor, codec: str, device) -> Q4Experts:
    """Encode a frozen ``[E, N, K]`` host tensor (K a multiple of 128, so the
    flat groups of the stack are exactly each expert's groups)."""
    E, N, K = weights.shape
    rec = encode(weights.reshape(E * N, K).contiguous(), codec)
    return Q4Experts(rec.parts["payload"].to(device), rec.parts["scales"].to(device), E, N, K,
                     codec)


@dataclass
class ExpertLoRA:
    """Per-expert fp32 LoRA of one expert projection: ``A [E, R, K]``,
    ``B [E, N, r]`` with ``R = segments * r`` (gate|up share one object:
    rows ``[s r, (s+1) r)`` of A and ``[s N/segments, ...)`` of B belong to
    segment s).  Same field names as ``LoRAProjection`` so the optimizer and
    checkpoint code treat it alike."""
    name: str
    rank: int
    alpha: float
    experts: int
    in_features: int
    out_features: int
    segments: int = 1
    A: torch.Tensor = None
    B: torch.Tensor = None
    grad_A: torch.Tensor = field(default=None)
    grad_B: torch.Tensor = field(default=None)
    m_A: torch.Tensor = field(default=None)
    v_A: torch.Tensor = field(default=None)
    m_B: torch.Tensor = field(default=None)
    v_B: torch.Tensor = field(default=None)
    target_path: Optional[str] = None
    layer: Optional[int] = None

    def __post_init__(self):
        E, r, s = self.experts, self.rank, self.segments
        if self.out_features % s:
            raise ValueError("out_features must split evenly into the segments")
        shape_a, shape_b = (E, s * r, self.in_features), (E, self.out_features, r)
        for name, t, shape in (("A", self.A, shape_a), ("B", self.B, shape_b)):
            if t is None or t.dtype != _F32 or tuple(t.shape) != shape:
                raise ValueError(f"{self.name}.{name} must be fp32 {shape}")
        self.A = self.A.detach().clone().requires_grad_(True)
        self.B = self.B.detach().clone().requires_grad_(True)
        for suffix, ref in (("grad_A", self.A), ("grad_B", self.B), ("m_A", self.A),
                            ("v_A", self.A), ("m_B", self.B), ("v_B", self.B)):
            if getattr(self, suffix) is None:
                setattr(self, suffix, torch.zeros_like(ref.detach()))
        self.target_path = self.target_path or self.name

    @property
    def scale(self) -> float:
        return self.alpha / self.rank

    def zero_grad(self) -> None:
        self.grad_A.zero_()
        self.grad_B.zero_()
        self.A.grad = None
        self.B.grad = None


def make_expert_lora(name, experts, in_features, out_features, *, rank, alpha, device,
                     segments=1, generator=None, b_std=0.0) -> ExpertLoRA:
    """``A = randn * 0.02`` and ``B = 0`` (or ``N(0, b_std)``) per expert, the
    reference's projection init (finetune/lora.py:319-388) applied per expert."""
    A = torch.randn(experts, segments * rank, in_features, generator=generator).mul_(0.02)
    B = torch.zeros(experts, out_features, rank)
    if b_std:
        B.normal_(0.0, b_std, generator=generator)
    return ExpertLoRA(name, rank, alpha, experts, in_features, out_features, segments,
                      A.to(device), B.to(device))


# ----------------------------------------------------------------- the function
def _stream(dev):
    return _lib.stream_handle(dev)


def _router_parts(router: torch.Tensor) -> torch.Tensor:
    """``[hi; mid; lo]`` bf16 rows [3E, H] of an fp32 router with
    hi + mid + lo == router exactly (normal-range values).  The router is
    frozen: the split is kept on the tensor itself, remade only when its
    version counter moves."""
    cached = getattr(router, "_st_parts", None)
    if cached is not None and cached[0] == router._version:
        return cached[1]
    w = router.detach().float()
    hi = w.to(_BF16)
    r1 = w - hi.float()
    mid = r1.to(_BF16)
    lo = (r1 - mid.float()).to(_BF16)
    parts = torch.cat([hi, mid, lo], 0).contiguous()
    router._st_parts = (router._version, parts)
    return parts


def sigmoid_router_logits(flat: torch.Tensor, router: torch.Tensor) -> torch.Tensor:
    """fp32 router logits ``F.linear(flat.float(), router.float())`` of
    deepseek.py:117 for bf16 ``flat [T, H]`` and a bf16 or fp32 ``router [E, H]``.

    They run on the streaming MFMA rank-r kernel (every 64-expert slice in
    one launch), which splits its fp32 operand into three bf16 parts that sum to it
    exactly, so every product is the fp32 product, summed in fp32 -- for a
    bf16 router and for an fp32 one (the reference keeps DeepSeek routers in
    fp32)."""
    T, H = flat.shape
    E = router.shape[0]
    logits = torch.empty((T, E), dtype=_F32, device=flat.device)
    lora_gemm(T, E, H, flat, H, 1, router.float(), 1, H, 1.0, logits)
    return logits


class _MoEFeedForward(torch.autograd.Function):
    @staticmethod
    def forward(ctx, flat, router, bias, gate_up, down, cfg, *lora):
        top_k, norm, gu_rank, gu_scale, d_rank, d_scale, sig, groups, group_k, rscale = cfg
        T, H = flat.shape
        E = gate_up.experts
        I = down.in_features
        R = T * top_k
        dev = flat.device
        st = _stream(dev)
        lut_gu, lut_d = gate_up.lut(), down.lut()
        has_lora = bool(lora)
        has_gu, has_d = gu_rank > 0, d_rank > 0
        # 1. router
        weights = torch.empty((T, top_k), dtype=_F32, device=dev)
        indices = torch.empty((T, top_k), dtype=_I32, device=dev)
        if sig:
            # deepseek.py:117-125: fp32 logits F.linear(hidden.float(), weight.float()),
            # sigmoid group-limited selection with the bias, fp32 weights * scale
            logits = sigmoid_router_logits(flat, router)
            _lib.call("st_moe_route_sigmoid", _lib.ptr(logits), _lib.ptr(bias), T, E, groups,
                      group_k, top_k, int(norm), float(rscale), _lib.ptr(weights),
                      _lib.ptr(indices), st)
        else:
            logits = torch.empty((T, E), dtype=_BF16, device=dev)
            _lib.call("st_linear_bf16_fwd", _lib.ptr(flat), T, H, H, _lib.ptr(router), E, H,
                      _lib.ptr(logits), E, st)
            _lib.call("st_moe_route_softmax", _lib.ptr(logits), T, E, top_k, int(norm), 1,
                      _lib.ptr(weights), _lib.ptr(indices), st)
        # 2. permutation
        offsets = torch.empty(E + 1, dtype=_I32, device=dev)
        row_token = torch.empty(R, dtype=_I32, device=dev)
        pick_row = torch.empty(R, dtype=_I32, device=dev)
        _lib.call("st_moe_permute", _lib.ptr(indices), T, top_k, E, _lib.ptr(offsets),
                  _lib.ptr(row_token), _lib.ptr(pick_row), st)
        # 3. gate|up with per-expert LoRA (segments gate, up)
        A_gu = B_gu = A_d = B_d = T_gu = T_d = None
        if has_lora:
            A_gu, B_gu, A_d, B_d = (None if t is None else t.detach() for t in lora)
        if has_gu:
            T_gu = torch.empty((R, 2 * gu_rank), dtype=_F32, device=dev)
            _lib.call("st_moe_lora_rows", R, 2 * gu_rank, H, 1, _lib.ptr(flat), H, T,
                      _lib.ptr(row_token), _lib.ptr(A_gu), 1, H, 2 * gu_rank * H,
                      _lib.ptr(offsets), E, 1.0, _lib.ptr(T_gu), 2 * gu_rank, st)
        gu = torch.empty((R, 2 * I), dtype=_BF16, device=dev)
        _launch(("moe_fwd", R, 2 * I, H), lambda: _lib.call(
            "st_q4_grouped_fwd", _lib.ptr(flat), T, H, _lib.ptr(row_token), R, H,
            _lib.ptr(offsets), E, _lib.ptr(gate_up.payload), _lib.ptr(gate_up.scales), 2 * I,
            lut_gu, gate_up.flags, _lib.ptr(T_gu), 2 * gu_rank if has_gu else 0,
            _lib.ptr(B_gu), gu_rank if has_gu else 0, float(gu_scale),
            2 if has_gu else 0, _lib.i64_array([I, 2 * I]) if has_gu else None,
            _lib.ptr(gu), 2 * I, st))
        # 4. SwiGLU and down
        h = torch.empty((R, I), dtype=_BF16, device=dev)
        _lib.call("st_swiglu_fwd", _lib.ptr(gu), 2 * I, _lib.ptr(gu[:, I:]), 2 * I, R, I,
                  _lib.ptr(h), I, st)
        if has_d:
            T_d = torch.empty((R, d_rank), dtype=_F32, device=dev)
            _lib.call("st_moe_lora_rows", R, d_rank, I, 1, _lib.ptr(h), I, R, None,
                      _lib.ptr(A_d), 1, I, d_rank * I, _lib.ptr(offsets), E, 1.0,
                      _lib.ptr(T_d), d_rank, st)
        v = torch.empty((R, H), dtype=_BF16, device=dev)
        _launch(("moe_fwd", R, H, I), lambda: _lib.call(
            "st_q4_grouped_fwd", _lib.ptr(h), R, I, None, R, I, _lib.ptr(offsets), E,
            _lib.ptr(down.payload), _lib.ptr(down.scales), H, lut_d, down.flags,
            _lib.ptr(T_d), d_rank if has_d else 0, _lib.ptr(B_d), d_rank if has_d else 0,
            float(d_scale), 1 if has_d else 0, _lib.i64_array([H]) if has_d else None,
            _lib.ptr(v), H, st))
        # 5. combine
        out = torch.empty((T, H), dtype=_BF16, device=dev)
        _lib.call("st_moe_combine", _lib.ptr(v), R, _lib.ptr(weights), _lib.ptr(indices),
                  _lib.ptr(pick_row), T, top_k, H, _lib.ptr(out), st)
        ctx.meta = (gate_up, down, cfg, has_lora, has_gu, has_d)
        ctx.save_for_backward(flat, router, logits, weights, indices, offsets, row_token,
                              pick_row, gu, h, v, T_gu, T_d, A_gu, B_gu, A_d, B_d)
        ctx.mark_non_differentiable(logits, weights, indices)
        return out, logits, weights, indices

    @staticmethod
    def backward(ctx, dout, _dlogits, _dweights, _dindices):
        gate_up, down, cfg, has_lora, has_gu, has_d = ctx.meta
        top_k, norm, gu_rank, gu_scale, d_rank, d_scale, sig, groups, group_k, rscale = cfg
        (flat, router, logits, weights, indices, offsets, row_token, pick_row, gu, h, v,
         T_gu, T_d, A_gu, B_gu, A_d, B_d) = ctx.saved_tensors
        dout = dout.contiguous()
        T, H = flat.shape
        E, I = gate_up.experts, down.in_features
        R = T * top_k
        dev = flat.device
        st = _stream(dev)
        # combine VJP
        dv = torch.empty((R, H), dtype=_BF16, device=dev)
        dw = torch.empty((T, top_k), dtype=_F32, device=dev)
        # bf16 routing weights (Qwen3) round the products and the sum; DeepSeek's
        # fp32 weights promote value * weight to fp32
        _lib.call("st_moe_combine_bwd", _lib.ptr(dout), _lib.ptr(v), R, _lib.ptr(weights),
                  _lib.ptr(pick_row), T, top_k, H, 0 if sig else 1, _lib.ptr(dv), _lib.ptr(dw),
                  st)
        grads = [None, None, None, None] if has_lora else []
        dT_d = dT_gu = None
        if has_d:
            dT_d = torch.empty((R, d_rank), dtype=_F32, device=dev)
            _lib.call("st_moe_lora_rows", R, d_rank, H, 1, _lib.ptr(dv), H, R, None,
                      _lib.ptr(B_d), d_rank, 1, H * d_rank, _lib.ptr(offsets), E,
                      float(d_scale), _lib.ptr(dT_d), d_rank, st)
            dB_d = torch.empty_like(B_d)
            _lib.call("st_moe_lora_grads", R, d_rank, H, 1, _lib.ptr(dv), H, R, None,
                      _lib.ptr(T_d), d_rank, 1, _lib.ptr(offsets), E, float(d_scale),
                      _lib.ptr(dB_d), H * d_rank, d_rank, 1, 0, st)
            dA_d = torch.empty_like(A_d)
            _lib.call("st_moe_lora_grads", R, d_rank, I, 1, _lib.ptr(h), I, R, None,
                      _lib.ptr(dT_d), d_rank, 1, _lib.ptr(offsets), E, 1.0,
                      _lib.ptr(dA_d), d_rank * I, 1, I, 0, st)
            grads[2:] = [dA_d, dB_d]
        # the down dgrad's epilogue applies the SwiGLU VJP: dgate|dup directly
        dgu = torch.empty((R, 2 * I), dtype=_BF16, device=dev)
        _launch(("moe_dgrad", R, H, I), lambda: _lib.call(
            "st_q4_grouped_dgrad_swiglu", _lib.ptr(dv), H, R, H, _lib.ptr(offsets), E,
            _lib.ptr(down.payload), _lib.ptr(down.scales), I, down.lut(), down.flags,
            _lib.ptr(dT_d), d_rank if has_d else 0, _lib.ptr(A_d), d_rank if has_d else 0,
            _lib.ptr(gu), 2 * I, _lib.ptr(dgu), 2 * I, st))
        if has_gu:
            dT_gu = torch.empty((R, 2 * gu_rank), dtype=_F32, device=dev)
            _lib.call("st_moe_lora_rows", R, gu_rank, I, 2, _lib.ptr(dgu), 2 * I, R, None,
                      _lib.ptr(B_gu), gu_rank, 1, 2 * I * gu_rank, _lib.ptr(offsets), E,
                      float(gu_scale), _lib.ptr(dT_gu), 2 * gu_rank, st)
            dB_gu = torch.empty_like(B_gu)
            _lib.call("st_moe_lora_grads", R, gu_rank, I, 2, _lib.ptr(dgu), 2 * I, R, None,
                      _lib.ptr(T_gu), 2 * gu_rank, 1, _lib.ptr(offsets), E, float(gu_scale),
                      _lib.ptr(dB_gu), 2 * I * gu_rank, gu_rank, 1, 0, st)
            dA_gu = torch.empty_like(A_gu)
            _lib.call("st_moe_lora_grads", R, 2 * gu_rank, H, 1, _lib.ptr(flat), H, T,
                      _lib.ptr(row_token), _lib.ptr(dT_gu), 2 * gu_rank, 1, _lib.ptr(offsets),
                      E, 1.0, _lib.ptr(dA_gu), 2 * gu_rank * H, 1, H, 0, st)
            grads[:2] = [dA_gu, dB_gu]
        dxs = torch.empty((R, H), dtype=_BF16, device=dev)
        _launch(("moe_dgrad", R, 2 * I, H), lambda: _lib.call(
            "st_q4_grouped_dgrad", _lib.ptr(dgu), 2 * I, R, 2 * I, _lib.ptr(offsets), E,
            _lib.ptr(gate_up.payload), _lib.ptr(gate_up.scales), H, gate_up.lut(),
            gate_up.flags, _lib.ptr(dT_gu), 2 * gu_rank if has_gu else 0, _lib.ptr(A_gu),
            2 * gu_rank if has_gu else 0, _lib.ptr(dxs), H, st))
        # router VJP and the input gradient over every use of flat
        if sig:
            # the router is frozen; its input gradient is fp32 dlogits @ W
            dlogits = torch.empty((T, E), dtype=_F32, device=dev)
            _lib.call("st_moe_route_sigmoid_bwd", _lib.ptr(logits), _lib.ptr(indices),
                      _lib.ptr(dw), T, E, top_k, int(norm), float(rscale), _lib.ptr(dlogits), st)
            drouter = torch.empty((T, H), dtype=_F32, device=dev)
            if router.dtype == _BF16:
                lora_gemm(T, H, E, dlogits, E, 1, router, H, 1, 1.0, drouter)
            else:
                # fp32 router: W = hi + mid + lo exactly (bf16 parts), so
                # dlogits @ W = [dlogits | dlogits | dlogits] @ [hi; mid; lo],
                # one streaming product with every term an fp32 product
                parts = _router_parts(router)
                lora_gemm(T, H, 3 * E, dlogits.repeat(1, 3), 3 * E, 1, parts, H, 1, 1.0, drouter)
            dflat = torch.empty((T, H), dtype=_BF16, device=dev)
            _lib.call("st_moe_gather_sum", _lib.ptr(dxs), R, _lib.ptr(pick_row), T, top_k, H,
                      _lib.ptr(drouter), _lib.ST_DTYPE_F32, _lib.ptr(dflat), st)
            return (dflat, None, None, None, None, None, *grads)
        dlogits = torch.empty((T, E), dtype=_BF16, device=dev)
        _lib.call("st_moe_route_softmax_bwd", _lib.ptr(logits), _lib.ptr(indices), _lib.ptr(dw),
                  T, E, top_k, int(norm), _lib.ptr(dlogits), st)
        Ec = E
        if E % 8:  # the GEMM contracts 16-byte chunks: zero-pad the expert dimension
            Ec = E + (-E) % 8
            padded = torch.zeros((T, Ec), dtype=_BF16, device=dev)
            padded[:, :E].copy_(dlogits)
            rpad = torch.zeros((Ec, H), dtype=_BF16, device=dev)
            rpad[:E].copy_(router)
            dlogits, router = padded, rpad
        drouter = torch.empty((T, H), dtype=_BF16, device=dev)
        _lib.call("st_linear_bf16_dgrad", _lib.ptr(dlogits), T, Ec, Ec, _lib.ptr(router), H, H,
                  _lib.ptr(drouter), H, st)
        dflat = torch.empty((T, H), dtype=_BF16, device=dev)
        _lib.call("st_moe_gather_sum", _lib.ptr(dxs), R, _lib.ptr(pick_row), T, top_k, H,
                  _lib.ptr(drouter), _lib.ST_DTYPE_BF16, _lib.ptr(dflat), st)
        return (dflat, None, None, None, None, None, *grads)


def moe_feed_forward(hidden, weights, *, num_experts, top_k, norm_topk_prob, lora_gate_up=None,
                     lora_down=None, return_routing=False):
    """``moe_feed_forward`` of qwen3_moe.py:95-113 on 4-bit experts.

    ``weights``: ``mlp.gate.weight`` (bf16 ``[E, H]`` router),
    ``mlp.experts.gate_up_proj`` and ``mlp.experts.down_proj``
    (:class:`Q4Experts`, ``[E, 2I, H]`` and ``[E, H, I]``).  Optional
    ``lora_gate_up`` (:class:`ExpertLoRA`, 2 segments) and ``lora_down``
    (1 segment), either or both, adapt every expert.  With ``return_routing`` also returns the
    ``(weights, indices)`` the router picked."""
    router = weights["mlp.gate.weight"]
    gate_up = weights["mlp.experts.gate_up_proj"]
    down = weights["mlp.experts.down_proj"]
    if not isinstance(gate_up, Q4Experts) or not isinstance(down, Q4Experts):
        raise ValueError("unsupported_capability: experts must be Q4Experts")
    shape = hidden.shape
    flat = hidden.reshape(-1, shape[-1])
    if flat.dtype != _BF16 or router.dtype != _BF16:
        raise ValueError("moe_feed_forward expects bf16 hidden states and router")
    E, H = router.shape
    I = down.in_features
    if (gate_up.experts, gate_up.out_features, gate_up.in_features) != (E, 2 * I, H) or \
            (down.experts, down.out_features) != (E, H) or E != num_experts:
        raise ValueError("expert shapes do not match the router")
    cfg, lora = _lora_cfg(top_k, norm_topk_prob, lora_gate_up, lora_down,
                          (False, 0, 0, 1.0))
    out, _, w, idx = _MoEFeedForward.apply(flat.contiguous(), router.detach().contiguous(), None,
                                           gate_up, down, cfg, *lora)
    out = out.reshape(shape)
    return (out, w, idx) if return_routing else out


def _lora_cfg(top_k, normalize, lora_gate_up, lora_down, router_cfg):
    """Router/LoRA configuration tuple and the adapter leaves (A_gu, B_gu,
    A_d, B_d; None for an absent adapter, nothing without any): gate_up and
    down are adapted independently."""
    if lora_gate_up is None and lora_down is None:
        return (int(top_k), bool(normalize), 0, 1.0, 0, 1.0) + router_cfg, ()
    if lora_gate_up is not None and lora_gate_up.segments != 2:
        raise ValueError("gate_up LoRA needs 2 segments")
    if lora_down is not None and lora_down.segments != 1:
        raise ValueError("down LoRA needs 1 segment")
    gu = (lora_gate_up.rank, lora_gate_up.scale) if lora_gate_up is not None else (0, 1.0)
    dn = (lora_down.rank, lora_down.scale) if lora_down is not None else (0, 1.0)
    leaves = (getattr(lora_gate_up, "A", None), getattr(lora_gate_up, "B", None),
              getattr(lora_down, "A", None), getattr(lora_down, "B", None))
    return (int(top_k), bool(normalize)) + gu + dn + router_cfg, leaves


def deepseek_moe_feed_forward(hidden, weights, *, num_experts, top_k, groups, group_k,
                              normalize, scale, lora_gate_up=None, lora_down=None,
                              lora_shared=None, return_routing=False):
    """The MoE part of ``deepseek_block`` (adapters/deepseek.py:115-126,
    158-174) on 4-bit experts: ``route`` (fp32 sigmoid scores, selection by
    score + ``e_score_correction_bias`` among the ``group_k`` best of
    ``groups`` expert groups, weights = scores of the picks, renormalised when
    ``normalize``, times ``scale``), the routed experts combined in ascending
    expert order with ``bf16(value * weight)`` accumulated into bf16
    (``index_add_``), plus the shared expert ``mlp.shared_experts.*`` when its
    weights are given: returns ``out + shared(x)`` in bf16, the operand the
    reference adds to the residual.

    ``weights``: ``mlp.gate.weight`` (fp32 or bf16 ``[E, H]``, frozen; the
    reference keeps DeepSeek routers in fp32, deepseek.py:81-83),
    ``mlp.gate.e_score_correction_bias`` (``[E]``), ``mlp.experts.gate_up_proj``
    / ``mlp.experts.down_proj`` (:class:`Q4Experts`) and optionally
    ``mlp.shared_experts.{gate,up,down}_proj.weight`` (:class:`~spilltune_amd.ops.Q4Weight`).
    ``lora_shared`` optionally maps ``"gate"``, ``"up"``, ``"down"`` to LoRA
    projections of the shared expert; ``lora_gate_up``/``lora_down`` adapt
    every routed expert (this build's extension, as for Qwen3)."""
    from . import ops
    router = weights["mlp.gate.weight"]
    bias = weights["mlp.gate.e_score_correction_bias"]
    gate_up = weights["mlp.experts.gate_up_proj"]
    down = weights["mlp.experts.down_proj"]
    if not isinstance(gate_up, Q4Experts) or not isinstance(down, Q4Experts):
        raise ValueError("unsupported_capability: experts must be Q4Experts")
    shape = hidden.shape
    flat = hidden.reshape(-1, shape[-1])
    if flat.dtype != _BF16 or router.dtype not in (_BF16, _F32):
        raise ValueError("deepseek_moe_feed_forward expects bf16 hidden states and a bf16 or "
                         "fp32 router")
    E, H = router.shape
    I = down.in_features
    if (gate_up.experts, gate_up.out_features, gate_up.in_features) != (E, 2 * I, H) or \
            (down.experts, down.out_features) != (E, H) or E != num_experts or \
            tuple(bias.shape) != (E,):
        raise ValueError("expert shapes do not match the router")
    cfg, lora = _lora_cfg(top_k, normalize, lora_gate_up, lora_down,
                          (True, int(groups), int(group_k), float(scale)))
    flat = flat.contiguous()
    out, _, w, idx = _MoEFeedForward.apply(flat, router.detach().contiguous(),
                                           bias.detach().float().contiguous(), gate_up, down,
                                           cfg, *lora)
    prefix = "mlp.shared_experts."
    if prefix + "gate_proj.weight" in weights:
        ls = lora_shared or {}
        wg, wu = weights[prefix + "gate_proj.weight"], weights[prefix + "up_proj.weight"]
        wd = weights[prefix + "down_proj.weight"]
        lg, lu, ldn = ls.get("gate"), ls.get("up"), ls.get("down")
        gu = ops.concat_rows([wg, wu])
        if gu is not None and ops.lora_fusable([lg, lu]):
            shared = ops.q4_lora_linear(ops.q4_lora_linear(flat, gu, [lg, lu]), wd, [ldn],
                                        swiglu=True)
        else:
            act = ops.swiglu_pair(ops.q4_lora_linear(flat, wg, [lg]),
                                  ops.q4_lora_linear(flat, wu, [lu]))
            shared = ops.q4_lora_linear(act, wd, [ldn])
        out = out + shared  # deepseek.py:174, bf16
    out = out.reshape(shape)
    return (out, w, idx) if return_routing else out
