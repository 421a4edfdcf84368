"""Differentiable ops of the per-layer path, each one call into the C ABI.

Every forward reproduces the reference expression it replaces and every
backward the VJP autograd computes for that expression (paths relative to
/root/reference/src/ram_vram_finetune):

* :func:`q4_lora_linear` -- ``LoRAProjection.forward`` (finetune/lora.py:
  205-220) on a frozen 4-bit weight, optionally over N-concatenated
  projections (fused q|k|v or gate|up) and with the decoder residual add
  (adapters/dense.py:149,153) folded into the epilogue.
* :func:`rms_norm` -- adapters/dense.py:115-117.
* :func:`rope_heads` -- adapters/dense.py:127-141 (q/k/v views, transpose,
  rotate) for one projection output.
* :func:`causal_attention` -- adapters/dense.py:142-148 (GQA repeat, fp32
  softmax with the causal mask, relayout to tokens) as flash attention.
* :func:`swiglu` -- adapters/dense.py:153 ``silu(gate) * up``.

Ops run on the current stream, allocate through PyTorch and never fall back
to another implementation.
"""
from __future__ import annotations

import math
from contextlib import contextmanager

from dataclasses import dataclass, field

import torch

from . import _lib
from .codecs import GROUP, codebook

_BF16 = torch.bfloat16
_F32 = torch.float32


# ----------------------------------------------------------------- weights
@dataclass
class Q4Weight:
    """A frozen ``[out, in]`` 4-bit matrix resident on the device (views into a
    slot).  ``segments`` lists the out-widths of N-concatenated projections."""
    payload: torch.Tensor
    scales: torch.Tensor
    shape: tuple
    codec: str
    segments: tuple = field(default=())
    flags: int = 0

    def __post_init__(self):
        self.shape = tuple(int(s) for s in self.shape)
        if not self.segments:
            self.segments = (self.shape[0],)
        if sum(self.segments) != self.shape[0]:
            raise ValueError("Q4Weight segments must sum to out_features")

    @property
    def out_features(self):
        return self.shape[0]

    @property
    def in_features(self):
        return self.shape[1]

    @property
    def device(self):
        return self.payload.device

    @property
    def requires_grad(self):
        return False

    @property
    def group(self):
        """Flat elements per scale: 128, or 64 with ST_FLAG_GROUP64."""
        return 64 if self.flags & _lib.ST_FLAG_GROUP64 else GROUP

    def lut(self):
        return _lib.lut_array(codebook(self.codec))

    def dequantize(self) -> torch.Tensor:
        """bf16 copy of the matrix (for checks / reference-side use only)."""
        out = torch.empty(self.shape, dtype=_BF16, device=self.device)
        _lib.call("st_dequant4", _lib.ptr(self.payload), _lib.ptr(self.scales),
                  self.shape[0] * self.shape[1], self.group, self.lut(), self.flags,
                  _lib.ptr(out), _lib.stream_handle(self.device))
        return out


MAX_LORA_COLS = 64  # LoRA columns (segments x rank) one fused GEMM epilogue stages


def lora_fusable(loras) -> bool:
    """Whether N-concatenated projections with these adapters can run as one
    fused GEMM: no adapter at all, or one on every part with a single rank and
    scale and at most MAX_LORA_COLS LoRA columns in all (the epilogue's
    limit).  Otherwise callers run the projections one by one."""
    loras = list(loras)
    if all(l is None for l in loras):
        return True
    if any(l is None for l in loras):
        return False
    ranks = {int(l.rank) for l in loras}
    scales = {float(l.scale) for l in loras}
    return len(ranks) == 1 and len(scales) == 1 and len(loras) * ranks.pop() <= MAX_LORA_COLS


def concat_rows(weights) -> Q4Weight | None:
    """Zero-copy view of row-concatenated 4-bit weights when their payloads and
    scales are adjacent in memory and each matrix holds whole groups (then the
    flat groups of the concatenation are exactly the parts' groups)."""
    weights = list(weights)
    if len(weights) < 2 or any(not isinstance(w, Q4Weight) for w in weights):
        return None
    first = weights[0]
    K = first.in_features
    if any(w.in_features != K or w.codec != first.codec or w.flags != first.flags
           or len(w.segments) != 1 for w in weights):
        return None
    if (K % first.group) != 0 or any(w.out_features % 32 for w in weights[:-1]):
        return None  # flat groups must not straddle parts; LoRA segments end on 32-column blocks
    # adjacency must hold inside ONE storage: two allocations that merely lie
    # back to back are not one buffer (the view below would run off the first)
    for part in ("payload", "scales"):
        ts = [getattr(w, part) for w in weights]
        storage = ts[0].untyped_storage()
        if any(not t.is_contiguous() or t.dim() != 1 for t in ts):
            return None
        off = ts[0].storage_offset()
        for t in ts:
            if t.untyped_storage().data_ptr() != storage.data_ptr() or t.storage_offset() != off:
                return None
            off += t.numel()
        if off * ts[0].element_size() > storage.nbytes():
            return None
    rows = sum(w.out_features for w in weights)
    base_p, base_s = first.payload, first.scales
    payload = torch.empty(0, dtype=torch.uint8, device=base_p.device).set_(
        base_p.untyped_storage(), base_p.storage_offset(), (rows * K // 2,), (1,))
    scales = torch.empty(0, dtype=_F32, device=base_s.device).set_(
        base_s.untyped_storage(), base_s.storage_offset(), (rows * K // first.group,), (1,))
    return Q4Weight(payload, scales, (rows, K), first.codec,
                    tuple(w.out_features for w in weights), first.flags)


# ----------------------------------------------------------------- timing hook
class KernelTimer:
    """Brackets fused 4-bit GEMM launches with HIP events on the launch
    stream, keyed ``(pass, M, N, K)``; durations are read after a sync.
    ``only``: time the launches with that key alone and run the others
    unbracketed (each timing event leaves the stream idle for a few
    microseconds, which a timed region should not carry for every launch)."""

    def __init__(self, only=None):
        self.events = {}
        self.only = only

    def record(self, key, fn):
        if self.only is not None and key != self.only:
            fn()
            return
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        self.events.setdefault(key, []).append((start, end))

    def summary(self):
        out = {}
        for key, evs in self.events.items():
            ms = [s.elapsed_time(e) for s, e in evs]
            out[key] = {"launches": len(ms), "avg_ms": sum(ms) / len(ms)}
        return out


TIMER: KernelTimer | None = None


def _launch(key, fn):
    if TIMER is None:
        fn()
    else:
        TIMER.record(key, fn)


# ----------------------------------------------------------------- workspace
class _Workspace:
    """Per-device scratch grown on demand through the PyTorch allocator."""

    def __init__(self):
        self._buf = {}

    def get(self, device, nbytes: int) -> torch.Tensor | None:
        if nbytes <= 0:
            return None
        key = (device.type, device.index)
        buf = self._buf.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(int(nbytes * 1.25) + 256, dtype=torch.uint8, device=device)
            self._buf[key] = buf
        return buf


_ws = _Workspace()


def lora_gemm(Mo, No, Kc, a, sam, sak, b, sbk, sbn, alpha, out, accumulate=False):
    """``out = (accumulate ? out : 0) + alpha * sum_k a(m,k) b(k,n)`` (fp32 out)."""
    need = _lib.query("st_lora_gemm_workspace_bytes", Mo, No, Kc)
    ws = _ws.get(out.device, need)
    dt = {_BF16: _lib.ST_DTYPE_BF16, _F32: _lib.ST_DTYPE_F32}
    _lib.call("st_lora_gemm", Mo, No, Kc, _lib.ptr(a), dt[a.dtype], sam, sak, _lib.ptr(b),
              dt[b.dtype], sbk, sbn, float(alpha), _lib.ptr(out), out.stride(0), int(accumulate),
              _lib.ptr(ws), 0 if ws is None else ws.numel(), _lib.stream_handle(out.device))


# ------------------------------------------------------- deferred adapter grads
class LoraGradSink:
    """Collects the adapter-gradient products of one layer's backward while
    autograd runs -- dB_s = s*dY_s^T*T_s and dA_s = dT_s^T*x of every
    projection -- and launches them together (``st_rk_batch``, 16 products per
    call) straight into each adapter's ``grad_A`` / ``grad_B``: added when
    ``accumulate`` (later microbatches of an accumulation window), written
    otherwise.  Only dT, which the input-gradient GEMM needs, runs inside
    autograd.  Each product keeps its split count and summation order, so the
    gradients equal the immediate path's bit for bit."""

    def __init__(self, device, accumulate: bool):
        self.device = torch.device(device)
        self.accumulate = bool(accumulate)
        self.products, self.keep = [], []
        self.written = set()
        self.stream = None

    def wants(self, lora) -> bool:
        """Fp32 contiguous gradient buffers shaped like A and B, and no product
        of this adapter taken yet (a second use in the layer returns its
        gradients through autograd, which the caller adds)."""
        if id(lora) in self.written:
            return False
        ga, gb = getattr(lora, "grad_A", None), getattr(lora, "grad_B", None)
        return all(isinstance(g, torch.Tensor) and g.dtype == _F32 and g.is_contiguous()
                   and g.device == self.device and tuple(g.shape) == tuple(t.shape)
                   for g, t in ((ga, lora.A), (gb, lora.B)))

    def add(self, lora, products, keep):
        # the products run on the stream the backward recorded them on
        if self.stream is None:
            self.stream = torch.cuda.current_stream(self.device)
        self.products += products
        self.keep += keep
        self.written.add(id(lora))

    def flush(self):
        if not self.products:
            return
        st = ctypes_stream(self.stream)
        for i in range(0, len(self.products), 16):
            chunk = self.products[i:i + 16]
            arr = (_lib.RkProduct * len(chunk))(*chunk)
            need = _lib.query("st_rk_batch_workspace_bytes", len(chunk), arr)
            ws = _ws.get(self.device, need)
            _lib.call("st_rk_batch", len(chunk), arr, _lib.ptr(ws),
                      0 if ws is None else ws.numel(), st)
        # the operands may be freed before the products finish: the allocator
        # must not hand their memory to another stream until they have
        for t in self.keep:
            if isinstance(t, torch.Tensor) and t.is_cuda:
                t.record_stream(self.stream)
        self.products, self.keep = [], []


_SINKS: dict = {}


def ctypes_stream(stream):
    return _lib.ctypes.c_void_p(stream.cuda_stream)


@contextmanager
def lora_grad_sink(device, accumulate: bool = False):
    """Route the adapter gradients of q4_lora_linear backwards on ``device``
    into a :class:`LoraGradSink` (call its ``flush()`` before reading them)."""
    key = torch.device(device).index
    prev = _SINKS.get(key)
    sink = LoraGradSink(device, accumulate)
    _SINKS[key] = sink
    try:
        yield sink
    finally:
        if prev is None:
            _SINKS.pop(key, None)
        else:
            _SINKS[key] = prev


def _rk(G, ldg, S, ssk, big, r, Kc, alpha, out, so_m, so_j, accumulate):
    """One column-form st_rk_product (contraction over G's rows)."""
    return _lib.RkProduct(G=G.data_ptr(), ldg=ldg, col=1, S=S.data_ptr(), ssk=ssk, ssj=1, big=big,
                          r=r, Kc=Kc, alpha=float(alpha), out=out.data_ptr(), so_m=so_m,
                          so_j=so_j, accumulate=int(accumulate))


# ----------------------------------------------------------------- projection
def _lora_meta(weight: Q4Weight, loras):
    loras = list(loras) if loras is not None else []
    if not loras or all(l is None for l in loras):
        return None
    if len(loras) != len(weight.segments) or any(l is None for l in loras):
        raise ValueError("unsupported_capability: fused projections need a LoRA on every segment")
    ranks = {int(l.rank) for l in loras}
    scales = {float(l.scale) for l in loras}
    if len(ranks) != 1 or len(scales) != 1:
        raise ValueError("unsupported_capability: fused projections need one rank and scale")
    return ranks.pop(), scales.pop()


def _stack_rows(ts):
    """Detached ``cat(ts, 0)`` of contiguous 2-D tensors of one width: a view
    when they already lie back to back in one storage (the layout
    ``lora.share_fused_storage`` gives fused groups), else a copy."""
    t0 = ts[0].detach()
    if len(ts) == 1:
        return t0.contiguous()
    width = t0.shape[1]
    off = t0.storage_offset()
    ptr = t0.untyped_storage().data_ptr()
    for t in ts:
        if (not t.is_contiguous() or t.dim() != 2 or t.shape[1] != width or t.dtype != t0.dtype
                or t.untyped_storage().data_ptr() != ptr or t.storage_offset() != off):
            return torch.cat([x.detach() for x in ts], 0).contiguous()
        off += t.numel()
    rows = sum(t.shape[0] for t in ts)
    return t0.as_strided((rows, width), (width, 1), t0.storage_offset())


class _Q4LoRALinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, residual, rank, scale, swiglu_I, loras, *ab):
        gu = None
        if swiglu_I:  # x is a fused gate|up pre-activation: the input is silu(gate) * up
            gu = x
            x = torch.empty((gu.shape[0], swiglu_I), dtype=_BF16, device=gu.device)
            _lib.call("st_swiglu_fwd", _lib.ptr(gu), gu.stride(0), _lib.ptr(gu[:, swiglu_I:]),
                      gu.stride(0), gu.shape[0], swiglu_I, _lib.ptr(x), swiglu_I,
                      _lib.stream_handle(gu.device))
        M, K = x.shape
        N = weight.out_features
        dev = x.device
        stream = _lib.stream_handle(dev)
        nseg = len(weight.segments)
        y = torch.empty((M, N), dtype=_BF16, device=dev)
        T = None
        if ab:
            A = [ab[2 * i] for i in range(nseg)]
            B = [ab[2 * i + 1] for i in range(nseg)]
            A_cat, B_cat = _stack_rows(A), _stack_rows(B)
            T = torch.empty((M, nseg * rank), dtype=_F32, device=dev)
            # T = x_f32 A_cat^T   (lora.py:219 inner linear)
            lora_gemm(M, nseg * rank, K, x, K, 1, A_cat, 1, K, 1.0, T)
            ends = _lib.i64_array(torch.tensor(weight.segments).cumsum(0).tolist())
        # split-K partials for shapes whose tiles leave CUs idle (0 otherwise)
        ws = _ws.get(dev, _lib.query("st_q4_linear_fwd_workspace_bytes", M, N, K))
        _launch(("fwd", M, N, K), lambda: _lib.call(
            "st_q4_linear_fwd", _lib.ptr(x), M, K, K, _lib.ptr(weight.payload),
            _lib.ptr(weight.scales), N, weight.lut(), weight.flags,
            _lib.ptr(T), 0 if T is None else T.stride(0),
            _lib.ptr(B_cat) if ab else None, rank if ab else 0, float(scale),
            nseg if ab else 0, ends if ab else None,
            _lib.ptr(residual), 0 if residual is None else residual.stride(0),
            _lib.ptr(y), N, _lib.ptr(ws), 0 if ws is None else ws.numel(), stream))
        ctx.weight, ctx.rank, ctx.scale = weight, rank, scale
        ctx.loras = loras
        ctx.has_residual = residual is not None
        ctx.nlora = len(ab)
        ctx.swiglu_I = swiglu_I
        if ab:
            ctx.save_for_backward(x, T, A_cat, B_cat, gu)
        else:
            ctx.save_for_backward(x, gu)
        return y

    @staticmethod
    def backward(ctx, dy):
        weight, rank, scale = ctx.weight, ctx.rank, ctx.scale
        dy = dy.contiguous()
        M, N = dy.shape
        K = weight.in_features
        dev = dy.device
        stream = _lib.stream_handle(dev)
        grads_ab = []
        dT = None
        A_cat = None
        sink = _SINKS.get(dev.index) if ctx.nlora else None
        if ctx.nlora:
            x, T, A_cat, B_cat, gu = ctx.saved_tensors
            nseg = len(weight.segments)
            dT = torch.empty((M, nseg * rank), dtype=_F32, device=dev)
            starts = [0]
            for width in weight.segments:
                starts.append(starts[-1] + width)
            if sink is not None and not (
                    ctx.loras is not None and rank <= 64 and all(sink.wants(l) for l in ctx.loras)
                    and all(st % 8 == 0 for st in starts) and N % 8 == 0 and K % 8 == 0
                    and dy.data_ptr() % 16 == 0 and x.data_ptr() % 16 == 0):
                sink = None
        if ctx.nlora and sink is not None:
            # dT now (the dgrad epilogue reads it); dB_s and dA_s go to the sink
            ends = _lib.i64_array(starts[1:])
            need = _lib.query("st_lora_bwd_dy_workspace_bytes", M, N, rank, nseg, ends)
            if need > 0:
                ws = _ws.get(dev, need)
                _lib.call("st_lora_bwd_dy", _lib.ptr(dy), M, N, N, _lib.ptr(B_cat), _lib.ptr(T),
                          T.stride(0), rank, nseg, ends, float(scale), _lib.ptr(dT), dT.stride(0),
                          None, _lib.ptr(ws), ws.numel(), stream)
            else:
                for s_ in range(nseg):
                    off, width = starts[s_], weight.segments[s_]
                    lora_gemm(M, rank, width, dy[:, off:off + width], N, 1,
                              B_cat[off:off + width], rank, 1, scale,
                              dT[:, s_ * rank:(s_ + 1) * rank])
            acc = sink.accumulate
            for s_, lo in enumerate(ctx.loras):
                off, width = starts[s_], weight.segments[s_]
                Ts, dTs = T[:, s_ * rank:], dT[:, s_ * rank:]
                sink.add(lo, [
                    # dB_s[n, j] = s * sum_m dY[m, off + n] T[m, s*r + j]
                    _rk(dy[:, off:], N, Ts, T.stride(0), width, rank, M, scale, lo.grad_B,
                        rank, 1, acc),
                    # dA_s[j, k] = sum_m dT[m, s*r + j] x[m, k]
                    _rk(x, K, dTs, dT.stride(0), K, rank, M, 1.0, lo.grad_A, 1, K, acc),
                ], (dy, T, dT, x))
            grads_ab = [None, None] * nseg
        elif ctx.nlora:
            dB_all = torch.empty((N, rank), dtype=_F32, device=dev)
            # dT_s = s * dY_s B_s and dB_s = s * dY_s^T T_s for every segment:
            # one launch of partial products and one reduction
            ends = _lib.i64_array(torch.tensor(weight.segments).cumsum(0).tolist())
            need = _lib.query("st_lora_bwd_dy_workspace_bytes", M, N, rank, nseg, ends)
            if need > 0:
                ws = _ws.get(dev, need)
                _lib.call("st_lora_bwd_dy", _lib.ptr(dy), M, N, N, _lib.ptr(B_cat), _lib.ptr(T),
                          T.stride(0), rank, nseg, ends, float(scale), _lib.ptr(dT), dT.stride(0),
                          _lib.ptr(dB_all), _lib.ptr(ws), ws.numel(), stream)
            else:  # segment layouts the batched kernel does not take: one product at a time
                off = 0
                for s, width in enumerate(weight.segments):
                    dys = dy[:, off:off + width]
                    lora_gemm(M, rank, width, dys, N, 1, B_cat[off:off + width], rank, 1, scale,
                              dT[:, s * rank:(s + 1) * rank])
                    lora_gemm(width, rank, M, dys, 1, N, T[:, s * rank:(s + 1) * rank],
                              T.stride(0), 1, scale, dB_all[off:off + width])
                    off += width
            dBs = []
            off = 0
            for width in weight.segments:
                dBs.append(dB_all[off:off + width])
                off += width
            # dA_cat = dT_cat^T x for every segment in one product
            R = nseg * rank
            dA_cat = torch.empty((R, K), dtype=_F32, device=dev)
            lora_gemm(R, K, M, dT, 1, R, x, K, 1, 1.0, dA_cat)
            for s in range(nseg):
                grads_ab += [dA_cat[s * rank:(s + 1) * rank], dBs[s]]
        else:
            x, gu = ctx.saved_tensors
        lora_args = (_lib.ptr(dT), 0 if dT is None else dT.stride(0), _lib.ptr(A_cat),
                     0 if dT is None else dT.shape[1])
        if ctx.swiglu_I:
            # the dgrad epilogue applies the SwiGLU VJP: the gradient of gate|up
            dx = torch.empty_like(gu)
            _launch(("dgrad", M, N, K), lambda: _lib.call(
                "st_q4_linear_dgrad_swiglu", _lib.ptr(dy), M, N, N, _lib.ptr(weight.payload),
                _lib.ptr(weight.scales), K, weight.lut(), weight.flags, *lora_args,
                _lib.ptr(gu), gu.stride(0), _lib.ptr(dx), dx.stride(0), None, 0, stream))
        else:
            dx = torch.empty((M, K), dtype=_BF16, device=dev)
            ws = _ws.get(dev, _lib.query("st_q4_linear_dgrad_workspace_bytes", M, N, K))
            _launch(("dgrad", M, N, K), lambda: _lib.call(
                "st_q4_linear_dgrad", _lib.ptr(dy), M, N, N, _lib.ptr(weight.payload),
                _lib.ptr(weight.scales), K, weight.lut(), weight.flags, *lora_args,
                _lib.ptr(dx), K, _lib.ptr(ws), 0 if ws is None else ws.numel(), stream))
        dres = dy if ctx.has_residual else None
        return (dx, None, dres, None, None, None, None, *grads_ab)


def q4_lora_linear(x: torch.Tensor, weight: Q4Weight, loras=None, residual=None,
                   swiglu: bool = False) -> torch.Tensor:
    """``bf16(bf16(x W^T) + s (x_f32 A^T) B^T)`` [``+ residual``] for a 2-D bf16 ``x``.

    ``loras`` holds one LoRA object (``A``, ``B``, ``rank``, ``scale``) per
    segment of ``weight`` or is None.  ``swiglu``: ``x`` is a fused gate|up
    pre-activation ``[M, 2I]`` and the projection reads ``silu(gate) * up``
    (dense.py:153); the backward applies the SwiGLU VJP inside the input-
    gradient GEMM and returns the gradient of gate|up."""
    if x.dtype != _BF16 or x.dim() != 2:
        raise ValueError("q4_lora_linear expects a 2-D bf16 input")
    width = x.shape[1] // 2 if swiglu else x.shape[1]
    if width != weight.in_features or (swiglu and x.shape[1] != 2 * width):
        raise ValueError(f"input width {x.shape[1]} does not match weight in_features "
                         f"{weight.in_features}{' (gate|up)' if swiglu else ''}")
    x = x.contiguous()
    swiglu_I = width if swiglu else 0
    meta = _lora_meta(weight, loras)
    if residual is not None:
        residual = residual.contiguous()
        if residual.shape != (x.shape[0], weight.out_features) or residual.dtype != _BF16:
            raise ValueError("residual must be a bf16 [M, out_features] tensor")
    if meta is None:
        return _Q4LoRALinear.apply(x, weight, residual, 0, 1.0, swiglu_I, None)
    rank, scale = meta
    ab = [t for l in loras for t in (l.A, l.B)]
    for l in loras:
        if l.A.dtype != _F32 or l.B.dtype != _F32:
            raise ValueError("LoRA A/B must be fp32")
    return _Q4LoRALinear.apply(x, weight, residual, rank, scale, swiglu_I, tuple(loras), *ab)


# ----------------------------------------------------------------- RMSNorm
class _RMSNorm(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, eps):
        rows, H = x.shape
        y = torch.empty_like(x)
        rstd = torch.empty(rows, dtype=_F32, device=x.device)
        _lib.call("st_rmsnorm_fwd", _lib.ptr(x), _lib.ptr(w), rows, H, float(eps), _lib.ptr(y),
                  _lib.ptr(rstd), _lib.stream_handle(x.device))
        ctx.save_for_backward(x, w, rstd)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, rstd = ctx.saved_tensors
        dy = dy.contiguous()
        rows, H = x.shape
        dx = torch.empty_like(x)
        _lib.call("st_rmsnorm_bwd", _lib.ptr(dy), _lib.ptr(x), _lib.ptr(w), _lib.ptr(rstd), None,
                  rows, H, _lib.ptr(dx), _lib.stream_handle(x.device))
        return dx, None, None


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    if x.dtype != _BF16 or weight.dtype != _BF16:
        raise ValueError("rms_norm expects bf16 input and weight")
    return _RMSNorm.apply(x.contiguous(), weight.detach().contiguous(), eps)


class _RMSNormResidual(torch.autograd.Function):
    """``(x, rms_norm(x))`` for a hidden state that also feeds a residual add
    (dense.py:120-153: ``residual = hidden`` next to ``rms(hidden)``).  The
    first output is ``x`` itself; the backward returns ``d_residual + VJP``
    from one st_rmsnorm_bwd call (its ``dres``), the sum autograd would
    otherwise form with a separate bf16 add."""

    @staticmethod
    def forward(ctx, x, w, eps):
        ctx.set_materialize_grads(False)
        rows, H = x.shape
        y = torch.empty_like(x)
        rstd = torch.empty(rows, dtype=_F32, device=x.device)
        _lib.call("st_rmsnorm_fwd", _lib.ptr(x), _lib.ptr(w), rows, H, float(eps), _lib.ptr(y),
                  _lib.ptr(rstd), _lib.stream_handle(x.device))
        ctx.save_for_backward(x, w, rstd)
        return x, y

    @staticmethod
    def backward(ctx, dres, dy):
        x, w, rstd = ctx.saved_tensors
        if dy is None:
            return dres, None, None
        dy = dy.contiguous()
        dres = None if dres is None else dres.contiguous()
        rows, H = x.shape
        dx = torch.empty_like(x)
        _lib.call("st_rmsnorm_bwd", _lib.ptr(dy), _lib.ptr(x), _lib.ptr(w), _lib.ptr(rstd),
                  _lib.ptr(dres), rows, H, _lib.ptr(dx), _lib.stream_handle(x.device))
        return dx, None, None


def rms_norm_residual(x: torch.Tensor, weight: torch.Tensor, eps: float):
    """``(x, rms_norm(x))`` with the residual gradient folded into the norm's VJP."""
    if x.dtype != _BF16 or weight.dtype != _BF16:
        raise ValueError("rms_norm expects bf16 input and weight")
    return _RMSNormResidual.apply(x.contiguous(), weight.detach().contiguous(), eps)


# ----------------------------------------------------------------- terminal
def linear_bf16(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``y = bf16(x w^T)`` on the MFMA GEMM (fp32 accumulation)."""
    M, K = x.shape
    N = w.shape[0]
    y = torch.empty((M, N), dtype=_BF16, device=x.device)
    _lib.call("st_linear_bf16_fwd", _lib.ptr(x), M, K, x.stride(0), _lib.ptr(w), N, w.stride(0),
              _lib.ptr(y), N, _lib.stream_handle(x.device))
    return y


def linear_bf16_dgrad(dy: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """``dx = bf16(dy w)`` on the MFMA GEMM (fp32 accumulation)."""
    M, N = dy.shape
    K = w.shape[1]
    dx = torch.empty((M, K), dtype=_BF16, device=dy.device)
    _lib.call("st_linear_bf16_dgrad", _lib.ptr(dy), M, N, dy.stride(0), _lib.ptr(w), K,
              w.stride(0), _lib.ptr(dx), K, _lib.stream_handle(dy.device))
    return dx


def supervised_chunk_intervals(labels: torch.Tensor, token_chunk: int) -> tuple:
    """Token chunks [start, end) of the shifted targets that hold at least one
    supervised label (native_terminal.py:44-46), from host labels (prepared
    once per batch, before the step)."""
    if type(token_chunk) is not int or token_chunk < 1:
        raise ValueError("invalid terminal token chunk")
    if labels.device.type != "cpu":
        raise RuntimeError("supervised chunks are prepared from host labels")
    S = labels.shape[1]
    return tuple((start, min(start + token_chunk, S - 1)) for start in range(0, S - 1, token_chunk)
                 if bool((labels[:, start + 1:min(start + token_chunk, S - 1) + 1] != -100).any()))


class _ChunkedCE(torch.autograd.Function):
    """Shifted, token-chunked causal-LM loss over the frozen head
    (quantization/native_terminal.py:11-37): per chunk one bf16 head GEMM,
    one in-place cross-entropy/gradient pass over the bf16 logits
    (``st_cross_entropy_rows``) and one bf16 GEMM back to the hidden size.
    The forward returns sum(CE)/normalization and keeps the full VJP; the
    backward scales it."""

    @staticmethod
    def forward(ctx, normalized, head, labels, normalization, token_chunk, chunks):
        if type(token_chunk) is not int or token_chunk < 1 or not math.isfinite(normalization) \
                or normalization <= 0:
            raise ValueError("invalid terminal token chunk/normalization")
        if labels.shape != normalized.shape[:2] or head.requires_grad:
            raise ValueError("invalid terminal labels/trainable frozen head")
        if normalized.dtype != _BF16 or head.dtype != _BF16:
            raise ValueError("terminal expects bf16 hidden states and head")
        B, S, H = normalized.shape
        V = head.shape[0]
        dev = normalized.device
        if labels.device.type == "cpu":
            # host labels are checked here, before the copy; device labels are
            # never scanned (a scan is a device->host sync inside the step,
            # native_terminal.py:1-5): st_cross_entropy_rows turns a label
            # outside [0, vocab) into a NaN row loss without reading the row
            bad = ((labels < 0) & (labels != -100)) | (labels >= V)
            if bool(bad.any()):
                raise ValueError("terminal labels must be -100 or in [0, vocab)")
        labels = labels.to(dev, torch.int64)
        head = head.detach().contiguous()
        vjp = torch.zeros_like(normalized)
        total = torch.zeros((), dtype=_F32, device=dev)
        scale = float(torch.tensor(1.0, dtype=_F32) / normalization)
        stream = _lib.stream_handle(dev)
        # rows per pass: the logits block stays below the GEMM's 2 GiB operand limit
        max_rows = max(1, ((1 << 31) - 1) // (2 * V))
        for start, end in chunks:
            h = normalized[:, start:end].detach().contiguous().view(-1, H)
            target = labels[:, start + 1:end + 1].contiguous().view(-1)
            dh = torch.empty_like(h)
            for r0 in range(0, h.shape[0], max_rows):
                r1 = min(r0 + max_rows, h.shape[0])
                logits = linear_bf16(h[r0:r1], head)
                loss_rows = torch.empty(r1 - r0, dtype=_F32, device=dev)
                _lib.call("st_cross_entropy_rows", _lib.ptr(logits), r1 - r0, V, V,
                          _lib.ptr(target[r0:r1]), -100, scale, _lib.ptr(loss_rows), stream)
                dh[r0:r1].copy_(linear_bf16_dgrad(logits, head))
                total += loss_rows.sum()
                del logits, loss_rows
            vjp[:, start:end].copy_(dh.view(B, end - start, H))
        ctx.save_for_backward(vjp)
        return total / normalization

    @staticmethod
    def backward(ctx, grad):
        (vjp,) = ctx.saved_tensors
        return vjp * grad, None, None, None, None, None


def chunked_causal_loss(normalized, head, labels, *, normalization, token_chunk,
                        supervised_chunks=None):
    """``sum CE(shifted) / normalization`` with the chunked terminal above
    (native_terminal.py:39-47); chunk intervals default to those of the host
    labels.  Device labels need prepared ``supervised_chunks``: they are never
    scanned on the host (native_terminal.py:41-42)."""
    if supervised_chunks is None:
        if labels.device.type != "cpu":
            raise RuntimeError("device terminal requires startup-prepared supervised chunks")
        supervised_chunks = supervised_chunk_intervals(labels, token_chunk)
    return _ChunkedCE.apply(normalized, head, labels, normalization, token_chunk,
                            tuple(supervised_chunks))


# ----------------------------------------------------------------- RoPE
class _RopeHeads(torch.autograd.Function):
    """Token-major projection output columns -> [B, heads, S, D] (rotated)."""

    @staticmethod
    def forward(ctx, y, col0, B, S, heads, D, cos, sin, rotate):
        ld = y.stride(0)
        out = torch.empty((B, heads, S, D), dtype=_BF16, device=y.device)
        base = y[:, col0:]
        _lib.call("st_rope_fwd", _lib.ptr(base), ld, _lib.ptr(cos), _lib.ptr(sin), B, S, heads,
                  D, int(rotate), _lib.ptr(out), _lib.stream_handle(y.device))
        ctx.meta = (y.shape, col0, B, S, heads, D, rotate, ld)
        ctx.save_for_backward(cos, sin)
        return out

    @staticmethod
    def backward(ctx, dout):
        shape, col0, B, S, heads, D, rotate, ld = ctx.meta
        cos, sin = ctx.saved_tensors
        dout = dout.contiguous()
        dy = torch.zeros(shape, dtype=_BF16, device=dout.device) if col0 or shape[1] != heads * D \
            else torch.empty(shape, dtype=_BF16, device=dout.device)
        _lib.call("st_rope_bwd", _lib.ptr(dout), _lib.ptr(cos), _lib.ptr(sin), B, S, heads, D,
                  int(rotate), _lib.ptr(dy[:, col0:]), ld, _lib.stream_handle(dout.device))
        return dy, None, None, None, None, None, None, None, None


class _RopeQKV(torch.autograd.Function):
    """Fused q|k|v projection output -> rotated q, k and plain v in head layout;
    the VJP writes straight into one fused gradient buffer."""

    @staticmethod
    def forward(ctx, y, B, S, heads, kv_heads, D, cos, sin):
        ld = y.stride(0)
        dev = y.device
        st = _lib.stream_handle(dev)
        q = torch.empty((B, heads, S, D), dtype=_BF16, device=dev)
        k = torch.empty((B, kv_heads, S, D), dtype=_BF16, device=dev)
        v = torch.empty((B, kv_heads, S, D), dtype=_BF16, device=dev)
        offs = (0, heads * D, (heads + kv_heads) * D)
        _lib.call("st_rope_qkv_fwd", _lib.ptr(y), ld, _lib.ptr(cos), _lib.ptr(sin), B, S, heads,
                  kv_heads, D, _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), st)
        ctx.meta = (y.shape, B, S, heads, kv_heads, D, offs)
        ctx.save_for_backward(cos, sin)
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        shape, B, S, heads, kv_heads, D, offs = ctx.meta
        cos, sin = ctx.saved_tensors
        dev = cos.device
        st = _lib.stream_handle(dev)
        dy = torch.empty(shape, dtype=_BF16, device=dev)
        gs = [torch.zeros((B, h, S, D), dtype=_BF16, device=dev) if g is None else g.contiguous()
              for g, h in ((dq, heads), (dk, kv_heads), (dv, kv_heads))]
        _lib.call("st_rope_qkv_bwd", *(_lib.ptr(g) for g in gs), _lib.ptr(cos), _lib.ptr(sin), B,
                  S, heads, kv_heads, D, _lib.ptr(dy), shape[1], st)
        return dy, None, None, None, None, None, None, None


def rope_qkv(y, B, S, heads, kv_heads, D, cos, sin):
    return _RopeQKV.apply(y, B, S, heads, kv_heads, D, cos.contiguous(), sin.contiguous())


class _RopeQKVNorm(torch.autograd.Function):
    """Qwen3 qk_norm + rotation of a fused q|k|v projection output in one
    launch each way (dense.py:128-141): per-head RMSNorm of q and k, then the
    rotation, v copied to head layout."""

    @staticmethod
    def forward(ctx, y, B, S, heads, kv_heads, D, cos, sin, wq, wk, eps):
        ld = y.stride(0)
        dev = y.device
        st = _lib.stream_handle(dev)
        q = torch.empty((B, heads, S, D), dtype=_BF16, device=dev)
        k = torch.empty((B, kv_heads, S, D), dtype=_BF16, device=dev)
        v = torch.empty((B, kv_heads, S, D), dtype=_BF16, device=dev)
        rstd = torch.empty((B * S, heads + kv_heads), dtype=_F32, device=dev)
        _lib.call("st_rope_qkv_norm_fwd", _lib.ptr(y), ld, _lib.ptr(cos), _lib.ptr(sin), B, S,
                  heads, kv_heads, D, _lib.ptr(wq), _lib.ptr(wk), float(eps), _lib.ptr(q),
                  _lib.ptr(k), _lib.ptr(v), _lib.ptr(rstd), st)
        ctx.meta = (y.shape, ld, B, S, heads, kv_heads, D)
        ctx.save_for_backward(y, cos, sin, wq, wk, rstd)
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        shape, ld, B, S, heads, kv_heads, D = ctx.meta
        y, cos, sin, wq, wk, rstd = ctx.saved_tensors
        dev = cos.device
        st = _lib.stream_handle(dev)
        dy = torch.empty(shape, dtype=_BF16, device=dev)
        gs = [torch.zeros((B, h, S, D), dtype=_BF16, device=dev) if g is None else g.contiguous()
              for g, h in ((dq, heads), (dk, kv_heads), (dv, kv_heads))]
        _lib.call("st_rope_qkv_norm_bwd", *(_lib.ptr(g) for g in gs), _lib.ptr(y), ld,
                  _lib.ptr(cos), _lib.ptr(sin), _lib.ptr(wq), _lib.ptr(wk), _lib.ptr(rstd), B, S,
                  heads, kv_heads, D, _lib.ptr(dy), shape[1], st)
        return dy, None, None, None, None, None, None, None, None, None, None


def rope_qkv_norm(y, B, S, heads, kv_heads, D, cos, sin, wq, wk, eps):
    """q, k, v head-major from a fused q|k|v output with Qwen3's per-head
    q/k RMSNorm applied before the rotation (one kernel each way)."""
    if y.dtype != _BF16 or wq.dtype != _BF16 or wk.dtype != _BF16:
        raise ValueError("rope_qkv_norm expects bf16 inputs and norm weights")
    return _RopeQKVNorm.apply(y, B, S, heads, kv_heads, D, cos.contiguous(), sin.contiguous(),
                              wq.detach().contiguous(), wk.detach().contiguous(), eps)


def rope_heads(y, col0, B, S, heads, D, cos, sin, rotate=True):
    return _RopeHeads.apply(y, col0, B, S, heads, D, cos.contiguous(), sin.contiguous(), rotate)


# ----------------------------------------------------------------- attention
def _kv_len_arg(kv_len, B, dev):
    """Device int32 [B] of valid key counts (right padding) or None."""
    if kv_len is None:
        return None
    if kv_len.dtype != torch.int32 or kv_len.device != dev or tuple(kv_len.shape) != (B,):
        raise ValueError("unsupported_capability: kv_len must be an int32 [batch] tensor on the "
                         "attention's device")
    return kv_len.contiguous()


class _CausalAttention(torch.autograd.Function):
    """GQA causal attention of dense.py:142-148 as flash attention: no
    [S, S] scores in memory; the backward recomputes probabilities from the
    saved base-2 log-sum-exp.  ``kv_len`` masks the keys past each row's
    valid prefix (right padding, dense.py:237-246)."""

    @staticmethod
    def forward(ctx, q, k, v, scale, kv_len):
        B, H, S, D = q.shape
        Hkv = k.shape[1]
        dev = q.device
        out = torch.empty((B, S, H * D), dtype=_BF16, device=dev)
        lse = torch.empty((B, H, S), dtype=_F32, device=dev)
        ws = _ws.get(dev, _lib.query("st_flash_attn_workspace_bytes", B, S, H, Hkv, D, 0))
        _lib.call("st_flash_attn_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), B, S, H, Hkv, D,
                  float(scale), _lib.ptr(kv_len), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws),
                  0 if ws is None else ws.numel(), _lib.stream_handle(dev))
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.scale, ctx.kv_len = scale, kv_len
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        B, H, S, D = q.shape
        Hkv = k.shape[1]
        dev = q.device
        dout = dout.contiguous()
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        ws = _ws.get(dev, _lib.query("st_flash_attn_workspace_bytes", B, S, H, Hkv, D, 1))
        _lib.call("st_flash_attn_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out),
                  _lib.ptr(lse), _lib.ptr(dout), B, S, H, Hkv, D, float(ctx.scale),
                  _lib.ptr(ctx.kv_len), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws),
                  0 if ws is None else ws.numel(), _lib.stream_handle(dev))
        return dq, dk, dv, None, None


def causal_attention(q, k, v, scale, kv_len=None):
    """q [B,H,S,D], k/v [B,Hkv,S,D] -> token-major [B,S,H*D]; ``kv_len``
    (int32 [B] on the device, or None) gives each row's valid key count."""
    return _CausalAttention.apply(q.contiguous(), k.contiguous(), v.contiguous(), float(scale),
                                  _kv_len_arg(kv_len, q.shape[0], q.device))


# ----------------------------------------------------------------- MLA (DeepSeek-V3)
class _MLARope(torch.autograd.Function):
    """q [M, H*(nope+rope)], kv [M, H*(nope+v)] and the shared rope key
    ``comp[:, kv_rank:kv_rank+rope]`` -> Q, K [B,H,S,nope+rope], V [B,H,S,v]
    (deepseek.py:137-150).  The VJP returns dq, dkv and a gradient of ``comp``
    holding only the rope key's columns (the latent columns get theirs through
    the kv path)."""

    @staticmethod
    def forward(ctx, q, kv, comp, cos, sin, B, S, heads, nope, rope, v_dim, kv_rank, interleave):
        dev = q.device
        st = _lib.stream_handle(dev)
        Q = torch.empty((B, heads, S, nope + rope), dtype=_BF16, device=dev)
        K = torch.empty_like(Q)
        V = torch.empty((B, heads, S, v_dim), dtype=_BF16, device=dev)
        kr = comp[:, kv_rank:]
        _lib.call("st_mla_rope_fwd", _lib.ptr(q), q.stride(0), _lib.ptr(kv), kv.stride(0),
                  _lib.ptr(kr), comp.stride(0), _lib.ptr(cos), _lib.ptr(sin), B, S, heads, nope,
                  rope, v_dim, int(interleave), _lib.ptr(Q), _lib.ptr(K), _lib.ptr(V), st)
        ctx.meta = (q.shape, kv.shape, comp.shape, B, S, heads, nope, rope, v_dim, kv_rank,
                    interleave)
        ctx.save_for_backward(cos, sin)
        return Q, K, V

    @staticmethod
    def backward(ctx, dQ, dK, dV):
        qs, kvs, cs, B, S, heads, nope, rope, v_dim, kv_rank, interleave = ctx.meta
        cos, sin = ctx.saved_tensors
        dev = cos.device
        z = lambda shape: torch.zeros(shape, dtype=_BF16, device=dev)  # noqa: E731
        dQ = z((B, heads, S, nope + rope)) if dQ is None else dQ.contiguous()
        dK = z((B, heads, S, nope + rope)) if dK is None else dK.contiguous()
        dV = z((B, heads, S, v_dim)) if dV is None else dV.contiguous()
        dq = torch.empty(qs, dtype=_BF16, device=dev)
        dkv = torch.empty(kvs, dtype=_BF16, device=dev)
        dcomp = torch.zeros(cs, dtype=_BF16, device=dev)
        _lib.call("st_mla_rope_bwd", _lib.ptr(dQ), _lib.ptr(dK), _lib.ptr(dV), _lib.ptr(cos),
                  _lib.ptr(sin), B, S, heads, nope, rope, v_dim, int(interleave), _lib.ptr(dq),
                  dq.stride(0), _lib.ptr(dkv), dkv.stride(0), _lib.ptr(dcomp[:, kv_rank:]),
                  dcomp.stride(0), _lib.stream_handle(dev))
        return (dq, dkv, dcomp) + (None,) * 10


def mla_rope(q, kv, comp, cos, sin, *, batch, seq, heads, nope, rope, v_dim, kv_rank,
             interleave):
    """Q, K, V of DeepSeek's multi-head latent attention (deepseek.py:137-150)
    from the q_b (or q_proj) output ``q``, the kv_b output ``kv`` and the
    kv_a_proj_with_mqa output ``comp`` (its columns ``kv_rank:kv_rank+rope`` are
    the shared rope key; ``comp`` may be a column slice of a wider output)."""
    if comp.stride(1) != 1 or q.stride(1) != 1 or kv.stride(1) != 1:
        raise ValueError("mla_rope expects row-major operands")
    return _MLARope.apply(q.contiguous(), kv.contiguous(), comp, cos.contiguous(),
                          sin.contiguous(), batch, seq, heads, nope, rope, v_dim, kv_rank,
                          bool(interleave))


class _MLAAttention(torch.autograd.Function):
    """Causal attention with query/key heads of DQ and value heads of DV
    (deepseek.py:151-153) on the flash kernels; ``kv_len`` as in
    :func:`causal_attention`."""

    @staticmethod
    def forward(ctx, q, k, v, scale, kv_len):
        B, H, S, DQ = q.shape
        DV = v.shape[-1]
        dev = q.device
        out = torch.empty((B, S, H * DV), dtype=_BF16, device=dev)
        lse = torch.empty((B, H, S), dtype=_F32, device=dev)
        ws = _ws.get(dev, _lib.query("st_mla_attn_workspace_bytes", B, S, H, DQ, DV, 0))
        _lib.call("st_mla_attn_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), B, S, H, DQ, DV,
                  float(scale), _lib.ptr(kv_len), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws),
                  0 if ws is None else ws.numel(), _lib.stream_handle(dev))
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.scale, ctx.kv_len = scale, kv_len
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, lse = ctx.saved_tensors
        B, H, S, DQ = q.shape
        DV = v.shape[-1]
        dev = q.device
        dout = dout.contiguous()
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        ws = _ws.get(dev, _lib.query("st_mla_attn_workspace_bytes", B, S, H, DQ, DV, 1))
        _lib.call("st_mla_attn_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out),
                  _lib.ptr(lse), _lib.ptr(dout), B, S, H, DQ, DV, float(ctx.scale),
                  _lib.ptr(ctx.kv_len), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws),
                  0 if ws is None else ws.numel(), _lib.stream_handle(dev))
        return dq, dk, dv, None, None


def mla_attention(q, k, v, scale, kv_len=None):
    """q, k [B,H,S,DQ], v [B,H,S,DV] -> token-major [B,S,H*DV]."""
    return _MLAAttention.apply(q.contiguous(), k.contiguous(), v.contiguous(), float(scale),
                               _kv_len_arg(kv_len, q.shape[0], q.device))


# ----------------------------------------------------------------- SwiGLU
class _SwiGLU(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gu, I, gate_col, up_col):
        rows = gu.shape[0]
        ld = gu.stride(0)
        a = torch.empty((rows, I), dtype=_BF16, device=gu.device)
        _lib.call("st_swiglu_fwd", _lib.ptr(gu[:, gate_col:]), ld, _lib.ptr(gu[:, up_col:]), ld,
                  rows, I, _lib.ptr(a), I, _lib.stream_handle(gu.device))
        ctx.save_for_backward(gu)
        ctx.meta = (I, gate_col, up_col)
        return a

    @staticmethod
    def backward(ctx, da):
        (gu,) = ctx.saved_tensors
        I, gate_col, up_col = ctx.meta
        da = da.contiguous()
        rows, ld = gu.shape[0], gu.stride(0)
        dgu = torch.empty_like(gu) if gu.shape[1] == 2 * I else torch.zeros_like(gu)
        _lib.call("st_swiglu_bwd", _lib.ptr(da), I, _lib.ptr(gu[:, gate_col:]), ld,
                  _lib.ptr(gu[:, up_col:]), ld, rows, I, _lib.ptr(dgu[:, gate_col:]), ld,
                  _lib.ptr(dgu[:, up_col:]), ld, _lib.stream_handle(gu.device))
        return dgu, None, None, None


class _SwiGLUPair(torch.autograd.Function):
    """silu(g) * u on two separate tensors (unfused gate/up projections)."""

    @staticmethod
    def forward(ctx, g, u):
        rows, I = g.shape
        a = torch.empty_like(g)
        _lib.call("st_swiglu_fwd", _lib.ptr(g), I, _lib.ptr(u), I, rows, I, _lib.ptr(a), I,
                  _lib.stream_handle(g.device))
        ctx.save_for_backward(g, u)
        return a

    @staticmethod
    def backward(ctx, da):
        g, u = ctx.saved_tensors
        da = da.contiguous()
        rows, I = g.shape
        dg, du = torch.empty_like(g), torch.empty_like(u)
        _lib.call("st_swiglu_bwd", _lib.ptr(da), I, _lib.ptr(g), I, _lib.ptr(u), I, rows, I,
                  _lib.ptr(dg), I, _lib.ptr(du), I, _lib.stream_handle(g.device))
        return dg, du


def swiglu(gu: torch.Tensor, I: int) -> torch.Tensor:
    """``silu(gu[:, :I]) * gu[:, I:2I]`` for a fused gate|up output."""
    return _SwiGLU.apply(gu, I, 0, I)


def swiglu_pair(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    return _SwiGLUPair.apply(g.contiguous(), u.contiguous())


def attention_scale(head_dim: int) -> float:
    return float(head_dim) ** -0.5


__all__ = ["Q4Weight", "concat_rows", "lora_fusable", "q4_lora_linear", "rms_norm", "rope_qkv", "rope_heads",
           "causal_attention", "swiglu", "swiglu_pair", "lora_gemm", "attention_scale",
           "mla_rope", "mla_attention",
           "rms_norm_residual",
           "linear_bf16", "linear_bf16_dgrad", "supervised_chunk_intervals",
           "chunked_causal_loss"]
