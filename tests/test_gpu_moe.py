"""MoE HIP path vs the CPU oracle (oracle/moe.py), through the C ABI.

Routers: the picks must be the oracle's lowest-index top-k exactly (ties in
bf16 logits included) and the weights within a bf16 ulp.  Permutation and
combine are integer/byte work: exact.  Grouped GEMMs: the oracle's bf16
result up to fp32 summation order.  The whole feed-forward (forward and
backward, with per-expert LoRA): outputs rel err <= 2e-2, gradients cosine
>= 0.999, against the oracle's expert loop run on the GPU's picks."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe as OM
from spilltune_amd import _lib, moe

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _st(dev):
    return _lib.stream_handle(dev)


class _Held:
    """Device copies kept alive until the test ends (a raw pointer does not
    keep its tensor alive, and kernels run after the call returns)."""

    def __init__(self, dev):
        self.dev, self.items = dev, []

    def __call__(self, t):
        self.items.append(t.to(self.dev))
        return _lib.ptr(self.items[-1])


def _experts(oc, w: torch.Tensor, dev, fmt="nf4-g128"):
    """Encode [E, N, K] with the oracle; return (Q4Experts, exact bf16 W)."""
    E, N, K = w.shape
    w32 = w.reshape(E * N, K).numpy().astype(np.float32)
    enc = oc.encode_nf4 if fmt == "nf4-g128" else oc.encode_int4
    payload, scales = enc(w32)
    lut = oc.NF4_LUT if fmt == "nf4-g128" else oc.INT4_LUT
    bits = np.asarray(oc.decode4(payload, scales, w32.size, lut=lut), dtype=np.uint16)
    W = torch.from_numpy(bits.astype(np.int16)).view(BF).view(E, N, K)
    q = moe.Q4Experts(torch.from_numpy(payload).to(dev), torch.from_numpy(scales).to(dev), E, N,
                      K, fmt)
    return q, W


def _cos(a, b):
    a, b = a.detach().double().flatten().cpu(), b.detach().double().flatten().cpu()
    return float(a @ b / (a.norm() * b.norm()).clamp_min(1e-300))


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


# ----------------------------------------------------------------- routers
@pytest.mark.parametrize("T,E,k,norm", [(300, 128, 8, True), (77, 64, 2, False), (5, 512, 32, True),
                                        (64, 16, 16, False)])
def test_route_softmax_picks_and_weights(dev, T, E, k, norm):
    g = torch.Generator().manual_seed(T + E + k)
    H_ = _Held(dev)
    logits = torch.randn(T, E, generator=g).to(BF)        # bf16: many exact ties
    w = torch.empty(T, k, device=dev)
    idx = torch.empty(T, k, dtype=torch.int32, device=dev)
    _lib.call("st_moe_route_softmax", H_(logits), T, E, k, int(norm), 1,
              _lib.ptr(w), _lib.ptr(idx), _st(dev))
    torch.cuda.synchronize()
    probs = F.softmax(logits.float(), dim=-1)
    _, ref_idx = OM.topk_lowest_index(probs, k)
    assert torch.equal(idx.cpu().long(), ref_idx)
    ref = probs.gather(1, ref_idx)
    if norm:
        ref = ref / ref.sum(-1, keepdim=True)
    ref = ref.to(BF).float()
    assert ((w.cpu() - ref).abs() <= ref.abs() * 2 ** -7 + 1e-30).all()


def test_route_softmax_bwd_matches_autograd(dev):
    g = torch.Generator().manual_seed(2)
    H_ = _Held(dev)
    T, H, E, k = 96, 64, 32, 4
    flat = torch.randn(T, H, generator=g).to(BF)
    router = torch.randn(E, H, generator=g).to(BF)
    logits = F.linear(flat, router)
    for norm in (True, False):
        _, idx = OM.topk_lowest_index(F.softmax(logits.float(), -1), k)
        lg = logits.clone().requires_grad_(True)
        probs = F.softmax(lg, dtype=torch.float32, dim=-1)
        r = probs.gather(1, idx)
        if norm:
            r = r / r.sum(-1, keepdim=True)
        r = r.to(BF)
        dw = torch.randn(T, k, generator=g).to(BF)
        (ref,) = torch.autograd.grad(r, lg, dw)
        out = torch.empty(T, E, dtype=BF, device=dev)
        _lib.call("st_moe_route_softmax_bwd", H_(logits),
                  H_(idx.int()), H_(dw.float()), T, E, k, int(norm),
                  _lib.ptr(out), _st(dev))
        torch.cuda.synchronize()
        assert _rel(out, ref) < 1e-2 and _cos(out, ref) > 0.9999


@pytest.mark.parametrize("E,groups,group_k,k", [(256, 8, 4, 8), (64, 8, 3, 6), (32, 4, 2, 5)])
def test_route_sigmoid_vs_oracle(dev, E, groups, group_k, k):
    g = torch.Generator().manual_seed(E + k)
    H_ = _Held(dev)
    T, H = 200, 96
    flat = torch.randn(T, H, generator=g).to(BF)
    wr = torch.randn(E, H, generator=g).to(BF)
    bias = torch.randn(E, generator=g) * 0.05
    logits, wref, iref = OM.deepseek_route(flat, wr, bias, groups=groups, group_k=group_k,
                                           top_k=k, normalize=True, scale=2.5)
    w = torch.empty(T, k, device=dev)
    idx = torch.empty(T, k, dtype=torch.int32, device=dev)
    _lib.call("st_moe_route_sigmoid", H_(logits), H_(bias), T, E,
              groups, group_k, k, 1, 2.5, _lib.ptr(w), _lib.ptr(idx), _st(dev))
    torch.cuda.synchronize()
    got = {(t, int(e)): float(v) for t in range(T) for e, v in zip(idx[t].cpu(), w[t].cpu())}
    ref = {(t, int(e)): float(v) for t in range(T) for e, v in zip(iref[t], wref[t])}
    assert got.keys() == ref.keys()
    for key in ref:
        assert got[key] == pytest.approx(ref[key], rel=2e-6, abs=1e-7)
    # VJP w.r.t. the fp32 logits for the same picks
    lg = logits.clone().requires_grad_(True)
    wg = OM.deepseek_weights_given(lg, idx.cpu().long(), normalize=True, scale=2.5)
    dw = torch.randn(T, k, generator=g)
    (dref,) = torch.autograd.grad(wg, lg, dw)
    dl = torch.empty(T, E, device=dev)
    _lib.call("st_moe_route_sigmoid_bwd", H_(logits), _lib.ptr(idx), H_(dw),
              T, E, k, 1, 2.5, _lib.ptr(dl), _st(dev))
    torch.cuda.synchronize()
    torch.testing.assert_close(dl.cpu(), dref, rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------------- permutation / combine
@pytest.mark.parametrize("T,E,k,invalid", [(4096, 128, 8, False), (33, 7, 3, False), (1, 4, 4, False),
                                           (500, 256, 1, False), (2048, 256, 8, False),
                                           (300, 16, 2, True)])
def test_permute_exact(dev, T, E, k, invalid):
    """Rows grouped by expert in ascending pick order (skewed loads, fewer
    picks than threads, more picks than a thread run); picks of an expert id
    outside [0, E) get row -1 and count nowhere."""
    g = torch.Generator().manual_seed(T * k + E)
    H_ = _Held(dev)
    hot = max(k, 5)     # skewed load: a third of the tokens pick among the first experts only
    idx = torch.stack([torch.randperm(hot if t < T // 3 else E, generator=g)[:k]
                       for t in range(T)]).int()
    if invalid:
        bad = torch.randperm(T * k, generator=g)[:T // 4]
        idx.view(-1)[bad[: len(bad) // 2]] = -1
        idx.view(-1)[bad[len(bad) // 2:]] = E
        valid = (idx.flatten() >= 0) & (idx.flatten() < E)
        offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
        row_token = torch.full((T * k,), -7, dtype=torch.int32, device=dev)
        pick_row = torch.empty(T * k, dtype=torch.int32, device=dev)
        _lib.call("st_moe_permute", H_(idx), T, k, E, _lib.ptr(offsets),
                  _lib.ptr(row_token), _lib.ptr(pick_row), _st(dev))
        torch.cuda.synchronize()
        flat = idx.flatten().long()
        counts = torch.bincount(flat[valid], minlength=E)
        assert torch.equal(offsets.cpu().long(),
                           torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]))
        picks = torch.arange(T * k)[valid]
        order = picks[torch.argsort(flat[valid] * (T * k) + picks, stable=True)]
        n = int(valid.sum())
        assert torch.equal(row_token.cpu().long()[:n], order // k)
        expect = torch.full((T * k,), -1, dtype=torch.long)
        expect[order] = torch.arange(n)
        assert torch.equal(pick_row.cpu().long(), expect)
        return
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    row_token = torch.empty(T * k, dtype=torch.int32, device=dev)
    pick_row = torch.empty(T * k, dtype=torch.int32, device=dev)
    _lib.call("st_moe_permute", H_(idx), T, k, E, _lib.ptr(offsets),
              _lib.ptr(row_token), _lib.ptr(pick_row), _st(dev))
    torch.cuda.synchronize()
    flat = idx.flatten().long()
    counts = torch.bincount(flat, minlength=E)
    assert torch.equal(offsets.cpu().long(), torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]))
    order = torch.argsort(flat * (T * k) + torch.arange(T * k), stable=True)   # by expert, then pick
    assert torch.equal(row_token.cpu().long(), order // k)
    inv = torch.empty_like(order)
    inv[order] = torch.arange(T * k)
    assert torch.equal(pick_row.cpu().long(), inv)


def test_combine_bit_exact_and_vjp(dev):
    g = torch.Generator().manual_seed(8)
    H_ = _Held(dev)
    T, E, k, H = 257, 16, 4, 264
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).int()
    R = T * k
    v = torch.randn(R, H, generator=g).to(BF)
    w = torch.rand(T, k, generator=g).to(BF).float()
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    row_token = torch.empty(R, dtype=torch.int32, device=dev)
    pick_row = torch.empty(R, dtype=torch.int32, device=dev)
    _lib.call("st_moe_permute", H_(idx), T, k, E, _lib.ptr(offsets),
              _lib.ptr(row_token), _lib.ptr(pick_row), _st(dev))
    out = torch.empty(T, H, dtype=BF, device=dev)
    vd, wd = v.to(dev), w.to(dev)
    _lib.call("st_moe_combine", _lib.ptr(vd), R, _lib.ptr(wd), H_(idx),
              _lib.ptr(pick_row), T, k, H, _lib.ptr(out), _st(dev))
    torch.cuda.synchronize()
    pr = pick_row.cpu().long().view(T, k)
    # reference: the oracle's index_add_ loop over experts in ascending order
    ref = torch.zeros(T, H, dtype=BF)
    for e in range(E):
        pos, tok = torch.where(idx.T.long() == e)
        if tok.numel():
            val = v[pr[tok, pos]] * w[tok, pos, None].to(BF)
            ref.index_add_(0, tok, val)
    assert torch.equal(out.cpu().view(torch.int16), ref.view(torch.int16))
    # VJP (bf16 weights): autograd of the same expression
    vr = v.clone().requires_grad_(True)
    wr = w.to(BF).clone().requires_grad_(True)
    acc = torch.zeros(T, H, dtype=BF)
    for e in range(E):
        pos, tok = torch.where(idx.T.long() == e)
        if tok.numel():
            acc = acc.index_add(0, tok, vr[pr[tok, pos]] * wr[tok, pos, None])
    dout = torch.randn(T, H, generator=g).to(BF)
    dv_ref, dw_ref = torch.autograd.grad(acc, (vr, wr), dout)
    dv = torch.empty(R, H, dtype=BF, device=dev)
    dw = torch.empty(T, k, device=dev)
    _lib.call("st_moe_combine_bwd", H_(dout), _lib.ptr(vd), R, _lib.ptr(wd),
              _lib.ptr(pick_row), T, k, H, 1, _lib.ptr(dv), _lib.ptr(dw), _st(dev))
    torch.cuda.synchronize()
    assert torch.equal(dv.cpu().view(torch.int16), dv_ref.view(torch.int16))
    assert ((dw.cpu() - dw_ref.float()).abs() <= dw_ref.float().abs() * 2 ** -7 + 1e-3).all()
    # gather-sum: input gradient of flat[tokens] over all picks plus an extra term
    extra = torch.randn(T, H, generator=g).to(BF)
    gs = torch.empty(T, H, dtype=BF, device=dev)
    _lib.call("st_moe_gather_sum", _lib.ptr(dv), R, _lib.ptr(pick_row), T, k, H,
              H_(extra), _lib.ST_DTYPE_BF16, _lib.ptr(gs), _st(dev))
    torch.cuda.synchronize()
    ref_gs = (dv.cpu().float()[pr].sum(1) + extra.float()).to(BF)
    assert _rel(gs, ref_gs) < 4e-3


# ----------------------------------------------------------------- grouped GEMMs
@pytest.mark.parametrize("tile", ["128", "2562", "2566", "2568"])
@pytest.mark.parametrize("E,N,K,T,k", [(8, 256, 256, 100, 2), (16, 96, 384, 333, 4),
                                       (32, 1536, 2048, 512, 8)])
def test_grouped_fwd_and_dgrad_vs_oracle(dev, oracle_codec, monkeypatch, E, N, K, T, k, tile):
    """Grouped forward on the default 128x128 tile, the warp-specialised
    256x128 tile (forward and dgrad; N = 96 leaves the dgrad a ragged k-tile)
    and the register-operand 256x256 and 128x256 tiles (ST_GROUPED_TILE;
    K = 384 is not a multiple of 256 and keeps the 128x128 tile), and the
    grouped dgrad."""
    monkeypatch.setenv("ST_GROUPED_TILE", tile)
    g = torch.Generator().manual_seed(E + N + K)
    H_ = _Held(dev)
    q, W = _experts(oracle_codec, torch.randn(E, N, K, generator=g) * 0.02, dev)
    x = torch.randn(T, K, generator=g).to(BF)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).int()
    R = T * k
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    row_token = torch.empty(R, dtype=torch.int32, device=dev)
    pick_row = torch.empty(R, dtype=torch.int32, device=dev)
    _lib.call("st_moe_permute", H_(idx), T, k, E, _lib.ptr(offsets),
              _lib.ptr(row_token), _lib.ptr(pick_row), _st(dev))
    y = torch.empty(R, N, dtype=BF, device=dev)
    _lib.call("st_q4_grouped_fwd", H_(x), T, K, _lib.ptr(row_token), R, K,
              _lib.ptr(offsets), E, _lib.ptr(q.payload), _lib.ptr(q.scales), N, q.lut(), 0,
              None, 0, None, 0, 1.0, 0, None, _lib.ptr(y), N, _st(dev))
    dy = torch.randn(R, N, generator=g).to(BF)
    dx = torch.empty(R, K, dtype=BF, device=dev)
    _lib.call("st_q4_grouped_dgrad", H_(dy), N, R, N, _lib.ptr(offsets), E,
              _lib.ptr(q.payload), _lib.ptr(q.scales), K, q.lut(), 0, None, 0, None, 0,
              _lib.ptr(dx), K, _st(dev))
    torch.cuda.synchronize()
    off = offsets.cpu().long()
    tok = row_token.cpu().long()
    y_ref = torch.empty(R, N, dtype=BF)
    dx_ref = torch.empty(R, K, dtype=BF)
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            y_ref[a:b] = F.linear(x[tok[a:b]].float(), W[e].float()).to(BF)
            dx_ref[a:b] = (dy[a:b].float() @ W[e].float()).to(BF)
    for got, ref, what in ((y, y_ref, "fwd"), (dx, dx_ref, "dgrad")):
        got, ref = got.float().cpu(), ref.float()
        err = (got - ref).abs()
        bad = (err > ref.abs() * 2 ** -7 + 1e-6).float().mean().item()
        assert _rel(got, ref) < 4e-3 and bad < 1e-3, what


@pytest.mark.parametrize("tile", ["128", "2562", "2566", "2568"])
@pytest.mark.parametrize("r,nseg", [(8, 2), (5, 1), (40, 2), (80, 1)])
def test_grouped_lora_epilogue_vs_reference(dev, oracle_codec, monkeypatch, tile, r, nseg):
    """Per-expert LoRA terms in the grouped GEMM epilogues on every grouped
    tile: forward y = bf16(bf16(x W_e^T) + s T B_e^T) with nseg segments of
    rank r, dgrad dx = bf16(bf16(dy W_e) + bf16(dT A_e)) with nseg * r LoRA
    rows.  80 and 2 x 40 LoRA columns exceed what the 128x256 and 256x128
    tiles' LDS stages and run on the 128x128 kernel, which stages 2 x 40 and
    reads rank 80 from global memory."""
    monkeypatch.setenv("ST_GROUPED_TILE", tile)
    E, N, K, T, k = 8, 256, 256, 100, 2
    g = torch.Generator().manual_seed(r * 7 + nseg)
    H_ = _Held(dev)
    q, W = _experts(oracle_codec, torch.randn(E, N, K, generator=g) * 0.02, dev)
    x = torch.randn(T, K, generator=g).to(BF)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).int()
    R, C = T * k, nseg * r
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    row_token = torch.empty(R, dtype=torch.int32, device=dev)
    pick_row = torch.empty(R, dtype=torch.int32, device=dev)
    _lib.call("st_moe_permute", H_(idx), T, k, E, _lib.ptr(offsets),
              _lib.ptr(row_token), _lib.ptr(pick_row), _st(dev))
    Tm = torch.randn(R, C, generator=g) * 0.5
    Bl = torch.randn(E, N, r, generator=g) * 0.05
    dT = torch.randn(R, C, generator=g) * 0.5
    Al = torch.randn(E, C, K, generator=g) * 0.05
    scale = 2.0
    ends = [N // nseg * (i + 1) for i in range(nseg)]
    y = torch.empty(R, N, dtype=BF, device=dev)
    _lib.call("st_q4_grouped_fwd", H_(x), T, K, _lib.ptr(row_token), R, K,
              _lib.ptr(offsets), E, _lib.ptr(q.payload), _lib.ptr(q.scales), N, q.lut(), 0,
              H_(Tm), C, H_(Bl), r, scale, nseg, _lib.i64_array(ends), _lib.ptr(y), N, _st(dev))
    dy = torch.randn(R, N, generator=g).to(BF)
    dx = torch.empty(R, K, dtype=BF, device=dev)
    _lib.call("st_q4_grouped_dgrad", H_(dy), N, R, N, _lib.ptr(offsets), E,
              _lib.ptr(q.payload), _lib.ptr(q.scales), K, q.lut(), 0, H_(dT), C, H_(Al), C,
              _lib.ptr(dx), K, _st(dev))
    torch.cuda.synchronize()
    off = offsets.cpu().long()
    tok = row_token.cpu().long()
    y_ref = torch.empty(R, N, dtype=BF)
    dx_ref = torch.empty(R, K, dtype=BF)
    seg = torch.zeros(N, dtype=torch.long)
    for e_ in ends[:-1]:
        seg[e_:] += 1
    for e in range(E):
        a, b = int(off[e]), int(off[e + 1])
        if b > a:
            base = F.linear(x[tok[a:b]].float(), W[e].float()).to(BF).double()
            Ts = Tm[a:b].double().view(b - a, nseg, r)[:, seg, :]       # [rows, N, r]
            lora = (Ts * Bl[e].double().unsqueeze(0)).sum(-1) * scale
            y_ref[a:b] = (base + lora).to(BF)
            dbase = (dy[a:b].float() @ W[e].float()).to(BF).double()
            dx_ref[a:b] = (dbase + (dT[a:b].double() @ Al[e].double()).to(BF).double()).to(BF)
    for got, ref, what in ((y, y_ref, "fwd"), (dx, dx_ref, "dgrad")):
        got, ref = got.float().cpu(), ref.float()
        err = (got - ref).abs()
        bad = (err > ref.abs() * 2 ** -7 + 1e-6).float().mean().item()
        assert _rel(got, ref) < 4e-3 and bad < 1e-3, (what, _rel(got, ref), bad)


@pytest.mark.parametrize("E,H,I,T,k,r,tile", [
    (8, 256, 256, 100, 2, 8, None), (16, 384, 128, 333, 4, 0, None), (32, 2048, 768, 512, 8, 8, None),
    # LoRA operands that fill the tile's LDS up to or past the SwiGLU staging:
    # 128x128 at 256*(r+1) + 2304 > 18432 dwords for r >= 63, the 256x128
    # warp-specialised tile at lora_k >= 79
    (8, 256, 256, 100, 2, 62, None), (8, 256, 256, 100, 2, 63, None), (8, 256, 256, 100, 2, 64, None),
    (8, 256, 256, 100, 2, 71, None), (8, 256, 256, 100, 2, 72, None),
    (8, 256, 256, 100, 2, 78, "2562"), (8, 256, 256, 100, 2, 80, "2562"),
])
def test_grouped_dgrad_swiglu_equals_dgrad_then_swiglu_bwd(dev, oracle_codec, monkeypatch,
                                                           E, H, I, T, k, r, tile):
    """st_q4_grouped_dgrad_swiglu (the SwiGLU VJP in the experts' down dgrad
    epilogue) == st_q4_grouped_dgrad then st_swiglu_bwd, bit for bit, with
    and without the per-expert LoRA term, over ragged expert groups.  Ranks
    whose LoRA operands leave no room for the SwiGLU staging run on the
    global-operand kernel instead of failing."""
    if tile is not None:
        monkeypatch.setenv("ST_GROUPED_TILE", tile)
    lora = r > 0
    g = torch.Generator().manual_seed(E + H + I)
    H_ = _Held(dev)
    q, _ = _experts(oracle_codec, torch.randn(E, H, I, generator=g) * 0.02, dev)
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(T)]).int()
    R = T * k
    offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
    row_token = torch.empty(R, dtype=torch.int32, device=dev)
    pick_row = torch.empty(R, dtype=torch.int32, device=dev)
    _lib.call("st_moe_permute", H_(idx), T, k, E, _lib.ptr(offsets),
              _lib.ptr(row_token), _lib.ptr(pick_row), _st(dev))
    dy = torch.randn(R, H, generator=g).to(BF).to(dev)
    gu = torch.randn(R, 2 * I, generator=g).to(BF).to(dev)
    dt = (torch.randn(R, r, generator=g) * 0.1).to(dev) if lora else None
    a = (torch.randn(E, r, I, generator=g) * 0.05).to(dev) if lora else None
    kr = r if lora else 0
    dh = torch.empty(R, I, dtype=BF, device=dev)
    _lib.call("st_q4_grouped_dgrad", _lib.ptr(dy), H, R, H, _lib.ptr(offsets), E,
              _lib.ptr(q.payload), _lib.ptr(q.scales), I, q.lut(), 0, _lib.ptr(dt), kr,
              _lib.ptr(a), kr, _lib.ptr(dh), I, _st(dev))
    ref = torch.empty(R, 2 * I, dtype=BF, device=dev)
    _lib.call("st_swiglu_bwd", _lib.ptr(dh), I, _lib.ptr(gu), 2 * I, _lib.ptr(gu[:, I:]), 2 * I,
              R, I, _lib.ptr(ref), 2 * I, _lib.ptr(ref[:, I:]), 2 * I, _st(dev))
    got = torch.empty(R, 2 * I, dtype=BF, device=dev)
    _lib.call("st_q4_grouped_dgrad_swiglu", _lib.ptr(dy), H, R, H, _lib.ptr(offsets), E,
              _lib.ptr(q.payload), _lib.ptr(q.scales), I, q.lut(), 0, _lib.ptr(dt), kr,
              _lib.ptr(a), kr, _lib.ptr(gu), 2 * I, _lib.ptr(got), 2 * I, _st(dev))
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


# ----------------------------------------------------------------- whole feed-forward
def _oracle_ffn(flat, router, Wgu, Wd, idx, norm, lora):
    """Oracle forward + VJP on the GPU's picks; returns out and grads."""
    x = flat.clone().requires_grad_(True)
    _, routing = OM.qwen3_route_given(x, router, idx, norm_topk_prob=norm)
    loras, leaves = None, []
    if lora is not None:
        A_gu, B_gu, A_d, B_d, r, s_gu, s_d = lora
        leaves = [None if t is None else t.clone().requires_grad_(True)
                  for t in (A_gu, B_gu, A_d, B_d)]
        I = Wd.shape[2]
        loras = {}
        if A_gu is not None:
            loras["gate"] = (leaves[0][:, :r], leaves[1][:, :I], s_gu)
            loras["up"] = (leaves[0][:, r:], leaves[1][:, I:], s_gu)
        if A_d is not None:
            loras["down"] = (leaves[2], leaves[3], s_d)
    out = OM.expert_loop(x, routing, idx, Wgu, Wd, num_experts=Wgu.shape[0], loras=loras)
    return x, out, leaves


@pytest.mark.parametrize("T,H,I,E,k,norm,use_lora,r", [
    (64, 256, 128, 8, 2, True, True, 8),
    (203, 256, 256, 16, 4, False, True, 8),
    (96, 128, 128, 4, 4, True, False, 8),
    (256, 2048, 768, 64, 8, True, True, 8),       # config 4 expert shapes, fewer experts/tokens
    (100, 256, 128, 8, 2, True, True, 80),        # rank 80: 160 gate|up LoRA columns
    (100, 256, 128, 8, 2, True, True, 62),        # down LoRA beside the SwiGLU staging
    (100, 256, 128, 8, 2, True, True, 63),
    (100, 256, 128, 8, 2, True, True, 64),
    (100, 256, 128, 8, 2, True, True, 71),
    (100, 256, 128, 8, 2, True, True, 72),
    (80, 256, 128, 8, 2, False, "gate_up", 8),
    (80, 256, 128, 8, 2, True, "down", 8),
])
def test_moe_ffn_fwd_bwd_vs_oracle(dev, oracle_codec, T, H, I, E, k, norm, use_lora, r):
    """Routed experts through the grouped GEMMs against the oracle's expert
    loop.  Rank 80 takes the expert LoRA products 64 columns per launch and
    the grouped GEMM epilogues' LoRA operands from global memory;
    "gate_up" / "down" adapt only that projection of every expert."""
    g = torch.Generator().manual_seed(T + H + I + E)
    router = (torch.randn(E, H, generator=g) * H ** -0.5).to(BF)
    qgu, Wgu = _experts(oracle_codec, torch.randn(E, 2 * I, H, generator=g) * 0.02, dev)
    qd, Wd = _experts(oracle_codec, torch.randn(E, H, I, generator=g) * 0.02, dev)
    flat = torch.randn(T, H, generator=g).to(BF)
    lgu = ld = None
    if use_lora in (True, "gate_up"):
        lgu = moe.make_expert_lora("mlp.experts.gate_up_proj", E, H, 2 * I, rank=r, alpha=16.0,
                                   device=dev, segments=2, generator=g, b_std=0.02)
    if use_lora in (True, "down"):
        ld = moe.make_expert_lora("mlp.experts.down_proj", E, I, H, rank=r, alpha=16.0,
                                  device=dev, generator=g, b_std=0.02)
    weights = {"mlp.gate.weight": router.to(dev), "mlp.experts.gate_up_proj": qgu,
               "mlp.experts.down_proj": qd}
    xd = flat.to(dev).requires_grad_(True)
    out, w, idx = moe.moe_feed_forward(xd, weights, num_experts=E, top_k=k, norm_topk_prob=norm,
                                       lora_gate_up=lgu, lora_down=ld, return_routing=True)
    dout = torch.randn(T, H, generator=g).to(BF)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    idx_c = idx.cpu().long()
    _, ref_idx = OM.topk_lowest_index(F.softmax(F.linear(flat, router).float(), -1), k)
    assert torch.equal(idx_c, ref_idx)
    lora = None
    if use_lora:
        cpu = lambda l, f: None if l is None else getattr(l, f).detach().cpu()  # noqa: E731
        lora = (cpu(lgu, "A"), cpu(lgu, "B"), cpu(ld, "A"), cpu(ld, "B"), r,
                1.0 if lgu is None else lgu.scale, 1.0 if ld is None else ld.scale)
    x, ref, leaves = _oracle_ffn(flat, router, Wgu, Wd, idx_c, norm, lora)
    ref.backward(dout)
    assert _rel(out, ref) < 2e-2, "output"
    assert _cos(xd.grad, x.grad) > 0.999, "input grad"
    if use_lora:
        for ad, i, name in ((lgu, 0, "gu"), (ld, 2, "d")):
            if ad is None:
                continue
            for got, leaf, part in ((ad.A.grad, leaves[i], "A"), (ad.B.grad, leaves[i + 1], "B")):
                assert _cos(got, leaf.grad) > 0.999, part + "_" + name


class _SharedLora:
    """LoRA of one shared-expert projection: fp32 leaves A [r, in], B [out, r]."""

    def __init__(self, g, r, fin, fout, alpha, dev):
        self.rank, self.scale = r, alpha / r
        self.A = (torch.randn(r, fin, generator=g) * 0.05).to(dev).requires_grad_(True)
        self.B = (torch.randn(fout, r, generator=g) * 0.05).to(dev).requires_grad_(True)


def _q4_dense(oc, w, dev):
    from spilltune_amd import ops
    w32 = w.numpy().astype(np.float32)
    payload, scales = oc.encode_nf4(w32)
    bits = np.asarray(oc.decode4(payload, scales, w32.size, lut=oc.NF4_LUT), dtype=np.uint16)
    exact = torch.from_numpy(bits.astype(np.int16)).view(BF).view(w.shape)
    return ops.Q4Weight(torch.from_numpy(payload).to(dev), torch.from_numpy(scales).to(dev),
                        tuple(w.shape), "nf4-g128"), exact


@pytest.mark.parametrize("T,H,I,E,groups,group_k,k,expert_lora", [
    (128, 256, 128, 16, 4, 2, 4, True),
    (77, 128, 128, 32, 8, 4, 8, False),
])
def test_deepseek_moe_ffn_fwd_bwd_vs_oracle(dev, oracle_codec, T, H, I, E, groups, group_k, k,
                                            expert_lora):
    """deepseek.py:115-126,158-174: sigmoid group-limited routing with the
    selection bias, fp32 routing weights, the routed experts and the shared
    expert (with LoRA on its three projections), forward and backward, vs the
    oracle on the GPU's picks; the picks equal the oracle router's."""
    from oracle import layer as OL
    g = torch.Generator().manual_seed(T + E + k)
    router = (torch.randn(E, H, generator=g) * 3 * H ** -0.5).to(BF)   # well-separated scores
    bias = torch.randn(E, generator=g) * 0.1
    qgu, Wgu = _experts(oracle_codec, torch.randn(E, 2 * I, H, generator=g) * 0.02, dev)
    qd, Wd = _experts(oracle_codec, torch.randn(E, H, I, generator=g) * 0.02, dev)
    Is = 2 * I
    qsg, Wsg = _q4_dense(oracle_codec, torch.randn(Is, H, generator=g) * 0.02, dev)
    qsu, Wsu = _q4_dense(oracle_codec, torch.randn(Is, H, generator=g) * 0.02, dev)
    qsd, Wsd = _q4_dense(oracle_codec, torch.randn(H, Is, generator=g) * 0.02, dev)
    flat = torch.randn(T, H, generator=g).to(BF)
    dout = torch.randn(T, H, generator=g).to(BF)
    r = 8
    lgu = ld = None
    if expert_lora:
        lgu = moe.make_expert_lora("mlp.experts.gate_up_proj", E, H, 2 * I, rank=r, alpha=16.0,
                                   device=dev, segments=2, generator=g, b_std=0.02)
        ld = moe.make_expert_lora("mlp.experts.down_proj", E, I, H, rank=r, alpha=16.0,
                                  device=dev, generator=g, b_std=0.02)
    ls = {"gate": _SharedLora(g, r, H, Is, 16.0, dev), "up": _SharedLora(g, r, H, Is, 16.0, dev),
          "down": _SharedLora(g, r, Is, H, 16.0, dev)}
    weights = {"mlp.gate.weight": router.to(dev), "mlp.gate.e_score_correction_bias": bias.to(dev),
               "mlp.experts.gate_up_proj": qgu, "mlp.experts.down_proj": qd,
               "mlp.shared_experts.gate_proj.weight": qsg, "mlp.shared_experts.up_proj.weight": qsu,
               "mlp.shared_experts.down_proj.weight": qsd}
    xd = flat.to(dev).requires_grad_(True)
    out, w, idx = moe.deepseek_moe_feed_forward(
        xd, weights, num_experts=E, top_k=k, groups=groups, group_k=group_k, normalize=True,
        scale=2.5, lora_gate_up=lgu, lora_down=ld, lora_shared=ls, return_routing=True)
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    idx_c = idx.cpu().long()
    _, _, ref_idx = OM.deepseek_route(flat, router, bias, groups=groups, group_k=group_k, top_k=k,
                                      normalize=True, scale=2.5)
    assert torch.equal(idx_c.sort(1)[0], ref_idx.sort(1)[0])
    # oracle on the GPU's picks
    x = flat.clone().requires_grad_(True)
    logits = F.linear(x.float(), router.float())
    routing = OM.deepseek_weights_given(logits, idx_c, normalize=True, scale=2.5)
    torch.testing.assert_close(w.cpu(), routing.detach(), rtol=1e-5, atol=1e-6)
    loras, leaves = None, []
    if expert_lora:
        leaves = [t.detach().cpu().clone().requires_grad_(True) for t in (lgu.A, lgu.B, ld.A, ld.B)]
        loras = {"gate": (leaves[0][:, :r], leaves[1][:, :I], lgu.scale),
                 "up": (leaves[0][:, r:], leaves[1][:, I:], lgu.scale),
                 "down": (leaves[2], leaves[3], ld.scale)}
    routed = OM.expert_loop(x, routing, idx_c, Wgu, Wd, num_experts=E, loras=loras)
    sl = {n: OL.Lora(n, l.A.detach().cpu(), l.B.detach().cpu(), 16.0) for n, l in ls.items()}
    act = F.silu(OL.lora_linear(x, Wsg, sl["gate"])) * OL.lora_linear(x, Wsu, sl["up"])
    ref = routed + OL.lora_linear(act, Wsd, sl["down"])
    ref.backward(dout)
    assert _rel(out, ref) < 2e-2, "output"
    assert _cos(xd.grad, x.grad) > 0.999, "input grad"
    for n in ("gate", "up", "down"):
        assert _cos(ls[n].A.grad, sl[n].A.grad) > 0.999, f"shared {n} A"
        assert _cos(ls[n].B.grad, sl[n].B.grad) > 0.999, f"shared {n} B"
    if expert_lora:
        for got, leaf, name in ((lgu.A.grad, leaves[0], "A_gu"), (lgu.B.grad, leaves[1], "B_gu"),
                                (ld.A.grad, leaves[2], "A_d"), (ld.B.grad, leaves[3], "B_d")):
            assert _cos(got, leaf.grad) > 0.999, name


def test_dense_block_with_moe_feed_forward(dev, oracle_codec):
    """A Qwen3-MoE-style decoder block: the HIP dense functional with the MoE
    feed-forward hook (dense.py:152) vs the oracle block with the oracle MoE."""
    import functools
    from oracle import layer as OL
    from spilltune_amd import dense, ops
    g = torch.Generator().manual_seed(77)
    B, S, H, heads, kv, D, E, I, k, r = 1, 96, 256, 4, 2, 64, 8, 128, 2, 8
    exact, wts = {}, {}
    for name, shape in (("self_attn.q_proj", (heads * D, H)), ("self_attn.k_proj", (kv * D, H)),
                        ("self_attn.v_proj", (kv * D, H)), ("self_attn.o_proj", (H, heads * D))):
        w32 = (torch.randn(shape, generator=g) * 0.02).numpy()
        payload, scales = oracle_codec.encode_nf4(w32)
        bits = np.asarray(oracle_codec.decode4(payload, scales, w32.size, lut=oracle_codec.NF4_LUT),
                          dtype=np.uint16)
        exact[name + ".weight"] = torch.from_numpy(bits.astype(np.int16)).view(BF).view(shape)
        wts[name + ".weight"] = ops.Q4Weight(torch.from_numpy(payload).to(dev),
                                             torch.from_numpy(scales).to(dev), shape, "nf4-g128")
    for nm in ("input_layernorm.weight", "post_attention_layernorm.weight"):
        exact[nm] = (1 + 0.05 * torch.randn(H, generator=g)).to(BF)
        wts[nm] = exact[nm].to(dev)
    router = (torch.randn(E, H, generator=g) * 3 * H ** -0.5).to(BF)   # well-separated logits
    qgu, Wgu = _experts(oracle_codec, torch.randn(E, 2 * I, H, generator=g) * 0.02, dev)
    qd, Wd = _experts(oracle_codec, torch.randn(E, H, I, generator=g) * 0.02, dev)
    wts.update({"mlp.gate.weight": router.to(dev), "mlp.experts.gate_up_proj": qgu,
                "mlp.experts.down_proj": qd})
    lgu = moe.make_expert_lora("mlp.experts.gate_up_proj", E, H, 2 * I, rank=r, alpha=16.0,
                               device=dev, segments=2, generator=g, b_std=0.02)
    ld = moe.make_expert_lora("mlp.experts.down_proj", E, I, H, rank=r, alpha=16.0, device=dev,
                              generator=g, b_std=0.02)
    hidden = torch.randn(B, S, H, generator=g).to(BF)
    dy = torch.randn(B, S, H, generator=g).to(BF)
    cos, sin = OL.rotary(B, S, D, 500000.0, BF)
    # HIP path
    ff = functools.partial(moe.moe_feed_forward, num_experts=E, top_k=k, norm_topk_prob=True,
                           lora_gate_up=lgu, lora_down=ld)
    h = hidden.to(dev).requires_grad_(True)
    out = dense.dense_block(h, (cos.to(dev), sin.to(dev)), dense.CausalMask(B, S), heads=heads,
                            kv_heads=kv, head_dim=D, eps=1e-6, feed_forward=ff, **wts)
    out.backward(dy.to(dev))
    torch.cuda.synchronize()
    # oracle
    leaves = [t.detach().cpu().clone().requires_grad_(True) for t in (lgu.A, lgu.B, ld.A, ld.B)]
    loras = {"gate": (leaves[0][:, :r], leaves[1][:, :I], lgu.scale),
             "up": (leaves[0][:, r:], leaves[1][:, I:], lgu.scale),
             "down": (leaves[2], leaves[3], ld.scale)}
    ffr = lambda x, w: M_ffn(x, router, Wgu, Wd, k, loras)
    x = hidden.clone().requires_grad_(True)
    ref = OL.dense_block(x, (cos, sin), OL.causal_mask(B, S, BF), heads=heads, kv_heads=kv,
                         head_dim=D, eps=1e-6, weights=exact, loras={}, feed_forward=ffr)
    ref.backward(dy)
    assert _rel(out, ref) < 2e-2
    assert _cos(h.grad, x.grad) > 0.999
    for got, leaf in zip((lgu.A.grad, lgu.B.grad, ld.A.grad, ld.B.grad), leaves):
        assert _cos(got, leaf.grad) > 0.999


def M_ffn(x, router, Wgu, Wd, k, loras):
    return OM.qwen3_moe_ffn(x, router, Wgu, Wd, top_k=k, norm_topk_prob=True, loras=loras)


def test_qwen3_moe_layer_streamed_whole_vs_oracle(dev, oracle_codec):
    """A Qwen3-MoE decoder layer built by make_dense_block(moe=...): attention,
    router and every expert stack in ONE slot image (qwen3_moe.py:146-152),
    streamed through two slots with the recompute driver, per-expert LoRA;
    against the oracle block with the oracle MoE feed-forward."""
    from oracle import layer as OL
    from spilltune_amd import slots
    from spilltune_amd.dense import CausalMask
    from spilltune_amd.recompute import streaming_block
    g = torch.Generator().manual_seed(78)
    B, S, H, heads, kv, D, E, I, k, r = 1, 80, 256, 4, 2, 64, 16, 128, 4, 8
    w = {}
    for name, shape in (("self_attn.q_proj", (heads * D, H)), ("self_attn.k_proj", (kv * D, H)),
                        ("self_attn.v_proj", (kv * D, H)), ("self_attn.o_proj", (H, heads * D))):
        w[name + ".weight"] = torch.randn(shape, generator=g) * 0.02
    for nm in ("input_layernorm.weight", "post_attention_layernorm.weight"):
        w[nm] = 1 + 0.05 * torch.randn(H, generator=g)
    w["mlp.gate.weight"] = torch.randn(E, H, generator=g) * 3 * H ** -0.5   # well-separated logits
    w["mlp.experts.gate_up_proj"] = torch.randn(E, 2 * I, H, generator=g) * 0.02
    w["mlp.experts.down_proj"] = torch.randn(E, H, I, generator=g) * 0.02
    block = slots.make_dense_block(0, w, codec="nf4-g128", heads=heads, kv_heads=kv, head_dim=D,
                                   eps=1e-6, rank=r, alpha=16.0,
                                   targets=("self_attn.q_proj", "self_attn.v_proj",
                                            "self_attn.o_proj"),
                                   device=dev, generator=g,
                                   moe={"num_experts": E, "top_k": k, "norm_topk_prob": True},
                                   expert_lora_rank=r)
    with torch.no_grad():
        for p in block.adapters.values():
            p.B.copy_(torch.randn(p.B.shape, generator=g) * 0.02)
    lay = slots.plan_layout(block)
    assert lay.entries["mlp.experts.gate_up_proj"][2] == (E, 2 * I, H)   # expert stacks in the image
    # oracle weights: exact bf16 decode of every stored record
    exact = {}
    for name, entry in block.storage_specs.items():
        spec = entry["spec"]
        bits = oracle_codec.decode4(block.host_weights[entry["parts"]["payload"]].numpy(),
                                    block.host_weights[entry["parts"]["scales"]].numpy(),
                                    spec["numel"], lut=oracle_codec.NF4_LUT)
        exact[name] = torch.from_numpy(np.asarray(bits, dtype=np.uint16).astype(np.int16)).view(
            BF).view(spec["shape"])
    for kk, v in block.host_weights.items():
        if not kk.startswith("@"):
            exact[kk] = v
    hidden = torch.randn(B, S, H, generator=g).to(BF)
    dy = torch.randn(B, S, H, generator=g).to(BF)
    cos, sin = OL.rotary(B, S, D, 500000.0, BF)
    session = slots.Q4SlotSession([block], dev, host_budget_bytes=1 << 34,
                                  device_budget_bytes=1 << 34, slots=2)
    h = hidden.to(dev).requires_grad_(True)
    with session.run():
        out = streaming_block(h, (cos.to(dev), sin.to(dev)), CausalMask(B, S), block.functional,
                              block.kwargs, session.reloader(block), block.adapters, block.index)
        out.backward(dy.to(dev))
    torch.cuda.synchronize()
    assert session.actual_h2d_bytes >= lay.nbytes
    lgu, ldn = block.adapters["mlp.experts.gate_up_proj"], block.adapters["mlp.experts.down_proj"]
    leaves = [t.detach().cpu().clone().requires_grad_(True) for t in (lgu.A, lgu.B, ldn.A, ldn.B)]
    loras = {"gate": (leaves[0][:, :r], leaves[1][:, :I], lgu.scale),
             "up": (leaves[0][:, r:], leaves[1][:, I:], lgu.scale),
             "down": (leaves[2], leaves[3], ldn.scale)}
    dense_l = {n: OL.Lora(n, p.A.detach().cpu(), p.B.detach().cpu(), p.alpha)
               for n, p in block.adapters.items() if not n.startswith("mlp.experts")}
    ffr = lambda x, wts: OM.qwen3_moe_ffn(x, exact["mlp.gate.weight"],  # noqa: E731
                                         exact["mlp.experts.gate_up_proj"],
                                         exact["mlp.experts.down_proj"], top_k=k,
                                         norm_topk_prob=True, loras=loras)
    x = hidden.clone().requires_grad_(True)
    ref = OL.dense_block(x, (cos, sin), OL.causal_mask(B, S, BF), heads=heads, kv_heads=kv,
                         head_dim=D, eps=1e-6, weights=exact, loras=dense_l, feed_forward=ffr)
    ref.backward(dy)
    assert _rel(out, ref) < 2e-2
    assert _cos(h.grad, x.grad) > 0.999
    for n, l in dense_l.items():
        assert _cos(block.adapters[n].grad_A, l.A.grad) > 0.999, n
        assert _cos(block.adapters[n].grad_B, l.B.grad) > 0.999, n
    for got, leaf, name in ((lgu.grad_A, leaves[0], "A_gu"), (lgu.grad_B, leaves[1], "B_gu"),
                            (ldn.grad_A, leaves[2], "A_d"), (ldn.grad_B, leaves[3], "B_d")):
        assert _cos(got, leaf.grad) > 0.999, name
    session.close()
