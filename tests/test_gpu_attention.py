"""Flash attention (HIP) vs a float32 PyTorch reference of the eager
attention of adapters/dense.py:142-148 (GQA repeat, causal mask, softmax,
probabilities @ v).  Tolerances: bf16 output rel err <= 1e-2; the base-2
log-sum-exp to 1e-4 relative."""
import math

import pytest
import torch

from spilltune_amd import _lib

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _blocked(B, S, lens, device):
    """dense.py:246: causal, and (right padding) keys past each row's prefix."""
    mask = torch.ones(S, S, dtype=torch.bool, device=device).triu(1)[None, None]
    if lens is not None:
        keys = torch.arange(S, device=device)[None, :] >= torch.tensor(lens, device=device)[:, None]
        mask = mask | keys[:, None, None, :]
    return mask


def _ref(q, k, v, scale, lens=None):
    B, H, S, D = q.shape
    g = H // k.shape[1]
    kf = k.float().repeat_interleave(g, 1)
    vf = v.float().repeat_interleave(g, 1)
    s = (q.float() @ kf.transpose(-1, -2)) * scale
    s = s.masked_fill(_blocked(B, S, lens, q.device), float("-inf"))
    lse2 = torch.logsumexp(s, -1) / math.log(2.0)
    o = torch.softmax(s, -1) @ vf
    return o.transpose(1, 2).reshape(B, S, H * D), lse2


def _kvl(lens, device):
    return None if lens is None else torch.tensor(lens, dtype=torch.int32, device=device)


def _fwd(q, k, v, scale, lens=None):
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    out = torch.empty(B, S, H * D, dtype=BF, device=q.device)
    lse = torch.empty(B, H, S, dtype=torch.float32, device=q.device)
    need = _lib.query("st_flash_attn_workspace_bytes", B, S, H, Hkv, D, 0)
    ws = torch.empty(need, dtype=torch.uint8, device=q.device)
    kvl = _kvl(lens, q.device)
    _lib.call("st_flash_attn_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), B, S, H, Hkv, D,
              float(scale), _lib.ptr(kvl), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws), ws.numel(),
              _lib.stream_handle(q.device))
    torch.cuda.synchronize()
    return out, lse


# sequence lengths of any size: 1, 17, 100 and 129 leave ragged key and
# query tiles (and a V^T staging row longer than S)
ODD_S = [(1, 2, 1, 1, 64), (2, 4, 2, 17, 128), (1, 4, 4, 100, 64), (1, 8, 2, 129, 128)]


@pytest.mark.parametrize("B,H,Hkv,S,D", [(1, 4, 2, 128, 64), (2, 4, 4, 200, 64), (1, 8, 2, 256, 128),
                                         (1, 4, 1, 72, 128), (1, 32, 8, 2048, 128)] + ODD_S)
def test_flash_fwd_vs_fp32(dev, B, H, Hkv, S, D):
    g = torch.Generator().manual_seed(B * 1000 + H * 10 + S + D)
    q = torch.randn(B, H, S, D, generator=g).to(BF).to(dev)
    k = torch.randn(B, Hkv, S, D, generator=g).to(BF).to(dev)
    v = torch.randn(B, Hkv, S, D, generator=g).to(BF).to(dev)
    scale = D ** -0.5
    out, lse = _fwd(q, k, v, scale)
    ref, lse_ref = _ref(q, k, v, scale)
    rel = ((out.float() - ref).norm() / ref.norm()).item()
    assert rel < 1e-2, rel
    torch.testing.assert_close(lse, lse_ref, rtol=1e-4, atol=1e-4)


def _bwd(q, k, v, out, lse, dout, scale, lens=None):
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    need = _lib.query("st_flash_attn_workspace_bytes", B, S, H, Hkv, D, 1)
    ws = torch.empty(need, dtype=torch.uint8, device=q.device)
    kvl = _kvl(lens, q.device)
    _lib.call("st_flash_attn_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out),
              _lib.ptr(lse), _lib.ptr(dout), B, S, H, Hkv, D, float(scale), _lib.ptr(kvl),
              _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws), ws.numel(),
              _lib.stream_handle(q.device))
    torch.cuda.synchronize()
    return dq, dk, dv


@pytest.mark.parametrize("B,H,Hkv,S,D", [(1, 4, 2, 128, 64), (2, 4, 4, 200, 64), (1, 8, 2, 256, 128),
                                         (1, 4, 1, 72, 128), (1, 32, 8, 2048, 128)] + ODD_S)
def test_flash_bwd_vs_fp32_autograd(dev, B, H, Hkv, S, D):
    g = torch.Generator().manual_seed(B * 999 + H * 7 + S + D)
    q = torch.randn(B, H, S, D, generator=g).to(BF).to(dev)
    k = torch.randn(B, Hkv, S, D, generator=g).to(BF).to(dev)
    v = torch.randn(B, Hkv, S, D, generator=g).to(BF).to(dev)
    dout = torch.randn(B, S, H * D, generator=g).to(BF).to(dev)
    scale = D ** -0.5
    out, lse = _fwd(q, k, v, scale)
    dq, dk, dv = _bwd(q, k, v, out, lse, dout, scale)
    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    ref, _ = _ref(qf, kf, vf, scale)
    ref.backward(dout.float())
    for got, want, name in ((dq, qf.grad, "dq"), (dk, kf.grad, "dk"), (dv, vf.grad, "dv")):
        if S == 1 and name != "dv":
            # one key: P = 1 and dS = P (dP - rowsum(dO o O)) = 0, so dq = dk = 0
            # (the fp32 reference leaves rounding noise)
            assert got.float().abs().max().item() < 1e-3 and want.abs().max().item() < 1e-3
            continue
        rel = ((got.float() - want).norm() / want.norm()).item()
        cos = torch.nn.functional.cosine_similarity(got.float().flatten(), want.flatten(), 0).item()
        assert rel < 2e-2 and cos > 0.9995, (name, rel, cos)


# ----------------------------------------------------------------- MLA (DeepSeek-V3)
def _ref_mla(q, k, v, scale, lens=None):
    B, H, S, DQ = q.shape
    DV = v.shape[-1]
    s = (q.float() @ k.float().transpose(-1, -2)) * scale
    s = s.masked_fill(_blocked(B, S, lens, q.device), float("-inf"))
    lse2 = torch.logsumexp(s, -1) / math.log(2.0)
    o = torch.softmax(s, -1) @ v.float()
    return o.transpose(1, 2).reshape(B, S, H * DV), lse2


def _mla(q, k, v, scale, dout=None, lens=None):
    B, H, S, DQ = q.shape
    DV = v.shape[-1]
    dev, st = q.device, _lib.stream_handle(q.device)
    kvl = _kvl(lens, dev)
    out = torch.empty(B, S, H * DV, dtype=BF, device=dev)
    lse = torch.empty(B, H, S, dtype=torch.float32, device=dev)
    ws = torch.empty(_lib.query("st_mla_attn_workspace_bytes", B, S, H, DQ, DV, 0),
                     dtype=torch.uint8, device=dev)
    _lib.call("st_mla_attn_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), B, S, H, DQ, DV,
              float(scale), _lib.ptr(kvl), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws), ws.numel(),
              st)
    if dout is None:
        torch.cuda.synchronize()
        return out, lse
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    wb = torch.empty(_lib.query("st_mla_attn_workspace_bytes", B, S, H, DQ, DV, 1),
                     dtype=torch.uint8, device=dev)
    _lib.call("st_mla_attn_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out),
              _lib.ptr(lse), _lib.ptr(dout), B, S, H, DQ, DV, float(scale), _lib.ptr(kvl),
              _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(wb), wb.numel(), st)
    torch.cuda.synchronize()
    return out, lse, dq, dk, dv


@pytest.mark.parametrize("B,H,S", [(1, 4, 128), (2, 3, 200), (1, 8, 72), (1, 128, 2048), (1, 2, 13),
                                   (2, 3, 130)])
def test_mla_attention_fwd_bwd_vs_fp32(dev, B, H, S):
    """Query/key heads of 192 against value heads of 128 (DeepSeek-V3 MLA),
    forward and VJP against float32 autograd; the last case is config 5's
    full attention shape (128 heads x 2048 tokens)."""
    DQ, DV = 192, 128
    g = torch.Generator().manual_seed(B * 31 + H * 7 + S)
    q = torch.randn(B, H, S, DQ, generator=g).to(BF).to(dev)
    k = torch.randn(B, H, S, DQ, generator=g).to(BF).to(dev)
    v = torch.randn(B, H, S, DV, generator=g).to(BF).to(dev)
    dout = torch.randn(B, S, H * DV, generator=g).to(BF).to(dev)
    scale = DQ ** -0.5
    out, lse, dq, dk, dv = _mla(q, k, v, scale, dout)
    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    ref, lse_ref = _ref_mla(qf, kf, vf, scale)
    rel = ((out.float() - ref.detach()).norm() / ref.detach().norm()).item()
    assert rel < 1e-2, rel
    torch.testing.assert_close(lse, lse_ref.detach(), rtol=1e-4, atol=1e-4)
    ref.backward(dout.float())
    for got, want, name in ((dq, qf.grad, "dq"), (dk, kf.grad, "dk"), (dv, vf.grad, "dv")):
        rel = ((got.float() - want).norm() / want.norm()).item()
        cos = torch.nn.functional.cosine_similarity(got.float().flatten(), want.flatten(), 0).item()
        assert rel < 2e-2 and cos > 0.9995, (name, rel, cos)


def test_mla_entry_with_equal_dims_matches_flash_attention(dev):
    """st_mla_attn_* with DQ = DV = 128 runs the dense kernels: the same bits
    as st_flash_attn_* with Hkv = H."""
    g = torch.Generator().manual_seed(9)
    B, H, S, D = 1, 4, 256, 128
    q, k, v = (torch.randn(B, H, S, D, generator=g).to(BF).to(dev) for _ in range(3))
    dout = torch.randn(B, S, H * D, generator=g).to(BF).to(dev)
    o1, l1, dq1, dk1, dv1 = _mla(q, k, v, D ** -0.5, dout)
    o2, l2 = _fwd(q, k, v, D ** -0.5)
    dq2, dk2, dv2 = _bwd(q, k, v, o2, l2, dout, D ** -0.5)
    for a, b in ((o1, o2), (l1, l2), (dq1, dq2), (dk1, dk2), (dv1, dv2)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,H,Hkv,S,D,lens", [(3, 4, 2, 200, 64, [200, 137, 1]),
                                              (2, 8, 2, 129, 128, [64, 129]),
                                              (2, 4, 4, 72, 128, [33, 8])])
def test_flash_right_padding_vs_fp32(dev, B, H, Hkv, S, D, lens):
    """Right-padded rows (dense.py:237-246): every query, the padded ones
    included, attends only to its row's first lens[b] keys (and causally);
    forward, lse and the VJP against fp32 autograd with the same mask."""
    g = torch.Generator().manual_seed(sum(lens) + S + D)
    q = torch.randn(B, H, S, D, generator=g).to(BF).to(dev)
    k = torch.randn(B, Hkv, S, D, generator=g).to(BF).to(dev)
    v = torch.randn(B, Hkv, S, D, generator=g).to(BF).to(dev)
    dout = torch.randn(B, S, H * D, generator=g).to(BF).to(dev)
    scale = D ** -0.5
    out, lse = _fwd(q, k, v, scale, lens)
    dq, dk, dv = _bwd(q, k, v, out, lse, dout, scale, lens)
    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    ref, lse_ref = _ref(qf, kf, vf, scale, lens)
    rel = ((out.float() - ref.detach()).norm() / ref.detach().norm()).item()
    assert rel < 1e-2, rel
    torch.testing.assert_close(lse, lse_ref.detach(), rtol=1e-4, atol=1e-4)
    ref.backward(dout.float())
    for got, want, name in ((dq, qf.grad, "dq"), (dk, kf.grad, "dk"), (dv, vf.grad, "dv")):
        rel = ((got.float() - want).norm() / want.norm()).item()
        cos = torch.nn.functional.cosine_similarity(got.float().flatten(), want.flatten(), 0).item()
        assert rel < 2e-2 and cos > 0.9995, (name, rel, cos)
    # keys past a row's prefix get no gradient at all
    for b, n in enumerate(lens):
        if n < S:
            assert dk[b, :, n:].abs().max().item() == 0 and dv[b, :, n:].abs().max().item() == 0


def test_mla_right_padding_vs_fp32(dev):
    """The same masking on the MLA heads (192 against 128)."""
    B, H, S, DQ, DV, lens = 2, 3, 130, 192, 128, [130, 57]
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, H, S, DQ, generator=g).to(BF).to(dev)
    k = torch.randn(B, H, S, DQ, generator=g).to(BF).to(dev)
    v = torch.randn(B, H, S, DV, generator=g).to(BF).to(dev)
    dout = torch.randn(B, S, H * DV, generator=g).to(BF).to(dev)
    scale = DQ ** -0.5
    out, lse, dq, dk, dv = _mla(q, k, v, scale, dout, lens)
    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    ref, lse_ref = _ref_mla(qf, kf, vf, scale, lens)
    rel = ((out.float() - ref.detach()).norm() / ref.detach().norm()).item()
    assert rel < 1e-2, rel
    torch.testing.assert_close(lse, lse_ref.detach(), rtol=1e-4, atol=1e-4)
    ref.backward(dout.float())
    for got, want, name in ((dq, qf.grad, "dq"), (dk, kf.grad, "dk"), (dv, vf.grad, "dv")):
        rel = ((got.float() - want).norm() / want.norm()).item()
        cos = torch.nn.functional.cosine_similarity(got.float().flatten(), want.flatten(), 0).item()
        assert rel < 2e-2 and cos > 0.9995, (name, rel, cos)
