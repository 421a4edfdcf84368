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


def _ref(q, k, v, scale):
    B, H, S, D = q.shape
    g = H // k.shape[1]
    kf = k.float().repeat_interleave(g, 1)
    vf = v.float().repeat_interleave(g, 1)
    s = (q.float() @ kf.transpose(-1, -2)) * scale
    mask = torch.ones(S, S, dtype=torch.bool, device=q.device).triu(1)
    s = s.masked_fill(mask, float("-inf"))
    lse2 = torch.logsumexp(s, -1) / math.log(2.0)
    o = torch.softmax(s, -1) @ vf
    return o.transpose(1, 2).reshape(B, S, H * D), lse2


def _fwd(q, k, v, scale):
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    out = torch.empty(B, S, H * D, dtype=BF, device=q.device)
    lse = torch.empty(B, H, S, dtype=torch.float32, device=q.device)
    need = _lib.query("st_flash_attn_workspace_bytes", B, S, H, Hkv, D, 0)
    ws = torch.empty(need, dtype=torch.uint8, device=q.device)
    _lib.call("st_flash_attn_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), B, S, H, Hkv, D,
              float(scale), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(ws), ws.numel(),
              _lib.stream_handle(q.device))
    torch.cuda.synchronize()
    return out, lse


@pytest.mark.parametrize("B,H,Hkv,S,D", [(1, 4, 2, 128, 64), (2, 4, 4, 200, 64), (1, 8, 2, 256, 128),
                                         (1, 4, 1, 72, 128), (1, 32, 8, 2048, 128)])
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


def _bwd(q, k, v, out, lse, dout, scale):
    B, H, S, D = q.shape
    Hkv = k.shape[1]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    need = _lib.query("st_flash_attn_workspace_bytes", B, S, H, Hkv, D, 1)
    ws = torch.empty(need, dtype=torch.uint8, device=q.device)
    _lib.call("st_flash_attn_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out),
              _lib.ptr(lse), _lib.ptr(dout), B, S, H, Hkv, D, float(scale), _lib.ptr(dq),
              _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws), ws.numel(), _lib.stream_handle(q.device))
    torch.cuda.synchronize()
    return dq, dk, dv


@pytest.mark.parametrize("B,H,Hkv,S,D", [(1, 4, 2, 128, 64), (2, 4, 4, 200, 64), (1, 8, 2, 256, 128),
                                         (1, 4, 1, 72, 128), (1, 32, 8, 2048, 128)])
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
        rel = ((got.float() - want).norm() / want.norm()).item()
        cos = torch.nn.functional.cosine_similarity(got.float().flatten(), want.flatten(), 0).item()
        assert rel < 2e-2 and cos > 0.9995, (name, rel, cos)
