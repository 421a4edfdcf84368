"""Pins oracle/layer.py (the PyTorch-CPU restatement of the reference's layer
math) against library routines: transformers' LlamaDecoderLayer with
LoRA-wrapped projections (the reference's own parity harness,
tests/test_dense_adapters.py:49-58), float64 closed forms for the LoRA VJP,
full-sequence cross-entropy and torch.optim.AdamW(foreach=False)."""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import layer as L

PROJ = L.PROJECTIONS


def _hf_layer(cfg, weights, loras, dtype, family="llama"):
    if family == "llama":
        from transformers.models.llama.configuration_llama import LlamaConfig as Config
        from transformers.models.llama.modeling_llama import (LlamaDecoderLayer as Layer,
                                                              LlamaRotaryEmbedding as Rotary)
    else:
        from transformers.models.qwen3.configuration_qwen3 import Qwen3Config as Config
        from transformers.models.qwen3.modeling_qwen3 import (Qwen3DecoderLayer as Layer,
                                                              Qwen3RotaryEmbedding as Rotary)
    c = Config(hidden_size=cfg["H"], intermediate_size=cfg["I"],
               num_attention_heads=cfg["heads"], num_key_value_heads=cfg["kv"],
               head_dim=cfg["D"], num_hidden_layers=1, vocab_size=32,
               rms_norm_eps=cfg["eps"], rope_theta=cfg["theta"])
    c._attn_implementation = "eager"
    layer = Layer(c, 0).to(dtype)
    sd = {k: v.to(dtype) for k, v in weights.items()}
    layer.load_state_dict(sd, strict=True)
    layer.requires_grad_(False)

    class Projection(torch.nn.Module):
        def __init__(self, original, lora):
            super().__init__()
            self.original = original
            self.A = torch.nn.Parameter(lora.A.detach().clone())
            self.B = torch.nn.Parameter(lora.B.detach().clone())
            self.scale = lora.scale

        def forward(self, x):
            base = self.original(x)
            upd = F.linear(F.linear(x.float(), self.A), self.B)
            return (base.float() + upd * self.scale).to(base.dtype)

    wrapped = {}
    for name, lora in loras.items():
        parent, leaf = name.rsplit(".", 1)
        mod = layer.get_submodule(parent)
        w = Projection(getattr(mod, leaf), lora)
        setattr(mod, leaf, w)
        wrapped[name] = w
    rot = Rotary(c)
    return layer, wrapped, rot


def _setup(dtype, seed=0, S=9, B=2, qk_norm=False):
    g = torch.Generator().manual_seed(seed)
    cfg = dict(H=64, I=96, heads=4, kv=2, D=16, eps=1e-5, theta=10000.0)
    H, I, D = cfg["H"], cfg["I"], cfg["D"]
    shapes = {"self_attn.q_proj": (cfg["heads"] * D, H), "self_attn.k_proj": (cfg["kv"] * D, H),
              "self_attn.v_proj": (cfg["kv"] * D, H), "self_attn.o_proj": (H, cfg["heads"] * D),
              "mlp.gate_proj": (I, H), "mlp.up_proj": (I, H), "mlp.down_proj": (H, I)}
    weights = {f"{n}.weight": torch.randn(s, generator=g) * 0.1 for n, s in shapes.items()}
    weights["input_layernorm.weight"] = 1 + 0.1 * torch.randn(H, generator=g)
    weights["post_attention_layernorm.weight"] = 1 + 0.1 * torch.randn(H, generator=g)
    if qk_norm:
        weights["self_attn.q_norm.weight"] = 1 + 0.1 * torch.randn(D, generator=g)
        weights["self_attn.k_norm.weight"] = 1 + 0.1 * torch.randn(D, generator=g)
    loras = {n: L.Lora(n, torch.randn(4, s[1], generator=g) * 0.1,
                       torch.randn(s[0], 4, generator=g) * 0.1, alpha=8.0) for n, s in shapes.items()}
    hidden = torch.randn(B, S, H, generator=g)
    dy = torch.randn(B, S, H, generator=g)
    return cfg, weights, loras, hidden.to(dtype), dy.to(dtype)


@pytest.mark.parametrize("family", ["llama", "qwen3"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dense_block_matches_transformers_layer(dtype, family):
    """Llama, and Qwen3 with per-head q/k RMSNorm (qk_norm)."""
    qk = family == "qwen3"
    cfg, weights, loras, hidden, dy = _setup(dtype, qk_norm=qk)
    B, S = hidden.shape[:2]
    layer, wrapped, rot = _hf_layer(cfg, weights, loras, dtype, family)
    pos = torch.arange(S)[None].expand(B, -1)
    cos, sin = rot(hidden, pos)
    cos, sin = cos.to(dtype), sin.to(dtype)
    mask = L.causal_mask(B, S, dtype)
    h = hidden.clone().requires_grad_(True)
    ref = layer(h, attention_mask=mask, position_ids=pos, position_embeddings=(cos, sin))
    ref = ref[0] if isinstance(ref, tuple) else ref
    ref.backward(dy)

    ours_rot = L.rotary(B, S, cfg["D"], cfg["theta"], dtype)
    tol = dict(rtol=2e-5, atol=2e-6) if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-3)
    torch.testing.assert_close(ours_rot[0], cos, **tol)
    torch.testing.assert_close(ours_rot[1], sin, **tol)
    w = {k: v.to(dtype) for k, v in weights.items()}
    kw = dict(heads=cfg["heads"], kv_heads=cfg["kv"], head_dim=cfg["D"], eps=cfg["eps"],
              qk_norm=qk)
    out, gh = L.streaming_step(hidden, ours_rot, mask, dy, weights=w, loras=loras, cfg=kw)
    torch.testing.assert_close(out, ref.detach(), **tol)
    torch.testing.assert_close(gh, h.grad, **tol)
    for n, lora in loras.items():
        torch.testing.assert_close(lora.grad_A, wrapped[n].A.grad, **tol)
        torch.testing.assert_close(lora.grad_B, wrapped[n].B.grad, **tol)


def test_lora_linear_vjp_closed_form():
    g = torch.Generator().manual_seed(5)
    M, K, N, r, alpha = 7, 24, 10, 4, 8.0
    x = torch.randn(M, K, generator=g).to(torch.bfloat16)
    W = (torch.randn(N, K, generator=g) * 0.1).to(torch.bfloat16)
    lora = L.Lora("p", torch.randn(r, K, generator=g), torch.randn(N, r, generator=g), alpha)
    xg = x.clone().requires_grad_(True)
    y = L.lora_linear(xg, W, lora)
    dy = torch.randn(M, N, generator=g).to(torch.bfloat16)
    y.backward(dy)
    s = alpha / r
    x64, W64, A64, B64, dy64 = (t.double() for t in (x, W, lora.A.detach(), lora.B.detach(), dy))
    y64 = x64 @ W64.T + s * (x64 @ A64.T) @ B64.T
    torch.testing.assert_close(y.double(), y64, rtol=2e-2, atol=2e-2)
    dT = s * dy64 @ B64
    torch.testing.assert_close(lora.A.grad.double(), dT.T @ x64, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(lora.B.grad.double(), s * dy64.T @ (x64 @ A64.T), rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(xg.grad.double(), dy64 @ W64 + dT @ A64, rtol=2e-2, atol=2e-2)
    # B = 0 reduces to the plain bf16 linear
    zero = L.Lora("p", lora.A, torch.zeros(N, r), alpha)
    assert torch.equal(L.lora_linear(x, W, zero), F.linear(x, W))


def test_terminal_chunked_ce_equals_full_sequence():
    g = torch.Generator().manual_seed(9)
    B, S, H, V = 2, 11, 16, 37
    hidden = torch.randn(B, S, H, generator=g)
    norm = 1 + 0.1 * torch.randn(H, generator=g)
    head = torch.randn(V, H, generator=g) * 0.2
    labels = torch.randint(0, V, (B, S), generator=g)
    labels[0, :4] = -100
    normalization = int((labels[:, 1:] != -100).sum())
    loss, grad = L.causal_lm_terminal(hidden, norm, head, labels, eps=1e-5,
                                      normalization=normalization, token_chunk=3)
    h = hidden.clone().requires_grad_(True)
    logits = F.linear(L.rms(h, norm, 1e-5), head)
    full = F.cross_entropy(logits[:, :-1].reshape(-1, V), labels[:, 1:].reshape(-1),
                           ignore_index=-100, reduction="sum") / normalization
    full.backward()
    assert loss == pytest.approx(float(full), rel=1e-6)
    torch.testing.assert_close(grad, h.grad, rtol=1e-5, atol=1e-6)
    # one chunk covering everything is bit-equal (test_terminal_vjp.py:9-39)
    l1, g1 = L.causal_lm_terminal(hidden, norm, head, labels, eps=1e-5,
                                  normalization=normalization, token_chunk=S)
    assert l1 == pytest.approx(float(full), rel=1e-7)


def test_adamw_matches_torch_optim():
    g = torch.Generator().manual_seed(2)
    p = torch.randn(5, 7, generator=g)
    ref = p.clone().requires_grad_(True)
    opt = torch.optim.AdamW([ref], lr=1e-3, weight_decay=0.1, foreach=False)
    m, v = torch.zeros_like(p), torch.zeros_like(p)
    for step in (1, 2, 3):
        grad = torch.randn(5, 7, generator=g)
        ref.grad = grad.clone()
        opt.step()
        L.adamw_step([(p, grad, m, v)], step=step, lr=1e-3, weight_decay=0.1)
        assert torch.equal(p, ref.detach())
