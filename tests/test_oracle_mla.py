"""Pins oracle/mla.py (the CPU restatement of adapters/deepseek.py:91-176)
against transformers' DeepseekV3DecoderLayer (eager attention and experts)
with LoRA-wrapped projections -- the reference's own harness pattern
(tests/test_dense_adapters.py:49-58) -- and its rotary tables against
DeepseekV3RotaryEmbedding, default and YaRN."""
import pytest
import torch
import torch.nn.functional as F

from oracle import layer as OL
from oracle import mla as OM

LORA_TARGETS = ("self_attn.q_a_proj", "self_attn.q_b_proj", "self_attn.q_proj",
                "self_attn.kv_a_proj_with_mqa", "self_attn.kv_b_proj", "self_attn.o_proj",
                "mlp.shared_experts.gate_proj", "mlp.shared_experts.up_proj",
                "mlp.shared_experts.down_proj")
YARN = {"rope_type": "yarn", "rope_theta": 10000.0, "factor": 4.0,
        "original_max_position_embeddings": 16, "beta_fast": 32.0, "beta_slow": 1.0,
        "mscale": 1.0, "mscale_all_dim": 1.0}


def _config(q_rank, interleave, moe, rope):
    from transformers.models.deepseek_v3.configuration_deepseek_v3 import DeepseekV3Config
    c = DeepseekV3Config(hidden_size=64, intermediate_size=96, moe_intermediate_size=32,
                         num_attention_heads=4, num_key_value_heads=4, q_lora_rank=q_rank,
                         kv_lora_rank=16, qk_nope_head_dim=16, qk_rope_head_dim=8,
                         v_head_dim=12, n_routed_experts=8, n_shared_experts=1, n_group=4,
                         topk_group=2, num_experts_per_tok=2, norm_topk_prob=True,
                         routed_scaling_factor=2.5, first_k_dense_replace=0 if moe else 1,
                         num_hidden_layers=2, vocab_size=32, rope_interleave=interleave,
                         rope_parameters=dict(rope), max_position_embeddings=64,
                         rms_norm_eps=1e-6)
    c._attn_implementation = "eager"
    return c


def _parameters(c, moe):
    return {"heads": c.num_attention_heads, "nope": c.qk_nope_head_dim,
            "rope": c.qk_rope_head_dim, "value": c.v_head_dim, "kv_rank": c.kv_lora_rank,
            "q_rank": c.q_lora_rank, "eps": c.rms_norm_eps,
            "attention_scale": OM.attention_scale(c.qk_nope_head_dim, c.qk_rope_head_dim,
                                                  c.rope_parameters),
            "interleave": c.rope_interleave, "moe": moe, "experts": c.n_routed_experts,
            "groups": c.n_group, "group_k": c.topk_group, "top_k": c.num_experts_per_tok,
            "normalize": c.norm_topk_prob, "router_scale": c.routed_scaling_factor}


class _Projection(torch.nn.Module):
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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("q_rank,interleave,moe,rope", [
    (24, True, True, {"rope_type": "default", "rope_theta": 10000.0}),
    (None, False, False, YARN),
    (24, False, True, YARN),
])
def test_deepseek_block_matches_transformers_layer(dtype, q_rank, interleave, moe, rope):
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import (
        DeepseekV3DecoderLayer, DeepseekV3RotaryEmbedding)
    c = _config(q_rank, interleave, moe, rope)
    g = torch.Generator().manual_seed(17)
    layer = DeepseekV3DecoderLayer(c, 0)   # layer 0: MoE when first_k_dense_replace = 0
    weights = {}
    for k, v in layer.state_dict().items():
        if k.endswith("layernorm.weight"):
            weights[k] = 1 + 0.1 * torch.randn(v.shape, generator=g)
        elif k.endswith("e_score_correction_bias"):
            weights[k] = 0.05 * torch.randn(v.shape, generator=g)
        else:
            weights[k] = 0.1 * torch.randn(v.shape, generator=g)
    layer = layer.to(dtype)
    layer.load_state_dict({k: v.to(dtype) for k, v in weights.items()}, strict=True)
    layer.requires_grad_(False)
    loras, wrapped = {}, {}
    for name in LORA_TARGETS:
        if name + ".weight" not in weights:
            continue
        out_f, in_f = weights[name + ".weight"].shape
        loras[name] = OL.Lora(name, torch.randn(4, in_f, generator=g) * 0.1,
                              torch.randn(out_f, 4, generator=g) * 0.1, alpha=8.0)
        parent, leaf = name.rsplit(".", 1)
        mod = layer.get_submodule(parent)
        wrapped[name] = _Projection(getattr(mod, leaf), loras[name])
        setattr(mod, leaf, wrapped[name])
    B, S = 2, 11
    hidden = torch.randn(B, S, c.hidden_size, generator=g).to(dtype)
    dy = torch.randn(B, S, c.hidden_size, generator=g).to(dtype)
    pos = torch.arange(S)[None].expand(B, -1)
    cos, sin = DeepseekV3RotaryEmbedding(c)(hidden, pos)
    cos, sin = cos.to(dtype), sin.to(dtype)
    mask = OL.causal_mask(B, S, dtype)
    h = hidden.clone().requires_grad_(True)
    ref = layer(h, attention_mask=mask, position_ids=pos, position_embeddings=(cos, sin))
    ref = ref[0] if isinstance(ref, tuple) else ref
    ref.backward(dy)

    tol = dict(rtol=2e-5, atol=2e-6) if dtype == torch.float32 else dict(rtol=2e-2, atol=4e-3)
    ours = OM.rotary(B, S, c.rope_parameters, c.qk_rope_head_dim, dtype)
    torch.testing.assert_close(ours[0], cos, **tol)
    torch.testing.assert_close(ours[1], sin, **tol)

    def close(a, b, elementwise=True):
        if dtype == torch.float32:
            torch.testing.assert_close(a, b, **tol)
            return
        # bf16: the MoE tolerance of the reference's own harness
        # (tests/test_qwen3_moe.py:59-62): rtol .03 plus a relative-L2 bound;
        # adapter gradients (sums over every token of bf16 intermediates):
        # relative L2 and cosine
        a, b = a.double().flatten(), b.double().flatten()
        assert ((a - b).norm() / b.norm()).item() < 1e-2
        if elementwise:
            torch.testing.assert_close(a, b, rtol=3e-2, atol=1e-2)
        else:
            assert (a @ b / (a.norm() * b.norm())).item() > 0.9999
    w = {k: v.to(dtype) for k, v in weights.items()}
    w["mlp.gate.weight"] = weights["mlp.gate.weight"].to(dtype).float() if moe else None
    w = {k: v for k, v in w.items() if v is not None}
    out, gh = OM.streaming_step(hidden, ours, mask, dy, parameters=_parameters(c, moe),
                                weights=w, loras=loras)
    close(out, ref.detach())
    close(gh, h.grad)
    for n, lora in loras.items():
        close(lora.grad_A, wrapped[n].A.grad, elementwise=False)
        close(lora.grad_B, wrapped[n].B.grad, elementwise=False)


def test_yarn_attention_scale_and_amplitude():
    """deepseek.py:91-112,205-206 against transformers' YaRN helpers: the
    amplitude of the rotary tables and the softmax scale."""
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3Attention
    c = _config(24, True, True, YARN)
    attn = DeepseekV3Attention(c, 0)
    assert OM.attention_scale(16, 8, c.rope_parameters) == pytest.approx(attn.scaling, rel=1e-7)
    inv, amp = OM.rope_parameters(c.rope_parameters, 8)
    assert amp == pytest.approx(1.0)          # mscale == mscale_all_dim
    default = OM.rope_parameters({"rope_type": "default", "rope_theta": 10000.0}, 8)
    assert torch.equal(default[0], 1.0 / 10000.0 ** (torch.arange(0, 8, 2).float() / 8))


def test_block_rows_equals_the_whole_block_on_its_rows():
    """oracle.mla.deepseek_block_rows (the MoE evaluated on a subset of rows,
    only the experts those rows hit stacked): output equal to the whole
    block's on those rows, and every gradient (input and each LoRA) equal to
    the whole block's under an upstream gradient that is zero off the rows."""
    torch.manual_seed(0)
    H, I, E, S, heads = 64, 32, 8, 24, 4
    c = {"heads": heads, "nope": 16, "rope": 8, "value": 12, "kv_rank": 16, "q_rank": 24,
         "eps": 1e-6, "attention_scale": 0.2, "interleave": True, "moe": True, "experts": E,
         "groups": 4, "group_k": 2, "top_k": 2, "normalize": True, "router_scale": 2.5}
    mats = {"self_attn.q_a_proj": (24, H), "self_attn.q_b_proj": (heads * 24, 24),
            "self_attn.kv_a_proj_with_mqa": (16 + 8, H), "self_attn.kv_b_proj": (heads * 28, 16),
            "self_attn.o_proj": (H, heads * 12), "mlp.shared_experts.gate_proj": (I, H),
            "mlp.shared_experts.up_proj": (I, H), "mlp.shared_experts.down_proj": (H, I)}
    w = {f"{n}.weight": (torch.randn(s) * 0.1)for n, s in mats.items()}
    for n, d in (("input_layernorm", H), ("post_attention_layernorm", H),
                 ("self_attn.q_a_layernorm", 24), ("self_attn.kv_a_layernorm", 16)):
        w[f"{n}.weight"] = 1 + 0.05 * torch.randn(d, dtype=torch.float32)
    w["mlp.gate.weight"] = torch.randn(E, H, dtype=torch.float32) * 0.3
    w["mlp.gate.e_score_correction_bias"] = torch.randn(E, dtype=torch.float32) * 0.05
    w["mlp.experts.gate_up_proj"] = torch.randn(E, 2 * I, H, dtype=torch.float32) * 0.1
    w["mlp.experts.down_proj"] = torch.randn(E, H, I, dtype=torch.float32) * 0.1
    loras = {n: OL.Lora(n, torch.randn(4, s[1]) * 0.1, torch.randn(s[0], 4) * 0.1, 8.0)
             for n, s in mats.items()}
    hidden = torch.randn(1, S, H, dtype=torch.float32)
    rot = OM.rotary(1, S, {"rope_type": "default", "rope_theta": 10000.0}, 8, torch.float32)
    mask = OL.causal_mask(1, S, torch.float32)
    rows = torch.tensor([2, 9, 10, 23])
    dy = torch.zeros(1, S, H, dtype=torch.float32)
    dy[0, rows] = torch.randn(len(rows), H, dtype=torch.float32)
    leaves = [t for lo in loras.values() for t in (lo.A, lo.B)]
    h1 = hidden.clone().requires_grad_(True)
    with torch.no_grad():
        x = OM.pre_moe_hidden(hidden, rot, mask, parameters=c, weights=w, loras=loras)
        from oracle import moe as OMoE
        _, _, idx = OMoE.deepseek_route(x, w["mlp.gate.weight"], w["mlp.gate.e_score_correction_bias"],
                                        groups=4, group_k=2, top_k=2, normalize=True, scale=2.5)
    whole = OM.deepseek_block(h1, rot, mask, parameters=c, weights=w, loras=loras, indices=idx)
    g1 = torch.autograd.grad(whole, [h1] + leaves, dy)
    hit = torch.unique(idx[rows]).tolist()
    sub = dict(w, **{"mlp.experts.gate_up_proj": w["mlp.experts.gate_up_proj"][hit],
                     "mlp.experts.down_proj": w["mlp.experts.down_proj"][hit]})
    h2 = hidden.clone().requires_grad_(True)
    part = OM.deepseek_block_rows(h2, rot, mask, parameters=c, weights=sub, loras=loras,
                                  rows=rows, indices=idx[rows], experts=hit)
    g2 = torch.autograd.grad(part, [h2] + leaves, dy[0, rows])
    # fp32 throughout: only the BLAS blocking of fewer rows differs
    torch.testing.assert_close(part, whole[0, rows], rtol=1e-5, atol=1e-6)
    for a, b in zip(g1, g2):
        torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-6)
