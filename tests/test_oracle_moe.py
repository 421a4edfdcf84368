"""Pins oracle/moe.py (the CPU restatement of the reference's MoE feed-forward
and routers) against transformers' own Qwen3-MoE block and DeepSeek-V3
router, a float64 closed form for the per-expert LoRA terms, and a
brute-force per-token combine."""
import pytest
import torch
import torch.nn.functional as F

from oracle import moe as M


def _qwen3_block(H, I, E, k, norm, dtype, g):
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock
    cfg = Qwen3MoeConfig(hidden_size=H, moe_intermediate_size=I, num_experts=E,
                         num_experts_per_tok=k, norm_topk_prob=norm, num_hidden_layers=1,
                         vocab_size=32)
    cfg._experts_implementation = "eager"
    block = Qwen3MoeSparseMoeBlock(cfg)
    router = torch.randn(E, H, generator=g) * 0.5
    gate_up = torch.randn(E, 2 * I, H, generator=g) * 0.1
    down = torch.randn(E, H, I, generator=g) * 0.1
    with torch.no_grad():
        block.gate.weight.copy_(router)
        block.experts.gate_up_proj.copy_(gate_up)
        block.experts.down_proj.copy_(down)
    block = block.to(dtype).requires_grad_(False)
    return block, router.to(dtype), gate_up.to(dtype), down.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("k,norm", [(1, False), (2, True), (4, False), (4, True)])
def test_qwen3_ffn_matches_transformers(dtype, k, norm):
    g = torch.Generator().manual_seed(11 + k)
    H, I, E, T = 32, 24, 8, 19
    block, router, gate_up, down = _qwen3_block(H, I, E, k, norm, dtype, g)
    x = torch.randn(1, T, H, generator=g).to(dtype)
    x1 = x.clone().requires_grad_(True)
    x2 = x.clone().requires_grad_(True)
    ours = M.qwen3_moe_ffn(x1, router, gate_up, down, top_k=k, norm_topk_prob=norm)
    ref = block(x2)
    if dtype == torch.float32:
        torch.testing.assert_close(ours, ref, rtol=3e-5, atol=3e-6)
    else:
        torch.testing.assert_close(ours, ref, rtol=0, atol=0)
    dy = torch.randn(ours.shape, generator=g).to(dtype)
    (ga,) = torch.autograd.grad(ours, x1, dy)
    (gb,) = torch.autograd.grad(ref, x2, dy)
    tol = dict(rtol=3e-5, atol=3e-6) if dtype == torch.float32 else dict(rtol=3e-2, atol=2e-3)
    torch.testing.assert_close(ga, gb, **tol)


def test_deepseek_route_matches_transformers():
    from transformers.models.deepseek_v3.configuration_deepseek_v3 import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3TopkRouter
    g = torch.Generator().manual_seed(5)
    H, E, groups, group_k, k, T = 48, 32, 4, 2, 6, 37
    cfg = DeepseekV3Config(hidden_size=H, n_routed_experts=E, n_group=groups,
                           topk_group=group_k, num_experts_per_tok=k, norm_topk_prob=True,
                           routed_scaling_factor=2.5, num_hidden_layers=1, vocab_size=32)
    router = DeepseekV3TopkRouter(cfg)
    w = torch.randn(E, H, generator=g).to(torch.bfloat16)
    bias = torch.randn(E, generator=g) * 0.1
    with torch.no_grad():
        router.weight.copy_(w.float())
        router.e_score_correction_bias.copy_(bias)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits, weights, idx = M.deepseek_route(x, w, bias, groups=groups, group_k=group_k, top_k=k,
                                            normalize=True, scale=2.5)
    rl, rw, ri = (t.detach() for t in router(x))
    torch.testing.assert_close(logits, rl, rtol=1e-6, atol=1e-6)
    ours = {(t, int(e)): float(v) for t in range(T) for e, v in zip(idx[t], weights[t])}
    theirs = {(t, int(e)): float(v) for t in range(T) for e, v in zip(ri[t], rw[t])}
    assert ours.keys() == theirs.keys()
    for key in ours:
        assert ours[key] == pytest.approx(theirs[key], rel=1e-6, abs=1e-7)


def test_expert_lora_terms_match_float64_closed_form():
    g = torch.Generator().manual_seed(3)
    E, H, I, r, rows, s = 3, 16, 12, 4, 7, 2.0
    x = torch.randn(rows, H, generator=g).to(torch.bfloat16)
    W = (torch.randn(E, I, H, generator=g) * 0.2).to(torch.bfloat16)
    A = torch.randn(E, r, H, generator=g).requires_grad_(True)
    B = torch.randn(E, I, r, generator=g).requires_grad_(True)
    e = 1
    y = M.expert_lora_linear(x, W[e], (A, B, s), e)
    base = (x.float() @ W[e].float().T).to(torch.bfloat16).double()
    upd = (x.double() @ A[e].detach().double().T) @ B[e].detach().double().T
    torch.testing.assert_close(y.double(), (base + s * upd).to(torch.bfloat16).double(),
                               rtol=1e-2, atol=1e-2)
    dy = torch.randn(rows, I, generator=g).to(torch.bfloat16)
    ga, gb = torch.autograd.grad(y, (A, B), dy)
    d = dy.double()
    t = x.double() @ A[e].detach().double().T
    torch.testing.assert_close(gb[e].double(), s * d.T @ t, rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(ga[e].double(), s * (d @ B[e].detach().double()).T @ x.double(),
                               rtol=1e-4, atol=1e-4)
    assert ga[0].abs().max() == 0 and gb[2].abs().max() == 0


def test_expert_loop_combine_is_ascending_bf16_sum():
    """The bf16 ``index_add_`` loop equals, per token, a sequential bf16 sum of
    ``bf16(y_e * w)`` in ascending expert order -- the rule the HIP combine
    kernel implements."""
    g = torch.Generator().manual_seed(9)
    H, I, E, T, k = 16, 8, 6, 11, 3
    flat = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gate_up = (torch.randn(E, 2 * I, H, generator=g) * 0.3).to(torch.bfloat16)
    down = (torch.randn(E, H, I, generator=g) * 0.3).to(torch.bfloat16)
    router = (torch.randn(E, H, generator=g)).to(torch.bfloat16)
    _, w, idx = M.qwen3_route(flat, router, top_k=k, norm_topk_prob=True)
    out = M.expert_loop(flat, w, idx, gate_up, down, num_experts=E)
    brute = torch.empty_like(flat)
    for t in range(T):
        acc = torch.zeros(H, dtype=torch.bfloat16)
        for j in sorted(range(k), key=lambda j: int(idx[t, j])):
            e = int(idx[t, j])
            gt, up = F.linear(flat[t:t + 1], gate_up[e]).chunk(2, dim=-1)
            v = F.linear(F.silu(gt) * up, down[e])[0]
            acc = (acc.float() + (v * w[t, j]).float()).to(torch.bfloat16)
        brute[t] = acc
    assert torch.equal(out, brute)


def test_given_pick_routers_match_topk_routers():
    g = torch.Generator().manual_seed(21)
    T, H, E, k = 13, 24, 10, 3
    flat = torch.randn(T, H, generator=g).to(torch.bfloat16)
    router = torch.randn(E, H, generator=g).to(torch.bfloat16)
    for norm in (False, True):
        x1 = flat.clone().requires_grad_(True)
        x2 = flat.clone().requires_grad_(True)
        _, w1, idx = M.qwen3_route(x1, router, top_k=k, norm_topk_prob=norm)
        _, w2 = M.qwen3_route_given(x2, router, idx, norm_topk_prob=norm)
        assert torch.equal(w1, w2)
        dw = torch.randn(T, k, generator=g).to(torch.bfloat16)
        (a,) = torch.autograd.grad(w1, x1, dw)
        (b,) = torch.autograd.grad(w2, x2, dw)
        assert torch.equal(a, b)
    bias = torch.randn(E, generator=g) * 0.1
    x1 = flat.clone().requires_grad_(True)
    logits, w1, idx = M.deepseek_route(x1, router, bias, groups=2, group_k=1, top_k=k,
                                       normalize=True, scale=1.5)
    w2 = M.deepseek_weights_given(logits, idx, normalize=True, scale=1.5)
    assert torch.equal(w1, w2)


def test_topk_lowest_index_matches_brute_force():
    g = torch.Generator().manual_seed(4)
    vals = torch.randint(0, 6, (40, 17), generator=g).float()   # many ties
    v, i = M.topk_lowest_index(vals, 5)
    for row in range(vals.shape[0]):
        brute = sorted(range(17), key=lambda j: (-float(vals[row, j]), j))[:5]
        assert i[row].tolist() == brute
        assert v[row].tolist() == [float(vals[row, j]) for j in brute]
