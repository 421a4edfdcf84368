"""The benchmark workloads at their real shapes on the HIP path, against the
CPU oracle (north-star criteria: outputs rel. err <= 2e-2, gradients cosine
>= 0.999, loss curves within 1e-2).

* config 2 -- one Llama-3-8B-shape layer step at 1 x 2048 tokens, nf4-g128,
  LoRA r=16 on all seven projections, compared whole with the oracle's
  streaming step;
* config 3 -- four Qwen3-8B-shape layers (qk_norm, 32/8 heads,
  intermediate 12288) at 4096 tokens streamed through two slots (so slots
  are overwritten within each phase), the vocabulary-151936 terminal inside
  every microbatch, layer-major window with gradient accumulation 4, two
  optimizer steps, against the oracle's training loop;
* config 4 -- the Qwen3-MoE-30B-A3B-shape feed-forward at 128 experts x 4096
  tokens with per-expert LoRA;
* config 5 -- the DeepSeek-V3-shape MoE feed-forward (256 experts of
  [2 x 2048, 7168] + [7168, 2048], sigmoid group-limited routing on an fp32
  router, shared expert with LoRA) at 2048 tokens, checked on 32 tokens
  spread over the sequence (at least 128 distinct experts, including ones
  whose packed gate|up lies past 2 GiB of the stack); the whole composed
  config-5 layer (MLA + MoE) is test_gpu_mla.py.

For the MoE layers the GPU runs the whole workload (every expert, ragged
row counts); the oracle checks a subset of tokens.  Each token's output and
input gradient depend only on that token's picks, so with the upstream
gradient nonzero only on the checked tokens every gradient the GPU returns
(input and LoRA) is the oracle's over the subset.  Router picks are checked
for every token, exactly, against the oracle's selection rule applied to the
GPU's own logits, and those logits against the oracle's.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import layer as OL
from oracle import moe as OM
from spilltune_amd import _lib, engine, moe, ops, slots

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def _cos(a, b):
    a, b = a.detach().double().flatten().cpu(), b.detach().double().flatten().cpu()
    return float(a @ b / (a.norm() * b.norm()).clamp_min(1e-300))


def _bits_to_bf16(bits, shape):
    return torch.from_numpy(np.asarray(bits, dtype=np.uint16).astype(np.int16)).view(BF).view(shape)


# ------------------------------------------------------------------ config 2
@pytest.mark.timeout(600)
def test_config2_llama8b_layer_step_2048_tokens(oracle_codec):
    from tests.test_gpu_layer import _assert, run_case
    cfg = dict(H=4096, I=14336, heads=32, kv=8, D=128, eps=1e-5, r=16, alpha=32.0, B=1, S=2048)
    res = run_case(cfg, 2048, oracle_codec)
    print({k: round(v, 6) for k, v in res.items()}, flush=True)
    _assert(res)


# ------------------------------------------------------------------ config 3
QWEN3_8B = dict(H=4096, I=12288, heads=32, kv=8, D=128, eps=1e-6, r=16, alpha=32.0,
                theta=1000000.0)


def _qwen3_layers(g, n):
    H, I, D, heads, kv = (QWEN3_8B[k] for k in ("H", "I", "D", "heads", "kv"))
    shapes = {"self_attn.q_proj": (heads * D, H), "self_attn.k_proj": (kv * D, H),
              "self_attn.v_proj": (kv * D, H), "self_attn.o_proj": (H, heads * D),
              "mlp.gate_proj": (I, H), "mlp.up_proj": (I, H), "mlp.down_proj": (H, I)}
    layers = []
    for _ in range(n):
        w = {f"{p}.weight": (torch.randn(s, generator=g) * 0.02).to(BF) for p, s in shapes.items()}
        for nm in ("input_layernorm.weight", "post_attention_layernorm.weight"):
            w[nm] = (1 + 0.05 * torch.randn(H, generator=g)).to(BF)
        w["self_attn.q_norm.weight"] = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
        w["self_attn.k_norm.weight"] = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
        layers.append(w)
    return layers


@pytest.mark.timeout(900)
def test_config3_qwen3_8b_streamed_layer_major_accumulation4(oracle_codec):
    from tests.test_gpu_train import decoded
    g = torch.Generator().manual_seed(3)
    c = QWEN3_8B
    V, S, n_layers, acc, steps, lr = 151936, 4096, 4, 4, 2, 1e-3
    layers = _qwen3_layers(g, n_layers)
    emb = (torch.randn(V, c["H"], generator=g) * 0.5).to(BF)
    norm = (1 + 0.05 * torch.randn(c["H"], generator=g)).to(BF)
    head = (torch.randn(V, c["H"], generator=g) * 0.02).to(BF)
    dev = torch.device("cuda:0")
    model = engine.DenseModel(embedding=emb, norm=norm, head=head, layers=layers,
                              heads=c["heads"], kv_heads=c["kv"], head_dim=c["D"], eps=c["eps"],
                              theta=c["theta"], rank=c["r"], alpha=c["alpha"],
                              targets=OL.PROJECTIONS, device=dev, qk_norm=True)
    oracle_loras = []
    with torch.no_grad():
        for block in model.blocks:
            lo = {}
            for name in sorted(block.adapters):
                p = block.adapters[name]
                A = torch.randn(p.A.shape, generator=g) * 0.02
                B = torch.randn(p.B.shape, generator=g) * 0.02
                p.A.copy_(A)
                p.B.copy_(B)
                lo[name] = OL.Lora(name, A, B, p.alpha)
            oracle_loras.append(lo)
    gd = torch.Generator().manual_seed(7)
    rows = []
    for _ in range(acc):
        ids = torch.randint(0, V, (1, S), generator=gd)
        rows.append((ids, ids.clone()))
    session = slots.Q4SlotSession(model.blocks, dev, host_budget_bytes=1 << 36,
                                  device_budget_bytes=1 << 36, slots=2)
    gpu = engine.train(model, session, rows, steps=steps, accumulation=acc, lr=lr,
                       token_chunk=1024, layer_major=True)
    loads = session.reloads
    session.close()
    print(f"gpu losses {gpu}, layer loads {loads}", flush=True)
    oracle_layers = [decoded(b, oracle_codec) for b in model.blocks]
    cfg = dict(heads=c["heads"], kv_heads=c["kv"], head_dim=c["D"], eps=c["eps"], qk_norm=True)
    cpu = OL.train_reference(emb, norm, head, oracle_layers, oracle_loras, rows, cfg=cfg,
                             theta=c["theta"], steps=steps, lr=lr, token_chunk=1024,
                             accumulation=acc)
    print(f"cpu losses {cpu}", flush=True)
    diff = np.abs(np.array(gpu) - np.array(cpu))
    assert diff.max() <= 1e-2, (gpu, cpu)
    # layer-major: each layer loaded once per phase per window, not per microbatch
    assert loads == steps * 2 * n_layers, loads
    # the second step's accumulated adapter gradients (taken after one AdamW
    # update on both sides) agree with the oracle's
    for block, lo in zip(model.blocks, oracle_loras):
        for name, p in block.adapters.items():
            assert _cos(p.grad_A, lo[name].A.grad) > 0.999, (block.index, name, "A")
            assert _cos(p.grad_B, lo[name].B.grad) > 0.999, (block.index, name, "B")


# ------------------------------------------------------------------ MoE helpers
def _random_experts(E, N, K, dev, gen):
    """Packed nf4-g128 experts [E, N, K] drawn on the device: random codes,
    absmax uniform in [0.01, 0.05) (the cost and layout do not depend on the
    values; the oracle decodes the same bytes)."""
    payload = torch.randint(0, 256, (E * N * K // 2,), dtype=torch.uint8, device=dev,
                            generator=gen)
    scales = torch.rand(E * N * K // 128, device=dev, generator=gen) * 0.04 + 0.01
    return moe.Q4Experts(payload, scales, E, N, K, "nf4-g128")


def _decode_experts(oc, q: moe.Q4Experts, experts):
    """bf16 [len(experts), N, K] of the given experts, decoded by the oracle."""
    N, K = q.out_features, q.in_features
    pe, se = N * K // 2, N * K // 128
    out = torch.empty(len(experts), N, K, dtype=BF)
    for i, e in enumerate(experts):
        p = q.payload[e * pe:(e + 1) * pe].cpu().numpy()
        s = q.scales[e * se:(e + 1) * se].cpu().numpy()
        out[i] = _bits_to_bf16(oc.decode4(p, s, N * K, lut=oc.NF4_LUT), (N, K))
    return out


def _compact(idx_sub, E):
    """Hit experts of the checked tokens (ascending) and the picks renumbered
    into them: the ascending order, and so the combine order, is kept."""
    hit = torch.unique(idx_sub).tolist()
    remap = torch.full((E,), -1, dtype=torch.long)
    remap[torch.tensor(hit)] = torch.arange(len(hit))
    return hit, remap[idx_sub]


# ------------------------------------------------------------------ config 4
@pytest.mark.timeout(900)
def test_config4_qwen3_moe_128_experts_4096_tokens(dev, oracle_codec):
    T, H, I, E, k, r = 4096, 2048, 768, 128, 8, 8
    g = torch.Generator().manual_seed(4)
    gd = torch.Generator(device=dev).manual_seed(4)
    router = (torch.randn(E, H, generator=g) * H ** -0.5).to(BF)    # logits ~ N(0, 1)
    qgu = _random_experts(E, 2 * I, H, dev, gd)
    qd = _random_experts(E, H, I, dev, gd)
    lgu = moe.make_expert_lora("mlp.experts.gate_up_proj", E, H, 2 * I, rank=r, alpha=16.0,
                               device=dev, segments=2, generator=g, b_std=0.02)
    ld = moe.make_expert_lora("mlp.experts.down_proj", E, I, H, rank=r, alpha=16.0, device=dev,
                              generator=g, b_std=0.02)
    flat = torch.randn(T, H, generator=g).to(BF)
    check = torch.arange(0, T, 16)                     # 256 checked tokens
    dout = torch.zeros(T, H, dtype=BF)
    dout[check] = torch.randn(len(check), H, generator=g).to(BF)
    weights = {"mlp.gate.weight": router.to(dev), "mlp.experts.gate_up_proj": qgu,
               "mlp.experts.down_proj": qd}
    xd = flat.to(dev).requires_grad_(True)
    out, w, idx = moe.moe_feed_forward(xd, weights, num_experts=E, top_k=k, norm_topk_prob=True,
                                       lora_gate_up=lgu, lora_down=ld, return_routing=True)
    out.backward(dout.to(dev))
    gpu_logits = ops.linear_bf16(flat.to(dev), router.to(dev)).cpu()   # the router GEMM alone
    torch.cuda.synchronize()
    idx_c = idx.cpu().long()
    counts = torch.bincount(idx_c.flatten(), minlength=E)
    print(f"rows per expert min {int(counts.min())} max {int(counts.max())}", flush=True)
    # router: logits within one bf16 ulp of the oracle's (plus the fp32
    # summation-order error for logits near zero), picks exactly the oracle's
    # selection rule on the GPU's logits, for every token
    cpu_logits = F.linear(flat, router)
    diff = (gpu_logits.float() - cpu_logits.float()).abs()
    assert (diff <= cpu_logits.float().abs() * 2 ** -7 + 1e-5).all()
    assert (diff == 0).float().mean() > 0.99
    _, sel = OM.topk_lowest_index(F.softmax(gpu_logits.float(), -1), k)
    assert torch.equal(idx_c, sel)
    # oracle on the checked tokens, on the GPU's picks
    hit, local = _compact(idx_c[check], E)
    Wgu, Wd = _decode_experts(oracle_codec, qgu, hit), _decode_experts(oracle_codec, qd, hit)
    x = flat[check].clone().requires_grad_(True)
    _, routing = OM.qwen3_route_given(x, router, idx_c[check], norm_topk_prob=True)
    leaves = [t.detach().cpu()[hit].clone().requires_grad_(True)
              for t in (lgu.A, lgu.B, ld.A, ld.B)]
    loras = {"gate": (leaves[0][:, :r], leaves[1][:, :I], lgu.scale),
             "up": (leaves[0][:, r:], leaves[1][:, I:], lgu.scale),
             "down": (leaves[2], leaves[3], ld.scale)}
    ref = OM.expert_loop(x, routing, local, Wgu, Wd, num_experts=len(hit), loras=loras)
    ref.backward(dout[check])
    assert _rel(out[check.to(dev)], ref) < 2e-2, "output"
    assert _cos(xd.grad[check.to(dev)], x.grad) > 0.999, "input grad"
    unchecked = torch.ones(T, dtype=torch.bool)
    unchecked[check] = False
    assert float(xd.grad.cpu()[unchecked].float().abs().max()) == 0.0
    hit_t = torch.tensor(hit)
    for got, leaf, name in ((lgu.A.grad, leaves[0], "A_gu"), (lgu.B.grad, leaves[1], "B_gu"),
                            (ld.A.grad, leaves[2], "A_d"), (ld.B.grad, leaves[3], "B_d")):
        assert _cos(got.cpu()[hit_t], leaf.grad) > 0.999, name
        others = torch.ones(E, dtype=torch.bool)
        others[hit_t] = False
        assert float(got.cpu()[others].abs().sum()) == 0.0, name   # experts the subset never hit


# ------------------------------------------------------------------ config 5
class _SharedLora:
    def __init__(self, g, r, fin, fout, alpha, dev):
        self.rank, self.scale = r, alpha / r
        self.A = (torch.randn(r, fin, generator=g) * 0.02).to(dev).requires_grad_(True)
        self.B = (torch.randn(fout, r, generator=g) * 0.02).to(dev).requires_grad_(True)


@pytest.mark.timeout(900)
def test_config5_deepseek_moe_256_experts_2048_tokens(dev, oracle_codec):
    T, H, I, E, groups, group_k, k, r, scale = 2048, 7168, 2048, 256, 8, 4, 8, 8, 2.5
    g = torch.Generator().manual_seed(5)
    gd = torch.Generator(device=dev).manual_seed(5)
    # fp32 router as the reference keeps it (storage.py:124), values not bf16-representable
    router = torch.randn(E, H, generator=g) * H ** -0.5
    assert not torch.equal(router, router.to(BF).float())
    bias = torch.randn(E, generator=g) * 0.05
    qgu = _random_experts(E, 2 * I, H, dev, gd)        # 3.76 GB of packed gate|up
    qd = _random_experts(E, H, I, dev, gd)
    # shared expert: gate and up adjacent in one buffer (one fused GEMM), down apart
    qsgu = _random_experts(2, I, H, dev, gd)
    qsd = _random_experts(1, H, I, dev, gd)
    half_p, half_s = I * H // 2, I * H // 128
    shared = {"mlp.shared_experts.gate_proj.weight":
              ops.Q4Weight(qsgu.payload[:half_p], qsgu.scales[:half_s], (I, H), "nf4-g128"),
              "mlp.shared_experts.up_proj.weight":
              ops.Q4Weight(qsgu.payload[half_p:], qsgu.scales[half_s:], (I, H), "nf4-g128"),
              "mlp.shared_experts.down_proj.weight":
              ops.Q4Weight(qsd.payload, qsd.scales, (H, I), "nf4-g128")}
    assert ops.concat_rows([shared["mlp.shared_experts.gate_proj.weight"],
                            shared["mlp.shared_experts.up_proj.weight"]]) is not None
    ls = {"gate": _SharedLora(g, r, H, I, 16.0, dev), "up": _SharedLora(g, r, H, I, 16.0, dev),
          "down": _SharedLora(g, r, I, H, 16.0, dev)}
    flat = torch.randn(T, H, generator=g).to(BF)
    check = torch.arange(3, T, 64)                     # 32 checked tokens
    dout = torch.zeros(T, H, dtype=BF)
    dout[check] = torch.randn(len(check), H, generator=g).to(BF)
    weights = {"mlp.gate.weight": router.to(dev), "mlp.gate.e_score_correction_bias": bias.to(dev),
               "mlp.experts.gate_up_proj": qgu, "mlp.experts.down_proj": qd, **shared}
    xd = flat.to(dev).requires_grad_(True)
    out, w, idx = moe.deepseek_moe_feed_forward(
        xd, weights, num_experts=E, top_k=k, groups=groups, group_k=group_k, normalize=True,
        scale=scale, lora_shared=ls, return_routing=True)
    out.backward(dout.to(dev))
    gpu_logits = moe.sigmoid_router_logits(flat.to(dev), router.to(dev)).cpu()
    torch.cuda.synchronize()
    idx_c = idx.cpu().long()
    counts = torch.bincount(idx_c.flatten(), minlength=E)
    print(f"rows per expert min {int(counts.min())} max {int(counts.max())}", flush=True)
    # router: fp32 logits against the oracle's fp32 F.linear; the picks are the
    # oracle's selection on the GPU's logits for every token (as sets: the
    # reference's topk(sorted=False) leaves the order open), weights to fp32
    cpu_logits = F.linear(flat.float(), router)
    assert _rel(gpu_logits, cpu_logits) < 1e-6
    _, wsel, sel = OM.deepseek_select(gpu_logits, bias, groups=groups, group_k=group_k,
                                      top_k=k, normalize=True, scale=scale)
    assert torch.equal(idx_c.sort(1)[0], sel.sort(1)[0])
    _, _, sel_cpu = OM.deepseek_select(cpu_logits, bias, groups=groups, group_k=group_k,
                                       top_k=k, normalize=True, scale=scale)
    same = (idx_c.sort(1)[0] == sel_cpu.sort(1)[0]).all(1)
    assert int((~same).sum()) <= 2, int((~same).sum())    # near-ties of fp32 summation order
    x = flat[check].clone().requires_grad_(True)
    logits = F.linear(x.float(), router)
    routing = OM.deepseek_weights_given(logits, idx_c[check], normalize=True, scale=scale)
    torch.testing.assert_close(w.cpu()[check], routing.detach(), rtol=1e-5, atol=1e-6)
    hit, local = _compact(idx_c[check], E)
    print(f"experts hit by the checked tokens: {len(hit)}, highest {max(hit)}", flush=True)
    # packed gate|up of expert e starts at e * 2I*H/2 bytes: past 2 GiB from e = 147
    assert len(hit) >= 128 and max(hit) * (2 * I * H // 2) >= 1 << 31
    Wgu, Wd = _decode_experts(oracle_codec, qgu, hit), _decode_experts(oracle_codec, qd, hit)
    routed = OM.expert_loop(x, routing, local, Wgu, Wd, num_experts=len(hit))
    Ws = [*_decode_experts(oracle_codec, qsgu, [0, 1]), _decode_experts(oracle_codec, qsd, [0])[0]]
    sl = {n: OL.Lora(n, l.A.detach().cpu(), l.B.detach().cpu(), 16.0) for n, l in ls.items()}
    act = F.silu(OL.lora_linear(x, Ws[0], sl["gate"])) * OL.lora_linear(x, Ws[1], sl["up"])
    ref = routed + OL.lora_linear(act, Ws[2], sl["down"])
    ref.backward(dout[check])
    cd = check.to(dev)
    assert _rel(out[cd], ref) < 2e-2, "output"
    assert _cos(xd.grad[cd], x.grad) > 0.999, "input grad"
    for n in ("gate", "up", "down"):
        assert _cos(ls[n].A.grad, sl[n].A.grad) > 0.999, f"shared {n} A"
        assert _cos(ls[n].B.grad, sl[n].B.grad) > 0.999, f"shared {n} B"


@pytest.mark.parametrize("E,groups,group_k", [(96, 8, 4), (256, 8, 4)])
def test_deepseek_router_slices_fp32_router(dev, E, groups, group_k):
    """Router logits over more than one 64-expert slice (E = 96: a partial
    last slice) with an fp32 router whose values bf16 cannot hold: logits to
    fp32 accuracy, picks equal the oracle router's selection on them."""
    T, H, k = 64, 128, 8
    g = torch.Generator().manual_seed(E)
    flat = torch.randn(T, H, generator=g).to(BF)
    router = torch.randn(E, H, generator=g) * 0.3
    bias = torch.randn(E, generator=g) * 0.05
    got = moe.sigmoid_router_logits(flat.to(dev), router.to(dev)).cpu()
    ref = F.linear(flat.double(), router.double())
    assert ((got.double() - ref).abs() <= 1e-5 * ref.abs().max()).all()
    w = torch.empty(T, k, device=dev)
    idx = torch.empty(T, k, dtype=torch.int32, device=dev)
    gl, bd = got.to(dev), bias.to(dev)
    _lib.call("st_moe_route_sigmoid", _lib.ptr(gl), _lib.ptr(bd), T, E, groups, group_k, k, 1,
              2.5, _lib.ptr(w), _lib.ptr(idx), _lib.stream_handle(dev))
    torch.cuda.synchronize()
    _, _, sel = OM.deepseek_select(got, bias, groups=groups, group_k=group_k, top_k=k,
                                   normalize=True, scale=2.5)
    assert torch.equal(idx.cpu().long().sort(1)[0], sel.sort(1)[0])
    _, wref, iref = OM.deepseek_route(flat, router, bias, groups=groups, group_k=group_k,
                                      top_k=k, normalize=True, scale=2.5)
    assert torch.equal(idx.cpu().long().sort(1)[0], iref.sort(1)[0])
    order_g, order_r = idx.cpu().long().argsort(1), iref.argsort(1)
    torch.testing.assert_close(w.cpu().gather(1, order_g), wref.gather(1, order_r), rtol=1e-5,
                               atol=1e-6)
