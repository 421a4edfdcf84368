"""DeepSeek-V3 MLA + MoE decoder layer on the HIP path against the CPU oracle
(oracle/mla.py, pinned to transformers' DeepseekV3DecoderLayer).

* the query/key/value assembly kernel (st_mla_rope_fwd/bwd) against the
  oracle's bf16 rotation and its autograd, both rotation conventions;
* whole layer steps (forward + recompute + backward through the streaming
  driver, weights streamed through two slots) at small shapes, MoE and dense
  layers, with and without q_lora_rank, default and interleaved rotary,
  default and YaRN tables;
* config 5's attention dimensions (hidden 7168, 128 heads, q_lora_rank 1536,
  kv_lora_rank 512, qk 128 + 64, v 128) at 256 tokens with 16 routed experts
  of width 2048;
* the composed config-5 layer at its real size -- 2048 tokens, 256 routed
  experts, shared expert, LoRA -- with the attention checked over every
  token and the MoE on 64 rows spread over the sequence (the upstream
  gradient is zero elsewhere, so every gradient is the whole layer's).
North-star criteria: output rel. err <= 2e-2, every gradient cosine >= 0.999."""
import numpy as np
import pytest
import torch

from oracle import layer as OL
from oracle import mla as OMLA
from spilltune_amd import deepseek, moe, ops, slots
from spilltune_amd.dense import CausalMask
from spilltune_amd.recompute import streaming_block

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
YARN = {"rope_type": "yarn", "rope_theta": 10000.0, "factor": 40.0,
        "original_max_position_embeddings": 4096, "beta_fast": 32, "beta_slow": 1,
        "mscale": 1.0, "mscale_all_dim": 1.0}
DEFAULT = {"rope_type": "default", "rope_theta": 10000.0}


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def _cos(a, b):
    a, b = a.detach().double().flatten().cpu(), b.detach().double().flatten().cpu()
    return float(a @ b / (a.norm() * b.norm()).clamp_min(1e-300))


# ----------------------------------------------------------------- assembly kernel
def _oracle_assembly(q, kv, comp, cos, sin, B, S, H, nope, rope, vdim, kv_rank, interleave):
    """deepseek.py:137-150 on the CPU in bf16 (oracle/mla.py's expressions)."""
    qh = q.view(B, S, H, nope + rope).transpose(1, 2)
    q_pass, q_rot = qh.split([nope, rope], -1)
    kvh = kv.view(B, S, H, nope + vdim).transpose(1, 2)
    k_pass, value = kvh.split([nope, vdim], -1)
    k_rot = comp[:, kv_rank:kv_rank + rope].reshape(B, 1, S, rope)
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)

    def rotate(t):
        if interleave:
            a, b = t[..., 0::2], t[..., 1::2]
            co, si = c[..., :rope // 2], s[..., :rope // 2]
            return torch.cat((a * co - b * si, b * co + a * si), -1)
        first, second = t.chunk(2, -1)
        return t * c + torch.cat((-second, first), -1) * s

    return (torch.cat((q_pass, rotate(q_rot)), -1),
            torch.cat((k_pass, rotate(k_rot).expand_as(q_rot)), -1), value)


@pytest.mark.parametrize("interleave", [True, False])
@pytest.mark.parametrize("B,S,H,nope,rope,vdim", [(1, 40, 4, 128, 64, 128), (2, 24, 3, 48, 16, 64)])
def test_mla_assembly_vs_oracle(dev, interleave, B, S, H, nope, rope, vdim):
    g = torch.Generator().manual_seed(H * 100 + S + interleave)
    kv_rank = 32
    M = B * S
    q = torch.randn(M, H * (nope + rope), generator=g).to(BF)
    kv = torch.randn(M, H * (nope + vdim), generator=g).to(BF)
    wide = torch.randn(M, kv_rank + rope + 24, generator=g).to(BF)   # a column slice, ld != width
    comp = wide[:, :kv_rank + rope]
    cos, sin = OMLA.rotary(B, S, YARN, rope, BF)
    ref = [t.contiguous() for t in _oracle_assembly(q, kv, comp, cos, sin, B, S, H, nope, rope,
                                                    vdim, kv_rank, interleave)]
    qd = q.to(dev).requires_grad_(True)
    kvd = kv.to(dev).requires_grad_(True)
    wd = wide.to(dev).requires_grad_(True)
    Q, K, V = ops.mla_rope(qd, kvd, wd[:, :kv_rank + rope], cos.to(dev), sin.to(dev), batch=B,
                           seq=S, heads=H, nope=nope, rope=rope, v_dim=vdim, kv_rank=kv_rank,
                           interleave=interleave)
    for got, want in zip((Q, K, V), ref):
        assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))
    # VJP against the oracle's autograd
    dQ = torch.randn(Q.shape, generator=g).to(BF)
    dK = torch.randn(K.shape, generator=g).to(BF)
    dV = torch.randn(V.shape, generator=g).to(BF)
    torch.autograd.backward((Q, K, V), (dQ.to(dev), dK.to(dev), dV.to(dev)))
    qc, kvc, wc = (t.clone().requires_grad_(True) for t in (q, kv, wide))
    out = _oracle_assembly(qc, kvc, wc[:, :kv_rank + rope], cos, sin, B, S, H, nope, rope, vdim,
                           kv_rank, interleave)
    torch.autograd.backward(out, (dQ, dK, dV))
    assert torch.equal(qd.grad.cpu().view(torch.int16), qc.grad.view(torch.int16))
    assert torch.equal(kvd.grad.cpu().view(torch.int16), kvc.grad.view(torch.int16))
    got, want = wd.grad.cpu().float(), wc.grad.float()
    assert torch.equal(got[:, :kv_rank], want[:, :kv_rank])          # zeros: no latent path here
    assert torch.equal(got[:, kv_rank + rope:], want[:, kv_rank + rope:])
    # the rope key's gradient sums every head's: fp32 sums in another order
    # round to bf16 at most one ulp apart
    d = (got[:, kv_rank:kv_rank + rope] - want[:, kv_rank:kv_rank + rope]).abs()
    assert (d <= want[:, kv_rank:kv_rank + rope].abs() * 2 ** -7 + 1e-6).all()


# ----------------------------------------------------------------- layer steps
def _layer_weights(g, c, H, I_moe, I_dense, E):
    """HF-named fp32 weights of one DeepSeek-V3 layer (N(0, 0.02) matrices)."""
    heads, nope, rope, vdim = c["heads"], c["nope"], c["rope"], c["value"]
    mats = {"self_attn.kv_a_proj_with_mqa": (c["kv_rank"] + rope, H),
            "self_attn.kv_b_proj": (heads * (nope + vdim), c["kv_rank"]),
            "self_attn.o_proj": (H, heads * vdim)}
    if c["q_rank"] is None:
        mats["self_attn.q_proj"] = (heads * (nope + rope), H)
    else:
        mats["self_attn.q_a_proj"] = (c["q_rank"], H)
        mats["self_attn.q_b_proj"] = (heads * (nope + rope), c["q_rank"])
    if c["moe"]:
        mats.update({"mlp.shared_experts.gate_proj": (I_moe, H),
                     "mlp.shared_experts.up_proj": (I_moe, H),
                     "mlp.shared_experts.down_proj": (H, I_moe)})
    else:
        mats.update({"mlp.gate_proj": (I_dense, H), "mlp.up_proj": (I_dense, H),
                     "mlp.down_proj": (H, I_dense)})
    w = {f"{n}.weight": torch.randn(s, generator=g) * 0.02 for n, s in mats.items()}
    w["input_layernorm.weight"] = 1 + 0.05 * torch.randn(H, generator=g)
    w["post_attention_layernorm.weight"] = 1 + 0.05 * torch.randn(H, generator=g)
    if c["q_rank"] is not None:
        w["self_attn.q_a_layernorm.weight"] = 1 + 0.05 * torch.randn(c["q_rank"], generator=g)
    w["self_attn.kv_a_layernorm.weight"] = 1 + 0.05 * torch.randn(c["kv_rank"], generator=g)
    if c["moe"]:
        # router with well-separated scores (fp32, as the reference keeps it)
        w["mlp.gate.weight"] = torch.randn(E, H, generator=g) * 3 * H ** -0.5
        w["mlp.gate.e_score_correction_bias"] = torch.randn(E, generator=g) * 0.05
        w["mlp.experts.gate_up_proj"] = torch.randn(E, 2 * I_moe, H, generator=g) * 0.02
        w["mlp.experts.down_proj"] = torch.randn(E, H, I_moe, generator=g) * 0.02
    return w


def _oracle_weights(block, oc):
    out = {}
    for name, entry in block.storage_specs.items():
        spec = entry["spec"]
        bits = oc.decode4(block.host_weights[entry["parts"]["payload"]].numpy(),
                          block.host_weights[entry["parts"]["scales"]].numpy(), spec["numel"],
                          lut=oc.NF4_LUT)
        out[name] = torch.from_numpy(np.asarray(bits, dtype=np.uint16).astype(np.int16)).view(
            BF).view(spec["shape"])
    for k, v in block.host_weights.items():
        if not k.startswith("@"):
            out[k] = v
    return out


def run_layer(c, *, H, I_moe=128, I_dense=256, E=16, S=64, B=1, seed=0, oracle_codec,
              streamed=True, shared_lora=True, monkeypatch=None):
    g = torch.Generator().manual_seed(seed)
    w = _layer_weights(g, c, H, I_moe, I_dense, E)
    dev = torch.device("cuda:0")
    block = deepseek.make_deepseek_block(0, w, codec="nf4-g128", parameters=c, rank=8, alpha=16.0,
                                         device=dev, shared_lora=shared_lora, generator=g)
    with torch.no_grad():
        for p in block.adapters.values():
            p.B.copy_(torch.randn(p.B.shape, generator=g) * 0.02)
    hidden = torch.randn(B, S, H, generator=g).to(BF)
    dy = torch.randn(B, S, H, generator=g).to(BF)
    rope_cfg = c["rope_cfg"]
    cos, sin = OMLA.rotary(B, S, rope_cfg, c["rope"], BF)
    lor = {n: OL.Lora(n, p.A.detach().cpu(), p.B.detach().cpu(), p.alpha)
           for n, p in block.adapters.items()}
    # the device path's expert picks (recorded from its MoE feed-forward)
    picks = []
    if c["moe"] and monkeypatch is not None:
        real = moe.deepseek_moe_feed_forward

        def recording(*args, **kwargs):
            out, _, idx = real(*args, return_routing=True, **kwargs)
            picks.append(idx.detach().cpu().long())
            return out
        monkeypatch.setattr(moe, "deepseek_moe_feed_forward", recording)
    # HIP path
    if streamed:
        session = slots.Q4SlotSession([block], dev, host_budget_bytes=1 << 40,
                                      device_budget_bytes=1 << 40, slots=2)
    else:
        session = slots.ResidentSession([block], dev)
    (dcos, dsin), mask = deepseek.positions_and_masks(torch.ones(B, S, dtype=torch.bool),
                                                      rope=rope_cfg, rope_dim=c["rope"],
                                                      device=dev)
    # the device-built tables agree with the oracle's host tables (device and
    # host cos/sin of large YaRN phases differ in the last fp32 bits, so a few
    # bf16 roundings differ); the step itself takes the oracle's
    for got, want in ((dcos, cos), (dsin, sin)):
        assert _rel(got.float(), want.float()) < 1e-3
    h = hidden.to(dev).requires_grad_(True)
    with session.run():
        out = streaming_block(h, (cos.to(dev), sin.to(dev)), mask, block.functional, block.kwargs,
                              session.reloader(block), block.adapters, block.index)
        out.backward(dy.to(dev))
    torch.cuda.synchronize()
    indices = None
    if picks:
        # forward and recompute pick alike; the oracle router agrees except at
        # near-ties of fp32 summation order, and the oracle runs on these picks
        assert torch.equal(picks[0], picks[-1])
        indices = picks[-1]
    wref = _oracle_weights(block, oracle_codec)
    out_ref, gh_ref = OMLA.streaming_step(hidden, (cos, sin), OL.causal_mask(B, S, BF), dy,
                                          parameters=c, weights=wref, loras=lor, indices=indices)
    if indices is not None:
        with torch.no_grad():
            x = OMLA.pre_moe_hidden(hidden, (cos, sin), OL.causal_mask(B, S, BF), parameters=c,
                                    weights=wref, loras=lor)
            from oracle import moe as OM
            _, _, own = OM.deepseek_route(x, wref["mlp.gate.weight"],
                                          wref["mlp.gate.e_score_correction_bias"],
                                          groups=c["groups"], group_k=c["group_k"],
                                          top_k=c["top_k"], normalize=True, scale=2.5)
        same = (own.sort(1)[0] == indices.sort(1)[0]).all(1).float().mean().item()
        print(f"tokens whose picks equal the oracle router's: {same:.4f}", flush=True)
        assert same >= 0.98
    res = {"out": _rel(out, out_ref), "dh": _cos(h.grad, gh_ref)}
    for n, p in block.adapters.items():
        res[n + ".A"] = _cos(p.grad_A, lor[n].grad_A)
        res[n + ".B"] = _cos(p.grad_B, lor[n].grad_B)
    session.close()
    return res


def _params(*, heads, nope, rope, vdim, kv_rank, q_rank, interleave, moe, rope_cfg, E=16,
            groups=4, group_k=2, top_k=4):
    return {"heads": heads, "nope": nope, "rope": rope, "value": vdim, "kv_rank": kv_rank,
            "q_rank": q_rank, "eps": 1e-6,
            "attention_scale": OMLA.attention_scale(nope, rope, rope_cfg),
            "interleave": interleave, "moe": moe, "experts": E, "groups": groups,
            "group_k": group_k, "top_k": top_k, "normalize": True, "router_scale": 2.5,
            "rope_cfg": rope_cfg}


def _assert(res):
    print({k: round(v, 6) for k, v in res.items()}, flush=True)
    assert res["out"] <= 2e-2, res
    bad = {k: v for k, v in res.items() if k != "out" and v < 0.999}
    assert not bad, bad


@pytest.mark.parametrize("q_rank,interleave,moe,rope_cfg", [
    (128, True, True, YARN),
    (None, False, True, DEFAULT),
    (128, False, False, YARN),
])
def test_deepseek_layer_step_v3_head_dims(oracle_codec, monkeypatch, q_rank, interleave, moe,
                                          rope_cfg):
    """V3 head dims (qk 128 + 64 against v 128) with few heads and experts."""
    c = _params(heads=4, nope=128, rope=64, vdim=128, kv_rank=128, q_rank=q_rank,
                interleave=interleave, moe=moe, rope_cfg=rope_cfg)
    _assert(run_layer(c, H=256, oracle_codec=oracle_codec, seed=11 + (q_rank or 0),
                      monkeypatch=monkeypatch))


@pytest.mark.parametrize("S", [40, 37])
def test_deepseek_layer_step_small_heads_resident(oracle_codec, monkeypatch, S):
    """qk 48 + 16 against v 64 (the 64/64 attention kernel), ragged tokens,
    batch 2, weights resident; S = 37 is no multiple of 8."""
    c = _params(heads=3, nope=48, rope=16, vdim=64, kv_rank=128, q_rank=128, interleave=True,
                moe=True, rope_cfg=DEFAULT, E=8, groups=4, group_k=2, top_k=2)
    _assert(run_layer(c, H=128, E=8, S=S, B=2, oracle_codec=oracle_codec, seed=5,
                      streamed=False, monkeypatch=monkeypatch))


@pytest.mark.timeout(900)
def test_config5_attention_dims_layer_step(oracle_codec, monkeypatch):
    """Config 5's MLA dimensions (hidden 7168, 128 heads, q_lora_rank 1536,
    kv_lora_rank 512, YaRN, interleaved rotary) with 16 routed experts of
    width 2048 (top 8 of 8 groups, best 4) and the shared expert with LoRA."""
    c = _params(heads=128, nope=128, rope=64, vdim=128, kv_rank=512, q_rank=1536,
                interleave=True, moe=True, rope_cfg=YARN, E=16, groups=8, group_k=4, top_k=8)
    _assert(run_layer(c, H=7168, I_moe=2048, E=16, S=256, oracle_codec=oracle_codec, seed=7,
                      monkeypatch=monkeypatch))


@pytest.mark.timeout(1200)
def test_config5_composed_layer_2048_tokens_256_experts(oracle_codec, monkeypatch):
    """Benchmark config 5 whole: one DeepSeek-V3-shape layer (MLA with 128
    heads, q_lora_rank 1536, kv_lora_rank 512, YaRN interleaved rotary; 256
    routed experts of width 2048, top 8 of 8 groups / best 4, shared expert;
    LoRA r=8 on the attention projections and the shared expert) at 2048
    tokens, streamed through a slot, forward + recompute + backward.  The
    4-bit records are random codes and scales written into the pinned image
    (the oracle decodes the same bytes).  The oracle
    (oracle.mla.deepseek_block_rows) runs the attention over all 2048 tokens
    and the MoE on 64 rows spread over the sequence, with only the experts
    those rows hit decoded (at least 64 of them, including experts whose
    packed gate|up lies past 2 GiB of the stack)."""
    from oracle import moe as OMoE
    T, H, I, E = 2048, 7168, 2048, 256
    c = _params(heads=128, nope=128, rope=64, vdim=128, kv_rank=512, q_rank=1536,
                interleave=True, moe=True, rope_cfg=YARN, E=E, groups=8, group_k=4, top_k=8)
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(55)
    heads, nope, rope, v = c["heads"], c["nope"], c["rope"], c["value"]
    mats = {"self_attn.q_a_proj": (c["q_rank"], H),
            "self_attn.q_b_proj": (heads * (nope + rope), c["q_rank"]),
            "self_attn.kv_a_proj_with_mqa": (c["kv_rank"] + rope, H),
            "self_attn.kv_b_proj": (heads * (nope + v), c["kv_rank"]),
            "self_attn.o_proj": (H, heads * v),
            "mlp.experts.gate_up_proj": (E, 2 * I, H), "mlp.experts.down_proj": (E, H, I),
            "mlp.shared_experts.gate_proj": (I, H), "mlp.shared_experts.up_proj": (I, H),
            "mlp.shared_experts.down_proj": (H, I)}
    weights = {}
    for name, shape in mats.items():
        n = int(np.prod(shape))
        key = name if ("experts." in name and "shared" not in name) else f"{name}.weight"
        weights[key] = codecs_record(shape, n)
    meta = lambda n, dt: torch.empty(n, dtype=dt, device="meta")  # noqa: E731
    weights.update({"input_layernorm.weight": meta(H, BF),
                    "post_attention_layernorm.weight": meta(H, BF),
                    "self_attn.q_a_layernorm.weight": meta(c["q_rank"], BF),
                    "self_attn.kv_a_layernorm.weight": meta(c["kv_rank"], BF),
                    "mlp.gate.weight": torch.empty(E, H, dtype=torch.float32, device="meta"),
                    "mlp.gate.e_score_correction_bias": meta(E, torch.float32)})
    block = deepseek.make_deepseek_block(0, weights, codec="nf4-g128", parameters=c, rank=8,
                                         alpha=16.0, device=dev, shared_lora=True, generator=g)
    with torch.no_grad():
        for p in block.adapters.values():
            p.B.copy_(torch.randn(p.B.shape, generator=g) * 0.02)
    gfill = torch.Generator().manual_seed(56)

    def fill(blk, layout, out):
        for name, e in layout.entries.items():
            if e[0] == "q4":
                _, _, _, po, pb, so, sb = e
                out[po:po + pb].random_(0, 256, generator=gfill)
                out[so:so + sb].view(torch.float32).uniform_(0.01, 0.03, generator=gfill)
            else:
                _, dtype, shape, o, nb = e
                view = out[o:o + nb].view(dtype)
                if name == "mlp.gate.weight":   # well-separated fp32 scores
                    view.normal_(0.0, 3 * H ** -0.5, generator=gfill)
                elif name.endswith("e_score_correction_bias"):
                    view.normal_(0.0, 0.05, generator=gfill)
                else:
                    view.copy_((1 + 0.05 * torch.randn(view.shape, generator=gfill)).to(dtype))
    session = slots.Q4SlotSession([block], dev, host_budget_bytes=1 << 40,
                                  device_budget_bytes=1 << 40, slots=2, image_loader=fill)
    layout, img = session.layouts[id(block)], session.images[id(block)]
    picks = []
    real = moe.deepseek_moe_feed_forward

    def recording(*args, **kwargs):
        out, _, idx = real(*args, return_routing=True, **kwargs)
        picks.append(idx.detach().cpu().long())
        return out
    monkeypatch.setattr(moe, "deepseek_moe_feed_forward", recording)
    hidden = torch.randn(1, T, H, generator=g).to(BF)
    rows = torch.arange(5, T, 32)                      # 64 rows over the whole sequence
    dy = torch.zeros(1, T, H, dtype=BF)
    dy[0, rows] = torch.randn(len(rows), H, generator=g).to(BF)
    cos, sin = OMLA.rotary(1, T, YARN, rope, BF)
    mask = CausalMask(1, T)
    h = hidden.to(dev).requires_grad_(True)
    with session.run():
        out = streaming_block(h, (cos.to(dev), sin.to(dev)), mask, block.functional, block.kwargs,
                              session.reloader(block), block.adapters, block.index)
        out.backward(dy.to(dev))
    torch.cuda.synchronize()
    print("device step done", flush=True)
    assert len(picks) == 2 and torch.equal(picks[0], picks[1])
    idx = picks[1]
    hit = torch.unique(idx[rows]).tolist()
    print(f"experts hit by the checked rows: {len(hit)}, highest {max(hit)}", flush=True)
    per_expert = 2 * I * H // 2
    assert len(hit) >= 64 and max(hit) * per_expert >= 1 << 31
    # oracle weights: every attention / shared matrix and the hit experts,
    # decoded from the pinned image the device copied
    wref = {}
    for name, e in layout.entries.items():
        if e[0] == "q4":
            _, _, shape, po, pb, so, sb = e
            if name.startswith("mlp.experts."):
                n_e = int(np.prod(shape[1:]))
                stack = torch.empty(len(hit), *shape[1:], dtype=BF)
                for i, ex in enumerate(hit):
                    p0, s0 = po + ex * n_e // 2, so + ex * (n_e // 128) * 4
                    bits = oracle_codec.decode4(img[p0:p0 + n_e // 2].numpy(),
                                                img[s0:s0 + n_e // 32].view(torch.float32).numpy(),
                                                n_e, lut=oracle_codec.NF4_LUT)
                    stack[i] = torch.from_numpy(bits.astype(np.int16)).view(BF).view(shape[1:])
                wref[name] = stack
            else:
                n = int(np.prod(shape))
                bits = oracle_codec.decode4(img[po:po + pb].numpy(),
                                            img[so:so + sb].view(torch.float32).numpy(), n,
                                            lut=oracle_codec.NF4_LUT)
                wref[name] = torch.from_numpy(bits.astype(np.int16)).view(BF).view(shape)
        else:
            _, dtype, shape, o, nb = e
            wref[name] = img[o:o + nb].view(dtype).view(shape).clone()
    lor = {n: OL.Lora(n, p.A.detach().cpu(), p.B.detach().cpu(), p.alpha)
           for n, p in block.adapters.items()}
    ordered = sorted(lor.values(), key=lambda q: q.name)
    hr = hidden.clone().requires_grad_(True)
    ref = OMLA.deepseek_block_rows(hr, (cos, sin), OL.causal_mask(1, T, BF), parameters=c,
                                   weights=wref, loras=lor, rows=rows, indices=idx[rows],
                                   experts=hit)
    grads = torch.autograd.grad(ref, [hr] + [t for q in ordered for t in (q.A, q.B)],
                                dy[0, rows])
    res = {"out": _rel(out.reshape(T, H)[rows.to(dev)], ref), "dh": _cos(h.grad, grads[0])}
    for i, q in enumerate(ordered):
        p = block.adapters[q.name]
        res[q.name + ".A"] = _cos(p.grad_A, grads[1 + 2 * i])
        res[q.name + ".B"] = _cos(p.grad_B, grads[2 + 2 * i])
    session.close()
    _assert(res)


def codecs_record(shape, n):
    """Layout-only 4-bit record (meta tensors) of an nf4-g128 matrix or stack."""
    from spilltune_amd import codecs
    groups = n // codecs.GROUP
    return codecs.Record({"version": 1, "shape": list(shape), "dtype": "bfloat16",
                          "codec": "nf4-g128", "group_size": codecs.GROUP, "numel": n},
                         {"payload": torch.empty(groups * codecs.STRIDE, dtype=torch.uint8,
                                                 device="meta"),
                          "scales": torch.empty(groups, dtype=torch.float32, device="meta")})
