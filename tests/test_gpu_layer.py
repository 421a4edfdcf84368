"""One streamed decoder-layer step on the HIP path vs the CPU oracle
(forward + recompute + backward through StreamingBlockFunction), plus the
elementwise kernels against the oracle's autograd.  North-star criteria:
rel. err <= 2e-2 on outputs, cosine >= 0.999 on gradients."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import layer as OL
from spilltune_amd import ops, slots
from spilltune_amd.dense import CausalMask
from spilltune_amd.recompute import streaming_block

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
PROJ = OL.PROJECTIONS


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def cosine(a, b):
    a, b = a.double().cpu().reshape(-1), b.double().cpu().reshape(-1)
    return (a @ b / (a.norm() * b.norm()).clamp_min(1e-300)).item()


def make_layer(cfg, seed, codec="nf4-g128", b_std=0.02, targets=PROJ, qk_norm=False):
    g = torch.Generator().manual_seed(seed)
    H, I, D, heads, kv = cfg["H"], cfg["I"], cfg["D"], cfg["heads"], cfg["kv"]
    shapes = {"self_attn.q_proj": (heads * D, H), "self_attn.k_proj": (kv * D, H),
              "self_attn.v_proj": (kv * D, H), "self_attn.o_proj": (H, heads * D),
              "mlp.gate_proj": (I, H), "mlp.up_proj": (I, H), "mlp.down_proj": (H, I)}
    weights = {f"{n}.weight": (torch.randn(s, generator=g) * 0.02).to(BF) for n, s in shapes.items()}
    weights["input_layernorm.weight"] = (1 + 0.05 * torch.randn(H, generator=g)).to(BF)
    weights["post_attention_layernorm.weight"] = (1 + 0.05 * torch.randn(H, generator=g)).to(BF)
    if qk_norm:
        weights["self_attn.q_norm.weight"] = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
        weights["self_attn.k_norm.weight"] = (1 + 0.1 * torch.randn(D, generator=g)).to(BF)
    block = slots.make_dense_block(0, weights, codec=codec, heads=heads, kv_heads=kv, head_dim=D,
                                   eps=cfg["eps"], rank=cfg["r"], alpha=cfg["alpha"],
                                   targets=targets, device="cuda:0", generator=g, qk_norm=qk_norm)
    with torch.no_grad():
        for p in block.adapters.values():
            p.B.copy_(torch.randn(p.B.shape, generator=g) * b_std)
    return block, weights


def oracle_weights(block, oracle_codec):
    """bf16 weights exactly as the reference's decode produces them."""
    out = {}
    for name, entry in block.storage_specs.items():
        spec = entry["spec"]
        p = block.host_weights[entry["parts"]["payload"]].numpy()
        s = block.host_weights[entry["parts"]["scales"]].numpy()
        lut = oracle_codec.NF4_LUT if spec["codec"] == "nf4-g128" else oracle_codec.INT4_LUT
        bits = oracle_codec.decode4(p, s, spec["numel"], lut=lut)
        out[name] = torch.from_numpy(bits.astype(np.int16)).view(BF).view(spec["shape"])
    for k, v in block.host_weights.items():
        if not k.startswith("@"):
            out[k] = v
    return out


def run_case(cfg, seed, oracle_codec, codec="nf4-g128", streamed=False, targets=PROJ,
             qk_norm=False, valid=None):
    block, _ = make_layer(cfg, seed, codec, targets=targets, qk_norm=qk_norm)
    g = torch.Generator().manual_seed(seed + 1)
    B, S, H = cfg["B"], cfg["S"], cfg["H"]
    hidden = torch.randn(B, S, H, generator=g).to(BF)
    dy = torch.randn(B, S, H, generator=g).to(BF)
    cos, sin = OL.rotary(B, S, cfg["D"], 500000.0, BF)
    # ---- oracle
    lor = {n: OL.Lora(n, p.A.detach().cpu(), p.B.detach().cpu(), p.alpha)
           for n, p in block.adapters.items()}
    kw = dict(heads=cfg["heads"], kv_heads=cfg["kv"], head_dim=cfg["D"], eps=cfg["eps"],
              qk_norm=qk_norm)
    out_ref, gh_ref = OL.streaming_step(hidden, (cos, sin), OL.causal_mask(B, S, BF, valid), dy,
                                        weights=oracle_weights(block, oracle_codec), loras=lor, cfg=kw)
    # ---- HIP path through the recompute driver
    dev = torch.device("cuda:0")
    if streamed:
        session = slots.Q4SlotSession([block], dev, host_budget_bytes=1 << 40,
                                      device_budget_bytes=1 << 40, slots=2)
    else:
        session = slots.ResidentSession([block], dev)
    h = hidden.to(dev).requires_grad_(True)
    with session.run():
        lengths = None if valid is None else valid.sum(1).to(device=dev, dtype=torch.int32)
        out = streaming_block(h, (cos.to(dev), sin.to(dev)), CausalMask(B, S, lengths),
                              block.functional,
                              block.kwargs, session.reloader(block), block.adapters, block.index)
        out.backward(dy.to(dev))
    torch.cuda.synchronize()
    res = {"out": rel(out.detach(), out_ref), "dh": cosine(h.grad, gh_ref)}
    for n, p in block.adapters.items():
        res[n + ".A"] = cosine(p.grad_A, lor[n].grad_A)
        res[n + ".B"] = cosine(p.grad_B, lor[n].grad_B)
    session.close()
    return res


TINY = dict(H=256, I=688, heads=4, kv=4, D=64, eps=1e-5, r=8, alpha=16.0, B=2, S=128)
GQA = dict(H=512, I=1024, heads=8, kv=2, D=64, eps=1e-5, r=16, alpha=32.0, B=1, S=192)


def _assert(res):
    assert res["out"] <= 2e-2, res
    bad = {k: v for k, v in res.items() if k != "out" and v < 0.999}
    assert not bad, bad


@pytest.mark.parametrize("codec", ["nf4-g128", "int4-sym-g128"])
def test_tiny_llama_layer_step_vs_oracle(oracle_codec, codec):
    _assert(run_case(TINY, 10, oracle_codec, codec))


def test_gqa_layer_step_streamed_vs_oracle(oracle_codec):
    _assert(run_case(GQA, 20, oracle_codec, streamed=True))


def test_reference_default_targets_qvo(oracle_codec):
    """q/v/o only (the reference's default dense targets): unfused q|k|v path."""
    _assert(run_case(TINY, 30, oracle_codec,
                     targets=("self_attn.q_proj", "self_attn.v_proj", "self_attn.o_proj")))


def test_qwen3_qk_norm_layer_step_vs_oracle(oracle_codec):
    """Qwen3 block: per-head q/k RMSNorm before RoPE, fused q|k|v and the
    separate-projection path (q/v/o targets)."""
    _assert(run_case(GQA, 50, oracle_codec, streamed=True, qk_norm=True))
    _assert(run_case(TINY, 51, oracle_codec, qk_norm=True,
                     targets=("self_attn.q_proj", "self_attn.v_proj", "self_attn.o_proj")))


@pytest.mark.parametrize("r", [5, 32, 80])
def test_layer_step_lora_ranks_vs_oracle(oracle_codec, r):
    """An odd rank (5: fused q|k|v and gate|up with 15 and 10 LoRA columns),
    rank 32 (q|k|v would need 96 LoRA columns: the functional runs q, k and v
    one by one; gate|up fused at 64) and rank 80 (every projection on its
    own, its LoRA operands read from global memory in the GEMM epilogues)."""
    _assert(run_case(dict(GQA, r=r, alpha=2.0 * r), 60 + r, oracle_codec))


def test_right_padded_batch_layer_step_vs_oracle(oracle_codec):
    """Right-padded rows (dense.py:237-246, the reference's additive
    finfo.min mask in the oracle): every output row, padded ones included,
    and every gradient."""
    valid = torch.ones(3, 100, dtype=torch.bool)
    valid[1, 61:] = False
    valid[2, 1:] = False
    _assert(run_case(dict(GQA, B=3, S=100), 26, oracle_codec, valid=valid))


def test_positions_and_masks_right_padding():
    """The lengths the mask marker carries, and the reference's rejections
    (a leading padded position, a valid position after padding)."""
    from spilltune_amd.dense import positions_and_masks
    valid = torch.tensor([[True] * 5, [True, True, False, False, False]])
    _, mask = positions_and_masks(valid, head_dim=8, theta=10000.0, device="cuda:0")
    assert mask.lengths.tolist() == [5, 2] and mask.lengths.dtype == torch.int32
    _, mask = positions_and_masks(torch.ones(2, 5, dtype=torch.bool), head_dim=8, theta=1e4,
                                  device="cuda:0")
    assert mask.lengths is None
    for bad in ([[False, True]], [[True, False, True]]):
        with pytest.raises(ValueError, match="unsupported_capability"):
            positions_and_masks(torch.tensor(bad), head_dim=8, theta=1e4, device="cuda:0")


def test_odd_sequence_length_layer_step_vs_oracle(oracle_codec):
    """A sequence length that is no multiple of 8 (or of any tile): 2 x 100
    tokens through the whole layer step, GQA, streamed."""
    _assert(run_case(dict(GQA, B=2, S=100), 25, oracle_codec, streamed=True))


def test_llama8b_dims_short_sequence(oracle_codec):
    cfg = dict(H=4096, I=14336, heads=32, kv=8, D=128, eps=1e-5, r=16, alpha=32.0, B=1, S=64)
    _assert(run_case(cfg, 40, oracle_codec))


# ---------------------------------------------------------------- elementwise
def test_rmsnorm_fwd_bwd_vs_oracle():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 1000, generator=g).to(BF)
    w = (1 + 0.1 * torch.randn(1000, generator=g)).to(BF)
    dy = torch.randn(64, 1000, generator=g).to(BF)
    xr = x.clone().requires_grad_(True)
    yr = OL.rms(xr, w, 1e-5)
    yr.backward(dy)
    xd = x.cuda().requires_grad_(True)
    yd = ops.rms_norm(xd, w.cuda(), 1e-5)
    yd.backward(dy.cuda())
    assert rel(yd, yr) < 4e-3 and rel(xd.grad, xr.grad) < 1e-2


@pytest.mark.parametrize("H", [512, 2048, 4096, 7168, 8192, 8200])
def test_rmsnorm_row_kernels_vs_oracle(H):
    """The 16-byte row kernels of st_rmsnorm_fwd/bwd at the hidden sizes of
    the benchmark models and around 8192 against the oracle's norm and its
    autograd VJP plus a residual gradient (the dres operand)."""
    g = torch.Generator().manual_seed(H)
    x = torch.randn(33, H, generator=g).to(BF)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(BF)
    dy = torch.randn(33, H, generator=g).to(BF)
    dres = torch.randn(33, H, generator=g).to(BF)
    xr = x.clone().requires_grad_(True)
    yr = OL.rms(xr, w, 1e-5)
    torch.autograd.backward([yr, xr], [dy, dres])
    xd = x.cuda().requires_grad_(True)
    res, yd = ops.rms_norm_residual(xd, w.cuda(), 1e-5)
    torch.autograd.backward([yd, res], [dy.cuda(), dres.cuda()])
    torch.cuda.synchronize()
    err = (yd.float().cpu() - yr.float()).abs()
    assert (err > yr.float().abs() * 2 ** -7 + 1e-6).float().mean().item() < 1e-3
    assert rel(yd, yr) < 4e-3 and rel(xd.grad, xr.grad) < 1e-2


def test_rope_relayout_vs_oracle():
    g = torch.Generator().manual_seed(1)
    B, S, heads, kv, D = 2, 16, 4, 2, 64
    cos, sin = OL.rotary(B, S, D, 10000.0, BF)
    y = torch.randn(B * S, (heads + 2 * kv) * D, generator=g).to(BF)
    yr = y.clone().requires_grad_(True)
    q = yr[:, :heads * D].reshape(B, S, heads, D).transpose(1, 2)
    k = yr[:, heads * D:(heads + kv) * D].reshape(B, S, kv, D).transpose(1, 2)
    v = yr[:, (heads + kv) * D:].reshape(B, S, kv, D).transpose(1, 2)
    c, s = cos.unsqueeze(1), sin.unsqueeze(1)
    qr, kr = OL._rotate(q, c, s), OL._rotate(k, c, s)
    gq, gk, gv = (torch.randn(t.shape, generator=g).to(BF) for t in (qr, kr, v))
    torch.autograd.backward([qr, kr, v], [gq, gk, gv])
    yd = y.cuda().requires_grad_(True)
    qd, kd, vd = ops.rope_qkv(yd, B, S, heads, kv, D, cos.cuda(), sin.cuda())
    torch.autograd.backward([qd, kd, vd], [gq.cuda(), gk.cuda(), gv.cuda()])
    for a, b in ((qd, qr), (kd, kr), (vd, v)):
        assert torch.equal(a.cpu().view(torch.int16), b.contiguous().view(torch.int16))
    assert torch.equal(yd.grad.cpu().view(torch.int16), yr.grad.view(torch.int16))


def test_swiglu_vs_oracle():
    g = torch.Generator().manual_seed(2)
    gu = torch.randn(50, 2 * 300, generator=g).to(BF)
    da = torch.randn(50, 300, generator=g).to(BF)
    r = gu.clone().requires_grad_(True)
    a = F.silu(r[:, :300]) * r[:, 300:]
    a.backward(da)
    d = gu.cuda().requires_grad_(True)
    ad = ops.swiglu(d, 300)
    ad.backward(da.cuda())
    assert rel(ad, a) < 4e-3 and rel(d.grad, r.grad) < 1e-2


@pytest.mark.parametrize("I", [1024, 300])
def test_swiglu_forward_elementwise_vs_torch(I):
    """silu(g) * u per element against torch's bf16 ops on the CPU (silu in
    fp32, rounded to bf16, then the bf16 product), over the range where silu
    changes shape.  The device exp may differ from the host's by an fp32 ulp
    and so move silu(g) across a bf16 rounding boundary (one ulp of silu,
    which the product with u can turn into at most two of the result) on a
    handful of elements.  (A hardware 2^x / reciprocal sigmoid, as in the
    VJP, measured 0.12% of elements off here, and the forward keeps expf and
    the IEEE division.)  I = 1024 takes the 8-wide kernel, 300 the scalar
    one."""
    g = torch.Generator().manual_seed(I)
    M = 2048
    gate = (torch.rand(M, I, generator=g) * 24 - 12).to(BF)
    up = torch.randn(M, I, generator=g).to(BF)
    ref = F.silu(gate) * up
    got = ops.swiglu(torch.cat([gate, up], 1).cuda(), I).cpu()
    diff = (got.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert int(diff.max()) <= 2
    assert (diff > 0).float().mean().item() < 1e-4


def test_causal_attention_vs_oracle():
    g = torch.Generator().manual_seed(3)
    B, H, kv, S, D = 2, 8, 2, 96, 64
    q = torch.randn(B, H, S, D, generator=g).to(BF)
    k = torch.randn(B, kv, S, D, generator=g).to(BF)
    v = torch.randn(B, kv, S, D, generator=g).to(BF)
    do = torch.randn(B, S, H * D, generator=g).to(BF)
    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    rep = lambda t: t[:, :, None].expand(B, kv, H // kv, S, D).reshape(B, H, S, D)
    scores = (qr @ rep(kr).transpose(-2, -1)) * D ** -0.5
    p = torch.softmax(scores + OL.causal_mask(B, S, BF), dim=-1, dtype=torch.float32).to(BF)
    o = (p @ rep(vr)).transpose(1, 2).reshape(B, S, H * D)
    o.backward(do)
    qd, kd, vd = (t.cuda().requires_grad_(True) for t in (q, k, v))
    od = ops.causal_attention(qd, kd, vd, D ** -0.5)
    od.backward(do.cuda())
    assert rel(od, o) < 1e-2
    for a, b in ((qd, qr), (kd, kr), (vd, vr)):
        assert cosine(a.grad, b.grad) > 0.999


def test_archive_backed_streamed_layer_matches_in_memory(tmp_path):
    """A layer whose pinned slot image is streamed straight from an nf4-g128
    archive gives bit-identical outputs and gradients to the same layer
    encoded in memory, through the streamed session and recompute driver."""
    from _ckpt import LAYER, make_checkpoint
    from spilltune_amd import archive
    tensors = make_checkpoint(tmp_path / "src", layers=1)
    archive.export_quantized(tmp_path / "src", tmp_path / "q", "llama", "nf4-g128")
    reader = archive.ArchiveReader(tmp_path / "q", "llama", "nf4-g128")
    dev = torch.device("cuda:0")
    kw = dict(heads=4, kv_heads=4, head_dim=64, eps=1e-5, rank=8, alpha=16.0, targets=PROJ,
              device=dev)
    a_block = slots.make_archive_block(reader, 0, **kw)
    m_block = slots.make_dense_block(0, {n: tensors["model.layers.0." + n] for n in LAYER},
                                     codec="nf4-g128", **kw)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        for n, p in a_block.adapters.items():
            A, B = torch.randn(p.A.shape, generator=g) * 0.05, torch.randn(p.B.shape, generator=g) * 0.02
            for blk in (a_block, m_block):
                blk.adapters[n].A.copy_(A)
                blk.adapters[n].B.copy_(B)
    hidden = torch.randn(2, 128, 256, generator=g).to(BF)
    dy = torch.randn(2, 128, 256, generator=g).to(BF)
    cos, sin = OL.rotary(2, 128, 64, 500000.0, BF)
    results = []
    for block, loader in ((a_block, reader.image_loader("model.layers.0.")), (m_block, None)):
        session = slots.Q4SlotSession([block], dev, host_budget_bytes=1 << 40,
                                      device_budget_bytes=1 << 40, slots=2, image_loader=loader)
        h = hidden.to(dev).requires_grad_(True)
        with session.run():
            out = streaming_block(h, (cos.to(dev), sin.to(dev)), CausalMask(2, 128),
                                  block.functional, block.kwargs, session.reloader(block),
                                  block.adapters, block.index)
            out.backward(dy.to(dev))
        torch.cuda.synchronize()
        results.append((out.detach().cpu(), h.grad.cpu(),
                        {n: (p.grad_A.cpu(), p.grad_B.cpu()) for n, p in block.adapters.items()}))
        session.close()
    (oa, ha, ga), (om, hm, gm) = results
    assert torch.equal(oa, om) and torch.equal(ha, hm)
    for n in ga:
        assert torch.equal(ga[n][0], gm[n][0]) and torch.equal(ga[n][1], gm[n][1]), n
