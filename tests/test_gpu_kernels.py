"""HIP kernels vs the CPU oracle, through the C ABI (MI355X only).

Dequantisation must be bit-exact; GEMM/LoRA outputs are compared with the
oracle's bf16 result allowing for fp32 summation order only (a bf16 ulp)."""
import os
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from spilltune_amd import _lib, codecs, ops

pytestmark = pytest.mark.gpu
GOLD = np.load(Path(__file__).parent / "golden" / "codec_vectors.npz")
BF = torch.bfloat16


def lut_for(fmt, oc):
    return oc.INT4_LUT if fmt.startswith("int4") else oc.NF4_LUT


def bits_tensor(bits):
    return torch.from_numpy(np.asarray(bits, dtype=np.uint16).astype(np.int16)).view(BF)


def dequant_dev(payload, scales, numel, fmt, dev, flags=0, group=128, out=None):
    if out is None:
        out = torch.empty(numel, dtype=BF, device=dev)
    lut = _lib.lut_array(codecs.CODEBOOKS[fmt])
    _lib.call("st_dequant4", _lib.ptr(payload), _lib.ptr(scales), numel, group, lut, flags,
              _lib.ptr(out), _lib.stream_handle(dev))
    torch.cuda.synchronize()
    return out


def q4_from_oracle(oc, w32: np.ndarray, fmt, dev):
    """Encode with the oracle, upload, return (Q4Weight, exact bf16 W on CPU)."""
    enc = oc.encode_int4 if fmt.startswith("int4") else oc.encode_nf4
    payload, scales = enc(w32)
    W = bits_tensor(oc.decode4(payload, scales, w32.size, lut=lut_for(fmt, oc))).view(w32.shape)
    q = ops.Q4Weight(torch.from_numpy(payload).to(dev), torch.from_numpy(scales).to(dev),
                     w32.shape, fmt)
    return q, W


@pytest.mark.parametrize("case", range(5))
@pytest.mark.parametrize("fmt", ["int4-sym-g128", "nf4-g128"])
def test_dequant_golden_cases_bit_exact(dev, case, fmt):
    short = "int4" if fmt.startswith("int4") else "nf4"
    p = torch.from_numpy(GOLD[f"case{case}_{short}_payload"]).to(dev)
    s = torch.from_numpy(GOLD[f"case{case}_{short}_scales"]).to(dev)
    n = GOLD[f"case{case}_x"].size
    got = dequant_dev(p, s, n, fmt, dev).cpu()
    assert torch.equal(got.view(torch.int16), bits_tensor(GOLD[f"case{case}_{short}_bits"]).view(torch.int16))


@pytest.mark.parametrize("fmt", ["int4-sym-g128", "nf4-g128"])
def test_dequant_codebook_tables_bit_exact(dev, fmt):
    short = "int4" if fmt.startswith("int4") else "nf4"
    payload = torch.tensor([c | ((c + 1) << 4) for c in range(0, 16, 2)] * 8, dtype=torch.uint8)
    for i, s in enumerate(GOLD[f"{short}_table_scales"]):
        got = dequant_dev(payload.to(dev), torch.tensor([s], dtype=torch.float32).to(dev), 16,
                          fmt, dev).cpu()
        assert torch.equal(got.view(torch.int16), bits_tensor(GOLD[f"{short}_table_bits"][i]).view(torch.int16))


@pytest.mark.parametrize("fmt", ["int4-sym-g128", "nf4-g128"])
@pytest.mark.parametrize("hi_first", [False, True])
@pytest.mark.parametrize("numel", [1, 31, 32, 4096 * 16 + 77, (1 << 21) + 3])
def test_dequant_random_vs_oracle(dev, oracle_codec, fmt, hi_first, numel):
    rng = np.random.default_rng(numel)
    groups = (numel + 127) // 128
    payload = rng.integers(0, 256, groups * 64, dtype=np.uint8)
    scales = (rng.standard_normal(groups).astype(np.float32) * 0.05)
    expect = oracle_codec.decode4(payload, scales, numel, lut=lut_for(fmt, oracle_codec),
                                  hi_first=hi_first)
    got = dequant_dev(torch.from_numpy(payload).to(dev), torch.from_numpy(scales).to(dev), numel,
                      fmt, dev, flags=_lib.ST_FLAG_HI_NIBBLE_FIRST if hi_first else 0)
    assert torch.equal(got.cpu().view(torch.int16), bits_tensor(expect).view(torch.int16))


def test_dequant_unaligned_output_and_group64(dev, oracle_codec):
    rng = np.random.default_rng(1)
    n = 64 * 40 + 9
    payload = rng.integers(0, 256, (n + 1) // 2 + 64, dtype=np.uint8)
    scales = rng.random((n + 63) // 64, dtype=np.float32)
    buf = torch.zeros(n + 8, dtype=BF, device=dev)
    out = buf[1:1 + n]  # 2-byte aligned only: exercises the element-wise path
    dequant_dev(torch.from_numpy(payload).to(dev), torch.from_numpy(scales).to(dev), n,
                "nf4-g128", dev, group=64, out=out)
    expect = oracle_codec.decode4(payload, scales, n, lut=oracle_codec.NF4_LUT, group=64)
    assert torch.equal(out.cpu().view(torch.int16), bits_tensor(expect).view(torch.int16))
    assert buf[0].item() == 0 and buf[n + 1:].float().abs().sum().item() == 0


# ---------------------------------------------------------------- GEMMs
class _L:
    def __init__(self, A, B, alpha):
        self.A, self.B, self.alpha = A, B, alpha
        self.rank = A.shape[0]
        self.scale = alpha / self.rank


def _close_bf16(got, ref, what):
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs()
    ulp = ref.abs().clamp_min(2 ** -20) * 2 ** -7
    frac_bad = (err > ulp + 1e-6).float().mean().item()
    rel = (err.norm() / ref.norm().clamp_min(1e-20)).item()
    assert rel < 4e-3 and frac_bad < 1e-3, f"{what}: rel {rel:.3e}, >1ulp fraction {frac_bad:.2e}"


SHAPES = [(64, 256, 256), (100, 384, 512), (37, 96, 688), (300, 512, 1024), (1, 128, 128)]


@pytest.mark.parametrize("tile", ["128", "2562", "256", "2566", "2567", "2568"])
@pytest.mark.parametrize("fmt", ["nf4-g128", "int4-sym-g128"])
@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("lora,residual", [(False, False), (True, False), (True, True)])
def test_q4_linear_fwd_vs_oracle(dev, oracle_codec, monkeypatch, tile, fmt, M, N, K, lora, residual):
    monkeypatch.setenv("ST_GEMM_TILE", tile)
    g = torch.Generator().manual_seed(M * 7 + N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    q, W = q4_from_oracle(oracle_codec, w, fmt, dev)
    x = torch.randn(M, K, generator=g).to(BF)
    ref = F.linear(x.float(), W.float()).to(BF)
    lo = None
    if lora:
        r = 8
        lo = _L(torch.randn(r, K, generator=g) * 0.05, torch.randn(N, r, generator=g) * 0.05, 16.0)
        T = x.float() @ lo.A.T
        ref = (ref.float() + (T @ lo.B.T) * lo.scale).to(BF)
        lo_dev = _L(lo.A.to(dev), lo.B.to(dev), 16.0)
    res = None
    if residual:
        res = torch.randn(M, N, generator=g).to(BF)
        ref = (res.float() + ref.float()).to(BF)
    y = ops.q4_lora_linear(x.to(dev), q, [lo_dev] if lora else None,
                           residual=None if res is None else res.to(dev))
    torch.cuda.synchronize()
    _close_bf16(y, ref, f"fwd {fmt} {M}x{N}x{K} tile{tile}")


@pytest.mark.parametrize("tile", ["128", "2562", "256", "2566", "2567", "2568"])
@pytest.mark.parametrize("r", [1, 3, 7, 65, 96, 128])
def test_q4_linear_fwd_odd_rank_vs_oracle(dev, oracle_codec, monkeypatch, tile, r):
    """Odd LoRA ranks on every forward tile, with a residual: the epilogue's
    fp32 MFMA takes the rank two at a time and reads a zero past the last
    rank column.  Ranks above 64 exceed what the 256-wide tiles' LDS
    stages: those calls run on the 128x128 kernel, which stages rank 65 and
    reads ranks 96 and 128 from global memory."""
    monkeypatch.setenv("ST_GEMM_TILE", tile)
    M, N, K = 300, 512, 1024
    g = torch.Generator().manual_seed(r * 101 + M)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    q, W = q4_from_oracle(oracle_codec, w, "nf4-g128", dev)
    x = torch.randn(M, K, generator=g).to(BF)
    lo = _L(torch.randn(r, K, generator=g) * 0.05, torch.randn(N, r, generator=g) * 0.05, 2.0 * r)
    res = torch.randn(M, N, generator=g).to(BF)
    ref = (F.linear(x.float(), W.float()).to(BF).float() + (x.float() @ lo.A.T @ lo.B.T) * lo.scale)
    ref = (res.float() + ref.to(BF).float()).to(BF)
    y = ops.q4_lora_linear(x.to(dev), q, [_L(lo.A.to(dev), lo.B.to(dev), 2.0 * r)],
                           residual=res.to(dev))
    torch.cuda.synchronize()
    _close_bf16(y, ref, f"odd rank {r} tile{tile}")


@pytest.mark.parametrize("tile", ["128", "2562", "256", "2566", "2568"])
@pytest.mark.parametrize("M,N,K", [(100, 384, 512), (300, 512, 1024)])
def test_q4_linear_high_nibble_first_vs_oracle(dev, oracle_codec, monkeypatch, tile, M, N, K):
    """bitsandbytes' packing (element 2i in the HIGH nibble of byte i,
    ST_FLAG_HI_NIBBLE_FIRST): forward and dgrad on every tile equal the
    oracle's decode of the same bytes, as for the low-nibble-first format."""
    monkeypatch.setenv("ST_GEMM_TILE", tile)
    g = torch.Generator().manual_seed(M + N + K + 1)
    w32 = (torch.randn(N, K, generator=g) * 0.02).numpy()
    payload, scales = oracle_codec.encode_nf4(w32, hi_first=True)
    W = bits_tensor(oracle_codec.decode4(payload, scales, w32.size, lut=oracle_codec.NF4_LUT,
                                         hi_first=True)).view(N, K)
    q = ops.Q4Weight(torch.from_numpy(payload).to(dev), torch.from_numpy(scales).to(dev),
                     (N, K), "nf4-g128", flags=_lib.ST_FLAG_HI_NIBBLE_FIRST)
    x = torch.randn(M, K, generator=g).to(BF)
    dy = torch.randn(M, N, generator=g).to(BF)
    xd = x.to(dev).requires_grad_(True)
    y = ops.q4_lora_linear(xd, q, None)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    _close_bf16(y, F.linear(x.float(), W.float()).to(BF), f"hi-first fwd tile{tile}")
    _close_bf16(xd.grad, (dy.float() @ W.float()).to(BF), f"hi-first dgrad tile{tile}")


@pytest.mark.parametrize("M,N,K", [(37, 96, 8), (64, 136, 200), (130, 256, 264), (5, 40, 1000)])
@pytest.mark.parametrize("fmt", ["nf4-g128", "int4-sym-g128"])
def test_q4_linear_flat_groups_vs_oracle(dev, oracle_codec, fmt, M, N, K):
    """K % 128 != 0: the flat 128-element scale groups straddle W's rows and
    the flat-group kernels give each packed word its own scale (forward and
    dgrad, from the packed weight, no workspace)."""
    g = torch.Generator().manual_seed(M + N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    q, W = q4_from_oracle(oracle_codec, w, fmt, dev)
    x = torch.randn(M, K, generator=g).to(BF)
    dy = torch.randn(M, N, generator=g).to(BF)
    xd = x.to(dev).requires_grad_(True)
    y = ops.q4_lora_linear(xd, q, None)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    _close_bf16(y, F.linear(x.float(), W.float()).to(BF), f"flat fwd {fmt} {M}x{N}x{K}")
    _close_bf16(xd.grad, (dy.float() @ W.float()).to(BF), f"flat dgrad {fmt} {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K", [(100, 384, 512), (37, 256, 1024)])
def test_q4_linear_fwd_flat_kernel_equals_aligned(dev, oracle_codec, monkeypatch, M, N, K):
    """A payload that is 4- but not 16-byte aligned takes the flat-group
    forward; with K % 128 == 0 its per-word scales are the per-tile ones, so
    it must equal the 128x128 tile on an aligned copy bit for bit."""
    monkeypatch.setenv("ST_GEMM_TILE", "128")
    g = torch.Generator().manual_seed(M + K)
    q, _ = q4_from_oracle(oracle_codec, (torch.randn(N, K, generator=g) * 0.02).numpy(),
                          "nf4-g128", dev)
    buf = torch.zeros(q.payload.numel() + 16, dtype=torch.uint8, device=dev)
    shifted = buf[4:4 + q.payload.numel()]
    shifted.copy_(q.payload)
    q2 = ops.Q4Weight(shifted, q.scales, (N, K), "nf4-g128")
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    y1 = ops.q4_lora_linear(x, q, None)
    y2 = ops.q4_lora_linear(x, q2, None)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


@pytest.mark.parametrize("tile", ["128", "2562", "256"])
@pytest.mark.parametrize("M,N,K", [(64, 256, 256), (100, 384, 512), (37, 128, 688), (300, 512, 1024),
                                   (77, 200, 256)])
@pytest.mark.parametrize("lora,r", [(False, 8), (True, 8), (True, 5), (True, 97)])
def test_q4_linear_dgrad_and_lora_grads_vs_oracle(dev, oracle_codec, monkeypatch, tile, M, N, K, lora,
                                                  r):
    """dX (and the LoRA grads) against autograd over the oracle's decode; N =
    200 leaves a ragged last k-tile of the dgrad contraction (8 of 64 rows);
    r = 5 is an odd rank (the epilogue takes the rank two at a time); r = 97
    is above what the tile's LDS stages (dT and A read from global memory,
    the rank-r products one by one on the general LoRA GEMM)."""
    monkeypatch.setenv("ST_GEMM_TILE", tile)
    g = torch.Generator().manual_seed(M + N * 3 + K)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    q, W = q4_from_oracle(oracle_codec, w, "nf4-g128", dev)
    x = torch.randn(M, K, generator=g).to(BF)
    dy = torch.randn(M, N, generator=g).to(BF)
    alpha = 2.0 * r
    A = torch.randn(r, K, generator=g) * 0.05
    B = torch.randn(N, r, generator=g) * 0.05
    # oracle: autograd of lora.py:218-220 on CPU
    xr = x.clone().requires_grad_(True)
    Ar, Br = A.clone().requires_grad_(True), B.clone().requires_grad_(True)
    base = F.linear(xr, W)
    out = (base.float() + F.linear(F.linear(xr.float(), Ar), Br) * (alpha / r)).to(BF) if lora else base
    out.backward(dy)
    xd = x.to(dev).requires_grad_(True)
    lo = _L(A.to(dev).requires_grad_(True), B.to(dev).requires_grad_(True), alpha)
    y = ops.q4_lora_linear(xd, q, [lo] if lora else None)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    _close_bf16(xd.grad, xr.grad, f"dgrad {M}x{N}x{K}")
    if lora:
        # fp32 reductions in a different order: tolerance scaled to the gradient's magnitude
        for got, ref in ((lo.A.grad.cpu(), Ar.grad), (lo.B.grad.cpu(), Br.grad)):
            torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-5 * ref.abs().max().item())


@pytest.mark.parametrize("splits", ["2", "3", "8"])
@pytest.mark.parametrize("M,N,K", [(300, 512, 1024), (517, 384, 2048), (64, 192, 4096),
                                   (300, 2048, 512)])
def test_split_k_vs_oracle(dev, oracle_codec, monkeypatch, splits, M, N, K):
    """Split-K (ST_GEMM_SPLITK forces the split count; contractions of 16
    k-steps or more split: the forward for K >= 1024, the dgrad for N = 2048):
    the forward (fused two segments with LoRA and a residual) and the dgrad
    with its LoRA term, against autograd over the oracle's decode.  The splits' fp32 partials
    are summed in split order, then the usual epilogue roundings apply."""
    monkeypatch.setenv("ST_GEMM_SPLITK", splits)
    g = torch.Generator().manual_seed(M + N + K + int(splits))
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    qw, W = q4_from_oracle(oracle_codec, w, "nf4-g128", dev)
    q = ops.Q4Weight(qw.payload, qw.scales, (N, K), "nf4-g128", (N // 2, N - N // 2))
    x = torch.randn(M, K, generator=g).to(BF)
    dy = torch.randn(M, N, generator=g).to(BF)
    res = torch.randn(M, N, generator=g).to(BF)
    r = 8
    A = [torch.randn(r, K, generator=g) * 0.05 for _ in range(2)]
    B = [torch.randn(N // 2, r, generator=g) * 0.05, torch.randn(N - N // 2, r, generator=g) * 0.05]
    xr = x.clone().requires_grad_(True)
    Ar = [a.clone().requires_grad_(True) for a in A]
    Br = [b.clone().requires_grad_(True) for b in B]
    base = F.linear(xr, W)
    # one fused projection: one x_f32 for both segments, so the LoRA input
    # gradient is rounded to bf16 once (as the fused epilogue does)
    xf = xr.float()
    lora = torch.cat([F.linear(F.linear(xf, Ar[i]), Br[i]) for i in range(2)], 1) * 2.0
    out = (res.float() + (base.float() + lora).to(BF).float()).to(BF)
    out.backward(dy)
    xd = x.to(dev).requires_grad_(True)
    los = [_L(A[i].to(dev).requires_grad_(True), B[i].to(dev).requires_grad_(True), 16.0)
           for i in range(2)]
    y = ops.q4_lora_linear(xd, q, los, residual=res.to(dev))
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    _close_bf16(y, out, f"split-K {splits} fwd {M}x{N}x{K}")
    _close_bf16(xd.grad, xr.grad, f"split-K {splits} dgrad {M}x{N}x{K}")
    for i in range(2):
        for got, ref in ((los[i].A.grad.cpu(), Ar[i].grad), (los[i].B.grad.cpu(), Br[i].grad)):
            torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-5 * ref.abs().max().item())


@pytest.mark.parametrize("N,K", [(32768, 512), (24576, 1536)])
def test_split_k_mla_dgrad_shapes_vs_torch_fp32(dev, N, K):
    """DeepSeek-V3 MLA input gradients at 2048 tokens (kv_b: 512 outputs from
    a 32768-long contraction; q_b: 1536 from 24576), where the dispatch
    splits the contraction on its own, with a LoRA term, against torch fp32
    matmul of the standalone decode (pinned bit-exact to the oracle)."""
    M = 2048
    assert _lib.query("st_q4_linear_dgrad_workspace_bytes", M, N, K) > 0
    g = torch.Generator().manual_seed(N + K)
    w = torch.randn(N, K, generator=g) * 0.02
    rec = codecs.encode(w, "nf4-g128")
    q = ops.Q4Weight(rec.parts["payload"].to(dev), rec.parts["scales"].to(dev), (N, K), "nf4-g128")
    Wd = q.dequantize().float()
    x = torch.randn(M, K, generator=g).to(BF).to(dev).requires_grad_(True)
    dy = torch.randn(M, N, generator=g).to(BF).to(dev)
    lo = _L((torch.randn(8, K, generator=g) * 0.05).to(dev).requires_grad_(True),
            (torch.randn(N, 8, generator=g) * 0.05).to(dev).requires_grad_(True), 16.0)
    y = ops.q4_lora_linear(x, q, [lo])
    y.backward(dy)
    dT = (dy.float() @ lo.B.detach()) * 2.0
    ref = ((dy.float() @ Wd).to(BF).float() + (dT @ lo.A.detach()).to(BF).float()).to(BF)
    torch.cuda.synchronize()
    _close_bf16(x.grad, ref, f"MLA dgrad {M}x{N}->{K}")


@pytest.mark.parametrize("tile", ["128", "2562", "256", "2566"])
@pytest.mark.parametrize("M", [1300, 1024])
def test_raster_order_gives_the_same_bits(dev, oracle_codec, monkeypatch, tile, M):
    """The grouped tile raster (4 row tiles per group; M = 1300 leaves a short
    last group) only reorders whole tiles: forward, dgrad and LoRA gradients
    equal the row-major order bit for bit."""
    monkeypatch.setenv("ST_GEMM_TILE", tile)
    g = torch.Generator().manual_seed(M)
    N, K = 1536, 512
    q, _ = q4_from_oracle(oracle_codec, (torch.randn(N, K, generator=g) * 0.02).numpy(), "nf4-g128",
                          dev)
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    dy = torch.randn(M, N, generator=g).to(BF).to(dev)
    A = torch.randn(8, K, generator=g) * 0.05
    B = torch.randn(N, 8, generator=g) * 0.05
    outs = []
    for raster in ("1", "4"):
        monkeypatch.setenv("ST_GEMM_RASTER", raster)
        xd = x.clone().requires_grad_(True)
        lo = _L(A.to(dev).requires_grad_(True), B.to(dev).requires_grad_(True), 16.0)
        y = ops.q4_lora_linear(xd, q, [lo])
        y.backward(dy)
        torch.cuda.synchronize()
        outs.append((y.view(torch.int16), xd.grad.view(torch.int16), lo.A.grad, lo.B.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("r", [4, 5])
def test_fused_segments_match_separate_projections(dev, oracle_codec, r):
    """q|k|v as one N-concatenated GEMM == three separate GEMMs (same bits for
    the forward: every output element has the same reduction), for an even
    and an odd rank."""
    g = torch.Generator().manual_seed(0)
    M, K, widths = 96, 256, (256, 64, 64)
    ws = [(torch.randn(n, K, generator=g) * 0.02).numpy() for n in widths]
    qs = [q4_from_oracle(oracle_codec, w, "nf4-g128", dev)[0] for w in ws]
    payload = torch.cat([q.payload for q in qs])
    scales = torch.cat([q.scales for q in qs])
    parts = []
    po = so = 0
    for q, n in zip(qs, widths):
        parts.append(ops.Q4Weight(payload[po:po + q.payload.numel()],
                                  scales[so:so + q.scales.numel()], (n, K), "nf4-g128"))
        po += q.payload.numel()
        so += q.scales.numel()
    fused = ops.concat_rows(parts)
    assert fused is not None and fused.segments == widths
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    loras = [_L((torch.randn(r, K, generator=g) * 0.05).to(dev), (torch.randn(n, r, generator=g) * 0.05).to(dev), 8.0)
             for n in widths]
    y = ops.q4_lora_linear(x, fused, loras)
    sep = torch.cat([ops.q4_lora_linear(x, p, [l]) for p, l in zip(parts, loras)], 1)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), sep.view(torch.int16))


@pytest.mark.parametrize("r", [40, 48])
def test_lora_epilogue_from_global_matches_lds(dev, oracle_codec, monkeypatch, r):
    """LoRA operands that do not fit a tile's LDS are read from global memory
    by the 128x128 kernel's epilogue: a fused q|k|v with 3r LoRA columns (120,
    144: beyond the 128x128 tile's LDS) gives the bits of three
    single-segment calls (r columns each, staged in LDS by the same kernel)
    on the same T and B, through the C ABI."""
    monkeypatch.setenv("ST_GEMM_TILE", "128")
    g = torch.Generator().manual_seed(r)
    M, K, widths = 300, 1024, (256, 128, 128)
    ws = [(torch.randn(n, K, generator=g) * 0.02).numpy() for n in widths]
    qs = [q4_from_oracle(oracle_codec, w, "nf4-g128", dev)[0] for w in ws]
    payload = torch.cat([q.payload for q in qs])
    scales = torch.cat([q.scales for q in qs])
    parts = []
    po = so = 0
    for q, n in zip(qs, widths):
        parts.append(ops.Q4Weight(payload[po:po + q.payload.numel()],
                                  scales[so:so + q.scales.numel()], (n, K), "nf4-g128"))
        po += q.payload.numel()
        so += q.scales.numel()
    fused = ops.concat_rows(parts)
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    T = (torch.randn(M, 3 * r, generator=g) * 0.5).to(dev)
    B = (torch.randn(sum(widths), r, generator=g) * 0.05).to(dev)

    def fwd(w, t, b, ends):
        y = torch.empty((M, w.out_features), dtype=BF, device=dev)
        _lib.call("st_q4_linear_fwd", _lib.ptr(x), M, K, K, _lib.ptr(w.payload),
                  _lib.ptr(w.scales), w.out_features, w.lut(), w.flags, _lib.ptr(t), 3 * r,
                  _lib.ptr(b), r, 2.0, len(ends), _lib.i64_array(ends), None, 0, _lib.ptr(y),
                  w.out_features, None, 0, _lib.stream_handle(dev))
        return y

    y = fwd(fused, T, B, [256, 384, 512])
    sep, off = [], 0
    for s_, (p, n) in enumerate(zip(parts, widths)):
        sep.append(fwd(p, T[:, s_ * r:], B[off:off + n], [n]))
        off += n
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), torch.cat(sep, 1).view(torch.int16))


@pytest.mark.parametrize("widths,r", [((256, 128, 128), 8), ((256, 128, 128), 16), ((384,), 64)])
def test_lora_grad_sink_matches_autograd_grads(dev, oracle_codec, widths, r):
    """Adapter gradients deferred to the sink (written into grad_A/grad_B by
    st_rk_batch after autograd) equal the ones the projection's backward
    returns, for a fused q|k|v of three segments: replace, then accumulate
    onto what the buffers hold (the second microbatch of a window)."""
    g = torch.Generator().manual_seed(5)
    M, K = 320, 512
    ws = [(torch.randn(n, K, generator=g) * 0.02).numpy() for n in widths]
    qs = [q4_from_oracle(oracle_codec, w, "nf4-g128", dev)[0] for w in ws]
    payload, scales = torch.cat([q.payload for q in qs]), torch.cat([q.scales for q in qs])
    parts, po, so = [], 0, 0
    for q, n in zip(qs, widths):
        parts.append(ops.Q4Weight(payload[po:po + q.payload.numel()],
                                  scales[so:so + q.scales.numel()], (n, K), "nf4-g128"))
        po, so = po + q.payload.numel(), so + q.scales.numel()
    fused = ops.concat_rows(parts) if len(parts) > 1 else parts[0]
    loras = []
    for n in widths:
        lo = _L((torch.randn(r, K, generator=g) * 0.05).to(dev).requires_grad_(True),
                (torch.randn(n, r, generator=g) * 0.05).to(dev).requires_grad_(True), 16.0)
        lo.grad_A, lo.grad_B = torch.zeros_like(lo.A), torch.zeros_like(lo.B)
        loras.append(lo)
    x = torch.randn(M, K, generator=g).to(BF).to(dev).requires_grad_(True)
    dy = torch.randn(M, sum(widths), generator=g).to(BF).to(dev)
    ab = [t for lo in loras for t in (lo.A, lo.B)]
    ref = torch.autograd.grad(ops.q4_lora_linear(x, fused, loras), [x] + ab, dy)
    prior = [torch.randn(t.shape, generator=g).to(dev) for t in ab]
    for accumulate in (False, True):
        for lo, (pa, pb) in zip(loras, zip(prior[::2], prior[1::2])):
            lo.grad_A.copy_(pa)
            lo.grad_B.copy_(pb)
        with ops.lora_grad_sink(dev, accumulate) as sink:
            got = torch.autograd.grad(ops.q4_lora_linear(x, fused, loras), [x] + ab, dy,
                                      allow_unused=True)
            sink.flush()
        torch.cuda.synchronize()
        assert all(t is None for t in got[1:]) and len(sink.written) == len(loras)
        assert torch.equal(got[0].view(torch.int16), ref[0].view(torch.int16))
        for i, lo in enumerate(loras):
            for buf, want, base in ((lo.grad_A, ref[1 + 2 * i], prior[2 * i]),
                                    (lo.grad_B, ref[2 + 2 * i], prior[2 * i + 1])):
                exp = (base + want) if accumulate else want
                torch.testing.assert_close(buf, exp, rtol=1e-5, atol=1e-6 * exp.abs().max().item())


def test_lora_grad_sink_adapter_used_twice(dev, oracle_codec):
    """An adapter used by two projections in one backward: the first use's
    products go to the sink, the second's come back through autograd, and
    their sum equals the autograd gradients of both uses."""
    g = torch.Generator().manual_seed(9)
    M, K, N, r = 256, 256, 128, 8
    q = q4_from_oracle(oracle_codec, (torch.randn(N, K, generator=g) * 0.02).numpy(),
                       "nf4-g128", dev)[0]
    lo = _L((torch.randn(r, K, generator=g) * 0.05).to(dev).requires_grad_(True),
            (torch.randn(N, r, generator=g) * 0.05).to(dev).requires_grad_(True), 16.0)
    lo.grad_A, lo.grad_B = torch.zeros_like(lo.A), torch.zeros_like(lo.B)
    x1 = torch.randn(M, K, generator=g).to(BF).to(dev)
    x2 = torch.randn(M, K, generator=g).to(BF).to(dev)
    dy = torch.randn(M, N, generator=g).to(BF).to(dev)

    def out():
        return ops.q4_lora_linear(x1, q, [lo]).float() + ops.q4_lora_linear(x2, q, [lo]).float()
    ref = torch.autograd.grad(out(), [lo.A, lo.B], dy.float())
    with ops.lora_grad_sink(dev, False) as sink:
        got = torch.autograd.grad(out(), [lo.A, lo.B], dy.float(), allow_unused=True)
        sink.flush()
    torch.cuda.synchronize()
    assert id(lo) in sink.written and got[0] is not None and got[1] is not None
    for buf, extra, want in ((lo.grad_A, got[0], ref[0]), (lo.grad_B, got[1], ref[1])):
        torch.testing.assert_close(buf + extra, want, rtol=1e-5, atol=1e-6 * want.abs().max().item())


def test_lora_gemm_strided_vs_float64(dev):
    """Both operand orders and layouts; (300, 150) and (97, 2000) have more
    than 64 columns on the fp32 operand's side (the rank-r kernel takes them
    64 at a time)."""
    g = torch.Generator().manual_seed(4)
    for Mo, No, Kc in [(2048, 16, 4096), (16, 4096, 2048), (4096, 16, 2048), (5, 7, 3), (70, 33, 1000),
                       (300, 150, 1024), (97, 2000, 512)]:
        a = torch.randn(Mo, Kc, generator=g).to(BF)
        b = torch.randn(Kc, No, generator=g)
        out = torch.empty(Mo, No, device=dev)
        # a transposed in memory (sam=1) for half the cases to cover both strides
        if Mo % 2:
            at = a.T.contiguous().to(dev)
            ops.lora_gemm(Mo, No, Kc, at, 1, Mo, b.to(dev), No, 1, 0.5, out)
        else:
            ops.lora_gemm(Mo, No, Kc, a.to(dev), Kc, 1, b.to(dev), No, 1, 0.5, out)
        ref = 0.5 * (a.double() @ b.double())
        torch.cuda.synchronize()
        # exact products summed in fp32: |error| ~ 5.5e-7 sqrt(Kc) for N(0, 1)
        # operands (numpy emulation of chunked fp32 sums); 7x margin
        tol = 4e-6 * Kc ** 0.5
        torch.testing.assert_close(out.cpu().double(), ref, rtol=1e-5, atol=tol)
        acc = out.clone()
        ops.lora_gemm(Mo, No, Kc, a.to(dev), Kc, 1, b.to(dev), No, 1, 0.5, acc, accumulate=True)
        torch.testing.assert_close(acc.cpu().double(), 2 * ref, rtol=1e-5, atol=2 * tol)
        # fp32 left operand, bf16 right operand (the dA = dT^T x shape), both layouts of b
        a32 = torch.randn(Mo, Kc, generator=g)
        b16 = torch.randn(Kc, No, generator=g).to(BF)
        ref2 = a32.double() @ b16.double()
        out2 = torch.empty(Mo, No, device=dev)
        ops.lora_gemm(Mo, No, Kc, a32.T.contiguous().to(dev), 1, Mo, b16.to(dev), No, 1, 1.0, out2)
        torch.testing.assert_close(out2.cpu().double(), ref2, rtol=1e-5, atol=tol)
        out3 = torch.empty(Mo, No, device=dev)
        ops.lora_gemm(Mo, No, Kc, a32.to(dev), Kc, 1, b16.T.contiguous().to(dev), 1, Kc, 1.0, out3)
        torch.testing.assert_close(out3.cpu().double(), ref2, rtol=1e-5, atol=tol)


@pytest.mark.parametrize("Kc", [256, 768])
def test_lora_gemm_wide_output_without_split(dev, Kc):
    """The router's input gradient shape: fp32 dlogits [2048, Kc] times a bf16
    router [Kc, 7168].  Enough row tiles and 64-column chunks (56 x 32) to
    fill the GPU, so every workgroup takes the whole contraction and writes
    its outputs directly (one launch, no partials, no reduction); against
    float64, written and accumulated."""
    g = torch.Generator().manual_seed(Kc)
    T, H = 2048, 7168
    dl = torch.randn(T, Kc, generator=g) * 1e-3
    w = (torch.randn(Kc, H, generator=g) * 0.02).to(BF)
    ref = dl.double() @ w.double()
    out = torch.empty(T, H, device=dev)
    ops.lora_gemm(T, H, Kc, dl.to(dev), Kc, 1, w.to(dev), H, 1, 1.0, out)
    torch.cuda.synchronize()
    tol = 4e-6 * Kc ** 0.5 * ref.abs().max().item()
    torch.testing.assert_close(out.cpu().double(), ref, rtol=1e-5, atol=tol)
    ops.lora_gemm(T, H, Kc, dl.to(dev), Kc, 1, w.to(dev), H, 1, 0.5, out, accumulate=True)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu().double(), 1.5 * ref, rtol=1e-5, atol=2 * tol)


def _lora_gemm_ws(dev, Mo, No, Kc, a, sam, sak, b, sbk, sbn, alpha, out, ws_bytes):
    """st_lora_gemm with a workspace of exactly ``ws_bytes``."""
    dt = {BF: _lib.ST_DTYPE_BF16, torch.float32: _lib.ST_DTYPE_F32}
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
    _lib.call("st_lora_gemm", Mo, No, Kc, _lib.ptr(a), dt[a.dtype], sam, sak, _lib.ptr(b),
              dt[b.dtype], sbk, sbn, float(alpha), _lib.ptr(out), out.stride(0), 0, _lib.ptr(ws),
              ws_bytes, _lib.stream_handle(dev))
    torch.cuda.synchronize()


@pytest.mark.parametrize("R", [65, 150])
def test_lora_gemm_chunks_in_one_launch_equal_chunk_by_chunk(dev, R):
    """More than 64 fp32 columns on the split path (too few row tiles to skip
    the split): with the workspace st_lora_gemm_workspace_bytes asks for, every
    64-column chunk runs in one launch and one reduction; with one chunk's
    partials only, the chunks run in turn.  Same splits, same summation order:
    the outputs are equal bit for bit, for the row form (T = x A^T) and the
    column form (dA = dT^T x), and match float64."""
    g = torch.Generator().manual_seed(R)
    M, K = 2048, 4096
    x = torch.randn(M, K, generator=g).to(BF)
    A = torch.randn(R, K, generator=g) * 0.02
    dT = torch.randn(M, R, generator=g)
    xd, Ad, dTd = x.to(dev), A.to(dev), dT.to(dev)
    # split counts (rk_ksplit: 512 workgroups over 128-row tiles, >= 256 contraction
    # elements each): 16 for the 2048 rows x 4096 row form, 8 for the 4096 x 2048 column form
    for Mo, No, Kc, args, big, ks, ref in (
            (M, R, K, (xd, K, 1, Ad, 1, K), M, 16, x.double() @ A.double().T),
            (R, K, M, (dTd, 1, R, xd, K, 1), K, 8, dT.double().T @ x.double())):
        full = _lib.query("st_lora_gemm_workspace_bytes", Mo, No, Kc)
        one = ks * big * 64 * 4  # one 64-column chunk's partials
        assert full >= ks * big * 64 * ((R + 63) // 64) * 4 > one
        outs = []
        for ws_bytes in (full, one):
            out = torch.empty(Mo, No, device=dev)
            _lora_gemm_ws(dev, Mo, No, Kc, *args, 1.0, out, ws_bytes)
            outs.append(out.cpu())
        assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32)), (Mo, No, Kc)
        tol = 4e-6 * Kc ** 0.5 * ref.abs().max().item()
        torch.testing.assert_close(outs[0].double(), ref, rtol=1e-5, atol=tol)
    with pytest.raises(ValueError, match="workspace"):
        out = torch.empty(M, R, device=dev)
        _lora_gemm_ws(dev, M, R, K, xd, K, 1, Ad, 1, K, 1.0, out, ks * M * 64 * 4 - 16)


@pytest.mark.parametrize("Mo,No,Kc", [(2048, 16, 4096), (300, 48, 1024), (16, 64, 2048)])
def test_lora_gemm_carries_fp32_operands_exactly(dev, Mo, No, Kc):
    """The fp32 operand keeps all 24 bits: with a one-hot bf16 operand every
    output is a single product 1 * s, so out == S[perm] bit for bit (a split
    into two bf16 parts would keep ~16 bits and miss by up to ~2^-17
    relative).  Both layouts of the fp32 operand."""
    g = torch.Generator().manual_seed(Mo + Kc)
    perm = torch.randperm(Kc, generator=g)[:Mo] if Mo <= Kc else torch.randint(0, Kc, (Mo,), generator=g)
    a = torch.zeros(Mo, Kc, dtype=BF)
    a[torch.arange(Mo), perm] = 1.0
    b = torch.randn(Kc, No, generator=g) * torch.exp2(torch.randint(-20, 20, (Kc, No), generator=g).float())
    out = torch.empty(Mo, No, device=dev)
    ops.lora_gemm(Mo, No, Kc, a.to(dev), Kc, 1, b.to(dev), No, 1, 1.0, out)
    out_t = torch.empty(Mo, No, device=dev)
    ops.lora_gemm(Mo, No, Kc, a.to(dev), Kc, 1, b.T.contiguous().to(dev), 1, Kc, 1.0, out_t)
    torch.cuda.synchronize()
    want = b[perm]
    assert torch.equal(out.cpu().view(torch.int32), want.view(torch.int32))
    assert torch.equal(out_t.cpu().view(torch.int32), want.view(torch.int32))


def test_q4_linear_full_size_vs_torch_fp32(dev):
    """Llama-3-8B gate|up shape at 2048 tokens against torch fp32 matmul on the
    dequantised weight (bit-exact dequant is pinned above)."""
    g = torch.Generator().manual_seed(1234)
    M, N, K = 2048, 2 * 14336, 4096
    w = torch.randn(N, K, generator=g) * 0.02
    rec = codecs.encode(w, "nf4-g128")
    q = ops.Q4Weight(rec.parts["payload"].to(dev), rec.parts["scales"].to(dev), (N, K), "nf4-g128",
                     (14336, 14336))
    W = q.dequantize()
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    y = ops.q4_lora_linear(x, q, None)
    ref = (x.float() @ W.float().T).to(BF)
    _close_bf16(y, ref, "full-size gate|up")
    dy = torch.randn(M, N, generator=g).to(BF).to(dev)
    xg = x.clone().requires_grad_(True)
    ops.q4_lora_linear(xg, q, None).backward(dy)
    ref_dx = (dy.float() @ W.float()).to(BF)
    _close_bf16(xg.grad, ref_dx, "full-size gate|up dgrad")


@pytest.mark.parametrize("rb", ["1", "0"])
@pytest.mark.parametrize("segments", [(16384, 33024), (32896, 33024)])
def test_q4_linear_tail_split_matches_single_launch(dev, oracle_codec, monkeypatch, segments, rb):
    """Shapes whose last round of tiles would leave CUs idle run as two
    launches over column ranges (256x256 tiles, then 256x128 ones: the
    register-operand pair by default, ST_GEMM_RB=0 the LDS-operand kernel and
    the warp-specialised one).  Every output element keeps its reduction
    order, so the split result equals the single launch bit for bit, LoRA
    segments (one ending before the split column, one straddling it) and
    residual included."""
    monkeypatch.setenv("ST_GEMM_RB", rb)
    g = torch.Generator().manual_seed(77)
    M, K = 512, 256
    N = segments[-1]
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    q, W = q4_from_oracle(oracle_codec, w, "nf4-g128", dev)
    q = ops.Q4Weight(q.payload, q.scales, (N, K), "nf4-g128",
                     (segments[0], segments[1] - segments[0]))
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    res = torch.randn(M, N, generator=g).to(BF).to(dev)
    loras = [_L((torch.randn(8, K, generator=g) * 0.05).to(dev),
                (torch.randn(n, 8, generator=g) * 0.05).to(dev), 16.0) for n in q.segments]
    outs = []
    for split in ("1", "0"):
        monkeypatch.setenv("ST_GEMM_SPLIT", split)
        outs.append(ops.q4_lora_linear(x, q, loras, residual=res))
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    # lora.py:218-220: bf16 base, fp32 adapter term, bf16 sum; then the residual
    ref = (x.float().cpu() @ W.float().T).to(BF).float()
    off = 0
    for lo, n in zip(loras, q.segments):
        ref[:, off:off + n] += (x.float().cpu() @ lo.A.cpu().T) @ lo.B.cpu().T * lo.scale
        off += n
    _close_bf16(outs[0], (ref.to(BF).float() + res.float().cpu()).to(BF), "split fwd")


@pytest.mark.parametrize("tile", ["128", "2562", "256"])
@pytest.mark.parametrize("M,N,K", [(300, 512, 1024), (77, 200, 256), (64, 100, 256)])
def test_vector_epilogue_matches_2byte_epilogue(dev, oracle_codec, monkeypatch, tile, M, N, K):
    """The epilogue that stages each 32x32 block through LDS and moves 16-byte
    rows gives the bits of the one that moves 2-byte elements: forward with
    the LoRA term and a residual, dgrad with the LoRA term, ragged row tiles.
    N = 100 (not a multiple of 8) takes the 2-byte path either way; its dgrad
    is not run (the dgrad contraction must be a multiple of 8)."""
    monkeypatch.setenv("ST_GEMM_TILE", tile)
    g = torch.Generator().manual_seed(M + N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    q, _ = q4_from_oracle(oracle_codec, w, "nf4-g128", dev)
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    res = torch.randn(M, N, generator=g).to(BF).to(dev)
    dy = torch.randn(M, N, generator=g).to(BF).to(dev)
    A = (torch.randn(8, K, generator=g) * 0.05).to(dev)
    Bm = (torch.randn(N, 8, generator=g) * 0.05).to(dev)
    outs = []
    for vec in ("1", "0"):
        monkeypatch.setenv("ST_GEMM_VEC_EPI", vec)
        xd = x.clone().requires_grad_(True)
        lo = _L(A.clone().requires_grad_(True), Bm.clone().requires_grad_(True), 16.0)
        y = ops.q4_lora_linear(xd, q, [lo], residual=res)
        if N % 8 == 0:
            y.backward(dy)
            outs.append((y, xd.grad))
        else:
            outs.append((y,))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("widths,rank", [((512, 128, 128), 16), ((1024, 1024), 8), ((384,), 40)])
def test_lora_bwd_dy_matches_per_product(dev, widths, rank):
    """st_lora_bwd_dy (every segment's dT and dB in one launch) gives the bits of
    the per-product st_lora_gemm calls (same splits, same summation order),
    and both match float64."""
    g = torch.Generator().manual_seed(sum(widths) + rank)
    M, N, nseg = 300, sum(widths), len(widths)
    dy = torch.randn(M, N, generator=g).to(BF).to(dev)
    B = (torch.randn(N, rank, generator=g) * 0.1).to(dev)
    T = torch.randn(M, nseg * rank, generator=g).to(dev)
    scale = 0.75
    ends = _lib.i64_array(torch.tensor(widths).cumsum(0).tolist())
    need = _lib.query("st_lora_bwd_dy_workspace_bytes", M, N, rank, nseg, ends)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    dT = torch.empty(M, nseg * rank, device=dev)
    dB = torch.empty(N, rank, device=dev)
    _lib.call("st_lora_bwd_dy", _lib.ptr(dy), M, N, N, _lib.ptr(B), _lib.ptr(T), T.stride(0), rank,
              nseg, ends, scale, _lib.ptr(dT), dT.stride(0), _lib.ptr(dB), _lib.ptr(ws), need,
              _lib.stream_handle(dev))
    dT2, dB2 = torch.empty_like(dT), torch.empty_like(dB)
    off = 0
    for s, w in enumerate(widths):
        dys = dy[:, off:off + w]
        ops.lora_gemm(M, rank, w, dys, N, 1, B[off:off + w], rank, 1, scale,
                      dT2[:, s * rank:(s + 1) * rank])
        ops.lora_gemm(w, rank, M, dys, 1, N, T[:, s * rank:(s + 1) * rank], T.stride(0), 1, scale,
                      dB2[off:off + w])
        off += w
    torch.cuda.synchronize()
    assert torch.equal(dT, dT2) and torch.equal(dB, dB2)
    off = 0
    for s, w in enumerate(widths):
        dys = dy[:, off:off + w].double()
        torch.testing.assert_close(dT[:, s * rank:(s + 1) * rank].double(),
                                   scale * dys @ B[off:off + w].double(), rtol=1e-5,
                                   atol=1e-4 * w ** 0.5)
        torch.testing.assert_close(dB[off:off + w].double(),
                                   scale * dys.T @ T[:, s * rank:(s + 1) * rank].double(),
                                   rtol=1e-5, atol=1e-4 * M ** 0.5)
        off += w
    # a segment start off the 8-element grid is refused by the query (callers fall back)
    bad = _lib.i64_array([100, N])
    assert _lib.query("st_lora_bwd_dy_workspace_bytes", M, N, rank, 2, bad) == 0


@pytest.mark.parametrize("I,lora,r,tile", [(512, True, 8, None), (384, False, 8, None),
                                         (688, True, 8, None), (512, True, 64, None),
                                         (512, True, 71, None), (512, True, 80, "2562")])
def test_swiglu_input_projection_matches_separate_ops(dev, oracle_codec, monkeypatch, I, lora, r,
                                                      tile):
    """q4_lora_linear(gate|up, W, swiglu=True) == q4_lora_linear(swiglu(gate|up), W):
    the forward and every gradient bit for bit (the dgrad epilogue applies the
    SwiGLU VJP with st_swiglu_bwd's roundings), on the 4-bit path and on the
    bf16 fallback (I % 128 != 0).  Ranks 64 and 71 (128x128) and 80 (256x128
    warp-specialised) leave no LDS for the SwiGLU staging beside the LoRA
    operands, so that dgrad reads them from global memory."""
    if tile is not None:
        monkeypatch.setenv("ST_GEMM_TILE", tile)
    g = torch.Generator().manual_seed(I)
    M, H = 200, 256
    w = (torch.randn(H, I, generator=g) * 0.02).numpy()
    q, _ = q4_from_oracle(oracle_codec, w, "nf4-g128", dev)
    gu0 = torch.randn(M, 2 * I, generator=g).to(BF).to(dev)
    dy = torch.randn(M, H, generator=g).to(BF).to(dev)
    A = torch.randn(r, I, generator=g) * 0.05
    Bm = torch.randn(H, r, generator=g) * 0.05
    outs = []
    for fused in (True, False):
        gu = gu0.clone().requires_grad_(True)
        lo = _L(A.to(dev).requires_grad_(True), Bm.to(dev).requires_grad_(True), 16.0) if lora else None
        if fused:
            y = ops.q4_lora_linear(gu, q, [lo] if lora else None, swiglu=True)
        else:
            y = ops.q4_lora_linear(ops.swiglu(gu, I), q, [lo] if lora else None)
        y.backward(dy)
        outs.append((y, gu.grad) + ((lo.A.grad, lo.B.grad) if lora else ()))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a.view(torch.int16),
                           b.view(torch.int32) if b.dtype == torch.float32 else b.view(torch.int16))


@pytest.mark.parametrize("D,pad", [(128, 0), (64, 0), (64, 4)])
def test_rope_qkv_fused_matches_separate_calls(dev, D, pad):
    """st_rope_qkv_fwd/bwd (one launch for q, k and v of a fused q|k|v row)
    give the bits of three st_rope_fwd/bwd calls; pad = 4 makes the row
    stride not a multiple of 8 (the per-segment path)."""
    g = torch.Generator().manual_seed(D + pad)
    B, S, H, Hkv = 2, 40, 4, 2
    W = (H + 2 * Hkv) * D
    big = torch.randn(B * S, W + pad, generator=g).to(BF).to(dev)
    y = big[:, :W]
    ang = torch.randn(B, S, D, generator=g)
    cos, sin = ang.cos().to(BF).to(dev), ang.sin().to(BF).to(dev)
    st = _lib.stream_handle(dev)
    outs = [torch.empty(B, h, S, D, dtype=BF, device=dev) for h in (H, Hkv, Hkv)]
    _lib.call("st_rope_qkv_fwd", _lib.ptr(y), y.stride(0), _lib.ptr(cos), _lib.ptr(sin), B, S, H,
              Hkv, D, *(_lib.ptr(o) for o in outs), st)
    refs = [torch.empty_like(o) for o in outs]
    for r, off, h, rot in zip(refs, (0, H * D, (H + Hkv) * D), (H, Hkv, Hkv), (1, 1, 0)):
        _lib.call("st_rope_fwd", _lib.ptr(y[:, off:]), y.stride(0), _lib.ptr(cos), _lib.ptr(sin),
                  B, S, h, D, rot, _lib.ptr(r), st)
    grads = [torch.randn(o.shape, generator=g).to(BF).to(dev) for o in outs]
    dbig = torch.zeros(B * S, W + pad, dtype=BF, device=dev)
    dx = dbig[:, :W]
    _lib.call("st_rope_qkv_bwd", *(_lib.ptr(t) for t in grads), _lib.ptr(cos), _lib.ptr(sin), B, S,
              H, Hkv, D, _lib.ptr(dx), dx.stride(0), st)
    dref = torch.zeros_like(dbig)
    for gr, off, h, rot in zip(grads, (0, H * D, (H + Hkv) * D), (H, Hkv, Hkv), (1, 1, 0)):
        _lib.call("st_rope_bwd", _lib.ptr(gr), _lib.ptr(cos), _lib.ptr(sin), B, S, h, D, rot,
                  _lib.ptr(dref[:, off:]), dref.stride(0), st)
    torch.cuda.synchronize()
    for a, b in zip(outs + [dbig], refs + [dref]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))

@pytest.mark.parametrize("D,H,Hkv", [(128, 4, 2), (64, 6, 2), (128, 32, 8)])
def test_rope_qkv_norm_matches_norm_then_rope(dev, D, H, Hkv):
    """st_rope_qkv_norm_fwd/bwd (Qwen3's per-head q/k RMSNorm fused with the
    rotation) against the separate ops it replaces: st_rmsnorm_fwd/bwd on the
    head rows, then st_rope_qkv_fwd/bwd.  The rounding points are the same;
    only the fp32 order of the per-head sums differs (the fused kernel sums a
    head across 16 lanes), so outputs and gradients agree to one bf16 ulp."""
    g = torch.Generator().manual_seed(D + H)
    B, S = 2, 40
    W = (H + 2 * Hkv) * D
    y = (torch.randn(B * S, W, generator=g) * 3).to(BF).to(dev)
    wq = (1 + 0.2 * torch.randn(D, generator=g)).to(BF).to(dev)
    wk = (1 + 0.2 * torch.randn(D, generator=g)).to(BF).to(dev)
    ang = torch.randn(B, S, D, generator=g)
    cos, sin = ang.cos().to(BF).to(dev), ang.sin().to(BF).to(dev)
    eps = 1e-6
    yf = y.clone().requires_grad_(True)
    q, k, v = ops.rope_qkv_norm(yf, B, S, H, Hkv, D, cos, sin, wq, wk, eps)
    yr = y.clone().requires_grad_(True)
    nq, nk = H * D, Hkv * D
    qn = ops.rms_norm(yr[:, :nq].reshape(-1, D), wq, eps).reshape(B * S, -1)
    kn = ops.rms_norm(yr[:, nq:nq + nk].reshape(-1, D), wk, eps).reshape(B * S, -1)
    qr, kr, vr = ops.rope_qkv(torch.cat((qn, kn, yr[:, nq + nk:]), 1), B, S, H, Hkv, D, cos, sin)
    grads = [torch.randn(t.shape, generator=g).to(BF).to(dev) for t in (q, k, v)]
    torch.autograd.backward((q, k, v), grads)
    torch.autograd.backward((qr, kr, vr), grads)
    torch.cuda.synchronize()

    def ulp_close(a, b, what):
        a, b = a.float().cpu(), b.float().cpu()
        err = (a - b).abs()
        tol = b.abs().clamp_min(2 ** -20) * 2 ** -7 + 1e-30
        assert bool((err <= tol).all()), f"{what}: beyond one bf16 ulp"
        assert (err == 0).float().mean().item() > 0.97, f"{what}: too many 1-ulp differences"
    for a, b, n in ((q, qr, "q"), (k, kr, "k"), (v, vr, "v"), (yf.grad, yr.grad, "dy")):
        ulp_close(a, b, n)
    assert torch.equal(v.view(torch.int16), vr.view(torch.int16))


@pytest.mark.parametrize("M,N,K,ldw_pad", [(64, 256, 256, 0), (100, 384, 520, 8), (37, 1000, 136, 0),
                                           (1024, 4096, 2048, 0), (1800, 6200, 6152, 8)])
def test_linear_bf16_fwd_and_dgrad_vs_fp32(dev, M, N, K, ldw_pad):
    """The plain bf16 GEMMs (terminal head, MoE router): y = bf16(x W^T) and
    dx = bf16(dy W) with fp32 accumulation against torch fp32 matmul, ragged
    M/N/K and a padded W row stride; the last shape takes the 256x256 tiles
    both ways (>= 192 tiles)."""
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(BF)
    dy = torch.randn(M, N, generator=g).to(BF)
    wbig = (torch.randn(N, K + ldw_pad, generator=g) * 0.05).to(BF)
    w = wbig[:, :K]
    y = ops.linear_bf16(x.to(dev), wbig.to(dev)[:, :K])
    dx = ops.linear_bf16_dgrad(dy.to(dev), wbig.to(dev)[:, :K])
    torch.cuda.synchronize()
    _close_bf16(y, (x.float() @ w.float().T).to(BF), f"bf16 fwd {M}x{N}x{K}")
    _close_bf16(dx, (dy.float() @ w.float()).to(BF), f"bf16 dgrad {M}x{N}x{K}")
