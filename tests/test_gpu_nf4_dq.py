"""bitsandbytes NF4 + double-quantisation state on the GPU, through the C ABI
(MI355X only): the device conversion of the block statistics bit-exact
against the oracle, and the fused GEMMs reading the state's packed bytes as
they lie (group 64, high nibble first) against the oracle's decode.

bitsandbytes itself is absent (no reference test holds its bytes), so the
states come from the oracle's test encoder; the decode of a given state is
what is checked, exactly."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from spilltune_amd import _lib, nf4_state, ops

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def _bits(b):
    return torch.from_numpy(np.asarray(b, dtype=np.uint16).astype(np.int16)).view(BF)


def _state(oc, w, seed=0):
    """(packed [bytes,1], parts, exact bf16 W on the CPU) of a test state."""
    packed, q, nested, off, m = oc.encode_nf4_dq(w)
    meta = {"quant_type": "nf4", "blocksize": 64, "dtype": "bfloat16", "shape": list(w.shape),
            "nested_blocksize": 256, "nested_dtype": "float32", "nested_offset": off}
    parts = {"absmax": torch.from_numpy(q), "nested_absmax": torch.from_numpy(nested),
             "nested_quant_map": torch.from_numpy(m), "quant_map": torch.tensor(oc.NF4_LUT),
             nf4_state.PACKED_STATE_KEY: nf4_state.pack_metadata(meta)}
    absmax = oc.dq_absmax(q, nested, m, off)
    W = _bits(oc.decode4(packed, absmax, w.size, lut=oc.NF4_LUT, group=64,
                         hi_first=True)).view(w.shape)
    return torch.from_numpy(packed).view(-1, 1), parts, W


@pytest.mark.parametrize("blocks", [1, 255, 256 * 3 + 77, 1_000_003])
def test_dq_scales_device_bit_exact(dev, oracle_codec, blocks):
    rng = np.random.default_rng(blocks)
    q = rng.integers(0, 256, blocks, dtype=np.uint8)
    nested = (rng.random((blocks + 255) // 256, dtype=np.float32) * 0.05).astype(np.float32)
    m = oracle_codec.dynamic_map()
    for off in (0.0, float(np.float32(0.0123456))):
        got = nf4_state.dq_scales_device(torch.from_numpy(q).to(dev), torch.from_numpy(nested).to(dev),
                                         torch.from_numpy(m).to(dev), off)
        torch.cuda.synchronize()
        expect = oracle_codec.dq_absmax(q, nested, m, off)
        assert torch.equal(got.cpu().view(torch.int32), torch.from_numpy(expect).view(torch.int32))


def test_dq_scales_device_rounds_the_product_before_the_offset(dev, oracle_codec):
    """(1 + 2**-12)/2 * 2(1 + 2**-12) - 1: 2**-11 with the product rounded,
    2**-11 + 2**-24 if the kernel fused the multiply and the add."""
    m = np.zeros(256, np.float32)
    m[9] = np.float32((1 + 2.0 ** -12) / 2)
    q = np.array([9], dtype=np.uint8)
    nested = np.array([2 * (1 + 2.0 ** -12)], dtype=np.float32)
    got = nf4_state.dq_scales_device(torch.from_numpy(q).to(dev), torch.from_numpy(nested).to(dev),
                                     torch.from_numpy(m).to(dev), -1.0)
    assert got.item() == 2.0 ** -11


def _close_bf16(got, ref, what):
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs()
    ulp = ref.abs().clamp_min(2 ** -20) * 2 ** -7
    frac_bad = (err > ulp + 1e-6).float().mean().item()
    rel = (err.norm() / ref.norm().clamp_min(1e-20)).item()
    assert rel < 4e-3 and frac_bad < 1e-3, f"{what}: rel {rel:.3e}, >1ulp fraction {frac_bad:.2e}"


class _L:
    def __init__(self, A, B, alpha):
        self.A, self.B, self.alpha = A, B, alpha
        self.rank = A.shape[0]
        self.scale = alpha / self.rank


@pytest.mark.parametrize("tile", ["128", "2562", "256", "2566"])
@pytest.mark.parametrize("M,N,K", [(100, 384, 512), (64, 256, 192), (37, 96, 320), (130, 136, 200),
                                   (5, 40, 8)])
@pytest.mark.parametrize("lora", [False, True])
def test_group64_linear_fwd_dgrad_vs_oracle(dev, oracle_codec, monkeypatch, tile, M, N, K, lora):
    """A staged state through the fused forward and dgrad (and the LoRA
    gradients) against autograd over the oracle's decode of the same bytes.
    K % 64 == 0 reads one scale per k-step of 64 on every tile (K = 192, 320:
    not multiples of 128); K % 64 != 0 takes the flat-group kernel; the
    register-operand tile (2566) is not built for 64-element groups and its
    request runs on 128x128."""
    monkeypatch.setenv("ST_GEMM_TILE", tile)
    g = torch.Generator().manual_seed(M + 3 * N + K)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    packed, parts, W = _state(oracle_codec, w)
    staged = nf4_state.PinnedNF4State(packed, parts).stage(dev)
    x = torch.randn(M, K, generator=g).to(BF)
    dy = torch.randn(M, N, generator=g).to(BF)
    r, alpha = 8, 16.0
    A = torch.randn(r, K, generator=g) * 0.05
    B = torch.randn(N, r, generator=g) * 0.05
    xr = x.clone().requires_grad_(True)
    Ar, Br = A.clone().requires_grad_(True), B.clone().requires_grad_(True)
    base = F.linear(xr, W)
    out = (base.float() + F.linear(F.linear(xr.float(), Ar), Br) * (alpha / r)).to(BF) if lora else base
    out.backward(dy)
    xd = x.to(dev).requires_grad_(True)
    lo = _L(A.to(dev).requires_grad_(True), B.to(dev).requires_grad_(True), alpha)
    staged.wait_on(torch.cuda.current_stream(dev))
    y = ops.q4_lora_linear(xd, staged.weight, [lo] if lora else None)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    _close_bf16(y, out, f"g64 fwd {M}x{N}x{K} tile{tile}")
    _close_bf16(xd.grad, xr.grad, f"g64 dgrad {M}x{N}x{K} tile{tile}")
    if lora:
        # fp32 reductions in another order: tolerance scaled to the gradient's magnitude
        for got, ref in ((lo.A.grad.cpu(), Ar.grad), (lo.B.grad.cpu(), Br.grad)):
            torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-5 * ref.abs().max().item())


def test_group64_dequant_and_linear_cuda_shapes(dev, oracle_codec):
    """linear_cuda on a [B, S, K] input (nf4_backend_cuda.py:888-917) equals
    the 2-D call, and the staged weight's standalone decode equals the
    oracle bit for bit."""
    g = torch.Generator().manual_seed(7)
    w = (torch.randn(256, 192, generator=g) * 0.02).numpy()
    packed, parts, W = _state(oracle_codec, w)
    staged = nf4_state.PinnedNF4State(packed, parts).stage(dev)
    staged.synchronize_ready()
    assert torch.equal(staged.weight.dequantize().cpu().view(torch.int16), W.view(torch.int16))
    x = torch.randn(2, 33, 192, generator=g).to(BF).to(dev)
    y = nf4_state.linear_cuda(x, staged)
    y2 = ops.q4_lora_linear(x.reshape(-1, 192), staged.weight, None)
    torch.cuda.synchronize()
    assert y.shape == (2, 33, 256)
    assert torch.equal(y.reshape(-1, 256).view(torch.int16), y2.view(torch.int16))
    with pytest.raises(ValueError, match="does not match NF4 weight size"):
        nf4_state.linear_cuda(torch.zeros(4, 100, dtype=BF, device=dev), staged)
    with pytest.raises(TypeError, match="bfloat16"):
        nf4_state.linear_cuda(torch.zeros(4, 192, device=dev), staged)


@pytest.mark.parametrize("M,N,K", [(2048, 6144, 4096), (2048, 4096, 14336)])
def test_group64_llama_shapes_vs_fp32_matmul(dev, oracle_codec, M, N, K):
    """Llama-8B projection shapes (q|k|v forward; down with its 14336-long
    contraction) on the default dispatch with 64-element groups (the 256x256
    LDS-operand forward and the warp-specialised dgrad), against torch fp32
    matmul of the standalone decode, which the test above pins to the
    oracle."""
    rng = np.random.default_rng(M + N)
    blocks = N * K // 64
    q = torch.from_numpy(rng.integers(0, 256, blocks, dtype=np.uint8)).to(dev)
    nested = torch.from_numpy((rng.random((blocks + 255) // 256, dtype=np.float32) * 0.02)).to(dev)
    m = torch.from_numpy(oracle_codec.dynamic_map()).to(dev)
    scales = nf4_state.dq_scales_device(q, nested, m, 0.01)
    payload = torch.from_numpy(rng.integers(0, 256, N * K // 2, dtype=np.uint8)).to(dev)
    wt = ops.Q4Weight(payload, scales, (N, K), nf4_state.CODEC, flags=nf4_state.FLAGS)
    W = wt.dequantize().float()
    x = torch.randn(M, K, device=dev).to(BF)
    dy = torch.randn(M, N, device=dev).to(BF)
    xd = x.clone().requires_grad_(True)
    y = ops.q4_lora_linear(xd, wt, None)
    y.backward(dy)
    ref_y = (x.float() @ W.T).to(BF)
    ref_dx = (dy.float() @ W).to(BF)
    torch.cuda.synchronize()
    _close_bf16(y, ref_y, f"g64 fwd {M}x{N}x{K}")
    _close_bf16(xd.grad, ref_dx, f"g64 dgrad {M}x{N}x{K}")
