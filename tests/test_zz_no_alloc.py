"""The allocation-free LoRA product (st_lora_gemm_noalloc, static device
scratch) against the workspace entry point st_lora_gemm, through the C ABI:
bit-equal outputs on two calls in a row, the second with a smaller input
(the scratch keeps the first call's partials), on both kernel paths (the
streaming rank-r MFMA path and the generic fp32 path), plus the size limit."""
import ctypes

import pytest
import torch

from spilltune_amd import _lib

pytestmark = pytest.mark.gpu
BF = torch.bfloat16
DT = {BF: _lib.ST_DTYPE_BF16, torch.float32: _lib.ST_DTYPE_F32}


def _run(noalloc, Mo, No, Kc, a, sam, sak, b, sbk, sbn, alpha, out, accumulate, dev):
    st = _lib.stream_handle(dev)
    if noalloc:
        _lib.call("st_lora_gemm_noalloc", Mo, No, Kc, _lib.ptr(a), DT[a.dtype], sam, sak,
                  _lib.ptr(b), DT[b.dtype], sbk, sbn, float(alpha), _lib.ptr(out), out.stride(0),
                  int(accumulate), st)
    else:
        need = _lib.query("st_lora_gemm_workspace_bytes", Mo, No, Kc)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        _lib.call("st_lora_gemm", Mo, No, Kc, _lib.ptr(a), DT[a.dtype], sam, sak, _lib.ptr(b),
                  DT[b.dtype], sbk, sbn, float(alpha), _lib.ptr(out), out.stride(0),
                  int(accumulate), _lib.ptr(ws), ws.numel(), st)
        torch.cuda.synchronize()
        del ws


def _case(dev, g, M, K, R, a_dtype, accumulate=False):
    """T = alpha * x A^T (x [M, K] bf16, A [R, K]) plus a column-form product
    dA = dT^T x ([R, K], contraction over M)."""
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    A = (torch.randn(R, K, generator=g) * 0.02).to(a_dtype).to(dev)
    dT = torch.randn(M, R, generator=g).to(dev)
    outs = []
    for noalloc in (False, True):
        T = torch.full((M, R), 0.5, device=dev)
        dA = torch.full((R, K), -0.25, device=dev)
        _run(noalloc, M, R, K, x, K, 1, A, 1, K, 0.75, T, accumulate, dev)
        _run(noalloc, R, K, M, dT, 1, R, x, K, 1, 1.0, dA, accumulate, dev)
        torch.cuda.synchronize()
        outs.append((T.cpu(), dA.cpu()))
    return outs


@pytest.mark.parametrize("a_dtype", [torch.float32, BF])
def test_noalloc_equals_workspace_entry_two_calls(dev, a_dtype):
    g = torch.Generator().manual_seed(11)
    # first call large (fills the scratch), second smaller: stale partials of
    # the first call must not leak into the second
    for M, K, R, acc in ((2048, 4096, 48, False), (300, 1024, 16, True)):
        (t0, a0), (t1, a1) = _case(dev, g, M, K, R, a_dtype, acc)
        assert torch.equal(t0, t1) and torch.equal(a0, a1), (M, K, R)


def test_noalloc_generic_path_and_limit(dev):
    """A product with more than 64 output columns on both sides runs the
    generic fp32 kernel; the same two-call check, then a product whose
    partials exceed the static scratch is rejected before any launch."""
    g = torch.Generator().manual_seed(12)
    for Mo, No, Kc in ((256, 96, 640), (64, 80, 200)):
        a = torch.randn(Mo, Kc, generator=g).to(dev)
        b = torch.randn(Kc, No, generator=g).to(dev)
        res = []
        for noalloc in (False, True):
            out = torch.zeros(Mo, No, device=dev)
            _run(noalloc, Mo, No, Kc, a, Kc, 1, b, No, 1, 1.0, out, False, dev)
            torch.cuda.synchronize()
            res.append(out.cpu())
        assert torch.equal(res[0], res[1]), (Mo, No, Kc)
    big = (1 << 14, 1 << 10, 1 << 16)
    assert _lib.query("st_lora_gemm_workspace_bytes", *big) > 32 << 20
    with pytest.raises(ValueError, match="static scratch"):
        _lib.call("st_lora_gemm_noalloc", *big, ctypes.c_void_p(16), _lib.ST_DTYPE_F32, 1, 1,
                  ctypes.c_void_p(16), _lib.ST_DTYPE_F32, 1, 1, 1.0, ctypes.c_void_p(16),
                  big[1], 0, _lib.stream_handle(dev))
