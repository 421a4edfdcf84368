"""Causal-LM terminal on the HIP path (RMSNorm + token-chunked head GEMM +
in-place cross-entropy/gradient + GEMM back) against the CPU oracle of
training/engine.py:58-79 (oracle.layer.causal_lm_terminal).  Loss within
1e-4 relative (fp32 sums in another order), gradients within bf16 tolerance."""
import pytest
import torch
import torch.nn.functional as F

from oracle import layer as OL
from spilltune_amd import ops

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def rel(a, b):
    a, b = a.float().cpu(), b.float().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def cosine(a, b):
    a, b = a.double().cpu().reshape(-1), b.double().cpu().reshape(-1)
    return (a @ b / (a.norm() * b.norm()).clamp_min(1e-300)).item()


def case(B, S, H, V, chunk, seed, ignore_every=0, dead_chunk=False, oracle_chunk=None):
    g = torch.Generator().manual_seed(seed)
    hidden = torch.randn(B, S, H, generator=g).to(BF)
    norm = (1 + 0.1 * torch.randn(H, generator=g)).to(BF)
    head = (0.05 * torch.randn(V, H, generator=g)).to(BF)
    labels = torch.randint(0, V, (B, S), generator=g)
    labels[:, 0] = -100
    if ignore_every:
        labels[:, ::ignore_every] = -100
    if dead_chunk:
        labels[:, 1:chunk + 1] = -100  # the first chunk has no supervised target
    normalization = float((labels[:, 1:] != -100).sum().clamp_min(1))
    # the oracle's chunking does not change the sum it computes; a smaller
    # chunk only bounds its fp32 logits in host memory
    loss_ref, grad_ref = OL.causal_lm_terminal(hidden, norm, head, labels, eps=1e-5,
                                               normalization=normalization,
                                               token_chunk=oracle_chunk or chunk)
    dev = torch.device("cuda:0")
    x = hidden.to(dev).requires_grad_(True)
    normalized = ops.rms_norm(x.view(B * S, H), norm.to(dev), 1e-5).view(B, S, H)
    # host labels: checked and turned into supervised chunks on the host
    loss = ops.chunked_causal_loss(normalized, head.to(dev), labels,
                                   normalization=normalization, token_chunk=chunk)
    (gx,) = torch.autograd.grad(loss, x)
    torch.cuda.synchronize()
    got = float(loss.detach())
    assert abs(got - loss_ref) <= 1e-4 * abs(loss_ref), (got, loss_ref)
    assert rel(gx, grad_ref) < 2e-2 and cosine(gx, grad_ref) > 0.999, (rel(gx, grad_ref),
                                                                      cosine(gx, grad_ref))


def test_terminal_tiny_llama_vocab():
    case(2, 128, 256, 1024, 64, 0)


def test_terminal_ignored_targets_and_unsupervised_chunk():
    case(2, 130, 256, 1024, 48, 1, ignore_every=3, dead_chunk=True)


def test_terminal_qwen3_vocab_rows():
    case(1, 96, 512, 151936, 40, 2)


@pytest.mark.timeout(600)
def test_terminal_qwen3_vocab_row_split():
    """Config 3's vocabulary with a token chunk of 2 x 4095 = 8190 rows: the
    bf16 logits block would pass the GEMM's 2 GiB operand limit, so the chunk
    runs as 7067 + 1123 rows (ops._ChunkedCE's row split)."""
    V = 151936
    assert 2 * 4095 > ((1 << 31) - 1) // (2 * V)
    case(2, 4096, 128, V, 4096, 4, ignore_every=5, oracle_chunk=512)


def test_terminal_device_labels_with_prepared_chunks():
    """Device labels with startup-prepared chunks (the reference's CUDA
    terminal contract, native_terminal.py:39-47): no host scan, same loss."""
    g = torch.Generator().manual_seed(5)
    B, S, H, V, chunk = 2, 64, 128, 512, 16
    hidden = torch.randn(B, S, H, generator=g).to(BF)
    head = (0.05 * torch.randn(V, H, generator=g)).to(BF)
    labels = torch.randint(0, V, (B, S), generator=g)
    chunks = ops.supervised_chunk_intervals(labels, chunk)
    dev = torch.device("cuda:0")
    h = hidden.to(dev)
    host = ops.chunked_causal_loss(h, head.to(dev), labels, normalization=100.0,
                                   token_chunk=chunk)
    device = ops.chunked_causal_loss(h, head.to(dev), labels.to(dev), normalization=100.0,
                                     token_chunk=chunk, supervised_chunks=chunks)
    assert float(host) == float(device)


def test_cross_entropy_rows_matches_fp32_softmax():
    """The row kernel alone: loss and bf16 gradient against fp32 torch math,
    including a row of equal logits, an ignored row and a non-multiple-of-8 row stride."""
    g = torch.Generator().manual_seed(3)
    rows, V, ld = 6, 1000, 1003
    x = torch.randn(rows, ld, generator=g).mul(4).to(BF)
    x[2, :V] = 1.5
    labels = torch.randint(0, V, (rows,), generator=g)
    labels[4] = -100
    ref = x[:, :V].float()
    lse = torch.logsumexp(ref, 1)
    valid = labels != -100
    loss_ref = torch.where(valid, lse - ref[torch.arange(rows), labels.clamp_min(0)], torch.zeros(()))
    p = torch.softmax(ref, 1)
    onehot = F.one_hot(labels.clamp_min(0), V).float()
    grad_ref = ((p - onehot) * 0.125 * valid[:, None]).to(BF)
    dev = torch.device("cuda:0")
    xd = x.to(dev)
    loss = torch.empty(rows, device=dev)
    from spilltune_amd import _lib
    _lib.call("st_cross_entropy_rows", _lib.ptr(xd), rows, V, ld, _lib.ptr(labels.to(dev)), -100,
              0.125, _lib.ptr(loss), _lib.stream_handle(dev))
    torch.cuda.synchronize()
    assert torch.allclose(loss.cpu(), loss_ref, rtol=1e-5, atol=1e-5)
    got = xd.cpu()
    assert (got[:, :V].float() - grad_ref.float()).abs().max() <= 2 ** -7 * 0.125  # one bf16 ulp
    assert torch.equal(got[:, V:], x[:, V:])  # padding columns untouched
