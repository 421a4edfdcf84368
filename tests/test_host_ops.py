"""Host-side logic of the differentiable ops that runs before any kernel
(CPU only): when fused projections may share one weight view, and the
terminal's label rules (native_terminal.py:39-47: device labels are never
scanned on the host)."""
import pytest
import torch

from spilltune_amd import ops


def _q4(payload, scales, rows, K=128):
    return ops.Q4Weight(payload, scales, (rows, K), "nf4-g128")


def test_concat_rows_views_one_storage():
    rows = (64, 32)
    K = 128
    pay = torch.zeros(sum(rows) * K // 2, dtype=torch.uint8)
    sc = torch.ones(sum(rows) * K // 128, dtype=torch.float32)
    a = _q4(pay[:rows[0] * K // 2], sc[:rows[0]], rows[0])
    b = _q4(pay[rows[0] * K // 2:], sc[rows[0]:], rows[1])
    fused = ops.concat_rows([a, b])
    assert fused is not None and fused.shape == (96, K) and fused.segments == rows
    assert fused.payload.data_ptr() == pay.data_ptr() and fused.payload.numel() == pay.numel()
    assert fused.scales.numel() == sc.numel()


def test_concat_rows_rejects_adjacent_separate_allocations():
    """Two allocations that lie back to back in memory are not one buffer:
    the fused view would run off the first storage."""
    K = 128
    raw_p = bytearray(96 * K // 2)
    raw_s = bytearray(96 * K // 128 * 4)
    pa = torch.frombuffer(raw_p, dtype=torch.uint8, count=64 * K // 2, offset=0)
    pb = torch.frombuffer(raw_p, dtype=torch.uint8, count=32 * K // 2, offset=64 * K // 2)
    sa = torch.frombuffer(raw_s, dtype=torch.float32, count=64, offset=0)
    sb = torch.frombuffer(raw_s, dtype=torch.float32, count=32, offset=64 * 4)
    assert pa.data_ptr() + pa.numel() == pb.data_ptr()          # adjacent pointers ...
    assert pa.untyped_storage().data_ptr() != pb.untyped_storage().data_ptr()  # ... two storages
    assert ops.concat_rows([_q4(pa, sa, 64), _q4(pb, sb, 32)]) is None
    # one storage but a gap between the parts is not adjacent either
    pay = torch.zeros(100 * K // 2, dtype=torch.uint8)
    sc = torch.ones(100, dtype=torch.float32)
    a = _q4(pay[:64 * K // 2], sc[:64], 64)
    b = _q4(pay[68 * K // 2:], sc[68:], 32)
    assert ops.concat_rows([a, b]) is None


def test_terminal_device_labels_need_prepared_chunks():
    normalized = torch.zeros(1, 8, 16, dtype=torch.bfloat16, device="meta")
    head = torch.zeros(32, 16, dtype=torch.bfloat16, device="meta")
    labels = torch.zeros(1, 8, dtype=torch.int64, device="meta")
    with pytest.raises(RuntimeError, match="prepared supervised chunks"):
        ops.chunked_causal_loss(normalized, head, labels, normalization=7.0, token_chunk=4)
    with pytest.raises(RuntimeError, match="host labels"):
        ops.supervised_chunk_intervals(labels, 4)


def test_supervised_chunk_intervals_host_rule():
    labels = torch.full((2, 10), -100)
    labels[1, 6] = 3                       # only the target of position 5 is supervised
    assert ops.supervised_chunk_intervals(labels, 4) == ((4, 8),)
    with pytest.raises(ValueError, match="token chunk"):
        ops.supervised_chunk_intervals(labels, 0)


def test_router_parts_sum_exactly_and_follow_the_version():
    """The fp32 router's bf16 parts [hi; mid; lo] (the operand of its input
    gradient on the rank-r kernel) sum back to every fp32 value exactly,
    including values far from 1 and with low-order bits set; they are kept
    on the tensor and remade only after an in-place change (version)."""
    from spilltune_amd import moe
    g = torch.Generator().manual_seed(5)
    E, H = 8, 96
    w = torch.randn(E, H, generator=g) * torch.exp2(torch.randint(-30, 30, (E, H), generator=g).float())
    w[0, :4] = torch.tensor([1.0 + 2 ** -23, -(2 - 2 ** -22), 2 ** -100, 3.0e20])
    parts = moe._router_parts(w)
    assert parts.shape == (3 * E, H) and parts.dtype == torch.bfloat16
    back = parts[:E].double() + parts[E:2 * E].double() + parts[2 * E:].double()
    assert torch.equal(back, w.double())
    assert moe._router_parts(w) is parts  # unchanged tensor: the kept split
    w.mul_(0.5)
    again = moe._router_parts(w)
    assert again is not parts
    back = again[:E].double() + again[E:2 * E].double() + again[2 * E:].double()
    assert torch.equal(back, w.double())
