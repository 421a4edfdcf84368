"""bitsandbytes NF4 + double-quantisation state (CPU): the oracle's block
statistics pinned by closed forms, the product's host conversion against the
oracle, and the reference's state rules (nf4_backend.py:184-240,
nf4_backend_cuda.py:314-380 of /root/reference/src/ram_vram_finetune)."""
import numpy as np
import pytest
import torch

from spilltune_amd import nf4_state

F32 = np.float32


# --------------------------------------------------------- oracle statistics
def test_zero_map_gives_the_offset_exactly(oracle_codec):
    rng = np.random.default_rng(0)
    q = rng.integers(0, 256, 1000, dtype=np.uint8)
    nested = rng.random(4, dtype=np.float32) * 3
    out = oracle_codec.dq_absmax(q, nested, np.zeros(256, F32), 0.8125)
    assert np.all(out == F32(0.8125))


def test_nested_scale_changes_every_256_blocks(oracle_codec):
    """nested[k] = 2**k with a map of ones: block j reads 2**(j // 256); an
    index of j // 64 (the primary blocksize) would read 2**(j // 64)."""
    blocks = 256 * 3 + 77
    nested = F32(2.0) ** np.arange(4, dtype=F32)
    m = np.ones(256, F32)
    q = np.arange(blocks, dtype=np.int64).astype(np.uint8)
    out = oracle_codec.dq_absmax(q, nested, m, 0.0)
    np.testing.assert_array_equal(out, (2.0 ** (np.arange(blocks) // 256)).astype(F32))


def test_offset_is_added_after_the_rounded_product(oracle_codec):
    """Exact dyadic case: map 0.75, nested 3 -> 2.25, + 0.5 = 2.75 (scaling the
    offset, 0.75 * (3 + 0.5) = 2.625, fails).  Rounding case: a = (1 +
    2**-12) / 2, b = 2 (1 + 2**-12): a*b = 1 + 2**-11 + 2**-24 rounds (tie to
    even) to 1 + 2**-11 in fp32, so with offset -1 the result is 2**-11; a
    fused multiply-add would keep 2**-11 + 2**-24."""
    m = np.zeros(256, F32)
    m[5] = 0.75
    a = F32((1 + 2.0 ** -12) / 2)
    m[9] = a
    q = np.array([5, 9], dtype=np.uint8)
    assert oracle_codec.dq_absmax(q[:1], np.array([3.0], F32), m, 0.5)[0] == F32(2.75)
    b = F32(2 * (1 + 2.0 ** -12))
    got = oracle_codec.dq_absmax(q[1:], np.array([b], F32), m, -1.0)[0]
    assert got == F32(2.0 ** -11)
    assert got != F32(2.0 ** -11 + 2.0 ** -24)


def test_power_of_two_operands_are_exact(oracle_codec):
    """Map entries k/128, nested scales 2**e and a dyadic offset: every step is
    exact, so the result equals Python float arithmetic."""
    rng = np.random.default_rng(3)
    m = (np.arange(256, dtype=F32) - 128) / F32(128)
    blocks = 256 * 5 + 13
    q = rng.integers(0, 256, blocks, dtype=np.uint8)
    e = rng.integers(-6, 6, 6)
    nested = (2.0 ** e).astype(F32)
    off = 0.375
    out = oracle_codec.dq_absmax(q, nested, m, off)
    expect = [float(m[q[j]]) * float(nested[j // 256]) + off for j in range(blocks)]
    np.testing.assert_array_equal(out, np.array(expect, dtype=F32))


def test_dynamic_map_shape(oracle_codec):
    m = oracle_codec.dynamic_map()
    assert m.dtype == F32 and m.size == 256 and np.all(np.diff(m) >= 0)
    assert m[-1] == 1.0 and (m == 0).sum() == 1 and np.all(np.abs(m) <= 1)
    np.testing.assert_array_equal(m[(m > 0) & (m < 1)], -m[m < 0][::-1])  # signed: mirrored


@pytest.mark.parametrize("shape", [(64, 256), (37, 200), (3, 5)])
def test_encoded_state_decodes_near_the_source(oracle_codec, shape):
    """The test encoder's state decodes (oracle statistics + group-64
    high-nibble-first decode) to within the NF4 quantisation error."""
    rng = np.random.default_rng(sum(shape))
    w = (rng.standard_normal(shape) * 0.02).astype(F32)
    packed, q, nested, off, m = oracle_codec.encode_nf4_dq(w)
    assert packed.size == (w.size + 1) // 2 and q.size == (w.size + 63) // 64
    absmax = oracle_codec.dq_absmax(q, nested, m, off)
    bits = oracle_codec.decode4(packed, absmax, w.size, lut=oracle_codec.NF4_LUT, group=64,
                                hi_first=True)
    back = oracle_codec.bf16_bits_to_f32(bits).reshape(shape)
    blockmax = np.abs(np.pad(w.reshape(-1), (0, q.size * 64 - w.size))).reshape(-1, 64).max(1)
    err = np.abs(back - w).reshape(-1)
    bound = np.repeat(blockmax, 64)[:w.size] * 0.17 + 1e-4
    assert np.all(err <= bound)


# ---------------------------------------------------------- product, host side
def test_host_conversion_equals_oracle(oracle_codec):
    rng = np.random.default_rng(5)
    blocks = 256 * 7 + 100
    q = rng.integers(0, 256, blocks, dtype=np.uint8)
    nested = (rng.random(8, dtype=np.float32) * 0.1).astype(F32)
    m = oracle_codec.dynamic_map()
    for off in (0.0, 0.013671875, 0.0123456):
        off = float(F32(off))
        np.testing.assert_array_equal(nf4_state.dq_scales_host(q, nested, m, off),
                                      oracle_codec.dq_absmax(q, nested, m, off))


def _parts(oracle_codec, shape=(16, 96)):
    w = (np.random.default_rng(1).standard_normal(shape) * 0.02).astype(F32)
    packed, q, nested, off, m = oracle_codec.encode_nf4_dq(w)
    meta = {"quant_type": "nf4", "blocksize": 64, "dtype": "bfloat16", "shape": list(shape),
            "nested_blocksize": 256, "nested_dtype": "float32", "nested_offset": off}
    parts = {"absmax": torch.from_numpy(q), "nested_absmax": torch.from_numpy(nested),
             "nested_quant_map": torch.from_numpy(m),
             "quant_map": torch.tensor(oracle_codec.NF4_LUT),
             nf4_state.PACKED_STATE_KEY: nf4_state.pack_metadata(meta)}
    return torch.from_numpy(packed).view(-1, 1), parts, meta


def test_validate_parts_accepts_a_state(oracle_codec):
    packed, parts, meta = _parts(oracle_codec)
    info = nf4_state.validate_parts(packed, parts)
    assert info.shape == (16, 96) and info.blocks == 24 and info.nested_blocks == 1
    assert info.offset == meta["nested_offset"]
    assert nf4_state.unpack_metadata(parts[nf4_state.PACKED_STATE_KEY]) == meta


def _bad_meta(**kw):
    def f(packed, parts, meta):
        m = dict(meta, **kw)
        parts[nf4_state.PACKED_STATE_KEY] = nf4_state.pack_metadata(m)
    return f


@pytest.mark.parametrize("mutate,msg", [
    (lambda p, s, m: s.pop("absmax"), "malformed quant_state_parts keys"),
    (lambda p, s, m: s.__setitem__("extra", torch.zeros(1)), "malformed quant_state_parts keys"),
    (_bad_meta(blocksize=128), "blocksize 64"),
    (_bad_meta(nested_blocksize=128), "secondary blocksize 256"),
    (_bad_meta(quant_type="fp4"), "only official NF4"),
    (_bad_meta(dtype="float16"), "unsupported compute or nested dtype"),
    (_bad_meta(shape=[16, 0]), "two positive integer dimensions"),
    (_bad_meta(shape=[16, 98]), "packed byte count"),
    (_bad_meta(nested_offset=-1.0), "finite and non-negative"),
    (_bad_meta(nested_offset=0.1), "does not match the canonical record"),
    (lambda p, s, m: s.__setitem__("absmax", s["absmax"][:-1].clone()), "primary NF4 absmax"),
    (lambda p, s, m: s.__setitem__("nested_absmax", s["nested_absmax"].double()), "secondary DQ absmax"),
    (lambda p, s, m: s.__setitem__("nested_quant_map", s["nested_quant_map"][:255].clone()),
     "256-entry"),
    (lambda p, s, m: s.__setitem__("quant_map", s["quant_map"] * 2), "official NF4 codebook"),
    (lambda p, s, m: s.__setitem__("nested_absmax", -s["nested_absmax"]), "non-negative"),
    (lambda p, s, m: s.__setitem__(nf4_state.PACKED_STATE_KEY, torch.tensor([1, 2], dtype=torch.uint8)),
     "malformed"),
])
def test_validate_parts_rejects(oracle_codec, mutate, msg):
    packed, parts, meta = _parts(oracle_codec)
    mutate(packed, parts, meta)
    with pytest.raises(ValueError, match=msg):
        nf4_state.validate_parts(packed, parts)


def test_validate_parts_layout(oracle_codec):
    packed, parts, _ = _parts(oracle_codec)
    with pytest.raises(ValueError, match=r"\[bytes, 1\] layout"):
        nf4_state.validate_parts(packed.view(-1), parts)
    with pytest.raises(TypeError, match="dtype"):
        nf4_state.validate_parts(packed.to(torch.int16), parts)
