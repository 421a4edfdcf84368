"""Pins the C codec oracle (and the product's host encoder) to the reference's
known answers, to the closed form evaluated independently, and to a scalar
decoder restated from tests/test_quantization.py:43-56 of the reference."""
from pathlib import Path

import numpy as np
import pytest
import torch

GOLD = np.load(Path(__file__).parent / "golden" / "codec_vectors.npz")


def scalar_decode_int4(payload: bytes, scales, numel):
    """Per-element restatement of the reference's independent decoder
    (test_quantization.py:43-56): ((b >> 4*(i%2)) & 15) - 8, times the
    group scale, rounded once to bf16."""
    vals = []
    for i in range(numel):
        code = ((payload[i // 2] >> (4 * (i % 2))) & 15) - 8
        vals.append(np.float32(code) * np.float32(scales[i // 128]))
    return torch.tensor(np.array(vals, dtype=np.float32)).to(torch.bfloat16)


def test_int4_reference_known_answer(oracle_codec):
    x = GOLD["int4_ka_values"]
    payload, scales = oracle_codec.encode_int4(x)
    assert scales[0] == 1.0
    assert payload[:3].tolist() == [0x61, 0x88, 0xfa]
    bits = oracle_codec.decode4(payload, scales, x.size, lut=oracle_codec.INT4_LUT)
    dec = oracle_codec.bf16_bits_to_f32(bits)
    assert dec[:6].tolist() == [-7, -2, 0, 0, 2, 7]
    assert payload.size == 64  # ceil(n/128)*64 (test_quantization.py:69)


def test_zero_group_scale_is_one(oracle_codec):
    x = np.zeros(257, dtype=np.float32)
    x[200] = 0.5
    _, s4 = oracle_codec.encode_int4(x)
    _, sn = oracle_codec.encode_nf4(x)
    assert s4[0] == 1.0 and s4[2] == 1.0 and sn[0] == 1.0 and sn[2] == 1.0
    assert sn[1] == np.float32(0.5) and s4[1] == np.float32(0.5) / np.float32(7)


@pytest.mark.parametrize("case", range(5))
@pytest.mark.parametrize("fmt", ["int4", "nf4"])
def test_oracle_matches_numpy_closed_form(oracle_codec, case, fmt):
    x = GOLD[f"case{case}_x"]
    enc = oracle_codec.encode_int4 if fmt == "int4" else oracle_codec.encode_nf4
    lut = oracle_codec.INT4_LUT if fmt == "int4" else oracle_codec.NF4_LUT
    payload, scales = enc(x)
    np.testing.assert_array_equal(payload, GOLD[f"case{case}_{fmt}_payload"])
    np.testing.assert_array_equal(scales, GOLD[f"case{case}_{fmt}_scales"])
    bits = oracle_codec.decode4(payload, scales, x.size, lut=lut)
    np.testing.assert_array_equal(bits, GOLD[f"case{case}_{fmt}_bits"])


@pytest.mark.parametrize("length", [128, 129, 257])
def test_oracle_matches_scalar_reference_decoder(oracle_codec, length):
    rng = np.random.default_rng(length)
    x = (rng.standard_normal(length) * 0.03).astype(np.float32)
    x[:128] = 0  # first group all-zero, as test_quantization.py:62
    payload, scales = oracle_codec.encode_int4(x)
    bits = oracle_codec.decode4(payload, scales, length, lut=oracle_codec.INT4_LUT)
    expect = scalar_decode_int4(bytes(payload.tolist()), scales.tolist(), length)
    assert torch.equal(torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16), expect)


def test_chunk_boundary_reencode(oracle_codec):
    """codecs.py's 8192-group chunking must not change bytes
    (test_quantization.py:97-111): re-encoding the tail alone gives the same bytes."""
    length = 8192 * 128 + 129
    x = ((np.arange(length, dtype=np.float32) % 29) - 14) / 32
    payload, scales = oracle_codec.encode_int4(x)
    local_p, local_s = oracle_codec.encode_int4(x[(8192 - 1) * 128:].copy())
    np.testing.assert_array_equal(payload[-3 * 64:], local_p)
    np.testing.assert_array_equal(scales[-3:], local_s)


@pytest.mark.parametrize("fmt", ["nf4", "int4"])
def test_codebook_tables_all_codes_edge_scales(oracle_codec, fmt):
    lut = oracle_codec.NF4_LUT if fmt == "nf4" else oracle_codec.INT4_LUT
    scales = GOLD[f"{fmt}_table_scales"]
    expect = GOLD[f"{fmt}_table_bits"]
    for i, s in enumerate(scales):
        payload = np.array([c | ((c + 1) << 4) for c in range(0, 16, 2)], dtype=np.uint8)
        bits = oracle_codec.decode4(payload, np.array([s], np.float32), 16, lut=lut)
        np.testing.assert_array_equal(bits, expect[i])
        # brute force with Python floats rounded through float32 then bf16
        for c in range(16):
            prod = np.float32(np.float32(lut[c]) * np.float32(s))
            assert bits[c] == oracle_codec.f32_to_bf16_bits(np.array([prod]))[0]


def test_nf4_invariants(oracle_codec):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(128 * 64) * 0.02).astype(np.float32)
    payload, scales = oracle_codec.encode_nf4(x)
    dec = oracle_codec.bf16_bits_to_f32(oracle_codec.decode4(payload, scales, x.size,
                                                            lut=oracle_codec.NF4_LUT))
    amax = np.repeat(scales, 128)
    assert np.all(np.abs(dec) <= amax * (1 + 2 ** -8))
    codes = np.stack((payload & 15, payload >> 4), 1).reshape(-1)
    assert np.all(dec[codes == 7] == 0) and not np.signbit(dec[codes == 7]).any()
    np.testing.assert_allclose(dec[codes == 15], amax[codes == 15], rtol=2 ** -8)
    np.testing.assert_allclose(dec[codes == 0], -amax[codes == 0], rtol=2 ** -8)
    # every group's absmax element lands on code 0 or 15
    g = np.abs(x.reshape(-1, 128)).argmax(1) + np.arange(64) * 128
    assert set(codes[g].tolist()) <= {0, 15}
    # nearest-entry quantisation: the decoded error is at most half the widest gap
    gap = np.max(np.diff(oracle_codec.NF4_LUT))
    assert np.all(np.abs(dec - x) <= amax * (gap / 2 + 2 ** -8))


def test_hi_nibble_first_is_a_byte_swap(oracle_codec):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256) * 0.02).astype(np.float32)
    lo_p, s = oracle_codec.encode_nf4(x)
    hi_p, s2 = oracle_codec.encode_nf4(x, hi_first=True)
    np.testing.assert_array_equal(s, s2)
    np.testing.assert_array_equal(hi_p, ((lo_p & 15) << 4) | (lo_p >> 4))
    a = oracle_codec.decode4(lo_p, s, 256, lut=oracle_codec.NF4_LUT)
    b = oracle_codec.decode4(hi_p, s, 256, lut=oracle_codec.NF4_LUT, hi_first=True)
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("case", range(5))
@pytest.mark.parametrize("fmt", ["int4-sym-g128", "nf4-g128"])
def test_product_host_encoder_matches_oracle(oracle_codec, case, fmt):
    """The package's offline encoder must produce the oracle's bytes."""
    from spilltune_amd import codecs
    x = GOLD[f"case{case}_x"]
    rec = codecs.encode(torch.from_numpy(x.copy()), fmt)
    codecs.validate_spec(rec.spec, rec.parts)
    short = "int4" if fmt.startswith("int4") else "nf4"
    np.testing.assert_array_equal(rec.parts["payload"].numpy(), GOLD[f"case{case}_{short}_payload"])
    np.testing.assert_array_equal(rec.parts["scales"].numpy(), GOLD[f"case{case}_{short}_scales"])


def test_validate_spec_rejections():
    from spilltune_amd import codecs
    rec = codecs.encode(torch.ones(1, 129), "int4-sym-g128")
    bad = {k: v.clone() for k, v in rec.parts.items()}
    bad["scales"][0] = 0
    with pytest.raises(ValueError, match="scales"):
        codecs.validate_spec(rec.spec, bad)
    bad = {k: v.clone() for k, v in rec.parts.items()}
    bad["payload"][0] = 0
    with pytest.raises(ValueError, match="reserved"):
        codecs.validate_spec(rec.spec, bad)
    bad = {k: v.clone() for k, v in rec.parts.items()}
    bad["payload"][-1] ^= 1
    with pytest.raises(ValueError, match="padding"):
        codecs.validate_spec(rec.spec, bad)
    with pytest.raises(ValueError, match="unsupported_quantization"):
        codecs.encode(torch.ones(1, 128), "nf4")
    with pytest.raises(ValueError, match="nonfinite"):
        codecs.encode(torch.full((1, 128), float("nan")), "nf4-g128")


# ---- validation across bounded chunks (the reference's
# tests/test_validation_chunks.py:1-76, for the 4-bit formats of this build)
GROUPS_V = 2048 + 3   # codecs.VALIDATION_CHUNK_GROUPS + 3
POSITIONS_V = (0, 2047, 2048, GROUPS_V - 1)


def _zero_record(mode, tail=False):
    from spilltune_amd import codecs
    assert codecs.VALIDATION_CHUNK_GROUPS == 2048
    return codecs.encode(torch.zeros(GROUPS_V * 128 - (1 if tail else 0)), mode)


@pytest.mark.parametrize("group", POSITIONS_V)
def test_reserved_code_at_chunk_boundaries(group):
    from spilltune_amd import codecs
    r = _zero_record("int4-sym-g128")
    r.parts["payload"][group * 64] = 0
    with pytest.raises(ValueError, match="reserved"):
        codecs.validate_spec(r.spec, r.parts)


@pytest.mark.parametrize("mode", ["int4-sym-g128", "nf4-g128"])
@pytest.mark.parametrize("group", POSITIONS_V)
@pytest.mark.parametrize("bad", [0.0, -1.0, float("nan"), float("inf")])
def test_invalid_scale_at_chunk_boundaries(mode, group, bad):
    from spilltune_amd import codecs
    r = _zero_record(mode)
    r.parts["scales"][group] = bad
    with pytest.raises(ValueError, match="scales"):
        codecs.validate_spec(r.spec, r.parts)


@pytest.mark.parametrize("mode", ["int4-sym-g128", "nf4-g128"])
@pytest.mark.parametrize("group", POSITIONS_V)
def test_finite_fp32_product_but_bf16_overflow_is_rejected(mode, group):
    from spilltune_amd import codecs
    r = _zero_record(mode)
    p = r.parts["payload"]
    # first element of the group decodes to +1: int4 code 9, NF4 code 15
    p[group * 64] = (int(p[group * 64]) & 0xF0) | (9 if mode == "int4-sym-g128" else 15)
    r.parts["scales"][group] = 3.4e38
    assert torch.isfinite(r.parts["scales"][group]) and \
        not torch.isfinite(r.parts["scales"][group].bfloat16())
    with pytest.raises(ValueError, match="BF16"):
        codecs.validate_spec(r.spec, r.parts)


@pytest.mark.parametrize("mode", ["int4-sym-g128", "nf4-g128"])
def test_large_scale_with_small_codes_is_accepted(mode):
    """The overflow rule is per decoded value: a scale of 1e38 whose group
    holds only +-1 (int4) or 0.0796 (NF4 code 8) fits bf16, though 7x or 1x
    of it might not."""
    from spilltune_amd import codecs
    r = _zero_record(mode)
    p = r.parts["payload"]
    p[5] = (int(p[5]) & 0xF0) | (9 if mode == "int4-sym-g128" else 8)
    r.parts["scales"][0] = 1e38 if mode == "int4-sym-g128" else 3.3e38
    codecs.validate_spec(r.spec, r.parts)
    if mode == "int4-sym-g128":  # code 15 (+7) in the same group overflows
        p[6] = (int(p[6]) & 0xF0) | 15
        with pytest.raises(ValueError, match="BF16"):
            codecs.validate_spec(r.spec, r.parts)


@pytest.mark.parametrize("mode", ["int4-sym-g128", "nf4-g128"])
def test_tail_of_last_chunk_is_checked(mode):
    from spilltune_amd import codecs
    r = _zero_record(mode, tail=True)
    r.parts["payload"][-1] ^= 16
    with pytest.raises(ValueError, match="padding"):
        codecs.validate_spec(r.spec, r.parts)


@pytest.mark.parametrize("mode", ["int4-sym-g128", "nf4-g128"])
def test_valid_multichunk_storage_bytes_remain_frozen(mode):
    from spilltune_amd import codecs
    g = torch.Generator().manual_seed(3)
    r = codecs.encode(torch.randn(GROUPS_V * 128 - 5, generator=g), mode)
    saved = {k: t.clone() for k, t in r.parts.items()}
    codecs.validate_spec(r.spec, r.parts)
    assert all(torch.equal(t, saved[k]) for k, t in r.parts.items())


@pytest.mark.parametrize("mode", ["int4-sym-g128", "nf4-g128"])
def test_fp32_multiply_overflow_remains_rejected(mode):
    from spilltune_amd import codecs
    r = codecs.encode(torch.ones(128), mode)
    r.parts["scales"].fill_(1e38 if mode == "int4-sym-g128" else 3.4e38)
    with pytest.raises(ValueError, match="BF16"):
        codecs.validate_spec(r.spec, r.parts)
