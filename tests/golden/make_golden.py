"""Writes tests/golden/codec_vectors.npz: small codec fixtures.

Every array here is computed with numpy float32 arithmetic written from the
closed forms (not with oracle/codec.c and not with the reference), so the C
oracle, the host encoder and the HIP kernels are all checked against an
independent statement:

* ``int4_ka_*`` -- the reference's own known-answer vector
  (tests/test_quantization.py:73-81 in /root/reference): values
  [-7,-1.5,-.5,.5,1.5,7] in a zero 128-group encode to scale 1, payload bytes
  0x61,0x88,0xfa and decode to [-7,-2,0,0,2,7].
* ``nf4_table_*`` / ``int4_table_*`` -- every code x edge scales ->
  bf16 bits of bf16_rne(fp32(codebook[c]) * fp32(scale)).
* ``case<i>_*`` -- seeded matrices with tails (128, 129, 257 elements and a
  [4, 688] matrix whose flat 128-groups straddle rows) encoded in both formats.

Run: python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np

NF4 = np.array([
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634,
    0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
    0.7229568362236023, 1.0], dtype=np.float32)
INT4 = (np.arange(16) - 8).astype(np.float32)


def bf16_bits(x):
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def pad_groups(x):
    n = x.size
    g = (n + 127) // 128
    out = np.zeros(g * 128, dtype=np.float32)
    out[:n] = x.reshape(-1)
    return out.reshape(g, 128)


def pack(codes):
    c = codes.reshape(-1, 2).astype(np.uint8)
    return (c[:, 0] | (c[:, 1] << 4)).astype(np.uint8)


def encode_int4(x):
    ch = pad_groups(x)
    scale = (np.abs(ch).max(1) / np.float32(7)).astype(np.float32)
    scale[scale == 0] = 1
    n = np.clip(ch / scale[:, None], -7, 7).astype(np.float32)
    codes = (np.rint(n) + 8).astype(np.uint8)  # rint = round half to even
    return pack(codes), scale


def encode_nf4(x):
    ch = pad_groups(x)
    amax = np.abs(ch).max(1).astype(np.float32)
    scale = np.where(amax == 0, np.float32(1), amax).astype(np.float32)
    n = (ch / scale[:, None]).astype(np.float32)
    mids = ((NF4[:-1] + NF4[1:]) * np.float32(0.5)).astype(np.float32)
    codes = (n[..., None] > mids).sum(-1).astype(np.uint8)
    return pack(codes), scale


def decode(payload, scales, numel, lut):
    codes = np.stack((payload & 15, payload >> 4), 1).reshape(-1)[:numel]
    idx = np.arange(numel) // 128
    return bf16_bits(lut[codes] * scales[idx])


def main():
    out = {}
    # reference known answer (test_quantization.py:73-81)
    ka = np.zeros(128, dtype=np.float32)
    ka[:6] = [-7, -1.5, -.5, .5, 1.5, 7]
    p, s = encode_int4(ka)
    assert s[0] == 1 and p[:3].tolist() == [0x61, 0x88, 0xfa]
    out["int4_ka_values"] = ka
    out["int4_ka_payload_prefix"] = np.array([0x61, 0x88, 0xfa], dtype=np.uint8)
    out["int4_ka_decoded_prefix"] = np.array([-7, -2, 0, 0, 2, 7], dtype=np.float32)

    scales = np.array([1.0, 0.5, 3.0, 1e-3, 0.02, 0.0123456, 65504.0, 1e30, 1e-38, 7.0],
                      dtype=np.float32)
    for name, lut in (("nf4", NF4), ("int4", INT4)):
        out[f"{name}_table_scales"] = scales
        out[f"{name}_table_bits"] = bf16_bits(lut[None, :] * scales[:, None])

    rng = np.random.default_rng(20261201)
    shapes = [(128,), (129,), (257,), (4, 688), (3, 256)]
    for i, shape in enumerate(shapes):
        x = (rng.standard_normal(shape) * 0.02).astype(np.float32)
        if i == 4:
            x[1] = 0.0  # an all-zero row -> zero groups take scale 1
        out[f"case{i}_x"] = x
        for name, enc, lut in (("int4", encode_int4, INT4), ("nf4", encode_nf4, NF4)):
            p, s = enc(x)
            out[f"case{i}_{name}_payload"] = p
            out[f"case{i}_{name}_scales"] = s
            out[f"case{i}_{name}_bits"] = decode(p, s, x.size, lut)
    path = Path(__file__).with_name("codec_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
