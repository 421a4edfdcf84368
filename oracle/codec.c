/*
 * CPU restatement of the 4-bit storage codecs on the SpillTune per-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP kernels in
 * spilltune_amd/csrc; nothing in the product links it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Formats restated (reference paths relative to /root/reference):
 *   int4-sym-g128  src/ram_vram_finetune/quantization/codecs.py:55-63 (unpack),
 *                  :66-116 (encode), :158-170 (decode_into).  Codes 1..15 map to
 *                  -7..7, code 0 (-8) is reserved, two codes per byte low nibble
 *                  first, one fp32 scale per 128 *flattened* elements.
 *   nf4-g128       The benchmark storage format: same container as int4-sym-g128
 *                  (payload uint8[ceil(n/128)*64] low nibble first, fp32 absmax
 *                  per flat 128-group) with the published NF4 codebook (QLoRA,
 *                  Dettmers et al. 2023, arXiv:2305.14314, appendix E) in place
 *                  of code-8.  The reference compares its table against the
 *                  bitsandbytes one at nf4_backend.py:252-255.
 *
 * Every decode is value = bf16_rne( fp32(code_value) * fp32(scale_of_group) ),
 * i.e. one IEEE fp32 multiply followed by round-to-nearest-even to bfloat16,
 * which is what codecs.py:168 (fp32 tensor product) followed by the bf16
 * copy_ at codecs.py:170 computes.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* Published NF4 codebook, fp32 (QLoRA appendix E). */
const float st_oracle_nf4_lut[16] = {
    -1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f,
    -0.28444138169288635f, -0.18477343022823334f, -0.09105003625154495f, 0.0f,
    0.07958029955625534f, 0.16093020141124725f, 0.24611230194568634f,
    0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,
    0.7229568362236023f, 1.0f};

static inline uint32_t f32_bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bits_f32(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* fp32 -> bf16 round-to-nearest-even (quiet NaN kept quiet). */
uint16_t st_oracle_bf16_rne(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float st_oracle_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* code value of element i of a low-nibble-first (or high-first) payload */
static inline unsigned nibble(const uint8_t* payload, int64_t i, int hi_first) {
  unsigned b = payload[i >> 1];
  unsigned sh = ((unsigned)(i & 1) ^ (unsigned)(hi_first != 0)) * 4u;
  return (b >> sh) & 15u;
}

/*
 * Generic flat-group decode: out[i] = bf16(lut[code_i] * scales[i / group]).
 * Covers int4-sym-g128 (lut[c] = c - 8, codecs.py:60,168) and nf4-g128.
 */
void st_oracle_decode4(const uint8_t* payload, const float* scales, int64_t numel,
                       int group, const float* lut16, int hi_first, uint16_t* out) {
  for (int64_t i = 0; i < numel; ++i) {
    float v = lut16[nibble(payload, i, hi_first)] * scales[i / group];
    out[i] = st_oracle_bf16_rne(v);
  }
}

/* round-half-to-even of an fp32 value (torch.round semantics). */
static float round_half_even(float x) {
  float r = nearbyintf(x); /* default FE_TONEAREST is ties-to-even */
  return r;
}

/*
 * int4-sym-g128 encoder, codecs.py:81-116: per flat 128-group (zero padded
 * tail), scale = absmax/7 (scale 0 -> 1), q = round_half_even(clamp(x/scale,
 * -7, 7)) + 8, packed low nibble first.  Returns 0, or -1 on a non-finite input
 * (the reference raises ValueError there).
 */
int st_oracle_encode_int4(const float* x, int64_t numel, uint8_t* payload, float* scales) {
  int64_t groups = (numel + 127) / 128;
  for (int64_t g = 0; g < groups; ++g) {
    float chunk[128];
    float amax = 0.0f;
    for (int k = 0; k < 128; ++k) {
      int64_t i = g * 128 + k;
      chunk[k] = i < numel ? x[i] : 0.0f;
      if (!isfinite(chunk[k])) return -1;
      float a = fabsf(chunk[k]);
      if (a > amax) amax = a;
    }
    float scale = amax / 7.0f;
    if (scale == 0.0f) scale = 1.0f;
    scales[g] = scale;
    for (int k = 0; k < 128; k += 2) {
      unsigned q[2];
      for (int t = 0; t < 2; ++t) {
        float n = chunk[k + t] / scale;
        if (n < -7.0f) n = -7.0f;
        if (n > 7.0f) n = 7.0f;
        q[t] = (unsigned)((int)round_half_even(n) + 8);
      }
      payload[g * 64 + k / 2] = (uint8_t)(q[0] | (q[1] << 4));
    }
  }
  return 0;
}

/*
 * nf4-g128 encoder (this build's format; offline, not on the hot path):
 * absmax per flat 128-group (0 -> 1, as codecs.py:94 does for int4), code =
 * number of codebook midpoints strictly below x/absmax, i.e. nearest entry with
 * ties going to the lower code.  Zero-padded tail codes are the code of 0.0
 * (7), so a padded tail decodes to +0.
 */
int st_oracle_encode_nf4(const float* x, int64_t numel, int hi_first, uint8_t* payload,
                         float* scales) {
  float mids[15];
  for (int i = 0; i < 15; ++i) mids[i] = 0.5f * (st_oracle_nf4_lut[i] + st_oracle_nf4_lut[i + 1]);
  int64_t groups = (numel + 127) / 128;
  for (int64_t g = 0; g < groups; ++g) {
    float amax = 0.0f;
    for (int k = 0; k < 128; ++k) {
      int64_t i = g * 128 + k;
      float v = i < numel ? x[i] : 0.0f;
      if (!isfinite(v)) return -1;
      if (fabsf(v) > amax) amax = fabsf(v);
    }
    float scale = amax == 0.0f ? 1.0f : amax;
    scales[g] = scale;
    for (int k = 0; k < 128; k += 2) {
      unsigned q[2];
      for (int t = 0; t < 2; ++t) {
        int64_t i = g * 128 + k + t;
        float n = i < numel ? x[i] / scale : 0.0f;
        unsigned c = 0;
        for (int m = 0; m < 15; ++m) c += (n > mids[m]) ? 1u : 0u;
        q[t] = c;
      }
      payload[g * 64 + k / 2] =
          hi_first ? (uint8_t)((q[0] << 4) | q[1]) : (uint8_t)(q[0] | (q[1] << 4));
    }
  }
  return 0;
}

/*
 * bitsandbytes NF4 double-quantised block statistics (bitsandbytes==0.50.2,
 * absent here; the reference's call sites are nf4_backend.py:292-298
 * quantize_4bit(blocksize=64, compress_statistics=True) and
 * nf4_backend_cuda.py:888-917 matmul_4bit; state layout nf4_backend.py:
 * 219-240).  The library's published dequantisation of the statistics is a
 * blockwise dequantize of the uint8 codes with the nested state followed by
 * `absmax += offset`:
 *   absmax_j = fp32( fp32(map[q_j] * nested[j / nested_block]) + offset ).
 * Each operation rounds to fp32 (no contraction: -ffp-contract=off, SSE).
 */
void st_oracle_dq_absmax(const uint8_t* q, const float* nested, int64_t blocks, int nested_block,
                         const float* map256, float offset, float* out) {
  for (int64_t j = 0; j < blocks; ++j) {
    float prod = map256[q[j]] * nested[j / nested_block];
    out[j] = prod + offset;
  }
}
