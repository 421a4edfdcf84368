// DeepSeek-V3 multi-head latent attention: the query/key/value assembly
// around the attention kernel (adapters/deepseek.py:137-150), forward and VJP.
//
//   q   [M, H*(NOPE+ROPE)]   per head: [q_nope | q_rope]        (q_b / q_proj output)
//   kv  [M, H*(NOPE+DV)]     per head: [k_nope | value]         (kv_b output)
//   kr  [M, ROPE]            the shared rope key (kv_a_proj_with_mqa columns)
//   Q[b,h,s]  = cat(q_nope, rotate(q_rope))     [B,H,S,NOPE+ROPE]
//   K[b,h,s]  = cat(k_nope, rotate(kr))         (the same rotated key for every head)
//   V[b,h,s]  = value                           [B,H,S,DV]
//
// rotate(t) with bf16 cos/sin [B,S,ROPE] (= cat(freqs, freqs) * amplitude):
//   default:     t*cos + cat(-t2, t1)*sin                                  (t1, t2 halves)
//   interleave:  cat(t[0::2]*c - t[1::2]*s, t[1::2]*c + t[0::2]*s),  c, s = cos, sin[:ROPE/2]
// with every product, sum and difference rounded to bf16, as the reference's
// bf16 tensor ops do.  One workgroup per token; 16-byte vectors; HBM-bound.
#include "common.h"

namespace {

constexpr int NT = 256;
constexpr int MAXROPE = 128;

struct MlaDims {
  int H, NOPE, ROPE, DV, interleave;
  int64_t S;
};

__device__ __forceinline__ float bf(float x) { return st::bf16r(x); }

__device__ __forceinline__ void unpack8(uint4 v, float* f) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(w[e] << 16);
    f[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 pack8(const float* f) {
  return make_uint4(st::pack_bf16x2(f[0], f[1]), st::pack_bf16x2(f[2], f[3]),
                    st::pack_bf16x2(f[4], f[5]), st::pack_bf16x2(f[6], f[7]));
}

// rotated output chunk c (elements 8c .. 8c+7) of rotate(t); t, cs, sn are the
// token's ROPE values (fp32 copies of bf16) in LDS or registers
__device__ __forceinline__ void rotate_chunk(const float* t, const float* cs, const float* sn,
                                             int ROPE, int interleave, int c, float* o) {
  const int half = ROPE / 2;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int j = 8 * c + e;
    if (!interleave) {
      const float rot = j < half ? -t[j + half] : t[j - half];
      o[e] = bf(bf(t[j] * cs[j]) + bf(rot * sn[j]));
    } else if (j < half) {
      const float a = t[2 * j], b = t[2 * j + 1];
      o[e] = bf(bf(a * cs[j]) - bf(b * sn[j]));
    } else {
      const int i = j - half;
      const float a = t[2 * i], b = t[2 * i + 1];
      o[e] = bf(bf(b * cs[i]) + bf(a * sn[i]));
    }
  }
}

// VJP of rotate for output-gradient g (bf16 values as fp32): element j of dt
__device__ __forceinline__ float rotate_vjp(const float* g, const float* cs, const float* sn,
                                            int ROPE, int interleave, int j) {
  const int half = ROPE / 2;
  if (!interleave) {
    // t*cos: bf16(g*cos); cat(-t2, t1)*sin: u = bf16(g*sin), t1 gets u[j+half], t2 gets -u[j-half]
    const float direct = bf(g[j] * cs[j]);
    return j < half ? bf(direct + bf(g[j + half] * sn[j + half]))
                    : bf(direct - bf(g[j - half] * sn[j - half]));
  }
  const int i = j >> 1;
  const float g1 = g[i], g2 = g[half + i];
  // a = t[2i]: a*c (out1) and a*s (out2); b = t[2i+1]: -b*s (out1) and b*c (out2)
  return (j & 1) ? bf(bf(g2 * cs[i]) - bf(g1 * sn[i])) : bf(bf(g1 * cs[i]) + bf(g2 * sn[i]));
}

__device__ __forceinline__ uint4 ldg16(const uint16_t* p) { return *(const uint4*)p; }

// Output chunk cr (elements 8cr .. 8cr+7) of rotate(t) for a head's rope
// values t in global memory; it reads two 16-byte chunks of t.  Default:
// chunk cr and its partner cr +- R8/2 (t[j +- half]); interleave: chunks 2p
// and 2p+1, p = cr mod R8/2 (the pairs t[2i], t[2i+1]).  Same roundings as
// rotate_chunk.
__device__ __forceinline__ uint4 rotate_chunk_g(const uint16_t* t, const float* cs,
                                                const float* sn, int ROPE, int interleave,
                                                int cr) {
  const int hc = ROPE / 16;  // chunks per half
  float a[8], b[8], o[8];
  if (!interleave) {
    const int pc = cr < hc ? cr + hc : cr - hc;
    unpack8(ldg16(t + 8 * cr), a);
    unpack8(ldg16(t + 8 * pc), b);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = 8 * cr + e;
      const float rot = cr < hc ? -b[e] : b[e];
      o[e] = bf(bf(a[e] * cs[j]) + bf(rot * sn[j]));
    }
  } else {
    const int pr = cr < hc ? cr : cr - hc;
    unpack8(ldg16(t + 16 * pr), a);
    unpack8(ldg16(t + 16 * pr + 8), b);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = 8 * pr + e;  // pair index within the half
      const float x0 = e < 4 ? a[2 * e] : b[2 * e - 8], x1 = e < 4 ? a[2 * e + 1] : b[2 * e - 7];
      o[e] = cr < hc ? bf(bf(x0 * cs[i]) - bf(x1 * sn[i])) : bf(bf(x1 * cs[i]) + bf(x0 * sn[i]));
    }
  }
  return pack8(o);
}

// Chunk cr of the rotation's VJP for a head's output gradient g in global
// memory (two 16-byte chunks of g; same roundings as rotate_vjp).  Default:
// chunk cr and its partner cr +- R8/2; interleave: element j of the chunk
// takes g[j/2] and g[half + j/2], chunks cr/2 and R8/2 + cr/2.
__device__ __forceinline__ uint4 rotate_vjp_chunk_g(const uint16_t* g, const float* cs,
                                                    const float* sn, int ROPE, int interleave,
                                                    int cr) {
  const int hc = ROPE / 16, half = ROPE / 2;
  float a[8], b[8], o[8];
  if (!interleave) {
    const int pc = cr < hc ? cr + hc : cr - hc;
    unpack8(ldg16(g + 8 * cr), a);
    unpack8(ldg16(g + 8 * pc), b);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int j = 8 * cr + e;
      const float direct = bf(a[e] * cs[j]);
      o[e] = cr < hc ? bf(direct + bf(b[e] * sn[j + half])) : bf(direct - bf(b[e] * sn[j - half]));
    }
  } else {
    unpack8(ldg16(g + 8 * (cr >> 1)), a);
    unpack8(ldg16(g + 8 * (hc + (cr >> 1))), b);
    const int e0 = 4 * (cr & 1);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = 4 * cr + (e >> 1);
      const float g1 = a[e0 + (e >> 1)], g2 = b[e0 + (e >> 1)];
      o[e] = (e & 1) ? bf(bf(g2 * cs[i]) - bf(g1 * sn[i])) : bf(bf(g1 * cs[i]) + bf(g2 * sn[i]));
    }
  }
  return pack8(o);
}

// dst[h*dst_h + 8c .. +7] = src[h*src_h + 8c .. +7] for H heads of n8
// 16-byte chunks: U chunks per thread are loaded before any is stored, so
// each thread keeps U loads in flight.
template <int U>
__device__ __forceinline__ void copy_heads(uint16_t* __restrict__ dst, int64_t dst_h,
                                           const uint16_t* __restrict__ src, int64_t src_h,
                                           int n8, int H) {
  const int total = H * n8;
  for (int i0 = threadIdx.x; i0 < total; i0 += NT * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * NT;
      if (i < total) {
        const int h = i / n8, c = i - h * n8;
        v[u] = ldg16(src + h * src_h + 8 * c);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int i = i0 + u * NT;
      if (i < total) {
        const int h = i / n8, c = i - h * n8;
        *(uint4*)(dst + h * dst_h + 8 * c) = v[u];
      }
    }
  }
}

// One workgroup per token, 16-byte chunks: the nope parts of Q and K and the
// value are copied head by head (several loads in flight per thread), then
// the rotated q_rope chunks (each reading its two input chunks straight from
// global memory) and the shared rotated key are written.
__global__ __launch_bounds__(NT) void mla_rope_fwd(const uint16_t* __restrict__ q, int64_t ldq,
                                                   const uint16_t* __restrict__ kv, int64_t ldkv,
                                                   const uint16_t* __restrict__ kr, int64_t ldkr,
                                                   const uint16_t* __restrict__ cos,
                                                   const uint16_t* __restrict__ sin, MlaDims d,
                                                   uint16_t* __restrict__ Q,
                                                   uint16_t* __restrict__ K,
                                                   uint16_t* __restrict__ V) {
  __shared__ float cs[MAXROPE], sn[MAXROPE], kt[MAXROPE];
  __shared__ uint4 kpk[MAXROPE / 8];  // the rotated shared key, packed
  const int64_t row = blockIdx.x;
  const int64_t b = row / d.S, s = row % d.S;
  const int tid = threadIdx.x;
  const int DQ = d.NOPE + d.ROPE, DKV = d.NOPE + d.DV;
  const int R8 = d.ROPE / 8;
  for (int j = tid; j < d.ROPE; j += NT) {
    cs[j] = st::bf16_to_f32(cos[row * d.ROPE + j]);
    sn[j] = st::bf16_to_f32(sin[row * d.ROPE + j]);
    kt[j] = st::bf16_to_f32(kr[row * ldkr + j]);
  }
  __syncthreads();
  if (tid < R8) {  // the shared rotated key, once per token
    float o[8];
    rotate_chunk(kt, cs, sn, d.ROPE, d.interleave, tid, o);
    kpk[tid] = pack8(o);
  }
  __syncthreads();
  const uint16_t* qr = q + row * ldq;
  const uint16_t* kvr = kv + row * ldkv;
  const int nq8 = d.NOPE / 8, nv8 = d.DV / 8;
  const int64_t t0 = (int64_t)b * d.H * d.S + s;  // (b, head 0, s)
  uint16_t* Qt = Q + t0 * DQ;
  uint16_t* Kt = K + t0 * DQ;
  const int64_t hq = d.S * DQ;  // head stride of Q and K
  copy_heads<4>(Qt, hq, qr, DQ, nq8, d.H);
  copy_heads<4>(Kt, hq, kvr, DKV, nq8, d.H);
  copy_heads<4>(V + t0 * d.DV, d.S * d.DV, kvr + d.NOPE, DKV, nv8, d.H);
  // rotated q_rope chunks (two input chunks each) and the shared rotated key
  const int nr = d.H * R8;
  for (int i0 = tid; i0 < nr; i0 += 2 * NT) {
    uint4 v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = i0 + u * NT;
      if (i < nr) {
        const int h = i / R8, cr = i - h * R8;
        v[u] = rotate_chunk_g(qr + (int64_t)h * DQ + d.NOPE, cs, sn, d.ROPE, d.interleave, cr);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = i0 + u * NT;
      if (i < nr) {
        const int h = i / R8, cr = i - h * R8;
        *(uint4*)(Qt + h * hq + d.NOPE + 8 * cr) = v[u];
        *(uint4*)(Kt + h * hq + d.NOPE + 8 * cr) = kpk[cr];
      }
    }
  }
}

__global__ __launch_bounds__(NT) void mla_rope_bwd(const uint16_t* __restrict__ dQ,
                                                   const uint16_t* __restrict__ dK,
                                                   const uint16_t* __restrict__ dV,
                                                   const uint16_t* __restrict__ cos,
                                                   const uint16_t* __restrict__ sin, MlaDims d,
                                                   uint16_t* __restrict__ dq, int64_t lddq,
                                                   uint16_t* __restrict__ dkv, int64_t lddkv,
                                                   uint16_t* __restrict__ dkr, int64_t lddkr) {
  __shared__ float cs[MAXROPE], sn[MAXROPE], gk[MAXROPE];
  __shared__ float gpart[NT * 8];  // [head group][rope element] partial sums
  const int64_t row = blockIdx.x;
  const int64_t b = row / d.S, s = row % d.S;
  const int tid = threadIdx.x;
  const int DQ = d.NOPE + d.ROPE, DKV = d.NOPE + d.DV;
  const int R8 = d.ROPE / 8, G = NT / R8;  // R8 divides NT (checked by the host)
  for (int j = tid; j < d.ROPE; j += NT) {
    cs[j] = st::bf16_to_f32(cos[row * d.ROPE + j]);
    sn[j] = st::bf16_to_f32(sin[row * d.ROPE + j]);
  }
  // gradient of the shared rope key before rotation: the sum over heads of
  // dK's rope part in fp32, rounded once to bf16.  Thread (head group hg,
  // chunk qc) sums heads hg, hg + G, ... of chunk qc with 16-byte loads; the
  // G group sums are then added in group order (a fixed order).
  {
    const int qc = tid % R8, hg = tid / R8;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int h = hg; h < d.H; h += G) {
      float v[8];
      unpack8(ldg16(dK + ((int64_t)(b * d.H + h) * d.S + s) * DQ + d.NOPE + 8 * qc), v);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += v[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) gpart[hg * d.ROPE + 8 * qc + e] = acc[e];
  }
  __syncthreads();
  if (tid < d.ROPE) {
    float a = 0.0f;
    for (int g = 0; g < G; ++g) a += gpart[g * d.ROPE + tid];
    gk[tid] = bf(a);
  }
  __syncthreads();
  if (tid < d.ROPE)
    dkr[row * lddkr + tid] = st::f32_to_bf16(rotate_vjp(gk, cs, sn, d.ROPE, d.interleave, tid));
  // per head: the dq row [nope copy | rope VJP] and the dkv row [k_nope | v]
  const int nq8 = d.NOPE / 8, nv8 = d.DV / 8;
  const int64_t t0 = (int64_t)b * d.H * d.S + s;  // (b, head 0, s)
  const uint16_t* dQt = dQ + t0 * DQ;
  const int64_t hq = d.S * DQ;
  uint16_t* dqr = dq + row * lddq;
  uint16_t* dkvr = dkv + row * lddkv;
  copy_heads<4>(dqr, DQ, dQt, hq, nq8, d.H);
  copy_heads<4>(dkvr, DKV, dK + t0 * DQ, hq, nq8, d.H);
  copy_heads<4>(dkvr + d.NOPE, DKV, dV + t0 * d.DV, d.S * d.DV, nv8, d.H);
  const int nr = d.H * R8;
  for (int i0 = tid; i0 < nr; i0 += 2 * NT) {
    uint4 v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = i0 + u * NT;
      if (i < nr) {
        const int h = i / R8, cr = i - h * R8;
        v[u] = rotate_vjp_chunk_g(dQt + h * hq + d.NOPE, cs, sn, d.ROPE, d.interleave, cr);
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = i0 + u * NT;
      if (i < nr) {
        const int h = i / R8, cr = i - h * R8;
        *(uint4*)(dqr + (int64_t)h * DQ + d.NOPE + 8 * cr) = v[u];
      }
    }
  }
}

bool a16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_dims(const char* name, int64_t B, int64_t S, int64_t H, int64_t NOPE, int64_t ROPE,
               int64_t DV) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && H > 0, "%s: bad shape", name);
  if (NOPE <= 0 || NOPE % 8 || DV <= 0 || DV % 8 || ROPE < 16 || ROPE % 16 || ROPE > MAXROPE ||
      NT % ROPE)
    return st::fail(ST_EUNSUPPORTED,
                    "%s: nope %lld and v %lld must be multiples of 8, rope %lld a multiple of 16 "
                    "dividing %d",
                    name, (long long)NOPE, (long long)DV, (long long)ROPE, NT);
  ST_CHECK_ARG(B * S < (1ll << 31), "%s: too many tokens", name);
  return ST_OK;
}

}  // namespace

extern "C" int st_mla_rope_fwd(const uint16_t* q, int64_t ldq, const uint16_t* kv, int64_t ldkv,
                               const uint16_t* kr, int64_t ldkr, const uint16_t* cos,
                               const uint16_t* sin, int64_t B, int64_t S, int64_t H, int64_t nope,
                               int64_t rope, int64_t v_dim, int32_t interleave, uint16_t* Q,
                               uint16_t* K, uint16_t* V, st_stream_t stream) {
  if (int rc = check_dims("st_mla_rope_fwd", B, S, H, nope, rope, v_dim)) return rc;
  if (B == 0 || S == 0) return ST_OK;
  ST_CHECK_ARG(q && kv && kr && cos && sin && Q && K && V, "st_mla_rope_fwd: NULL pointer");
  ST_CHECK_ARG(a16(q) && a16(kv) && a16(Q) && a16(K) && a16(V) && ldq % 8 == 0 && ldkv % 8 == 0,
               "st_mla_rope_fwd: q, kv and the outputs need 16-byte aligned rows");
  ST_CHECK_ARG(ldq >= H * (nope + rope) && ldkv >= H * (nope + v_dim) && ldkr >= rope,
               "st_mla_rope_fwd: leading dimension too small");
  MlaDims d{(int)H, (int)nope, (int)rope, (int)v_dim, interleave ? 1 : 0, S};
  mla_rope_fwd<<<(unsigned)(B * S), NT, 0, (hipStream_t)stream>>>(q, ldq, kv, ldkv, kr, ldkr, cos,
                                                                   sin, d, Q, K, V);
  return st::check_launch("st_mla_rope_fwd");
}

extern "C" int st_mla_rope_bwd(const uint16_t* dQ, const uint16_t* dK, const uint16_t* dV,
                               const uint16_t* cos, const uint16_t* sin, int64_t B, int64_t S,
                               int64_t H, int64_t nope, int64_t rope, int64_t v_dim,
                               int32_t interleave, uint16_t* dq, int64_t lddq, uint16_t* dkv,
                               int64_t lddkv, uint16_t* dkr, int64_t lddkr, st_stream_t stream) {
  if (int rc = check_dims("st_mla_rope_bwd", B, S, H, nope, rope, v_dim)) return rc;
  if (B == 0 || S == 0) return ST_OK;
  ST_CHECK_ARG(dQ && dK && dV && cos && sin && dq && dkv && dkr, "st_mla_rope_bwd: NULL pointer");
  ST_CHECK_ARG(a16(dQ) && a16(dK) && a16(dV) && a16(dq) && a16(dkv) && lddq % 8 == 0 &&
                   lddkv % 8 == 0,
               "st_mla_rope_bwd: gradients need 16-byte aligned rows");
  ST_CHECK_ARG(lddq >= H * (nope + rope) && lddkv >= H * (nope + v_dim) && lddkr >= rope,
               "st_mla_rope_bwd: leading dimension too small");
  MlaDims d{(int)H, (int)nope, (int)rope, (int)v_dim, interleave ? 1 : 0, S};
  mla_rope_bwd<<<(unsigned)(B * S), NT, 0, (hipStream_t)stream>>>(dQ, dK, dV, cos, sin, d, dq,
                                                                   lddq, dkv, lddkv, dkr, lddkr);
  return st::check_launch("st_mla_rope_bwd");
}
