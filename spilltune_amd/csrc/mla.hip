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

__global__ __launch_bounds__(NT) void mla_rope_fwd(const uint16_t* __restrict__ q, int64_t ldq,
                                                   const uint16_t* __restrict__ kv, int64_t ldkv,
                                                   const uint16_t* __restrict__ kr, int64_t ldkr,
                                                   const uint16_t* __restrict__ cos,
                                                   const uint16_t* __restrict__ sin, MlaDims d,
                                                   uint16_t* __restrict__ Q,
                                                   uint16_t* __restrict__ K,
                                                   uint16_t* __restrict__ V) {
  __shared__ float cs[MAXROPE], sn[MAXROPE], kt[MAXROPE], kout[MAXROPE];
  __shared__ float qt[NT / 64][MAXROPE];  // one head's q_rope per wave at a time
  const int64_t row = blockIdx.x;
  const int64_t b = row / d.S, s = row % d.S;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
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
#pragma unroll
    for (int e = 0; e < 8; ++e) kout[8 * tid + e] = o[e];
  }
  __syncthreads();
  const uint16_t* qr = q + row * ldq;
  const uint16_t* kvr = kv + row * ldkv;
  // nope parts of Q and K, the value, and the rotated key: 16-byte copies
  const int nq8 = d.NOPE / 8, nv8 = d.DV / 8;
  const int per_head = 2 * nq8 + nv8 + R8;
  for (int i = tid; i < d.H * per_head; i += NT) {
    const int h = i / per_head, c = i % per_head;
    const int64_t hs = ((int64_t)(b * d.H + h) * d.S + s);
    if (c < nq8) {
      *(uint4*)(Q + hs * DQ + 8 * c) = *(const uint4*)(qr + (int64_t)h * DQ + 8 * c);
    } else if (c < 2 * nq8) {
      const int cc = c - nq8;
      *(uint4*)(K + hs * DQ + 8 * cc) = *(const uint4*)(kvr + (int64_t)h * DKV + 8 * cc);
    } else if (c < 2 * nq8 + nv8) {
      const int cc = c - 2 * nq8;
      *(uint4*)(V + hs * d.DV + 8 * cc) = *(const uint4*)(kvr + (int64_t)h * DKV + d.NOPE + 8 * cc);
    } else {
      const int cc = c - 2 * nq8 - nv8;
      *(uint4*)(K + hs * DQ + d.NOPE + 8 * cc) = pack8(kout + 8 * cc);
    }
  }
  // rotated q_rope: each wave takes one head at a time (the rotation mixes
  // elements across the head's rope dims)
  for (int h = wave; h < d.H; h += NT / 64) {
    const uint16_t* src = qr + (int64_t)h * DQ + d.NOPE;
    for (int j = lane; j < d.ROPE; j += 64) qt[wave][j] = st::bf16_to_f32(src[j]);
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    if (lane < R8) {
      float o[8];
      rotate_chunk(qt[wave], cs, sn, d.ROPE, d.interleave, lane, o);
      const int64_t hs = ((int64_t)(b * d.H + h) * d.S + s);
      *(uint4*)(Q + hs * DQ + d.NOPE + 8 * lane) = pack8(o);
    }
    __builtin_amdgcn_wave_barrier();
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
  __shared__ float part[NT];
  __shared__ float gq[NT / 64][MAXROPE];
  const int64_t row = blockIdx.x;
  const int64_t b = row / d.S, s = row % d.S;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int DQ = d.NOPE + d.ROPE, DKV = d.NOPE + d.DV;
  for (int j = tid; j < d.ROPE; j += NT) {
    cs[j] = st::bf16_to_f32(cos[row * d.ROPE + j]);
    sn[j] = st::bf16_to_f32(sin[row * d.ROPE + j]);
  }
  // gradient of the shared rope key before rotation: the sum over heads of
  // dK's rope part (fp32, heads in a fixed order), rounded once to bf16
  {
    const int groups = NT / d.ROPE;  // ROPE divides NT
    const int j = tid % d.ROPE, grp = tid / d.ROPE;
    float acc = 0.0f;
    for (int h = grp; h < d.H; h += groups)
      acc += st::bf16_to_f32(dK[((int64_t)(b * d.H + h) * d.S + s) * DQ + d.NOPE + j]);
    part[grp * d.ROPE + j] = acc;
  }
  __syncthreads();
  if (tid < d.ROPE) {
    float acc = 0.0f;
    for (int g = 0; g < NT / d.ROPE; ++g) acc += part[g * d.ROPE + tid];
    gk[tid] = bf(acc);
  }
  __syncthreads();
  if (tid < d.ROPE)
    dkr[row * lddkr + tid] = st::f32_to_bf16(rotate_vjp(gk, cs, sn, d.ROPE, d.interleave, tid));
  // dq nope, dk nope and dv: 16-byte copies into the projection layouts
  const int nq8 = d.NOPE / 8, nv8 = d.DV / 8;
  const int per_head = 2 * nq8 + nv8;
  for (int i = tid; i < d.H * per_head; i += NT) {
    const int h = i / per_head, c = i % per_head;
    const int64_t hs = ((int64_t)(b * d.H + h) * d.S + s);
    if (c < nq8) {
      *(uint4*)(dq + row * lddq + (int64_t)h * DQ + 8 * c) = *(const uint4*)(dQ + hs * DQ + 8 * c);
    } else if (c < 2 * nq8) {
      const int cc = c - nq8;
      *(uint4*)(dkv + row * lddkv + (int64_t)h * DKV + 8 * cc) =
          *(const uint4*)(dK + hs * DQ + 8 * cc);
    } else {
      const int cc = c - 2 * nq8;
      *(uint4*)(dkv + row * lddkv + (int64_t)h * DKV + d.NOPE + 8 * cc) =
          *(const uint4*)(dV + hs * d.DV + 8 * cc);
    }
  }
  // q_rope gradient: VJP of the rotation, one head per wave at a time
  for (int h = wave; h < d.H; h += NT / 64) {
    const int64_t hs = ((int64_t)(b * d.H + h) * d.S + s);
    for (int j = lane; j < d.ROPE; j += 64) gq[wave][j] = st::bf16_to_f32(dQ[hs * DQ + d.NOPE + j]);
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_wave_barrier();
    for (int j = lane; j < d.ROPE; j += 64)
      dq[row * lddq + (int64_t)h * DQ + d.NOPE + j] =
          st::f32_to_bf16(rotate_vjp(gq[wave], cs, sn, d.ROPE, d.interleave, j));
    __builtin_amdgcn_wave_barrier();
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
