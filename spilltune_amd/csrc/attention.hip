// Causal GQA flash attention for gfx950 (forward, and backward in two
// deterministic passes), replacing the eager scores/softmax/probabilities
// chain of adapters/dense.py:142-148.
//
// Layout: q [B, H, S, D], k/v [B, Hkv, S, D] (head-major bf16); the output is
// written token-major [B, S, H*D]; lse [B, H, S] fp32 is the base-2 log-sum-exp
// of each query row of x = scale * log2(e) * q.k.
//
// Transposed formulation: every MFMA tile is S^T = K Q^T (rows = keys,
// columns = queries), so one lane owns one query column: the softmax max/sum
// are in-lane reductions plus one exchange between the two half-waves, and
// the probabilities are already in the B-operand layout of O^T += V^T P^T.
#include "common.h"

namespace {

constexpr int NTH = 256;
constexpr int BQ = 128;  // queries per workgroup (4 waves x 32)
constexpr int BKT = 64;  // keys per tile
constexpr float LOG2E = 1.4426950408889634f;

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 ld_global16(const uint16_t* p) { return *(const uint4*)p; }

// K tile [64 keys][D] in LDS, 16-byte chunks XOR-swizzled by row
template <int D>
__device__ __forceinline__ int kswz(int row, int chunk) {
  return row * (D / 8) + (chunk ^ (row & (D / 8 - 1)));
}
// V^T tile [D][64 keys] in LDS, 8-byte chunks (4 keys) XOR-swizzled by d
__device__ __forceinline__ int vswz8(int d, int kc) { return d * 16 + (kc ^ ((d >> 1) & 15)); }

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// ---------------------------------------------------------------- transpose
// dst[n][d][s] = src[n][s][d] for n < N heads (64x64 tiles through LDS)
__global__ __launch_bounds__(NTH) void transpose_heads(const uint16_t* __restrict__ src,
                                                       uint16_t* __restrict__ dst, int64_t S,
                                                       int D) {
  __shared__ uint16_t t[64][66];
  const int64_t n = blockIdx.z;
  const int64_t s0 = (int64_t)blockIdx.x * 64, d0 = (int64_t)blockIdx.y * 64;
  const uint16_t* in = src + n * S * D;
  uint16_t* out = dst + n * S * D;
  for (int i = threadIdx.x; i < 64 * 64; i += NTH) {
    const int r = i / 64, c = i % 64;
    t[r][c] = (s0 + r < S && d0 + c < D) ? in[(s0 + r) * D + d0 + c] : 0;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += NTH) {
    const int r = i / 64, c = i % 64;  // r: d, c: s
    if (d0 + r < D && s0 + c < S) out[(d0 + r) * S + s0 + c] = t[c][r];
  }
}

// ---------------------------------------------------------------- forward
template <int D>
__global__ __launch_bounds__(NTH, 2) void fa_fwd(const uint16_t* __restrict__ q,
                                              const uint16_t* __restrict__ k,
                                              const uint16_t* __restrict__ vt, int S, int H,
                                              int Hkv, float sl2, uint16_t* __restrict__ out,
                                              float* __restrict__ lse) {
  constexpr int DS = D / 16;   // contraction steps over d
  constexpr int DB = D / 32;   // 32-row d blocks of O^T
  constexpr int LDK = BKT * D; // bf16 per K tile
  constexpr int LDV = D * BKT; // bf16 per V^T tile
  constexpr int PER = D / 32;  // 16-byte chunks per thread per tile (K and V^T each)
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * (LDK + LDV)];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c = lane & 31;
  const int qt = gridDim.x - 1 - blockIdx.x;  // longest (diagonal-most) tiles first
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (H / Hkv);
  const uint16_t* qb = q + ((int64_t)(b * H + h) * S) * D;
  const uint16_t* kb = k + ((int64_t)(b * Hkv + hk) * S) * D;
  const uint16_t* vb = vt + ((int64_t)(b * Hkv + hk) * D) * S;
  const int q0 = qt * BQ + wave * 32;
  const int myq = q0 + c;

  bf16x8 qf[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s)
    qf[s] = as_bf16x8(myq < S ? ld_global16(qb + (int64_t)myq * D + 16 * s + 8 * g)
                              : make_uint4(0, 0, 0, 0));

  f32x16 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) oacc[i][v] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  const int qlast = min(qt * BQ + BQ, S) - 1;   // last query of the workgroup
  const int ntiles = qlast / BKT + 1;           // causal: keys <= qlast
  uint4 kr[PER], vr[PER];
  auto load = [&](int t) {
    const int k0 = t * BKT;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int id = tid + i * NTH;
      const int row = id / (D / 8), ch = id % (D / 8);  // K: key row, chunk
      kr[i] = (k0 + row < S) ? ld_global16(kb + (int64_t)(k0 + row) * D + ch * 8)
                             : make_uint4(0, 0, 0, 0);
      const int d = id / 8, kc2 = id % 8;                 // V^T: d row, 16-byte key chunk
      vr[i] = (k0 + kc2 * 8 < S) ? ld_global16(vb + (int64_t)d * S + k0 + kc2 * 8)
                                 : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
    uint16_t* ks = lds + buf * (LDK + LDV);
    uint16_t* vs = ks + LDK;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int id = tid + i * NTH;
      const int row = id / (D / 8), ch = id % (D / 8);
      *(uint4*)(ks + kswz<D>(row, ch) * 8) = kr[i];
      const int d = id / 8, kc2 = id % 8;
      const int f = (d >> 1) & 15;
      const int slot = kc2 ^ (f >> 1);
      uint4 w = vr[i];
      if (f & 1) w = make_uint4(w.z, w.w, w.x, w.y);
      *(uint4*)(vs + d * BKT + slot * 8) = w;
    }
  };

  load(0);
  store(0);
  __syncthreads();
  // one barrier per tile: tile t+1 is stored into the other buffer, whose
  // readers (tile t-1) all passed the previous barrier
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load(t + 1);
    const uint16_t* ks = lds + buf * (LDK + LDV);
    const uint16_t* vs = ks + LDK;
    const int k0 = t * BKT;
    // 32-key blocks, each: S^T = K Q^T, online softmax, O^T += V^T P^T.  A
    // block wholly above this wave's queries (or past S) is skipped.
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      const int kb0 = k0 + jb * 32;
      if (kb0 > q0 + 31 || kb0 >= S) continue;  // wave-uniform
      f32x16 sacc;
#pragma unroll
      for (int v = 0; v < 16; ++v) sacc[v] = 0.0f;
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const bf16x8 a = as_bf16x8(*(const uint4*)(ks + kswz<D>(jb * 32 + c, 2 * s + g) * 8));
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[s], sacc, 0, 0, 0);
      }
      const bool diag = kb0 + 31 > q0 || kb0 + 31 >= S;
      float mt = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int key = kb0 + (v >> 2) * 8 + g * 4 + (v & 3);
        float x = sacc[v] * sl2;
        if (diag && (key > myq || key >= S)) x = -INFINITY;
        sacc[v] = x;
        mt = fmaxf(mt, x);
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32));
      const float m_new = fmaxf(m_run, mt);
      if (__ballot(m_new > m_run)) {
        const float alpha = exp2f(m_run - m_new);
#pragma unroll
        for (int i = 0; i < DB; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) oacc[i][v] *= alpha;
        l_run *= alpha;
      }
      m_run = m_new;
      bf16x8 pf[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p[e] = exp2f(sacc[8 * hh + e] - m_new);
          l_run += p[e];
        }
        pf[hh] = as_bf16x8(make_uint4(st::pack_bf16x2(p[0], p[1]), st::pack_bf16x2(p[2], p[3]),
                                      st::pack_bf16x2(p[4], p[5]), st::pack_bf16x2(p[6], p[7])));
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int cc = jb * 2 + hh;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int d = db * 32 + c;
          const u32x2 lo = *(const u32x2*)(vs + vswz8(d, 4 * cc + g) * 4);
          const u32x2 hi = *(const u32x2*)(vs + vswz8(d, 4 * cc + 2 + g) * 4);
          const bf16x8 a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[hh], oacc[db], 0, 0, 0);
        }
      }
    }
    if (t + 1 < ntiles) store(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  if (g == 0 && myq < S) lse[((int64_t)(b * H + h)) * S + myq] = m_run + log2f(l_tot);
  // stage O (query rows) through LDS for 16-byte token-major stores
  constexpr int LDO = D + 8;
  uint16_t* os = lds + wave * 32 * LDO;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const int d = db * 32 + v4 * 8 + g * 4;
      const u32x2 w = {st::pack_bf16x2(oacc[db][4 * v4] * inv, oacc[db][4 * v4 + 1] * inv),
                       st::pack_bf16x2(oacc[db][4 * v4 + 2] * inv, oacc[db][4 * v4 + 3] * inv)};
      *(u32x2*)(os + c * LDO + d) = w;
    }
  __syncthreads();
  const int64_t ld_out = (int64_t)H * D;
  for (int i = lane; i < 32 * (D / 8); i += 64) {
    const int r = i / (D / 8), ch = i % (D / 8);
    const int qq = q0 + r;
    if (qq < S) {
      const u32x2 a = *(const u32x2*)(os + r * LDO + ch * 8);
      const u32x2 bb = *(const u32x2*)(os + r * LDO + ch * 8 + 4);
      *(uint4*)(out + ((int64_t)b * S + qq) * ld_out + (int64_t)h * D + ch * 8) =
          make_uint4(a.x, a.y, bb.x, bb.y);
    }
  }
}

// ---------------------------------------------------------------- backward
// Row-major [rows][D] LDS tile, 16-byte chunks XOR-swizzled so that both
// 16-byte row reads and the transposing 8-byte reads below avoid conflicts.
template <int D>
__device__ __forceinline__ int tswz(int row, int chunk) {
  return row * D + ((chunk ^ (((row & 7) << 1) & (D / 8 - 1))) << 3);
}
template <int D>
__device__ __forceinline__ bf16x8 tile_row(const uint16_t* t, int row, int s, int g) {
  return as_bf16x8(*(const uint4*)(t + tswz<D>(row, 2 * s + g)));
}
// Transposed MFMA operand from a row-major tile: lane (row n = nb + lane%32,
// half g = lane/32) gets tile[kb + (s>>2)*8 + g*4 + (s&3)][n] for s = 0..7,
// the contraction order of a probability block held in MFMA accumulators.
// ds_read_b64_tr_b16: within 16 lanes, lane i receives element (i % 4) of the
// 4-element rows supplied by lanes 4j + i/4, j = 0..3.
template <int D>
__device__ __forceinline__ bf16x8 tile_tr(const uint16_t* t, int kb, int nb, int lane) {
  const int G = lane >> 4, i = lane & 15, g = lane >> 5;
  const int col = nb + 16 * (G & 1) + 4 * (i & 3);
  typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
  v4bf r[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = kb + 8 * h + 4 * g + (i >> 2);
    const uint16_t* p = t + tswz<D>(row, col >> 3) + (col & 7);
    r[h] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) v4bf*)p);
  }
  return __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7);
}

// dQ (and Delta = rowsum(dO * O)) per 128-query tile: S^T = K Q^T,
// P^T = exp2(S^T - lse), dP^T = V dO^T, dS^T = P^T (dP^T - Delta),
// dQ^T += K^T dS^T; keys up to the diagonal.
template <int D>
__global__ __launch_bounds__(NTH, 2) void fa_bwd_dq(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ o,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse, int S, int H, int Hkv,
    float sl2, float scale, float* __restrict__ delta, uint16_t* __restrict__ dq) {
  constexpr int DS = D / 16, DB = D / 32;
  constexpr int LT = BKT * D;           // bf16 per K (or V) tile
  constexpr int PER = D / 32;           // 16-byte chunks per thread per tile
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * 2 * LT];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c = lane & 31;
  const int qt = gridDim.x - 1 - blockIdx.x;
  const int h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (H / Hkv);
  const int64_t ldt = (int64_t)H * D;  // token-major row stride
  const uint16_t* qb = q + ((int64_t)(b * H + h) * S) * D;
  const uint16_t* kb = k + ((int64_t)(b * Hkv + hk) * S) * D;
  const uint16_t* vb = v + ((int64_t)(b * Hkv + hk) * S) * D;
  const int q0 = qt * BQ + wave * 32;
  const int myq = q0 + c;
  const bool qok = myq < S;
  const int64_t trow = ((int64_t)b * S + myq) * ldt + (int64_t)h * D;

  bf16x8 qf[DS], dof[DS];
  float dl = 0.0f;
#pragma unroll
  for (int s = 0; s < DS; ++s) {
    const int d = 16 * s + 8 * g;
    const uint4 z = make_uint4(0, 0, 0, 0);
    const uint4 qv = qok ? ld_global16(qb + (int64_t)myq * D + d) : z;
    const uint4 gv = qok ? ld_global16(dout + trow + d) : z;
    const uint4 ov = qok ? ld_global16(o + trow + d) : z;
    qf[s] = as_bf16x8(qv);
    dof[s] = as_bf16x8(gv);
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, ow[4] = {ov.x, ov.y, ov.z, ov.w};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      dl += st::bf16_to_f32((uint16_t)(gw[e >> 1] >> (16 * (e & 1)))) *
            st::bf16_to_f32((uint16_t)(ow[e >> 1] >> (16 * (e & 1))));
  }
  dl += __shfl_xor(dl, 32);
  const int64_t srow = (int64_t)(b * H + h) * S;
  if (g == 0 && qok) delta[srow + myq] = dl;
  const float lq = qok ? lse[srow + myq] : 0.0f;

  f32x16 dqacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) dqacc[i][e] = 0.0f;

  const int qlast = min(qt * BQ + BQ, S) - 1;
  const int ntiles = qlast / BKT + 1;
  uint4 kr[PER], vr[PER];
  auto load = [&](int t) {
    const int k0 = t * BKT;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int id = tid + i * NTH;
      const int row = id / (D / 8), ch = id % (D / 8);
      const bool ok = k0 + row < S;
      kr[i] = ok ? ld_global16(kb + (int64_t)(k0 + row) * D + ch * 8) : make_uint4(0, 0, 0, 0);
      vr[i] = ok ? ld_global16(vb + (int64_t)(k0 + row) * D + ch * 8) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
    uint16_t* ks = lds + buf * 2 * LT;
    uint16_t* vs = ks + LT;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int id = tid + i * NTH;
      const int row = id / (D / 8), ch = id % (D / 8);
      *(uint4*)(ks + tswz<D>(row, ch)) = kr[i];
      *(uint4*)(vs + tswz<D>(row, ch)) = vr[i];
    }
  };
  load(0);
  store(0);
  __syncthreads();
  for (int t = 0; t < ntiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < ntiles) load(t + 1);
    const uint16_t* ks = lds + buf * 2 * LT;
    const uint16_t* vs = ks + LT;
    const int k0 = t * BKT;
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      const int kb0 = k0 + jb * 32;
      if (kb0 > q0 + 31 || kb0 >= S) continue;
      f32x16 sacc, pacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) { sacc[e] = 0.0f; pacc[e] = 0.0f; }
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_row<D>(ks, jb * 32 + c, s, g), qf[s],
                                                       sacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_row<D>(vs, jb * 32 + c, s, g), dof[s],
                                                       pacc, 0, 0, 0);
      }
      bf16x8 dsf[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float ds[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int vv = 8 * hh + e;
          const int key = kb0 + (vv >> 2) * 8 + g * 4 + (vv & 3);
          const bool keep = key <= myq && key < S && qok;
          const float p = keep ? exp2f(sacc[vv] * sl2 - lq) : 0.0f;
          ds[e] = p * (pacc[vv] - dl);
        }
        dsf[hh] = as_bf16x8(make_uint4(st::pack_bf16x2(ds[0], ds[1]), st::pack_bf16x2(ds[2], ds[3]),
                                       st::pack_bf16x2(ds[4], ds[5]), st::pack_bf16x2(ds[6], ds[7])));
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int db = 0; db < DB; ++db)
          dqacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              tile_tr<D>(ks, jb * 32 + 16 * hh, db * 32, lane), dsf[hh], dqacc[db], 0, 0, 0);
    }
    if (t + 1 < ntiles) store(buf ^ 1);
    __syncthreads();
  }
  // dQ = scale * dQ^T^T, staged through LDS as query rows, head-major out
  constexpr int LDO = D + 8;
  uint16_t* os = lds + wave * 32 * LDO;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const int d = db * 32 + v4 * 8 + g * 4;
      const u32x2 w = {st::pack_bf16x2(dqacc[db][4 * v4] * scale, dqacc[db][4 * v4 + 1] * scale),
                       st::pack_bf16x2(dqacc[db][4 * v4 + 2] * scale, dqacc[db][4 * v4 + 3] * scale)};
      *(u32x2*)(os + c * LDO + d) = w;
    }
  __syncthreads();
  uint16_t* dqb = dq + ((int64_t)(b * H + h) * S) * D;
  for (int i = lane; i < 32 * (D / 8); i += 64) {
    const int r = i / (D / 8), ch = i % (D / 8);
    const int qq = q0 + r;
    if (qq < S) {
      const u32x2 a = *(const u32x2*)(os + r * LDO + ch * 8);
      const u32x2 bb = *(const u32x2*)(os + r * LDO + ch * 8 + 4);
      *(uint4*)(dqb + (int64_t)qq * D + ch * 8) = make_uint4(a.x, a.y, bb.x, bb.y);
    }
  }
}

// dK, dV of one query head over a 128-key tile (8 waves: 4 key quarters x 2
// query halves), looping over 64-query tiles from the diagonal down:
// S = Q K^T, P = exp2(S - lse), dP = dO V^T, dS = P (dP - Delta),
// dV^T += dO^T P, dK^T += Q^T dS.  Writes fp32 per-query-head partials.
constexpr int KT2 = 128, QT2 = 64, NTH2 = 512;

template <int D>
__global__ __launch_bounds__(NTH2, 2) void fa_bwd_dkdv(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, int S, int H, int Hkv,
    float sl2, float scale, float* __restrict__ dk_part, float* __restrict__ dv_part) {
  constexpr int DS = D / 16, DB = D / 32;
  constexpr int LK = KT2 * D, LQ = QT2 * D;
  constexpr int PERQ = QT2 * D / 8 / NTH2;   // 16-byte chunks per thread per Q (dO) tile
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * LK + 2 * 2 * LQ];
  __shared__ float lse_s[2][QT2], dl_s[2][QT2];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, c = lane & 31;
  const int kq = wave & 3, qh = wave >> 2;
  const int kt = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int hk = h / (H / Hkv);
  const int64_t ldt = (int64_t)H * D;
  const uint16_t* qb = q + ((int64_t)(b * H + h) * S) * D;
  const uint16_t* kb = k + ((int64_t)(b * Hkv + hk) * S) * D;
  const uint16_t* vb = v + ((int64_t)(b * Hkv + hk) * S) * D;
  const uint16_t* gb = dout + (int64_t)b * S * ldt + (int64_t)h * D;
  const int64_t srow = (int64_t)(b * H + h) * S;
  uint16_t* Ks = lds;
  uint16_t* Vs = lds + LK;
  const int k0 = kt * KT2;

  // resident K and V tiles
  for (int id = tid; id < KT2 * D / 8; id += NTH2) {
    const int row = id / (D / 8), ch = id % (D / 8);
    const bool ok = k0 + row < S;
    *(uint4*)(Ks + tswz<D>(row, ch)) =
        ok ? ld_global16(kb + (int64_t)(k0 + row) * D + ch * 8) : make_uint4(0, 0, 0, 0);
    *(uint4*)(Vs + tswz<D>(row, ch)) =
        ok ? ld_global16(vb + (int64_t)(k0 + row) * D + ch * 8) : make_uint4(0, 0, 0, 0);
  }
  const int kw0 = k0 + kq * 32;   // this wave's keys
  const int mykey = kw0 + c;

  f32x16 dvacc[DB], dkacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) { dvacc[i][e] = 0.0f; dkacc[i][e] = 0.0f; }

  const int qt_first = k0 / QT2;
  const int qt_end = (S + QT2 - 1) / QT2;
  uint4 qr[PERQ], gr[PERQ];
  float lr = 0.0f, dr = 0.0f;
  auto load = [&](int qt) {
    const int q0 = qt * QT2;
#pragma unroll
    for (int i = 0; i < PERQ; ++i) {
      const int id = tid + i * NTH2;
      const int row = id / (D / 8), ch = id % (D / 8);
      const bool ok = q0 + row < S;
      qr[i] = ok ? ld_global16(qb + (int64_t)(q0 + row) * D + ch * 8) : make_uint4(0, 0, 0, 0);
      gr[i] = ok ? ld_global16(gb + (int64_t)(q0 + row) * ldt + ch * 8) : make_uint4(0, 0, 0, 0);
    }
    if (tid < QT2) {
      const bool ok = q0 + tid < S;
      lr = ok ? lse[srow + q0 + tid] : 0.0f;
      dr = ok ? delta[srow + q0 + tid] : 0.0f;
    }
  };
  auto store = [&](int buf) {
    uint16_t* qs = lds + 2 * LK + buf * 2 * LQ;
    uint16_t* gs = qs + LQ;
#pragma unroll
    for (int i = 0; i < PERQ; ++i) {
      const int id = tid + i * NTH2;
      const int row = id / (D / 8), ch = id % (D / 8);
      *(uint4*)(qs + tswz<D>(row, ch)) = qr[i];
      *(uint4*)(gs + tswz<D>(row, ch)) = gr[i];
    }
    if (tid < QT2) { lse_s[buf][tid] = lr; dl_s[buf][tid] = dr; }
  };
  if (qt_first < qt_end) {
    load(qt_first);
    store(0);
  }
  __syncthreads();
  for (int qt = qt_first; qt < qt_end; ++qt) {
    const int buf = (qt - qt_first) & 1;
    if (qt + 1 < qt_end) load(qt + 1);
    const uint16_t* qs = lds + 2 * LK + buf * 2 * LQ;
    const uint16_t* gs = qs + LQ;
    const int qw0 = qt * QT2 + qh * 32;   // this wave's queries
    if (qw0 + 31 >= kw0 && qw0 < S) {     // some query sees some key
      f32x16 sacc, pacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) { sacc[e] = 0.0f; pacc[e] = 0.0f; }
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_row<D>(qs, qh * 32 + c, s, g),
                                                       tile_row<D>(Ks, kq * 32 + c, s, g), sacc,
                                                       0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_row<D>(gs, qh * 32 + c, s, g),
                                                       tile_row<D>(Vs, kq * 32 + c, s, g), pacc,
                                                       0, 0, 0);
      }
      bf16x8 pf[2], dsf[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float p8[8], d8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int vv = 8 * hh + e;
          const int r = qh * 32 + (vv >> 2) * 8 + g * 4 + (vv & 3);  // query row in tile
          const int qq = qt * QT2 + r;
          const bool keep = mykey <= qq && mykey < S && qq < S;
          const float p = keep ? exp2f(sacc[vv] * sl2 - lse_s[buf][r]) : 0.0f;
          p8[e] = p;
          d8[e] = p * (pacc[vv] - dl_s[buf][r]);
        }
        pf[hh] = as_bf16x8(make_uint4(st::pack_bf16x2(p8[0], p8[1]), st::pack_bf16x2(p8[2], p8[3]),
                                      st::pack_bf16x2(p8[4], p8[5]), st::pack_bf16x2(p8[6], p8[7])));
        dsf[hh] = as_bf16x8(make_uint4(st::pack_bf16x2(d8[0], d8[1]), st::pack_bf16x2(d8[2], d8[3]),
                                       st::pack_bf16x2(d8[4], d8[5]), st::pack_bf16x2(d8[6], d8[7])));
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          dvacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              tile_tr<D>(gs, qh * 32 + 16 * hh, db * 32, lane), pf[hh], dvacc[db], 0, 0, 0);
          dkacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              tile_tr<D>(qs, qh * 32 + 16 * hh, db * 32, lane), dsf[hh], dkacc[db], 0, 0, 0);
        }
    }
    if (qt + 1 < qt_end) store(buf ^ 1);
    __syncthreads();
  }
  // the two query halves of each key quarter: qh = 1 parks its sums in LDS,
  // qh = 0 adds them and writes [key][d] fp32 partials
  float* red = (float*)lds;                 // 4 quarters x 2 arrays x (DB*16*64) floats
  constexpr int PART = DB * 16 * 64;
  if (qh == 1) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        red[(kq * 2 + 0) * PART + (db * 16 + e) * 64 + lane] = dvacc[db][e];
        red[(kq * 2 + 1) * PART + (db * 16 + e) * 64 + lane] = dkacc[db][e];
      }
  }
  __syncthreads();
  if (qh == 0 && mykey < S) {
    float* dvp = dv_part + (srow + mykey) * D;
    float* dkp = dk_part + (srow + mykey) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const int d = db * 32 + v4 * 8 + g * 4;
        float4 a, bq;
        float* pa = &a.x;
        float* pb = &bq.x;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int vv = 4 * v4 + e;
          pa[e] = dvacc[db][vv] + red[(kq * 2 + 0) * PART + (db * 16 + vv) * 64 + lane];
          pb[e] = (dkacc[db][vv] + red[(kq * 2 + 1) * PART + (db * 16 + vv) * 64 + lane]) * scale;
        }
        *(float4*)(dvp + d) = a;
        *(float4*)(dkp + d) = bq;
      }
  }
}

// dk[b,hk] = bf16(sum over the group's query heads of dk_part), same for dv
__global__ __launch_bounds__(NTH) void fa_bwd_reduce(const float* __restrict__ dk_part,
                                                     const float* __restrict__ dv_part,
                                                     int64_t B, int64_t S, int H, int Hkv, int D,
                                                     uint16_t* __restrict__ dk,
                                                     uint16_t* __restrict__ dv) {
  const int64_t per = S * D;
  const int64_t n = B * Hkv * per / 4;
  const int grp = H / Hkv;
  for (int64_t i = (int64_t)blockIdx.x * NTH + threadIdx.x; i < n; i += (int64_t)gridDim.x * NTH) {
    const int64_t e = i * 4;
    const int64_t bh = e / per, off = e % per;
    const int64_t b = bh / Hkv, hk = bh % Hkv;
    float4 sk = make_float4(0, 0, 0, 0), sv = make_float4(0, 0, 0, 0);
    for (int j = 0; j < grp; ++j) {
      const int64_t src = ((b * H + hk * grp + j) * per) + off;
      const float4 a = *(const float4*)(dk_part + src);
      const float4 bb = *(const float4*)(dv_part + src);
      sk.x += a.x; sk.y += a.y; sk.z += a.z; sk.w += a.w;
      sv.x += bb.x; sv.y += bb.y; sv.z += bb.z; sv.w += bb.w;
    }
    *(u32x2*)(dk + e) = u32x2{st::pack_bf16x2(sk.x, sk.y), st::pack_bf16x2(sk.z, sk.w)};
    *(u32x2*)(dv + e) = u32x2{st::pack_bf16x2(sv.x, sv.y), st::pack_bf16x2(sv.z, sv.w)};
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" int64_t st_flash_attn_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t Hkv,
                                                 int64_t D, int32_t backward) {
  const int64_t kv = B * Hkv * S * D * 2;
  if (!backward) return kv + 256;  // V^T
  // Delta [B,H,S] fp32, then fp32 dK and dV partials per query head
  const int64_t dl = (B * H * S * 4 + 255) / 256 * 256;
  return 256 + dl + 2 * B * H * S * D * 4;
}

extern "C" int st_flash_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 int64_t B, int64_t S, int64_t H, int64_t Hkv, int64_t D,
                                 float scale, uint16_t* out, float* lse, void* workspace,
                                 int64_t workspace_bytes, st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && H > 0 && Hkv > 0 && H % Hkv == 0,
               "st_flash_attn_fwd: bad head counts");
  if (B == 0 || S == 0) return ST_OK;
  if (D != 64 && D != 128)
    return st::fail(ST_EUNSUPPORTED, "st_flash_attn_fwd: head_dim %lld (64 or 128 only)",
                    (long long)D);
  ST_CHECK_ARG(S % 8 == 0 && S < (1 << 30), "st_flash_attn_fwd: S must be a multiple of 8");
  ST_CHECK_ARG(q && k && v && out && lse && al16(q) && al16(k) && al16(v) && al16(out),
               "st_flash_attn_fwd: NULL or unaligned pointer");
  const int64_t need = st_flash_attn_workspace_bytes(B, S, H, Hkv, D, 0);
  if (!workspace || workspace_bytes < need)
    return st::fail(ST_EWORKSPACE, "st_flash_attn_fwd: needs %lld workspace bytes",
                    (long long)need);
  hipStream_t s = (hipStream_t)stream;
  uint16_t* vt = (uint16_t*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  transpose_heads<<<dim3((unsigned)st::cdiv(S, 64), (unsigned)st::cdiv(D, 64),
                         (unsigned)(B * Hkv)), NTH, 0, s>>>(v, vt, S, (int)D);
  int rc = st::check_launch("transpose_heads");
  if (rc) return rc;
  dim3 grid((unsigned)st::cdiv(S, BQ), (unsigned)H, (unsigned)B);
  const float sl2 = scale * LOG2E;
  if (D == 128)
    fa_fwd<128><<<grid, NTH, 0, s>>>(q, k, vt, (int)S, (int)H, (int)Hkv, sl2, out, lse);
  else
    fa_fwd<64><<<grid, NTH, 0, s>>>(q, k, vt, (int)S, (int)H, (int)Hkv, sl2, out, lse);
  return st::check_launch("fa_fwd");
}

extern "C" int st_flash_attn_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* out, const float* lse, const uint16_t* dout,
                                 int64_t B, int64_t S, int64_t H, int64_t Hkv, int64_t D,
                                 float scale, uint16_t* dq, uint16_t* dk, uint16_t* dv,
                                 void* workspace, int64_t workspace_bytes, st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && H > 0 && Hkv > 0 && H % Hkv == 0,
               "st_flash_attn_bwd: bad head counts");
  if (B == 0 || S == 0) return ST_OK;
  if (D != 64 && D != 128)
    return st::fail(ST_EUNSUPPORTED, "st_flash_attn_bwd: head_dim %lld (64 or 128 only)",
                    (long long)D);
  ST_CHECK_ARG(S % 8 == 0 && S < (1 << 30), "st_flash_attn_bwd: S must be a multiple of 8");
  ST_CHECK_ARG(q && k && v && out && lse && dout && dq && dk && dv && al16(q) && al16(k) &&
                   al16(v) && al16(out) && al16(dout) && al16(dq) && al16(dk) && al16(dv),
               "st_flash_attn_bwd: NULL or unaligned pointer");
  const int64_t need = st_flash_attn_workspace_bytes(B, S, H, Hkv, D, 1);
  if (!workspace || workspace_bytes < need)
    return st::fail(ST_EWORKSPACE, "st_flash_attn_bwd: needs %lld workspace bytes",
                    (long long)need);
  hipStream_t s = (hipStream_t)stream;
  char* base = (char*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  float* delta = (float*)base;
  float* dk_part = (float*)(base + (B * H * S * 4 + 255) / 256 * 256);
  float* dv_part = dk_part + B * H * S * D;
  const float sl2 = scale * LOG2E;
  dim3 g1((unsigned)st::cdiv(S, BQ), (unsigned)H, (unsigned)B);
  dim3 g2((unsigned)st::cdiv(S, KT2), (unsigned)H, (unsigned)B);
  if (D == 128) {
    fa_bwd_dq<128><<<g1, NTH, 0, s>>>(q, k, v, out, dout, lse, (int)S, (int)H, (int)Hkv, sl2,
                                      scale, delta, dq);
    int rc = st::check_launch("fa_bwd_dq");
    if (rc) return rc;
    fa_bwd_dkdv<128><<<g2, NTH2, 0, s>>>(q, k, v, dout, lse, delta, (int)S, (int)H, (int)Hkv,
                                         sl2, scale, dk_part, dv_part);
  } else {
    fa_bwd_dq<64><<<g1, NTH, 0, s>>>(q, k, v, out, dout, lse, (int)S, (int)H, (int)Hkv, sl2,
                                     scale, delta, dq);
    int rc = st::check_launch("fa_bwd_dq");
    if (rc) return rc;
    fa_bwd_dkdv<64><<<g2, NTH2, 0, s>>>(q, k, v, dout, lse, delta, (int)S, (int)H, (int)Hkv,
                                        sl2, scale, dk_part, dv_part);
  }
  int rc = st::check_launch("fa_bwd_dkdv");
  if (rc) return rc;
  const int64_t n4 = B * Hkv * S * D / 4;
  const unsigned blocks = (unsigned)std::min<int64_t>(st::cdiv(n4, NTH), 4096);
  fa_bwd_reduce<<<blocks, NTH, 0, s>>>(dk_part, dv_part, B, S, (int)H, (int)Hkv, (int)D, dk, dv);
  return st::check_launch("fa_bwd_reduce");
}
