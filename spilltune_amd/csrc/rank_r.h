// Streaming rank-r product tile shared by the LoRA kernels (lora.hip) and the
// per-expert LoRA kernels (moe.hip).
//
//   acc[m, j] += sum_{k in [kb, ke)} g(m, k) S[k, j]      (m in [m0, m0 + RK_BM))
//
// g(m, k) = G[row(m) * ldg + gcol0 + k]  (ROW: contraction contiguous), or
// g(m, k) = G[row(k) * ldg + gcol0 + m]  (COL: contraction over G's rows),
// with row(r) = r, or (GATHER) the source row of permuted row r: ROW reads
// gather[r] (a value outside [0, g_rows) reads as zero); COL reads it from
// the caller's LDS copy idx[r - idx0] of the gather rows for [kb, ke).
// S is fp32, split into three bf16 parts hi = bf16(s), mid = bf16(s - hi),
// lo = bf16(s - hi - mid) with s == hi + mid + lo exactly (24 significant bits
// in three pieces of 8; normal range): each bf16 x bf16 product is exact in
// fp32, so g*hi + g*mid + g*lo on v_mfma_f32_32x32x16_bf16 with fp32
// accumulation is the fp32 product g*s summed in fp32, at bf16 matrix-core
// rate.
//
// Streaming pipeline: a ring of RK_PF chunks of G (4 x 16 bytes per thread)
// and S lives in registers; as soon as a chunk is staged into LDS its slot is
// refilled with the chunk RK_PF steps ahead, so each workgroup keeps about
// RK_PF x 16 KiB of loads in flight while it computes.  Loads go through
// buffer resources with 32-bit offsets (operand extents below 2 GiB, checked
// by the host); rows or chunks out of range read as zero.  G rows (ROW:
// contraction; COL: output columns) are 16-byte aligned multiples of 8
// elements (checked by the host).
#pragma once
#include "common.h"

namespace st {

constexpr int RK_NTH = 256;  // 4 waves, 32 output rows each
constexpr int RK_BM = 128, RK_BK = 64, RK_RP = 64;
constexpr int RK_LD = RK_BK + 8;  // bf16 per LDS row (144 bytes: 16-byte aligned, bank-spread)
constexpr int RK_PF = 3;          // chunks of loads in flight per workgroup
constexpr int RK_SPLIT = 3;       // bf16 parts of each fp32 S value
constexpr int RK_SS = RK_SPLIT * RK_RP * RK_LD;  // bf16 of the staged S parts

// s = hi + mid + lo exactly for normal-range fp32 s (each part bf16-exact)
__device__ __forceinline__ void split3(float s, uint16_t& hi, uint16_t& mid, uint16_t& lo) {
  hi = f32_to_bf16(s);
  const float r1 = s - bf16_to_f32(hi);
  mid = f32_to_bf16(r1);
  lo = f32_to_bf16(r1 - bf16_to_f32(mid));
}

// Gs: RK_BM * RK_LD bf16 (ROW: G as [m][k] rows; COL: [k][m] in the
// transposed-operand layout); Ss: RK_SS bf16 (S as [hi|mid|lo][j][k]).
template <bool COL, bool SK1, int NB, bool GATHER>
__device__ __forceinline__ void rk_accumulate(f32x16 (&acc)[NB], int64_t mend, int64_t R,
                                              int64_t m0, int kb, int ke,
                                              const uint16_t* __restrict__ G, int64_t ldg,
                                              int64_t g_bytes, int64_t gcol0,
                                              const float* __restrict__ S, int64_t ssk,
                                              int64_t ssj, int64_t s_bytes,
                                              const int32_t* __restrict__ gather, int64_t g_rows,
                                              const int* idx, int idx0,
                                              uint16_t* __restrict__ Gs,
                                              uint16_t* __restrict__ Ss) {
  constexpr int NTH = RK_NTH;
  constexpr int RP = NB * 32;            // staged S columns
  constexpr int SIT = RK_BK * RP / NTH;  // S values per thread per chunk (8 or 16)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const auto rsG = make_rsrc(G, g_bytes);
  const auto rsS = make_rsrc(S, s_bytes);
  const uint32_t ldg2 = (uint32_t)ldg * 2, ssk4 = (uint32_t)ssk * 4, ssj4 = (uint32_t)ssj * 4;

  // G: per-thread byte offset at contraction 0 (kOOB for rows/columns outside
  // the tile) and the contraction offset of each of its four 16-byte pieces
  uint32_t gbase[4];
  int gk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (!COL) {  // 128 rows x 64 contraction: 8 pieces of 8 per row, 4 pieces per thread
      const int id = tid + i * NTH, row = id >> 3, c = id & 7;
      const int64_t m = m0 + row;
      int64_t src = m;
      if (GATHER && m < mend) {
        src = gather[m];
        if (src < 0 || src >= g_rows) src = -1;
      }
      gbase[i] = (m < mend && src >= 0) ? (uint32_t)((src * ldg + gcol0) * 2) + c * 16 : kOOB;
      gk[i] = c * 8;
    } else {  // 64 contraction rows x 128 columns: 4 rows x 8 columns per thread
      const int64_t m = m0 + (tid & 15) * 8;
      gbase[i] = m < mend ? (uint32_t)((m + gcol0) * 2) : kOOB;
      gk[i] = (tid >> 4) * 4 + i;
    }
  }
  // S value i of a thread: (contraction kk, column j).  SK1 (S contiguous
  // along the contraction): kk = tid % 64, j = tid / 64 + 4i; otherwise
  // j = tid % RP, kk = tid / RP + (NTH / RP) i.
  auto s_kk = [&](int i) { return SK1 ? (tid & 63) : tid / RP + (NTH / RP) * i; };
  auto s_j = [&](int i) { return SK1 ? (tid >> 6) + 4 * i : tid % RP; };

  uint4 gr[RK_PF][4];
  float sr[RK_PF][SIT];
  auto load = [&](int k0, uint4 (&g)[4], float (&sv)[SIT]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int k = k0 + gk[i];
      uint32_t off = kOOB;
      if (gbase[i] != kOOB && k < ke) {
        if (COL) {
          int64_t src = k;
          if (GATHER) {
            src = idx[k - idx0];
            if (src < 0 || src >= g_rows) src = -1;
          }
          if (src >= 0) off = gbase[i] + (uint32_t)src * ldg2;
        } else {
          off = gbase[i] + (uint32_t)k0 * 2;
        }
      }
      // the offset is materialised before the load: left to itself the
      // compiler turns a select of two offsets into two loads on divergent
      // paths, each behind a wait for every load in flight
      asm volatile("" : "+v"(off));
      g[i] = ld16(rsG, off);
    }
#pragma unroll
    for (int i = 0; i < SIT; ++i) {
      const int k = k0 + s_kk(i), j = s_j(i);
      uint32_t off = (k < ke && j < R) ? (uint32_t)k * ssk4 + (uint32_t)j * ssj4 : kOOB;
      asm volatile("" : "+v"(off));
      sv[i] = __builtin_bit_cast(float, ld4(rsS, off));
    }
  };
  auto store = [&](const uint4 (&g)[4], const float (&sv)[SIT]) {
    if (!COL) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int id = tid + i * NTH, row = id >> 3, c = id & 7;
        *(uint4*)&Gs[row * RK_LD + c * 8] = g[i];
      }
    } else {  // [contraction][column] as loaded; the MFMA operand is read transposed
      const int kg = tid >> 4, mg = tid & 15;
#pragma unroll
      for (int h = 0; h < 4; ++h) ((uint4*)Gs)[trswz<RK_BM>(kg * 4 + h, mg)] = g[h];
    }
#pragma unroll
    for (int i = 0; i < SIT; ++i) {
      const int kk = s_kk(i), j = s_j(i);
      uint16_t hb, mb, lb;
      split3(sv[i], hb, mb, lb);
      Ss[j * RK_LD + kk] = hb;
      Ss[(RK_RP + j) * RK_LD + kk] = mb;
      Ss[(2 * RK_RP + j) * RK_LD + kk] = lb;
    }
  };

  auto chunk_mfmas = [&]() {
#pragma unroll
    for (int s = 0; s < RK_BK / 16; ++s) {
      const int ko = s * 16 + (lane >> 5) * 8;
      const bf16x8 a = COL ? tr_operand<RK_BM>((const uint4*)Gs, s * 16, wave * 32, lane)
                           : *(const bf16x8*)&Gs[(wave * 32 + (lane & 31)) * RK_LD + ko];
#pragma unroll
      for (int cc = 0; cc < NB; ++cc)
#pragma unroll
        for (int h = 0; h < RK_SPLIT; ++h) {
          const bf16x8 b = *(const bf16x8*)&Ss[(h * RK_RP + cc * 32 + (lane & 31)) * RK_LD + ko];
          acc[cc] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[cc], 0, 0, 0);
        }
    }
  };

#pragma unroll
  for (int c = 0; c < RK_PF; ++c)
    if (kb + c * RK_BK < ke) load(kb + c * RK_BK, gr[c], sr[c]);
  for (int kg = kb; kg < ke; kg += RK_PF * RK_BK) {
#pragma unroll
    for (int c = 0; c < RK_PF; ++c) {
      const int k0 = kg + c * RK_BK;
      if (k0 >= ke) break;
      store(gr[c], sr[c]);
      __syncthreads();
      if (k0 + RK_PF * RK_BK < ke) load(k0 + RK_PF * RK_BK, gr[c], sr[c]);
      chunk_mfmas();
      __syncthreads();
    }
  }
}

// Row m and column j of accumulator value v of block c for this lane.
__device__ __forceinline__ int rk_row(int v) {
  return (threadIdx.x >> 6) * 32 + (v >> 2) * 8 + ((threadIdx.x & 63) >> 5) * 4 + (v & 3);
}
__device__ __forceinline__ int rk_col(int c) { return c * 32 + (threadIdx.x & 31); }

}  // namespace st
