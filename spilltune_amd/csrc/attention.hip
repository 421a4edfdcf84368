// Causal GQA flash attention for gfx950 (forward, and backward in two
// deterministic passes), replacing the eager scores/softmax/probabilities
// chain of adapters/dense.py:142-148.
//
// Layout: q [B, H, S, DQ], k [B, Hkv, S, DQ], v [B, Hkv, S, DV] (head-major
// bf16); the output is written token-major [B, S, H*DV]; lse [B, H, S] fp32 is
// the base-2 log-sum-exp of each query row of x = scale * log2(e) * q.k.
// DQ = DV = D for the dense layers (adapters/dense.py:142-148); DeepSeek's
// multi-head latent attention has query/key heads of DQ = 192 (128 + 64 rope
// dims) against value heads of DV = 128 (adapters/deepseek.py:150-153).
//
// Transposed formulation: every MFMA tile is S^T = K Q^T (rows = keys,
// columns = queries), so one lane owns one query column: the softmax max/sum
// are in-lane reductions plus one exchange between the two half-waves, and
// the probabilities are already in the B-operand layout of O^T += V^T P^T.
#include <type_traits>

#include "common.h"

namespace {

constexpr int NTH = 256;
constexpr int BQ = 128;  // queries per workgroup (4 waves x 32)
constexpr float LOG2E = 1.4426950408889634f;

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint4 ld_global16(const uint16_t* p) { return *(const uint4*)p; }

// K tile [64 keys][D] in LDS, 16-byte chunks XOR-swizzled by row
template <int D>
__device__ __forceinline__ int kswz(int row, int chunk) {
  return row * (D / 8) + (chunk ^ (row & (D / 8 - 1)));
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// ---------------------------------------------------------------- transpose
// Position of key j inside its 16-key group in the staged V^T rows: bits 2
// and 3 swapped, so the keys {4g..4g+3, 8+4g..8+4g+3} a lane's MFMA operand
// needs (the row order of a 32x32 accumulator block) are 8 adjacent bf16.
__host__ __device__ __forceinline__ int vpos(int j) {
  return (j & ~12) | ((j & 4) << 1) | ((j & 8) >> 1);
}
// dst[n][d][vpos(s)] = src[n][s][d] (rows of Sp >= S elements, zero past S).
// A workgroup moves a 64-key x 64-d block: 16-byte loads of source rows into
// LDS, then each thread gathers 8 keys of one d column and writes them as one
// 16-byte store (Sp is a multiple of 16, so every output chunk is aligned).
// D is a multiple of 8 and src 16-byte aligned (checked by the host).
__global__ __launch_bounds__(NTH) void transpose_heads(const uint16_t* __restrict__ src,
                                                       uint16_t* __restrict__ dst, int64_t S,
                                                       int64_t Sp, int D) {
  __shared__ __attribute__((aligned(16))) uint16_t t[64][72];  // [key][d], 16-byte rows
  const int64_t n = blockIdx.z;
  const int64_t s0 = (int64_t)blockIdx.x * 64, d0 = (int64_t)blockIdx.y * 64;
  const uint16_t* in = src + n * S * D;
  uint16_t* out = dst + n * Sp * D;
  for (int i = threadIdx.x; i < 64 * 8; i += NTH) {
    const int r = i / 8, c = (i % 8) * 8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (s0 + r < S && d0 + c < D) v = *(const uint4*)(in + (s0 + r) * D + d0 + c);
    *(uint4*)&t[r][c] = v;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 8; i += NTH) {
    const int r = i / 8, c = (i % 8) * 8;  // r: d, c: first of 8 positions in the 64-key block
    if (d0 + r >= D || s0 + c >= Sp) continue;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      w[e] = (uint32_t)t[vpos(c + 2 * e)][r] | ((uint32_t)t[vpos(c + 2 * e + 1)][r] << 16);
    *(uint4*)(out + (d0 + r) * Sp + s0 + c) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Direct global -> LDS copy of 16 bytes per lane; the 64 lanes of a wave fill
// 1 KiB of LDS contiguously from `lds_wave` (wave-uniform), so layouts are
// formed by choosing each lane's source address.
__device__ __forceinline__ void g2lds16(const uint16_t* src, uint16_t* lds_wave) {
  __builtin_amdgcn_global_load_lds((const void*)src,
                                   (__attribute__((address_space(3))) void*)lds_wave, 16, 0, 0);
}

// Buffer copy of 16 bytes per lane into LDS, laid out like g2lds16; an
// offset at or past the resource's extent reads zeros.  Tiles move the
// resource base (scalar work) and keep each lane's offset fixed, so a copy
// costs no vector instructions.
__device__ __forceinline__ void b2lds16(__amdgpu_buffer_rsrc_t rs, uint32_t off,
                                        uint16_t* lds_wave) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rs, (__attribute__((address_space(3))) void*)lds_wave, 16, off, 0, 0, 0);
}

// Thread chunks of a row-major [rows][D] tile (tswz layout) copied by NT
// threads, copy i covering rows i*R .. i*R+R-1 (R = NT/(D/8)).  When R is a
// multiple of 16 every copy puts a thread at the same in-row position (the
// swizzle repeats every 16 rows): one lane offset serves all copies, and
// copy i moves the resource base by i*R rows instead.
template <int D, int NT>
struct RowCopy {
  static constexpr bool uniform = NT % (D / 8) == 0 && (NT / (D / 8)) % 16 == 0;
  static constexpr int rows = NT / (D / 8);
};

// Workgroup -> (x, h, b) for a 1-D grid of nx * H * B workgroups.  Blocks are
// dispatched round-robin over the 8 XCDs; remapping keeps consecutive logical
// indices on one XCD, and x runs fastest, then the query heads of a KV group,
// so each XCD streams the K/V of its own KV heads through its own L2.
struct WgIdx {
  int x, h, b;
};
__device__ __forceinline__ WgIdx wg_index(int nx, int H) {
  const int64_t L = st::xcd_remap(blockIdx.x, gridDim.x);
  WgIdx w;
  w.x = (int)(L % nx);
  const int64_t hb = L / nx;
  w.h = (int)(hb % H);
  w.b = (int)(hb / H);
  return w;
}

// ---------------------------------------------------------------- forward
// LDS tiles use padded rows (one spare 16-byte slot per row) rather than an
// XOR swizzle: 16-byte operand reads of 16 consecutive rows then hit 16
// distinct bank groups, and every operand address is a per-lane base plus an
// immediate.  Direct global->LDS copies fill whole slots, pads included (a
// pad slot receives a harmless in-bounds copy).
template <int D>
constexpr int KSLOTS = D / 8 + 1;        // 16-byte slots per padded K row
template <int BKT>
constexpr int VSLOTS = BKT / 8 + 1;      // per padded V^T row
constexpr float RESCALE_LOG2 = 8.0f;     // running max may lag by up to 2^8

template <int DQ, int DV, int BKT, int G>
constexpr int fwd_lds_elems() {
  return G * 2 * (BKT * KSLOTS<DQ> + DV * VSLOTS<BKT>) * 8;
}

// QW query waves per key group (32 queries each, 32*QW per workgroup).
// G = 1: one group over all keys.  G = 2: two groups over the same queries,
// group r taking K/V tiles r, r+2, ...; group 1's softmax state (max, partial
// sums, O) is merged into group 0's at the end.
template <int DQ, int DV, int BKT, int G, int QW>
__device__ __forceinline__ void fa_fwd_tile(const uint16_t* __restrict__ q,
                                            const uint16_t* __restrict__ k,
                                            const uint16_t* __restrict__ vt, int S, int H,
                                            int Hkv, float sl2, uint16_t* __restrict__ out,
                                            float* __restrict__ lse, int qt, int h, int b,
                                            int Sk, uint16_t* lds) {
  constexpr int DS = DQ / 16;  // contraction steps over the query/key dims
  constexpr int DB = DV / 32;  // 32-row blocks of O^T
  constexpr int KS = KSLOTS<DQ>, VS = VSLOTS<BKT>;
  constexpr int LK = BKT * KS * 8, LV = DV * VS * 8;  // bf16 per padded tile
  constexpr int KI = BKT * KS / 64, VI = DV * VS / 64;  // wave copies (1 KiB each) per tile
  static_assert((BKT * KS) % 64 == 0 && (DV * VS) % 64 == 0, "tiles are whole wave copies");

  const int tid = threadIdx.x, lane = tid & 63;
  // key group, wave in group (wave-uniform: tile indices and LDS bases are scalar)
  constexpr int BQW = 32 * QW;  // queries per workgroup
  const int grp = __builtin_amdgcn_readfirstlane((tid >> 6) / QW);
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) % QW);
  const int g = lane >> 5, c = lane & 31;
  const int hk = h / (H / Hkv);
  const uint16_t* qb = q + ((int64_t)(b * H + h) * S) * DQ;
  const uint16_t* kb = k + ((int64_t)(b * Hkv + hk) * S) * DQ;
  const int Sp = (S + 15) & ~15;                // staged V^T row length
  const uint16_t* vb = vt + ((int64_t)(b * Hkv + hk) * DV) * Sp;
  const int q0 = qt * BQW + wave * 32;
  const int myq = q0 + c;
  uint16_t* glds = lds + grp * 2 * (LK + LV);   // this group's two tile buffers

  bf16x8 qf[DS];
#pragma unroll
  for (int s = 0; s < DS; ++s)
    qf[s] = as_bf16x8(myq < S ? ld_global16(qb + (int64_t)myq * DQ + 16 * s + 8 * g)
                              : make_uint4(0, 0, 0, 0));

  f32x16 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int v = 0; v < 16; ++v) oacc[i][v] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  const int qlast = min(qt * BQW + BQW, S) - 1;  // last query of the workgroup
  // causal: keys <= qlast; keys >= Sk (right padding) are masked out
  const int ntiles = min(qlast, Sk - 1) / BKT + 1;
  const int nsteps = (ntiles + G - 1) / G;      // group steps (tile u*G + grp)
  // Copies: wave copy wi fills 1 KiB of the padded tile; pad slots repeat
  // the row's last chunk.  Lane offsets are fixed, the tile's first key moves
  // the resource base.  K rows past S read zeros; V^T columns past a row's
  // end read the next row's first columns (or zeros past the head): every
  // such key is masked out, so its probability is exactly 0.
  constexpr int KW = (KI + QW - 1) / QW, VW = (VI + QW - 1) / QW;
  uint32_t koff[KW], voff[VW];
#pragma unroll
  for (int i = 0; i < KW; ++i) {
    const int P = (i * QW + wave) * 64 + lane;
    const int row = min(P / KS, BKT - 1), ch = min(P % KS, DQ / 8 - 1);
    koff[i] = (uint32_t)(row * DQ + ch * 8) * 2;
  }
#pragma unroll
  for (int i = 0; i < VW; ++i) {
    const int P = (i * QW + wave) * 64 + lane;
    const int d = min(P / VS, DV - 1), ch = min(P % VS, BKT / 8 - 1);
    voff[i] = (uint32_t)(d * Sp + ch * 8) * 2;
  }
  auto issue = [&](int t, int buf) {
    const int k0 = t * BKT;
    const auto rk = st::make_rsrc(kb + (int64_t)k0 * DQ, (int64_t)(S - k0) * DQ * 2);
    const auto rv = st::make_rsrc(vb + k0, ((int64_t)DV * Sp - k0) * 2);
    uint16_t* ks = glds + buf * (LK + LV);
    uint16_t* vs = ks + LK;
#pragma unroll
    for (int i = 0; i < KW; ++i)
      if (i * QW + wave < KI) b2lds16(rk, koff[i], ks + (i * QW + wave) * 64 * 8);
#pragma unroll
    for (int i = 0; i < VW; ++i)
      if (i * QW + wave < VI) b2lds16(rv, voff[i], vs + (i * QW + wave) * 64 * 8);
  };

  if (grp < ntiles) issue(grp, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // one barrier per step: the next tile lands in the other buffer, whose
  // readers (step u-1) all passed the previous barrier
  for (int u = 0; u < nsteps; ++u) {
    const int buf = u & 1;
    const int t = u * G + grp;
    if (t + G < ntiles) issue(t + G, buf ^ 1);
    const uint16_t* ks = glds + buf * (LK + LV);
    const uint16_t* vs = ks + LK;
    const uint16_t* kl = ks + (c * KS + g) * 8;   // this lane's K operand row
    const uint16_t* vl = vs + (c * VS + g) * 8;   // this lane's V^T operand row
    const int k0 = t * BKT;
    // One code path for every tile: S^T = K Q^T for the tile's keys, the
    // causal / ragged mask as one per-lane key limit (entry v of block jb
    // holds key offset 32jb + 8(v>>2) + 4g + (v&3); offsets above the limit
    // become -inf), online softmax over the tile, O^T += V^T P^T.  A tile
    // wholly above this wave's queries is skipped (wave-uniform).
    if (t < ntiles && k0 <= q0 + 31) {
      const bool edge = k0 + BKT - 1 > q0 || k0 + BKT > Sk;  // wave-uniform
      const int limg = (edge ? min(myq, Sk - 1) - k0 : BKT) - g * 4;
      f32x16 sacc[BKT / 32];
#pragma unroll
      for (int jb = 0; jb < BKT / 32; ++jb)
#pragma unroll
        for (int v = 0; v < 16; ++v) sacc[jb][v] = 0.0f;
#pragma unroll
      for (int s = 0; s < DS; ++s)
#pragma unroll
        for (int jb = 0; jb < BKT / 32; ++jb) {
          const bf16x8 a = as_bf16x8(*(const uint4*)(kl + (jb * 32 * KS + 2 * s) * 8));
          sacc[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[s], sacc[jb], 0, 0, 0);
        }
      if (edge) {
#pragma unroll
        for (int jb = 0; jb < BKT / 32; ++jb)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            sacc[jb][v] = jb * 32 + (v >> 2) * 8 + (v & 3) <= limg ? sacc[jb][v] : -INFINITY;
      }
      float mt = sacc[0][0];
#pragma unroll
      for (int jb = 0; jb < BKT / 32; ++jb)
#pragma unroll
        for (int v = 0; v < 16; ++v) mt = fmaxf(mt, sacc[jb][v]);
      mt = fmaxf(mt, __shfl_xor(mt, 32)) * sl2;
      // rescale only when some query's max grew by more than 2^8
      if (__ballot(mt > m_run + RESCALE_LOG2)) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
        for (int i = 0; i < DB; ++i)
#pragma unroll
          for (int v = 0; v < 16; ++v) oacc[i][v] *= alpha;
        l_run *= alpha;
        m_run = m_new;
      }
      // a row with no visible key yet keeps m_run = -inf: its masked entries
      // give exp2(-inf) = 0 against an offset of 0
      const float m_use = m_run == -INFINITY ? 0.0f : m_run;
      bf16x8 pf[BKT / 16];
#pragma unroll
      for (int cc = 0; cc < BKT / 16; ++cc) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[cc >> 1][8 * (cc & 1) + e], sl2, -m_use));
          l_run += p[e];
        }
        pf[cc] = as_bf16x8(make_uint4(st::pack_bf16x2(p[0], p[1]), st::pack_bf16x2(p[2], p[3]),
                                      st::pack_bf16x2(p[4], p[5]), st::pack_bf16x2(p[6], p[7])));
      }
#pragma unroll
      for (int cc = 0; cc < BKT / 16; ++cc)
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const bf16x8 a = as_bf16x8(*(const uint4*)(vl + (db * 32 * VS + 2 * cc) * 8));
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[cc], oacc[db], 0, 0, 0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  if (G == 2) {  // group 1 parks (m, l, O) per lane; group 0 merges them
    float* park = (float*)lds + wave * 64 * (16 * DB + 2);
    if (grp == 1) {
#pragma unroll
      for (int i = 0; i < DB; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) park[(i * 16 + v) * 64 + lane] = oacc[i][v];
      park[(16 * DB) * 64 + lane] = m_run;
      park[(16 * DB + 1) * 64 + lane] = l_run;
    }
    __syncthreads();
    if (grp == 0) {
      const float mb = park[(16 * DB) * 64 + lane], lb = park[(16 * DB + 1) * 64 + lane];
      const float m = fmaxf(m_run, mb);
      const float aa = __builtin_amdgcn_exp2f(m_run - m), ab = __builtin_amdgcn_exp2f(mb - m);
#pragma unroll
      for (int i = 0; i < DB; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          oacc[i][v] = oacc[i][v] * aa + park[(i * 16 + v) * 64 + lane] * ab;
      l_run = l_run * aa + lb * ab;
      m_run = m;
    }
    __syncthreads();  // parked values read before the output staging reuses LDS
    if (grp == 1) return;
  }
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = 1.0f / l_tot;
  if (g == 0 && myq < S) lse[((int64_t)(b * H + h)) * S + myq] = m_run + log2f(l_tot);
  // stage O (query rows) through LDS for 16-byte token-major stores
  constexpr int LDO = DV + 8;
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
  // each wave reads back only its own rows: a wave-level fence suffices
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();
  const int64_t ld_out = (int64_t)H * DV;
  for (int i = lane; i < 32 * (DV / 8); i += 64) {
    const int r = i / (DV / 8), ch = i % (DV / 8);
    const int qq = q0 + r;
    if (qq < S) {
      const u32x2 a = *(const u32x2*)(os + r * LDO + ch * 8);
      const u32x2 bb = *(const u32x2*)(os + r * LDO + ch * 8 + 4);
      *(uint4*)(out + ((int64_t)b * S + qq) * ld_out + (int64_t)h * DV + ch * 8) =
          make_uint4(a.x, a.y, bb.x, bb.y);
    }
  }
}

// Valid keys of batch row b: all S, or (right padding) the first kvlen[b],
// clamped to [1, S] so no bound can pass S.
__device__ __forceinline__ int key_len(const int* __restrict__ kvlen, int b, int S) {
  return kvlen ? min(max(kvlen[b], 1), S) : S;
}

// Causal work per 128-query tile grows with its index; with `paired` each
// workgroup takes tiles i and n-1-i (equal total work per workgroup).
__device__ __forceinline__ int pair_tile(int x, int it, int nq, int paired) {
  if (!paired) return nq - 1 - x;  // longest tiles first
  return it == 0 ? nq - 1 - x : x;
}

template <int DQ, int DV, int BKT, int G, int QW = 4>
__global__ __launch_bounds__(64 * QW * G, G == 1 && QW == 4 && BKT == 64 && DQ <= 128 ? 2 : 1)
void fa_fwd(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
            const uint16_t* __restrict__ vt, int S, int H, int Hkv, float sl2,
            uint16_t* __restrict__ out, float* __restrict__ lse, int nq, int paired,
            const int* __restrict__ kvlen) {
  static_assert(QW * 32 * (DV + 8) <= fwd_lds_elems<DQ, DV, BKT, G>(), "output staging fits");
  __shared__ __attribute__((aligned(16))) uint16_t lds[fwd_lds_elems<DQ, DV, BKT, G>()];
  const WgIdx w = wg_index(paired ? (nq + 1) / 2 : nq, H);
  for (int it = 0; it < 1 + paired; ++it) {
    const int qt = pair_tile(w.x, it, nq, paired);
    if (it == 1) {
      if (qt == pair_tile(w.x, 0, nq, paired)) break;
      __syncthreads();  // the previous tile's output staging still reads LDS
    }
    fa_fwd_tile<DQ, DV, BKT, G, QW>(q, k, vt, S, H, Hkv, sl2, out, lse, qt, w.h, w.b,
                                    key_len(kvlen, w.b, S), lds);
  }
}

// ---------------------------------------------------------------- backward
// Row-major [rows][D] LDS tile, 16-byte chunks XOR-swizzled by row.  For
// D = 128 (rows of 256 bytes, each starting at bank 0) the XOR value
// ((row & 3) << 2) | ((row >> 2) & 3) is a permutation of row & 15, so the
// 16 rows of a quarter-wave 16-byte read (tile_row) land on 16 distinct chunk
// positions, and the 4 rows x 4 chunks of a half-wave transposing 8-byte read
// (tile_tr: rows 4 apart in bits 2-3 of the XOR value, chunks in bits 0-1)
// land on 16 distinct chunks: both are free of bank conflicts.  Other widths
// keep the XOR value ((row & 7) << 1), which stays inside the row's chunks.
template <int D>
__device__ __forceinline__ int swz(int row) {
  if constexpr (D == 128)
    return ((row & 3) << 2) | ((row >> 2) & 3);
  else
    return ((row & 7) << 1) & (D / 8 - 1);
}
template <int D>
__device__ __forceinline__ int tswz(int row, int chunk) {
  return row * D + ((chunk ^ swz<D>(row)) << 3);
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
template <int DQ, int DV, int BKT, int G, int QW>
__device__ __forceinline__ void fa_bwd_dq_tile(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ o,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse, int S, int H, int Hkv,
    float sl2, float scale, float* __restrict__ delta, uint16_t* __restrict__ dq, int qt, int h,
    int b, int Sk, uint16_t* lds) {
  constexpr int DSQ = DQ / 16, DSV = DV / 16, DB = DQ / 32;
  constexpr int LTK = BKT * DQ, LTV = BKT * DV;  // bf16 per K / V tile
  constexpr int NTG = 64 * QW;  // threads per key group
  constexpr int PERK = BKT * DQ / 8 / NTG, PERV = BKT * DV / 8 / NTG;  // 16-byte chunks per thread
  static_assert(PERK * NTG * 8 == LTK && PERV * NTG * 8 == LTV, "tiles are whole thread copies");
  const int tid = threadIdx.x, lane = tid & 63;
  // key group, wave in group (wave-uniform: tile indices and LDS bases are scalar)
  const int grp = __builtin_amdgcn_readfirstlane((tid >> 6) / QW);
  const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) % QW);
  const int gtid = tid % NTG;
  const int g = lane >> 5, c = lane & 31;
  const int hk = h / (H / Hkv);
  const int64_t ldt = (int64_t)H * DV;  // token-major row stride of O and dO
  const uint16_t* qb = q + ((int64_t)(b * H + h) * S) * DQ;
  const uint16_t* kb = k + ((int64_t)(b * Hkv + hk) * S) * DQ;
  const uint16_t* vb = v + ((int64_t)(b * Hkv + hk) * S) * DV;
  const int q0 = qt * (32 * QW) + wave * 32;
  const int myq = q0 + c;
  const bool qok = myq < S;
  const int64_t trow = ((int64_t)b * S + myq) * ldt + (int64_t)h * DV;
  uint16_t* glds = lds + grp * 2 * (LTK + LTV);  // this group's two K|V buffers

  bf16x8 qf[DSQ], dof[DSV];
  float dl = 0.0f;
  const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int s = 0; s < DSQ; ++s)
    qf[s] = as_bf16x8(qok ? ld_global16(qb + (int64_t)myq * DQ + 16 * s + 8 * g) : z);
#pragma unroll
  for (int s = 0; s < DSV; ++s) {
    const int d = 16 * s + 8 * g;
    const uint4 gv = qok ? ld_global16(dout + trow + d) : z;
    const uint4 ov = qok ? ld_global16(o + trow + d) : z;
    dof[s] = as_bf16x8(gv);
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w}, ow[4] = {ov.x, ov.y, ov.z, ov.w};
#pragma unroll
    for (int e = 0; e < 8; ++e)
      dl += st::bf16_to_f32((uint16_t)(gw[e >> 1] >> (16 * (e & 1)))) *
            st::bf16_to_f32((uint16_t)(ow[e >> 1] >> (16 * (e & 1))));
  }
  dl += __shfl_xor(dl, 32);
  const int64_t srow = (int64_t)(b * H + h) * S;
  if (grp == 0 && g == 0 && qok) delta[srow + myq] = dl;
  const float lq = qok ? lse[srow + myq] : INFINITY;  // rows past S: probability 0

  f32x16 dqacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) dqacc[i][e] = 0.0f;

  const int qlast = min(qt * (32 * QW) + 32 * QW, S) - 1;
  const int ntiles = min(qlast, Sk - 1) / BKT + 1;
  const int nsteps = (ntiles + G - 1) / G;
  // K and V tiles [key][D] (tswz layout) by buffer copies into LDS: fixed
  // lane offsets, the tile's first key in the resource base; keys past S
  // read zeros and are masked out below
  using CK = RowCopy<DQ, NTG>;
  using CV = RowCopy<DV, NTG>;
  uint32_t koff[CK::uniform ? 1 : PERK], voff[CV::uniform ? 1 : PERV];
#pragma unroll
  for (int i = 0; i < (CK::uniform ? 1 : PERK); ++i) {
    const int P = i * NTG + gtid;
    const int row = P / (DQ / 8);
    koff[i] = (uint32_t)(row * DQ + ((P % (DQ / 8)) ^ swz<DQ>(row)) * 8) * 2;
  }
#pragma unroll
  for (int i = 0; i < (CV::uniform ? 1 : PERV); ++i) {
    const int P = i * NTG + gtid;
    const int row = P / (DV / 8);
    voff[i] = (uint32_t)(row * DV + ((P % (DV / 8)) ^ swz<DV>(row)) * 8) * 2;
  }
  auto issue = [&](int t, int buf) {
    const int k0 = t * BKT;
    uint16_t* ks = glds + buf * (LTK + LTV);
    uint16_t* vs = ks + LTK;
#pragma unroll
    for (int i = 0; i < PERK; ++i) {
      const int r0 = k0 + (CK::uniform ? i * CK::rows : 0);
      const auto rk = st::make_rsrc(kb + (int64_t)r0 * DQ, (int64_t)max(S - r0, 0) * DQ * 2);
      b2lds16(rk, koff[CK::uniform ? 0 : i], ks + (i * NTG + wave * 64) * 8);
    }
#pragma unroll
    for (int i = 0; i < PERV; ++i) {
      const int r0 = k0 + (CV::uniform ? i * CV::rows : 0);
      const auto rv = st::make_rsrc(vb + (int64_t)r0 * DV, (int64_t)max(S - r0, 0) * DV * 2);
      b2lds16(rv, voff[CV::uniform ? 0 : i], vs + (i * NTG + wave * 64) * 8);
    }
  };
  // one 32-key block: S^T, dP^T, dS^T (masked when `edge`), dQ^T += K^T dS^T
  // `lim`: the largest kept key offset within the block less 4g (entry v of
  // the accumulator holds key offset 8(v>>2) + 4g + (v&3)); 31 keeps all
  auto block = [&](const uint16_t* ks, const uint16_t* vs, int jb, int lim) {
    f32x16 sacc, pacc;
#pragma unroll
    for (int e = 0; e < 16; ++e) { sacc[e] = 0.0f; pacc[e] = 0.0f; }
#pragma unroll
    for (int s = 0; s < DSQ; ++s) {
      sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_row<DQ>(ks, jb * 32 + c, s, g), qf[s],
                                                     sacc, 0, 0, 0);
      if (s < DSV)
        pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tile_row<DV>(vs, jb * 32 + c, s, g),
                                                       dof[s < DSV ? s : 0], pacc, 0, 0, 0);
    }
    bf16x8 dsf[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      float ds[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int vv = 8 * hh + e;
        float x = __builtin_fmaf(sacc[vv], sl2, -lq);
        x = (vv >> 2) * 8 + (vv & 3) <= lim ? x : -INFINITY;  // exp2(-inf) = 0
        ds[e] = __builtin_amdgcn_exp2f(x) * (pacc[vv] - dl);
      }
      dsf[hh] = as_bf16x8(make_uint4(st::pack_bf16x2(ds[0], ds[1]), st::pack_bf16x2(ds[2], ds[3]),
                                     st::pack_bf16x2(ds[4], ds[5]), st::pack_bf16x2(ds[6], ds[7])));
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int db = 0; db < DB; ++db)
        dqacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            tile_tr<DQ>(ks, jb * 32 + 16 * hh, db * 32, lane), dsf[hh], dqacc[db], 0, 0, 0);
  };
  if (grp < ntiles) issue(grp, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int u = 0; u < nsteps; ++u) {
    const int buf = u & 1;
    const int t = u * G + grp;
    if (t + G < ntiles) issue(t + G, buf ^ 1);
    const uint16_t* ks = glds + buf * (LTK + LTV);
    const uint16_t* vs = ks + LTK;
    const int k0 = t * BKT;
    if (t < ntiles) {
#pragma unroll
      for (int jb = 0; jb < BKT / 32; ++jb) {
        const int kb0 = k0 + jb * 32;
        if (kb0 > q0 + 31 || kb0 >= Sk) continue;  // wave-uniform
        const bool edge = kb0 + 31 > q0 || kb0 + 31 >= Sk || q0 + 31 >= S;
        block(ks, vs, jb, edge ? min(myq, Sk - 1) - kb0 - g * 4 : 31);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (G == 2) {  // dQ is additive over keys: group 1 parks, group 0 adds
    float* park = (float*)lds + wave * 64 * (16 * DB);
    if (grp == 1) {
#pragma unroll
      for (int i = 0; i < DB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) park[(i * 16 + e) * 64 + lane] = dqacc[i][e];
    }
    __syncthreads();
    if (grp == 0) {
#pragma unroll
      for (int i = 0; i < DB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) dqacc[i][e] += park[(i * 16 + e) * 64 + lane];
    }
    __syncthreads();
    if (grp == 1) return;
  }
  // dQ = scale * dQ^T^T, staged through LDS as query rows, head-major out;
  // with 8 query waves the two halves take turns with the staging space
  constexpr int LDO = DQ + 8;
  static_assert(4 * 32 * LDO <= G * 2 * BKT * (DQ + DV), "four waves' staging fits");
  uint16_t* os = lds + (wave % 4) * 32 * LDO;
  for (int half = 0; half < QW / 4; ++half) {
  if (half) __syncthreads();  // the previous half's read-back is done
  if (wave / 4 != half) continue;
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int v4 = 0; v4 < 4; ++v4) {
      const int d = db * 32 + v4 * 8 + g * 4;
      const u32x2 w = {st::pack_bf16x2(dqacc[db][4 * v4] * scale, dqacc[db][4 * v4 + 1] * scale),
                       st::pack_bf16x2(dqacc[db][4 * v4 + 2] * scale, dqacc[db][4 * v4 + 3] * scale)};
      *(u32x2*)(os + c * LDO + d) = w;
    }
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_wave_barrier();  // each wave reads back only its own rows
  uint16_t* dqb = dq + ((int64_t)(b * H + h) * S) * DQ;
  for (int i = lane; i < 32 * (DQ / 8); i += 64) {
    const int r = i / (DQ / 8), ch = i % (DQ / 8);
    const int qq = q0 + r;
    if (qq < S) {
      const u32x2 a = *(const u32x2*)(os + r * LDO + ch * 8);
      const u32x2 bb = *(const u32x2*)(os + r * LDO + ch * 8 + 4);
      *(uint4*)(dqb + (int64_t)qq * DQ + ch * 8) = make_uint4(a.x, a.y, bb.x, bb.y);
    }
  }
  }
}
template <int DQ, int DV, int BKT, int G, int QW = 4>
__global__ __launch_bounds__(64 * QW * G, G == 1 && QW == 4 && BKT == 64 && DQ <= 128 ? 2 : 1)
void fa_bwd_dq(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ o,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse, int S, int H, int Hkv,
    float sl2, float scale, float* __restrict__ delta, uint16_t* __restrict__ dq, int nq,
    int paired, const int* __restrict__ kvlen) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[G * 2 * BKT * (DQ + DV)];
  const WgIdx w = wg_index(paired ? (nq + 1) / 2 : nq, H);
  for (int it = 0; it < 1 + paired; ++it) {
    const int qt = pair_tile(w.x, it, nq, paired);
    if (it == 1) {
      if (qt == pair_tile(w.x, 0, nq, paired)) break;
      __syncthreads();
    }
    fa_bwd_dq_tile<DQ, DV, BKT, G, QW>(q, k, v, o, dout, lse, S, H, Hkv, sl2, scale, delta, dq,
                                       qt, w.h, w.b, key_len(kvlen, w.b, S), lds);
  }
}

// dK, dV of one query head over a 128-key tile, looping over 64-query tiles
// from the diagonal down: S = Q K^T, P = exp2(S - lse), dP = dO V^T,
// dS = P (dP - Delta), dV^T += dO^T P, dK^T += Q^T dS.  Writes fp32
// per-query-head partials.  DQ <= 128: 8 waves (4 key quarters x 2 query
// halves, two waves per SIMD; the halves' sums meet in LDS at the end), K and
// V tiles in LDS.  DQ = 192: 4 waves, one per key quarter, each taking both
// query halves in turn; a wave only ever reads its own 32 keys, so their K
// and V fragments stay in registers (one wave per SIMD has the whole register
// file: the dK and dV accumulators spilled 70 registers at two waves per
// SIMD) and LDS holds only the Q|dO tiles.  The Q|dO tiles are double
// buffered: the next tile's copy overlaps this one's MFMAs.  (The 4-wave form
// at DQ = 128 measured 172 us against 125 us for the 8-wave one: one wave per
// SIMD hides less latency than it saves in LDS reads.)
constexpr int KT2 = 128, QT2 = 64;
template <int DQ>
constexpr int dkdv_waves() {
  return DQ <= 128 ? 8 : 4;
}
template <int DQ, int DV>
constexpr int dkdv_lds_elems() {
  return (dkdv_waves<DQ>() == 8 ? KT2 + 2 * QT2 : 2 * QT2) * (DQ + DV);
}

template <int DQ, int DV>
__device__ __forceinline__ void fa_bwd_dkdv_tile(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, int S, int H, int Hkv,
    float sl2, float scale, float* __restrict__ dk_part, float* __restrict__ dv_part,
    uint16_t* __restrict__ dk_out, uint16_t* __restrict__ dv_out, int kt, int h, int b, int Sk,
    uint16_t* lds, float (*lse_s)[QT2], float (*dl_s)[QT2]) {
  constexpr int DSQ = DQ / 16, DSV = DV / 16, DBQ = DQ / 32, DBV = DV / 32;
  constexpr int LK = KT2 * DQ, LV = KT2 * DV, LQ = QT2 * DQ, LG = QT2 * DV;
  constexpr int NW = dkdv_waves<DQ>(), NTH2 = 64 * NW, QH = 8 / NW;  // query halves per wave
  constexpr bool KREG = NW == 4;  // K and V fragments in registers
  constexpr int PERQ = LQ / 8 / NTH2, PERG = LG / 8 / NTH2;  // 16-byte chunks per thread
  static_assert(PERQ * NTH2 * 8 == LQ && PERG * NTH2 * 8 == LG, "tiles are whole thread copies");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, c = lane & 31;
  const int kq = wave & 3, qh0 = NW == 8 ? wave >> 2 : 0;
  const int hk = h / (H / Hkv);
  const int64_t ldt = (int64_t)H * DV;
  const uint16_t* qb = q + ((int64_t)(b * H + h) * S) * DQ;
  const uint16_t* kb = k + ((int64_t)(b * Hkv + hk) * S) * DQ;
  const uint16_t* vb = v + ((int64_t)(b * Hkv + hk) * S) * DV;
  const uint16_t* gb = dout + (int64_t)b * S * ldt + (int64_t)h * DV;
  const int64_t srow = (int64_t)(b * H + h) * S;
  uint16_t* Ks = lds;
  uint16_t* Vs = lds + LK;
  uint16_t* qg = KREG ? lds : lds + LK + LV;  // Q|dO buffers
  const int k0 = kt * KT2;
  const int kw0 = k0 + kq * 32;   // this wave's keys
  const int mykey = kw0 + c;
  // KREG: the wave's K and V rows as MFMA operands (tile_row's fragments)
  bf16x8 kfr[KREG ? DSQ : 1], vfr[KREG ? DSV : 1];
  if constexpr (KREG) {
    const uint4 z = make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int s = 0; s < DSQ; ++s)
      kfr[s] = as_bf16x8(mykey < S ? ld_global16(kb + (int64_t)mykey * DQ + 16 * s + 8 * g) : z);
#pragma unroll
    for (int s = 0; s < DSV; ++s)
      vfr[s] = as_bf16x8(mykey < S ? ld_global16(vb + (int64_t)mykey * DV + 16 * s + 8 * g) : z);
  }

  // resident K and V tiles
  if constexpr (!KREG) {
  for (int id = tid; id < KT2 * DQ / 8; id += NTH2) {
    const int row = id / (DQ / 8), ch = id % (DQ / 8);
    *(uint4*)(Ks + tswz<DQ>(row, ch)) = k0 + row < S
        ? ld_global16(kb + (int64_t)(k0 + row) * DQ + ch * 8) : make_uint4(0, 0, 0, 0);
  }
  for (int id = tid; id < KT2 * DV / 8; id += NTH2) {
    const int row = id / (DV / 8), ch = id % (DV / 8);
    *(uint4*)(Vs + tswz<DV>(row, ch)) = k0 + row < S
        ? ld_global16(vb + (int64_t)(k0 + row) * DV + ch * 8) : make_uint4(0, 0, 0, 0);
  }
  }

  f32x16 dvacc[DBV], dkacc[DBQ];
#pragma unroll
  for (int i = 0; i < DBV; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) dvacc[i][e] = 0.0f;
#pragma unroll
  for (int i = 0; i < DBQ; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) dkacc[i][e] = 0.0f;

  const int qt_first = k0 / QT2;
  const int qt_end = (S + QT2 - 1) / QT2;
  float lr = 0.0f, dr = 0.0f;
  // Q and dO tiles [query][D] (tswz layout) by buffer copies into LDS:
  // fixed lane offsets, the tile's first query in the resource base; rows
  // past S read zeros (masked below); lse and Delta via VGPRs
  using CQ = RowCopy<DQ, NTH2>;
  using CG = RowCopy<DV, NTH2>;
  uint32_t qoff[CQ::uniform ? 1 : PERQ], goff[CG::uniform ? 1 : PERG];
#pragma unroll
  for (int i = 0; i < (CQ::uniform ? 1 : PERQ); ++i) {
    const int P = i * NTH2 + tid;
    const int row = P / (DQ / 8);
    qoff[i] = (uint32_t)(row * DQ + ((P % (DQ / 8)) ^ swz<DQ>(row)) * 8) * 2;
  }
#pragma unroll
  for (int i = 0; i < (CG::uniform ? 1 : PERG); ++i) {
    const int P = i * NTH2 + tid;
    const int row = P / (DV / 8);
    goff[i] = (uint32_t)(row * ldt + ((P % (DV / 8)) ^ swz<DV>(row)) * 8) * 2;
  }
  auto issue = [&](int qt, int buf) {
    const int q0 = qt * QT2;
    uint16_t* qs = qg + buf * (LQ + LG);
    uint16_t* gs = qs + LQ;
#pragma unroll
    for (int i = 0; i < PERQ; ++i) {
      const int r0 = q0 + (CQ::uniform ? i * CQ::rows : 0);
      const auto rq = st::make_rsrc(qb + (int64_t)r0 * DQ, (int64_t)max(S - r0, 0) * DQ * 2);
      b2lds16(rq, qoff[CQ::uniform ? 0 : i], qs + (i * NTH2 + wave * 64) * 8);
    }
#pragma unroll
    for (int i = 0; i < PERG; ++i) {
      const int r0 = q0 + (CG::uniform ? i * CG::rows : 0);
      const auto rg = st::make_rsrc(gb + (int64_t)r0 * ldt, (int64_t)max(S - r0, 0) * ldt * 2);
      b2lds16(rg, goff[CG::uniform ? 0 : i], gs + (i * NTH2 + wave * 64) * 8);
    }
    if (tid < QT2) {
      const bool ok = q0 + tid < S;
      lr = ok ? lse[srow + q0 + tid] : INFINITY;  // rows past S: probability 0
      dr = ok ? delta[srow + q0 + tid] : 0.0f;
    }
  };
  auto stats = [&](int buf) {
    if (tid < QT2) { lse_s[buf][tid] = lr; dl_s[buf][tid] = dr; }
  };
  if (qt_first < qt_end) {
    issue(qt_first, 0);
    stats(0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int qt = qt_first; qt < qt_end; ++qt) {
    const int buf = (qt - qt_first) & 1;
    if (qt + 1 < qt_end) issue(qt + 1, buf ^ 1);
    const uint16_t* qs = qg + buf * (LQ + LG);
    const uint16_t* gs = qs + LQ;
#pragma unroll
    for (int hq = 0; hq < QH; ++hq) {
    const int qh = NW == 8 ? qh0 : hq;
    const int qw0 = qt * QT2 + qh * 32;   // this wave's queries
    if (qw0 + 31 >= kw0 && qw0 < S) {     // some query sees some key
      // kept query rows (offsets within the block, less 4g) from lo on:
      // causal (query >= key), none for a key past Sk; rows past S carry an
      // lse of +inf, so their probabilities are 0 as well
      int lo = -64;
      if (qw0 < kw0 + 31 || kw0 + 31 >= Sk)  // wave-uniform
        lo = mykey < Sk ? mykey - qw0 - g * 4 : 64;
      f32x16 sacc, pacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) { sacc[e] = 0.0f; pacc[e] = 0.0f; }
#pragma unroll
      for (int s = 0; s < DSQ; ++s) {
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            tile_row<DQ>(qs, qh * 32 + c, s, g),
            KREG ? kfr[KREG ? s : 0] : tile_row<DQ>(Ks, kq * 32 + c, s, g), sacc, 0, 0, 0);
        if (s < DSV)
          pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              tile_row<DV>(gs, qh * 32 + c, s, g),
              KREG ? vfr[KREG && s < DSV ? s : 0] : tile_row<DV>(Vs, kq * 32 + c, s, g), pacc,
              0, 0, 0);
      }
      bf16x8 pf[2], dsf[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        float p8[8], d8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int vv = 8 * hh + e;
          const int ro = (vv >> 2) * 8 + (vv & 3);  // query row in the block, less 4g
          const int r = qh * 32 + ro + g * 4;      // query row in tile
          float x = __builtin_fmaf(sacc[vv], sl2, -lse_s[buf][r]);
          x = ro >= lo ? x : -INFINITY;  // exp2(-inf) = 0
          const float p = __builtin_amdgcn_exp2f(x);
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
        for (int db = 0; db < DBQ; ++db) {
          if (db < DBV)
            dvacc[db < DBV ? db : 0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                tile_tr<DV>(gs, qh * 32 + 16 * hh, db * 32, lane), pf[hh],
                dvacc[db < DBV ? db : 0], 0, 0, 0);
          dkacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              tile_tr<DQ>(qs, qh * 32 + 16 * hh, db * 32, lane), dsf[hh], dkacc[db], 0, 0, 0);
        }
    }
    }
    if (qt + 1 < qt_end) stats(buf ^ 1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  // 8 waves: the two query halves of each key quarter: qh = 1 parks its sums
  // in LDS, qh = 0 adds them and writes [key][d] fp32 partials; dV first,
  // then dK (4 quarters x DB*16*64 floats at a time).  4 waves: each writes
  // its own sums.
  const int qh = qh0;
  float* red = (float*)lds;
  constexpr int PARTV = DBV * 16 * 64, PARTK = DBQ * 16 * 64;
  static_assert(NW == 4 || 4 * PARTK * 4 <= dkdv_lds_elems<DQ, DV>() * 2, "dK partials fit in LDS");
  if (NW == 8 && qh == 1) {
#pragma unroll
    for (int db = 0; db < DBV; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[kq * PARTV + (db * 16 + e) * 64 + lane] = dvacc[db][e];
  }
  __syncthreads();
  if (qh == 0 && mykey < S) {
    float* dvp = dv_part + (srow + mykey) * DV;
#pragma unroll
    for (int db = 0; db < DBV; ++db)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        float4 a;
        float* pa = &a.x;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int vv = 4 * v4 + e;
          pa[e] = NW == 8 ? dvacc[db][vv] + red[kq * PARTV + (db * 16 + vv) * 64 + lane]
                          : dvacc[db][vv];
        }
        const int col = db * 32 + v4 * 8 + g * 4;
        if (dv_out)
          *(u32x2*)(dv_out + (srow + mykey) * DV + col) =
              u32x2{st::pack_bf16x2(a.x, a.y), st::pack_bf16x2(a.z, a.w)};
        else
          *(float4*)(dvp + col) = a;
      }
  }
  __syncthreads();
  if (NW == 8 && qh == 1) {
#pragma unroll
    for (int db = 0; db < DBQ; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) red[kq * PARTK + (db * 16 + e) * 64 + lane] = dkacc[db][e];
  }
  __syncthreads();
  if (qh == 0 && mykey < S) {
    float* dkp = dk_part + (srow + mykey) * DQ;
#pragma unroll
    for (int db = 0; db < DBQ; ++db)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        float4 bq;
        float* pb = &bq.x;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int vv = 4 * v4 + e;
          pb[e] = (NW == 8 ? dkacc[db][vv] + red[kq * PARTK + (db * 16 + vv) * 64 + lane]
                           : dkacc[db][vv]) * scale;
        }
        const int col = db * 32 + v4 * 8 + g * 4;
        if (dk_out)
          *(u32x2*)(dk_out + (srow + mykey) * DQ + col) =
              u32x2{st::pack_bf16x2(bq.x, bq.y), st::pack_bf16x2(bq.z, bq.w)};
        else
          *(float4*)(dkp + col) = bq;
      }
  }
}

// key tiles kt and n-1-kt in one workgroup: the causal query range of the two
// sums to a constant, so every workgroup does the same work
template <int DQ, int DV>
__global__ __launch_bounds__(64 * dkdv_waves<DQ>(), dkdv_waves<DQ>() == 8 ? 2 : 1) void fa_bwd_dkdv(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, const float* __restrict__ delta, int S, int H, int Hkv,
    float sl2, float scale, float* __restrict__ dk_part, float* __restrict__ dv_part,
    uint16_t* __restrict__ dk_out, uint16_t* __restrict__ dv_out, int nk, int paired,
    const int* __restrict__ kvlen) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[dkdv_lds_elems<DQ, DV>()];
  __shared__ __attribute__((aligned(16))) float lse_s[2][QT2];
  __shared__ __attribute__((aligned(16))) float dl_s[2][QT2];
  const WgIdx w = wg_index(paired ? (nk + 1) / 2 : nk, H);
  for (int it = 0; it < 1 + paired; ++it) {
    const int kt = paired ? (it == 0 ? w.x : nk - 1 - w.x) : w.x;
    if (it == 1) {
      if (kt == w.x) break;
      __syncthreads();  // the previous tile's partial sums still occupy LDS
    }
    fa_bwd_dkdv_tile<DQ, DV>(q, k, v, dout, lse, delta, S, H, Hkv, sl2, scale, dk_part, dv_part,
                             dk_out, dv_out, kt, w.h, w.b, key_len(kvlen, w.b, S), lds, lse_s,
                             dl_s);
  }
}

// dk[b,hk] = bf16(sum over the group's query heads of dk_part), same for dv
// (head dims DQ and DV; the sums run over the heads in ascending order)
__global__ __launch_bounds__(NTH) void fa_bwd_reduce(const float* __restrict__ dk_part,
                                                     const float* __restrict__ dv_part,
                                                     int64_t B, int64_t S, int H, int Hkv, int DQ,
                                                     int DV, uint16_t* __restrict__ dk,
                                                     uint16_t* __restrict__ dv) {
  const int64_t nk = B * Hkv * S * DQ / 4, n = nk + B * Hkv * S * DV / 4;
  const int grp = H / Hkv;
  for (int64_t i = (int64_t)blockIdx.x * NTH + threadIdx.x; i < n; i += (int64_t)gridDim.x * NTH) {
    const bool isk = i < nk;
    const int64_t per = S * (isk ? DQ : DV);
    const int64_t e = (isk ? i : i - nk) * 4;
    const int64_t bh = e / per, off = e % per;
    const int64_t b = bh / Hkv, hk = bh % Hkv;
    const float* part = isk ? dk_part : dv_part;
    float4 sk = make_float4(0, 0, 0, 0);
    for (int j = 0; j < grp; ++j) {
      const float4 a = *(const float4*)(part + ((b * H + hk * grp + j) * per) + off);
      sk.x += a.x; sk.y += a.y; sk.z += a.z; sk.w += a.w;
    }
    *(u32x2*)((isk ? dk : dv) + e) = u32x2{st::pack_bf16x2(sk.x, sk.y), st::pack_bf16x2(sk.z, sk.w)};
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// pair light and heavy query tiles in one workgroup when the unpaired grid
// would fit the GPU in one round anyway (then its longest tile sets the time)
int pair_mode(int nq, int64_t heads) {
  return nq >= 4 && nq * heads <= 1024 ? 1 : 0;
}

int64_t attn_workspace(int64_t B, int64_t S, int64_t H, int64_t Hkv, int64_t DQ, int64_t DV,
                       int backward) {
  if (!backward) return B * Hkv * ((S + 15) & ~15) * DV * 2 + 256;  // key-permuted V^T
  // Delta [B,H,S] fp32, then fp32 dK and dV partials per query head (none when
  // every KV head has one query head: the dK/dV pass then writes bf16)
  const int64_t dl = (B * H * S * 4 + 255) / 256 * 256;
  return 256 + dl + (H == Hkv ? 0 : B * H * S * (DQ + DV) * 4);
}

template <int DQ, int DV>
int attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t B, int64_t S,
             int64_t H, int64_t Hkv, float scale, const int32_t* kvlen, uint16_t* out, float* lse,
             void* workspace, hipStream_t s) {
  uint16_t* vt = (uint16_t*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  const int64_t Sp = (S + 15) & ~15;
  transpose_heads<<<dim3((unsigned)st::cdiv(Sp, 64), (unsigned)st::cdiv(DV, 64),
                         (unsigned)(B * Hkv)), NTH, 0, s>>>(v, vt, S, Sp, DV);
  int rc = st::check_launch("transpose_heads");
  if (rc) return rc;
  const float sl2 = scale * LOG2E;
  if constexpr (DQ > 128) {
    // two key groups' tiles do not fit in LDS: one group of 8 query waves
    // (256 queries) over every key tile, so each SIMD still holds two waves
    const int nq = (int)st::cdiv(S, 2 * BQ);
    const int paired = pair_mode(nq, B * H);
    dim3 grid((unsigned)((paired ? (nq + 1) / 2 : nq) * H * B));
    fa_fwd<DQ, DV, 64, 1, 8><<<grid, NTH * 2, 0, s>>>(q, k, vt, (int)S, (int)H, (int)Hkv, sl2, out,
                                                      lse, nq, paired, kvlen);
  } else {
    const int nq = (int)st::cdiv(S, BQ);
    // paired schedules use two key groups (8 waves) so each SIMD still holds
    // two waves
    const int paired = pair_mode(nq, B * H);
    dim3 grid((unsigned)((paired ? (nq + 1) / 2 : nq) * H * B));
    if (paired)
      fa_fwd<DQ, DV, 64, 2><<<grid, NTH * 2, 0, s>>>(q, k, vt, (int)S, (int)H, (int)Hkv, sl2, out,
                                                     lse, nq, paired, kvlen);
    else
      fa_fwd<DQ, DV, 64, 1><<<grid, NTH, 0, s>>>(q, k, vt, (int)S, (int)H, (int)Hkv, sl2, out,
                                                 lse, nq, paired, kvlen);
  }
  return st::check_launch("fa_fwd");
}

template <int DQ, int DV>
int attn_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* out,
             const float* lse, const uint16_t* dout, int64_t B, int64_t S, int64_t H, int64_t Hkv,
             float scale, const int32_t* kvlen, uint16_t* dq, uint16_t* dk, uint16_t* dv,
             void* workspace, hipStream_t s) {
  char* base = (char*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  float* delta = (float*)base;
  float* dk_part = (float*)(base + (B * H * S * 4 + 255) / 256 * 256);
  float* dv_part = dk_part + B * H * S * DQ;
  const float sl2 = scale * LOG2E;
  const int nk = (int)st::cdiv(S, KT2);
  const int paired_k = pair_mode(nk, B * H);
  dim3 g2((unsigned)((paired_k ? (nk + 1) / 2 : nk) * H * B));
  if constexpr (DQ > 128) {
    // two key groups' tiles do not fit in LDS: one group of 8 query waves
    // (256 queries), paired light and heavy query tiles
    const int nq = (int)st::cdiv(S, 2 * BQ);
    const int paired = pair_mode(nq, B * H);
    dim3 g1((unsigned)((paired ? (nq + 1) / 2 : nq) * H * B));
    fa_bwd_dq<DQ, DV, 64, 1, 8><<<g1, NTH * 2, 0, s>>>(q, k, v, out, dout, lse, (int)S, (int)H,
                                                      (int)Hkv, sl2, scale, delta, dq, nq, paired,
                                                      kvlen);
  } else {
    const int nq = (int)st::cdiv(S, BQ);
    const int paired = pair_mode(nq, B * H);
    dim3 g1((unsigned)((paired ? (nq + 1) / 2 : nq) * H * B));
    if (paired)
      fa_bwd_dq<DQ, DV, 64, 2><<<g1, NTH * 2, 0, s>>>(q, k, v, out, dout, lse, (int)S, (int)H,
                                                     (int)Hkv, sl2, scale, delta, dq, nq, paired,
                                                     kvlen);
    else
      fa_bwd_dq<DQ, DV, 64, 1><<<g1, NTH, 0, s>>>(q, k, v, out, dout, lse, (int)S, (int)H,
                                                  (int)Hkv, sl2, scale, delta, dq, nq, paired,
                                                  kvlen);
  }
  int rc = st::check_launch("fa_bwd_dq");
  if (rc) return rc;
  // one query head per KV head (MLA): the pass writes dK and dV in bf16 itself,
  // the rounding of the group sum over a single head
  const bool direct = H == Hkv;
  fa_bwd_dkdv<DQ, DV><<<g2, 64 * dkdv_waves<DQ>(), 0, s>>>(
      q, k, v, dout, lse, delta, (int)S, (int)H, (int)Hkv, sl2, scale, dk_part, dv_part,
      direct ? dk : nullptr, direct ? dv : nullptr, nk, paired_k, kvlen);
  rc = st::check_launch("fa_bwd_dkdv");
  if (rc || direct) return rc;
  const int64_t n4 = B * Hkv * S * (DQ + DV) / 4;
  const unsigned blocks = (unsigned)std::min<int64_t>(st::cdiv(n4, NTH), 4096);
  fa_bwd_reduce<<<blocks, NTH, 0, s>>>(dk_part, dv_part, B, S, (int)H, (int)Hkv, DQ, DV, dk, dv);
  return st::check_launch("fa_bwd_reduce");
}

// Tiles are copied through 32-bit buffer offsets from a head's base: the
// head's Q/K rows (S*DQ), its staged V^T (DV*Sp) and the token-major rows of
// the output gradient it reads (S rows of H*DV) must each span below 2 GiB.
bool extents_ok(int64_t S, int64_t H, int64_t DQ, int64_t DV) {
  const int64_t lim = (int64_t)1 << 31, Sp = (S + 15) & ~15;
  return S * DQ * 2 < lim && Sp * DV * 2 < lim && S * H * DV * 2 < lim;
}

bool dims_ok(int64_t DQ, int64_t DV) {
  return (DQ == 64 && DV == 64) || (DQ == 128 && DV == 128) || (DQ == 192 && DV == 128);
}

int fwd_common(const char* name, const uint16_t* q, const uint16_t* k, const uint16_t* v,
               int64_t B, int64_t S, int64_t H, int64_t Hkv, int64_t DQ, int64_t DV, float scale,
               const int32_t* kv_len, uint16_t* out, float* lse, void* workspace,
               int64_t workspace_bytes, st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "%s: bad head counts", name);
  if (B == 0 || S == 0) return ST_OK;
  if (!dims_ok(DQ, DV))
    return st::fail(ST_EUNSUPPORTED, "%s: head dims %lld/%lld (64/64, 128/128 or 192/128 only)",
                    name, (long long)DQ, (long long)DV);
  ST_CHECK_ARG(S < (1 << 30), "%s: S must be below 2^30", name);
  if (!extents_ok(S, H, DQ, DV))
    return st::fail(ST_EUNSUPPORTED, "%s: a head's rows must span below 2 GiB", name);
  ST_CHECK_ARG(q && k && v && out && lse && al16(q) && al16(k) && al16(v) && al16(out),
               "%s: NULL or unaligned pointer", name);
  const int64_t need = attn_workspace(B, S, H, Hkv, DQ, DV, 0);
  if (!workspace || workspace_bytes < need)
    return st::fail(ST_EWORKSPACE, "%s: needs %lld workspace bytes", name, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  if (DQ == 64)
    return attn_fwd<64, 64>(q, k, v, B, S, H, Hkv, scale, kv_len, out, lse, workspace, s);
  if (DQ == 128)
    return attn_fwd<128, 128>(q, k, v, B, S, H, Hkv, scale, kv_len, out, lse, workspace, s);
  return attn_fwd<192, 128>(q, k, v, B, S, H, Hkv, scale, kv_len, out, lse, workspace, s);
}

int bwd_common(const char* name, const uint16_t* q, const uint16_t* k, const uint16_t* v,
               const uint16_t* out, const float* lse, const uint16_t* dout, int64_t B, int64_t S,
               int64_t H, int64_t Hkv, int64_t DQ, int64_t DV, float scale, const int32_t* kv_len,
               uint16_t* dq, uint16_t* dk, uint16_t* dv, void* workspace, int64_t workspace_bytes,
               st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && H > 0 && Hkv > 0 && H % Hkv == 0, "%s: bad head counts", name);
  if (B == 0 || S == 0) return ST_OK;
  if (!dims_ok(DQ, DV))
    return st::fail(ST_EUNSUPPORTED, "%s: head dims %lld/%lld (64/64, 128/128 or 192/128 only)",
                    name, (long long)DQ, (long long)DV);
  ST_CHECK_ARG(S < (1 << 30), "%s: S must be below 2^30", name);
  if (!extents_ok(S, H, DQ, DV))
    return st::fail(ST_EUNSUPPORTED, "%s: a head's rows must span below 2 GiB", name);
  ST_CHECK_ARG(q && k && v && out && lse && dout && dq && dk && dv && al16(q) && al16(k) &&
                   al16(v) && al16(out) && al16(dout) && al16(dq) && al16(dk) && al16(dv),
               "%s: NULL or unaligned pointer", name);
  const int64_t need = attn_workspace(B, S, H, Hkv, DQ, DV, 1);
  if (!workspace || workspace_bytes < need)
    return st::fail(ST_EWORKSPACE, "%s: needs %lld workspace bytes", name, (long long)need);
  hipStream_t s = (hipStream_t)stream;
  if (DQ == 64)
    return attn_bwd<64, 64>(q, k, v, out, lse, dout, B, S, H, Hkv, scale, kv_len, dq, dk, dv,
                            workspace, s);
  if (DQ == 128)
    return attn_bwd<128, 128>(q, k, v, out, lse, dout, B, S, H, Hkv, scale, kv_len, dq, dk, dv,
                              workspace, s);
  return attn_bwd<192, 128>(q, k, v, out, lse, dout, B, S, H, Hkv, scale, kv_len, dq, dk, dv,
                            workspace, s);
}

}  // namespace

extern "C" int64_t st_flash_attn_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t Hkv,
                                                 int64_t D, int32_t backward) {
  return attn_workspace(B, S, H, Hkv, D, D, backward);
}

extern "C" int st_flash_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 int64_t B, int64_t S, int64_t H, int64_t Hkv, int64_t D,
                                 float scale, const int32_t* kv_len, uint16_t* out, float* lse,
                                 void* workspace, int64_t workspace_bytes, st_stream_t stream) {
  if (D != 64 && D != 128)
    return st::fail(ST_EUNSUPPORTED, "st_flash_attn_fwd: head_dim %lld (64 or 128 only)",
                    (long long)D);
  return fwd_common("st_flash_attn_fwd", q, k, v, B, S, H, Hkv, D, D, scale, kv_len, out, lse,
                    workspace, workspace_bytes, stream);
}

extern "C" int st_flash_attn_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                 const uint16_t* out, const float* lse, const uint16_t* dout,
                                 int64_t B, int64_t S, int64_t H, int64_t Hkv, int64_t D,
                                 float scale, const int32_t* kv_len, uint16_t* dq, uint16_t* dk,
                                 uint16_t* dv, void* workspace, int64_t workspace_bytes,
                                 st_stream_t stream) {
  if (D != 64 && D != 128)
    return st::fail(ST_EUNSUPPORTED, "st_flash_attn_bwd: head_dim %lld (64 or 128 only)",
                    (long long)D);
  return bwd_common("st_flash_attn_bwd", q, k, v, out, lse, dout, B, S, H, Hkv, D, D, scale,
                    kv_len, dq, dk, dv, workspace, workspace_bytes, stream);
}

extern "C" int64_t st_mla_attn_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t DQ,
                                               int64_t DV, int32_t backward) {
  return attn_workspace(B, S, H, H, DQ, DV, backward);
}

extern "C" int st_mla_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               int64_t B, int64_t S, int64_t H, int64_t DQ, int64_t DV,
                               float scale, const int32_t* kv_len, uint16_t* out, float* lse,
                               void* workspace, int64_t workspace_bytes, st_stream_t stream) {
  return fwd_common("st_mla_attn_fwd", q, k, v, B, S, H, H, DQ, DV, scale, kv_len, out, lse,
                    workspace, workspace_bytes, stream);
}

extern "C" int st_mla_attn_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                               const uint16_t* out, const float* lse, const uint16_t* dout,
                               int64_t B, int64_t S, int64_t H, int64_t DQ, int64_t DV,
                               float scale, const int32_t* kv_len, uint16_t* dq, uint16_t* dk,
                               uint16_t* dv, void* workspace, int64_t workspace_bytes,
                               st_stream_t stream) {
  return bwd_common("st_mla_attn_bwd", q, k, v, out, lse, dout, B, S, H, H, DQ, DV, scale, kv_len,
                    dq, dk, dv, workspace, workspace_bytes, stream);
}
