// Fused 4-bit dequant + bf16 MFMA GEMM for the frozen base projections.
//
//   forward  C[M,N]    = X[M,K]  * W[N,K]^T   (+ LoRA, + residual)   lora.py:218-220
//   dgrad    C[M,Kout] = dY[M,N] * W[N,Kout]  (+ LoRA dX term)      autograd of the same
//
// Generic form inside the kernel: C[M,P] = A[M,Q] * B[Q,P], Q = contraction.
// The packed weight is streamed from HBM (0.53 B/element), dequantised in
// registers (codebook in LDS, one fp32 multiply + RNE per element, the exact
// arithmetic of codecs.py:168-170) and written to LDS as bf16, so W never
// exists in HBM as bf16.  The A tile and the forward B tile are stored
// contraction-contiguous in padded 144-byte rows; the dgrad B tile keeps W's
// natural [contraction][output] orientation and its MFMA operand is read with
// the transposing ds_read_b64_tr_b16.
//
// Tiling: 128x128 (4 waves, 2x2) or 256x256 (8 waves, 2x4, two per SIMD),
// BK = 64, LDS double buffered, one barrier per k-step; operand fragments are
// read one 16-wide slice ahead of the MFMAs (v_mfma_f32_32x32x16_bf16).
// The LoRA epilogue runs on v_mfma_f32_32x32x2_f32 (fp32 operands and
// accumulation), so the adapter term keeps the reference's fp32 arithmetic.
#include <type_traits>

#include "common.h"
#include "decode4.h"

namespace {

constexpr int BK = 64;

enum Mode { FWD_Q4 = 0, DGRAD_Q4 = 1, FWD_BF16 = 2, DGRAD_BF16 = 3 };

struct GemmParams {
  const uint16_t* A;
  int64_t lda;
  const uint8_t* Wq;
  const float* Ws;
  const uint16_t* Wb;
  int64_t ldw;  // elements per row of W
  int64_t M, P, Q;
  Lut16 lut;
  int hi_first;
  // log2 of the flat scale group: 7 (128 elements) or 6 (64, ST_FLAG_GROUP64:
  // bitsandbytes' blocksize).  The register-operand kernel takes 7 only.
  int gshift;
  uint16_t* C;
  int64_t ldc;
  const uint16_t* R;
  int64_t ldr;
  const float* T;
  int64_t ldt;
  const float* L;
  int64_t ldl;
  int lora_k;
  int lora_cols;  // columns of T staged (fwd: nseg*rank, dgrad: lora_k)
  int lora_global;  // LoRA operands read from global memory (gemm_kernel<..., LG = true>)
  float lora_scale;
  int nseg;
  int64_t seg_end[4];
  int64_t a_bytes, w_bytes, s_bytes;  // extents of A, W (payload or bf16), scales
  // grouped (per-expert) GEMM: rows of group g are [goff[g], goff[g+1]) and use
  // W/scales/LoRA operand g (strides below); A row r reads source row gather[r]
  const int32_t* gather;  // nullptr: row r
  const int32_t* goff;    // nullptr: one group of M rows
  int ngroups;
  int64_t w_gstride, s_gstride, l_gstride;  // payload bytes (or bf16 elements), floats, floats
  // dgrad only: C = the gradient of a fused gate|up pre-activation [M, 2*swi_I]
  // (row stride ldc) instead of dX; the epilogue applies the SwiGLU VJP to
  // each dX value with gate|up read from swi_gu (row stride swi_ld)
  const uint16_t* swi_gu;
  int64_t swi_ld, swi_I;
  // set by the launcher: the epilogue stages each 32x32 block through LDS
  // and moves 16-byte rows (C, residual, gate|up 16-byte aligned with row
  // strides and P multiples of 8, and the staging fits the tile's LDS)
  int vec_epi;
  // row tiles per raster group (st::raster); grouped launches take 1
  int raster_m;
  // split-K (gemm_ws_kernel, dense launches): the grid holds `splits` copies
  // of the tiles, copy s taking contraction k-steps [s*ks_len, (s+1)*ks_len),
  // and each writes its raw fp32 sums to part[s][M][P] (no epilogue);
  // splitk_epilogue then sums them in split order and applies the epilogue
  float* part;
  int splits, ks_len;
};

// LDS tile rows hold 64 bf16 (8 chunks of 16 bytes) plus one chunk of padding:
// a 144-byte stride puts the 16 rows of each quarter-wave of a fragment read
// on distinct banks, and every fragment of a wave is its lane base plus an
// immediate offset.  Index in 16-byte units.
constexpr int RS = 9;
__device__ __forceinline__ int pad(int row, int c) { return row * RS + c; }

// DGRAD_Q4 B tile: W[n][k] rows of BN bf16 in the transposed-operand layout
// (st::trswz / st::tr_operand).
#define dswz(n, c) st::trswz<BN>(n, c)
#define b_tr(bs, n0, kc, lane) st::tr_operand<BN>(bs, n0, kc, lane)

using st::kOOB;
using st::ld16;
using st::ld4;
using st::make_rsrc;

using st::Tbl;
using st::make_tbl;
using st::deq8;
using st::deq8o;

// WAVES = 4 or 8 (two waves per SIMD), arranged WAVES_M x (WAVES / WAVES_M)
template <int MODE, int BM, int BN, int WAVES, int WAVES_M>
struct Tile {
  static constexpr int NT = 64 * WAVES;
  static constexpr int WAVES_N = WAVES / WAVES_M;
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int FM = WM / 32, FN = WN / 32;
  static constexpr int A_IT = BM * 8 / NT;  // 16-byte chunks per thread
  static constexpr bool Q4 = (MODE == FWD_Q4 || MODE == DGRAD_Q4);
  static constexpr bool DGRAD = (MODE == DGRAD_Q4 || MODE == DGRAD_BF16);
  static constexpr int BF_IT = BN * 8 / NT;        // FWD_BF16 chunks per thread
  static constexpr int LDS_CHUNKS = 2 * (BM + BN) * RS;
};

// Copies a rows x cols block of fp32 values into LDS, dst[r*ls + c] = element
// (row0 + r, col0 + c) of a row-major array with row stride ld read through
// rs; rows r >= vrows and columns c >= vcols read as zero.  Each thread keeps
// eight loads in flight before its LDS writes, and walks its elements
// e = tid + NT*i as (r, c) pairs without divisions.
template <int NT>
__device__ __forceinline__ void stage_f32(float* dst, int ls, __amdgpu_buffer_rsrc_t rs,
                                          int64_t ld, int64_t row0, int64_t col0, int rows,
                                          int cols, int64_t vrows, int64_t vcols, int tid) {
  const int total = rows * cols;
  int r = tid / cols, c = tid % cols;
  const int dr = NT / cols, dc = NT % cols;
  for (int e0 = 0; e0 < total; e0 += 8 * NT) {
    float v[8];
    int d[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const bool in = e0 + u * NT + tid < total;
      const bool ok = in && r < vrows && c < vcols;
      v[u] = __builtin_bit_cast(
          float, ld4(rs, ok ? (uint32_t)(((row0 + r) * ld + col0 + c) * 4) : kOOB));
      d[u] = in ? r * ls + c : -1;
      r += dr;
      c += dc;
      if (c >= cols) {
        c -= cols;
        ++r;
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (d[u] >= 0) dst[d[u]] = v[u];
  }
}

struct EpiIn {
  uint4 a0, a1, b0, b1;
};

// Per-wave LDS staging of the vector epilogue (dwords), placed after the LoRA
// operands the epilogue stages (16-byte aligned).
constexpr int EPI_STG = 16 * 36;
// Dwords of LDS the LoRA epilogue stages T and the right operand in, rounded
// to 16 bytes (none when they are read from global memory)
template <bool DGRAD, int BM, int BN>
__host__ __device__ __forceinline__ int64_t epi_stage_offset(const GemmParams& p) {
  if (!p.T || p.lora_global) return 0;
  const int64_t f = (int64_t)BM * (p.lora_cols + 1) +
                    (int64_t)BN * (p.lora_k + 1);
  return (f + 3) & ~(int64_t)3;
}
// Whether the LoRA operands staged in LDS leave room for what the epilogue
// cannot do without: the SwiGLU VJP always moves 16-byte rows, so it needs
// `waves` staging areas after them.  When they do not fit, the GEMM runs on
// the 128x128 kernel that reads the LoRA operands from global memory.
template <bool DGRAD, int BM, int BN>
__host__ __forceinline__ bool lora_staged_fits(const GemmParams& p, int64_t lds_dwords,
                                               int waves) {
  if (!p.T || p.lora_global) return true;
  return epi_stage_offset<DGRAD, BM, BN>(p) + (p.swi_gu ? (int64_t)waves * EPI_STG : 0) <=
         lds_dwords;
}

// Epilogue shared by the GEMM kernels: y = bf16(acc) (+ LoRA term, + residual)
// for this tile; waves with `has_acc` false only help stage the LoRA operands.
// LG: T and the LoRA right operand are read from global memory instead of
// being staged in LDS (only the 128x128 kernel is built with it, for LoRA
// operands that do not fit its LDS; the other kernels keep the staged form
// only, so their register allocation does not carry the global loop).
// LDS (`lds`, at least BM*(lora_cols+1) + the LoRA right operand floats) is
// reused, so the caller has finished every LDS read of the main loop.
// Residual loads and output stores go through buffer resources with masked
// 32-bit offsets (the host keeps C and R below 2 GiB): a 32x32 block's 16
// residual loads are all in flight before the LoRA products, and rows or
// columns outside the problem are skipped without branches.
template <bool DGRAD, int BM, int BN, int NT, int FM, int FN, int WM, int WN, bool LG = false>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p, const f32x16 (&acc)[FM][FN],
                                              uint4* lds, int64_t m0, int64_t mend, int64_t p0,
                                              int wm, int wn, int tid, int lane, bool has_acc,
                                              const float* Lg) {
  const bool lora = p.T != nullptr;
  float* Ts = (float*)lds;
  const int tstride = p.lora_cols + 1;
  float* Ls = Ts + BM * tstride;
  const int lstride = DGRAD ? BN : (p.lora_k + 1);
  if (!LG && lora) {
    // T rows [m0, m0+BM) x [0, lora_cols) and the LoRA right operand
    // (dgrad: A_cat [lora_k, P] columns p0..; forward: B_lora [P, rank] rows p0..)
    stage_f32<NT>(Ts, tstride, make_rsrc(p.T, 0x7fffffff), p.ldt, m0, 0, BM, p.lora_cols,
                  mend - m0, p.lora_cols, tid);
    if (DGRAD)
      stage_f32<NT>(Ls, lstride, make_rsrc(Lg, 0x7fffffff), p.ldl, 0, p0, p.lora_k, BN, p.lora_k,
                    p.P - p0, tid);
    else
      stage_f32<NT>(Ls, lstride, make_rsrc(Lg, 0x7fffffff), p.ldl, p0, 0, BN, p.lora_k, p.P - p0,
                    p.lora_k, tid);
    // zeros past the contraction (T's spare column, the right operand's spare
    // column or row): lora_term takes the rank two at a time, so an odd rank
    // reads index lora_k once, as 0 x (a finite T value or 0)
    for (int r = tid; r < BM; r += NT) Ts[r * tstride + p.lora_cols] = 0.0f;
    for (int c = tid; c < BN; c += NT) {
      if (DGRAD)
        Ls[p.lora_k * lstride + c] = 0.0f;
      else
        Ls[c * lstride + p.lora_k] = 0.0f;
    }
    __syncthreads();
  }
  if (!has_acc) return;
  const auto rsC = make_rsrc(p.C, 0x7fffffff);
  const auto rsR = make_rsrc(p.R, 0x7fffffff);
  const auto rsG = make_rsrc(p.swi_gu, 0x7fffffff);
  const uint32_t ldc2 = (uint32_t)p.ldc * 2, ldr2 = (uint32_t)p.ldr * 2;
  // this wave's staging area for one 32x32 block: 16 row pairs x 36 dwords
  // (dword = the bf16 values of rows 2q, 2q+1 of one column; 36 makes the
  // 16-byte row-pair reads of a quarter-wave cover all 64 banks once)
  uint32_t* stg = (uint32_t*)lds + epi_stage_offset<DGRAD, BM, BN>(p) + (tid >> 6) * EPI_STG;

  // LoRA term of block (i, j) on v_mfma_f32_32x32x2_f32.  LG: the same
  // operands (same guards, same products in the same order) come from global
  // memory through L2.
  auto lora_term = [&](int rl, int cl, int coff) {
    f32x16 la;
#pragma unroll
    for (int v = 0; v < 16; ++v) la[v] = 0.0f;
    if constexpr (!LG) {
      for (int kk = 0; kk < p.lora_k; kk += 2) {
        int kx = kk + (lane >> 5);
        float av = Ts[(rl + (lane & 31)) * tstride + coff + kx];
        float bv = DGRAD ? Ls[kx * lstride + cl + (lane & 31)]
                         : Ls[(cl + (lane & 31)) * lstride + kx];
        la = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, la, 0, 0, 0);
      }
    } else {
      const auto rsTg = make_rsrc(p.T, 0x7fffffff), rsLg = make_rsrc(Lg, 0x7fffffff);
      const int64_t row = m0 + rl + (lane & 31), col = p0 + cl + (lane & 31);
      const bool rok = row < mend, cok = col < p.P;
      for (int kk = 0; kk < p.lora_k; kk += 2) {
        const int kx = kk + (lane >> 5);
        const bool kok = kx < p.lora_k;
        const uint32_t ta = rok && kok ? (uint32_t)((row * p.ldt + coff + kx) * 4) : kOOB;
        const uint32_t tb = !(cok && kok) ? kOOB
                            : DGRAD ? (uint32_t)(((int64_t)kx * p.ldl + col) * 4)
                                    : (uint32_t)((col * p.ldl + kx) * 4);
        const float av = __builtin_bit_cast(float, ld4(rsTg, ta));
        const float bv = __builtin_bit_cast(float, ld4(rsLg, tb));
        la = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, la, 0, 0, 0);
      }
    }
    return la;
  };
  auto seg_off = [&](int cl) {
    int coff = 0;
    if (lora && !DGRAD) {
      int64_t pblk = p0 + cl;
      int s = 0;
      for (int q = 0; q < p.nseg; ++q) s += (p.seg_end[q] <= pblk) ? 1 : 0;
      coff = s * p.lora_k;
    }
    return coff;
  };

  // VEC: block staged through LDS, each lane then owns rows 2q, 2q+1 (q =
  // lane % 16) x columns 8k..8k+7 (k = lane / 16) of the block and moves
  // them with 16-byte accesses.  Otherwise one 2-byte access per element.
  // Separate copies of the loop nest per mode keep each fully unrolled.
  // VEC operands of block (i, j) for this lane's rows 2q, 2q+1 and 8 columns:
  // residual rows in a0, a1, or (SWI) gate rows in a0, a1 and up rows in b0, b1
  auto fetch = [&](auto swi, int i, int j) {
    constexpr bool SWI = decltype(swi)::value;
    const int q = lane & 15, kc = lane >> 4;
    const int64_t row0 = m0 + wm * WM + i * 32 + 2 * q, col = p0 + wn * WN + j * 32 + 8 * kc;
    const bool cok = col < p.P;
    const bool ok0 = cok && row0 < mend, ok1 = cok && row0 + 1 < mend;
    EpiIn in;
    in.a0 = in.a1 = in.b0 = in.b1 = make_uint4(0, 0, 0, 0);
    if (SWI) {
      const uint32_t gb = (uint32_t)((row0 * p.swi_ld + col) * 2);
      const uint32_t ldg2 = (uint32_t)p.swi_ld * 2, uo = (uint32_t)p.swi_I * 2;
      in.a0 = ld16(rsG, ok0 ? gb : kOOB);
      in.a1 = ld16(rsG, ok1 ? gb + ldg2 : kOOB);
      in.b0 = ld16(rsG, ok0 ? gb + uo : kOOB);
      in.b1 = ld16(rsG, ok1 ? gb + ldg2 + uo : kOOB);
    } else if (p.R) {
      const uint32_t rb = (uint32_t)((row0 * p.ldr + col) * 2);
      in.a0 = ld16(rsR, ok0 ? rb : kOOB);
      in.a1 = ld16(rsR, ok1 ? rb + ldr2 : kOOB);
    }
    return in;
  };

  auto blocks = [&](auto swi, auto vec) {
    constexpr bool SWI = decltype(swi)::value, VEC = decltype(vec)::value;
    EpiIn cur;
    if constexpr (VEC) cur = fetch(swi, 0, 0);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int cl = wn * WN + j * 32;  // tile-local first column of this block
      const int coff = seg_off(cl);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int rl = wm * WM + i * 32;
        if constexpr (VEC) {
          const int q = lane & 15, kc = lane >> 4;
          const int64_t row0 = m0 + rl + 2 * q, col = p0 + cl + 8 * kc;
          const bool cok = col < p.P;
          const bool ok0 = cok && row0 < mend, ok1 = cok && row0 + 1 < mend;
          // this block's operands were issued one block ahead; issue the next one's
          const EpiIn in = cur;
          if (j * FM + i + 1 < FM * FN)
            cur = fetch(swi, (j * FM + i + 1) % FM, (j * FM + i + 1) / FM);
          const uint4 &r0 = in.a0, &r1 = in.a1, &g0 = in.a0, &g1 = in.a1, &u0 = in.b0,
                      &u1 = in.b1;
          f32x16 la;
          if (lora) la = lora_term(rl, cl, coff);
          // y = bf16(acc) (+ LoRA) into the staging area, two rows per dword
#pragma unroll
          for (int qq = 0; qq < 4; ++qq)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
              float y2[2];
#pragma unroll
              for (int h = 0; h < 2; ++h) {
                const int v = 4 * qq + 2 * t + h;
                float y = st::bf16r(acc[i][j][v]);
                if (lora) {
                  if (DGRAD)
                    y = st::bf16r(y + st::bf16r(la[v]));
                  else
                    y = st::bf16r(y + la[v] * p.lora_scale);
                }
                y2[h] = y;
              }
              const int pr = qq * 4 + (lane >> 5) * 2 + t;  // row pair
              stg[pr * 36 + (lane & 31)] = st::pack_bf16x2(y2[0], y2[1]);
            }
          // the wave reads back only its own area: LDS accesses of one wave
          // complete in order, the fence keeps the compiler from moving them
          __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
          const uint4 lo4 = *(const uint4*)&stg[q * 36 + 8 * kc];
          const uint4 hi4 = *(const uint4*)&stg[q * 36 + 8 * kc + 4];
          // dword c of the pair holds (row 2q, row 2q+1) of column 8k + c
          const uint32_t d[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
          uint32_t e0[4], e1[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            e0[c] = __builtin_amdgcn_perm(d[2 * c + 1], d[2 * c], 0x05040100u);
            e1[c] = __builtin_amdgcn_perm(d[2 * c + 1], d[2 * c], 0x07060302u);
          }
          __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // before the next block's writes
          const uint32_t cb = (uint32_t)((row0 * p.ldc + col) * 2);
          auto emit = [&](const uint32_t (&e)[4], bool okr, uint32_t off, const uint4& rr,
                          const uint4& gg, const uint4& uu) {
            float yv[8];
            const uint32_t ew[4] = {e[0], e[1], e[2], e[3]};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              yv[2 * c] = __uint_as_float(ew[c] << 16);
              yv[2 * c + 1] = __uint_as_float(ew[c] & 0xffff0000u);
            }
            if constexpr (SWI) {
              // SwiGLU VJP of dense.py:153 on the bf16 dX value (st::swiglu_vjp,
              // as the standalone SwiGLU backward)
              const uint32_t gw[4] = {gg.x, gg.y, gg.z, gg.w}, uw[4] = {uu.x, uu.y, uu.z, uu.w};
              uint32_t og[4], ou[4];
#pragma unroll
              for (int c = 0; c < 4; ++c) {
                float rg[2], ru[2];
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                  const float gv = st::bf16_to_f32((uint16_t)(gw[c] >> (16 * h)));
                  const float uv = st::bf16_to_f32((uint16_t)(uw[c] >> (16 * h)));
                  st::swiglu_vjp(gv, uv, yv[2 * c + h], rg[h], ru[h]);
                }
                og[c] = st::pack_bf16x2(rg[0], rg[1]);
                ou[c] = st::pack_bf16x2(ru[0], ru[1]);
              }
              const uint32_t uo = (uint32_t)p.swi_I * 2;
              __builtin_amdgcn_raw_buffer_store_b128(
                  st::u32x4{og[0], og[1], og[2], og[3]}, rsC, (int)(okr ? off : kOOB), 0, 0);
              __builtin_amdgcn_raw_buffer_store_b128(
                  st::u32x4{ou[0], ou[1], ou[2], ou[3]}, rsC, (int)(okr ? off + uo : kOOB), 0, 0);
            } else {
              uint32_t o[4];
              if (p.R) {
                const uint32_t rw[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
                for (int c = 0; c < 4; ++c)
                  o[c] = st::pack_bf16x2(
                      st::bf16_to_f32((uint16_t)rw[c]) + yv[2 * c],
                      st::bf16_to_f32((uint16_t)(rw[c] >> 16)) + yv[2 * c + 1]);
              } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) o[c] = ew[c];
              }
              __builtin_amdgcn_raw_buffer_store_b128(st::u32x4{o[0], o[1], o[2], o[3]}, rsC,
                                                     (int)(okr ? off : kOOB), 0, 0);
            }
          };
          emit(e0, ok0, cb, r0, g0, u0);
          emit(e1, ok1, cb + ldc2, r1, g1, u1);
        } else {
          const int64_t pcol = p0 + cl + (lane & 31);
          const bool colok = pcol < p.P;
          const int64_t rbase = m0 + rl + (lane >> 5) * 4;  // row of v = 0
          // element v sits at row rbase + dv(v), dv = (v/4)*8 + v%4
          auto ok = [&](int v) { return colok && rbase + (v >> 2) * 8 + (v & 3) < mend; };
          uint16_t rv[16];  // raw bf16: converted where used, after the LoRA products
          if (p.R) {
            const uint32_t rb = (uint32_t)((rbase * p.ldr + pcol) * 2);
#pragma unroll
            for (int v = 0; v < 16; ++v)
              rv[v] = __builtin_amdgcn_raw_buffer_load_b16(
                  rsR, (int)(ok(v) ? rb + (uint32_t)((v >> 2) * 8 + (v & 3)) * ldr2 : kOOB), 0,
                  0);
          }
          f32x16 la;
          if (lora) la = lora_term(rl, cl, coff);
          const uint32_t cb = (uint32_t)((rbase * p.ldc + pcol) * 2);
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            float y = st::bf16r(acc[i][j][v]);
            if (lora) {
              if (DGRAD)
                y = st::bf16r(y + st::bf16r(la[v]));
              else
                y = st::bf16r(y + la[v] * p.lora_scale);
            }
            if (p.R) y = st::bf16r(st::bf16_to_f32(rv[v]) + y);
            __builtin_amdgcn_raw_buffer_store_b16(
                st::f32_to_bf16(y), rsC,
                (int)(ok(v) ? cb + (uint32_t)((v >> 2) * 8 + (v & 3)) * ldc2 : kOOB), 0, 0);
          }
        }
      }
    }
  };
  if constexpr (DGRAD) {
    if (p.swi_gu) {  // the launcher only sets swi_gu with vec_epi
      blocks(std::true_type{}, std::true_type{});
      return;
    }
  }
  if (p.vec_epi)
    blocks(std::false_type{}, std::true_type{});
  else
    blocks(std::false_type{}, std::false_type{});
}

// FLAT (4-bit modes, 128x128 tiles): K is not a multiple of the scale group
// (128, or 64 with gshift 6), so the flat groups of W straddle its rows; every
// packed word (8 weights, which K % 8 == 0 keeps inside one group) then reads
// its own scale at (flat element index) >> gshift and gets its own decode
// table.  Otherwise a k-step of 64 lies inside one group: its scale is group
// kt >> (gshift - 6) of the row, and with 64-element groups every k-step
// rebuilds the decode table.
template <int MODE, int BM, int BN, int WAVES, int WAVES_M, bool FLAT = false, bool LG = false>
__global__ __launch_bounds__(64 * WAVES) void gemm_kernel(GemmParams p) {
  using TL = Tile<MODE, BM, BN, WAVES, WAVES_M>;
  constexpr int NT = TL::NT;
  constexpr int WM = TL::WM, WN = TL::WN, FM = TL::FM, FN = TL::FN;
  __shared__ uint4 lds[TL::LDS_CHUNKS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / TL::WAVES_N, wn = wave % TL::WAVES_N;
  const int64_t tiles_p = st::cdiv(p.P, BN);
  const int64_t t = st::xcd_remap(blockIdx.x, gridDim.x);
  int64_t mt, pt;
  st::raster(t, st::cdiv(p.M, BM), tiles_p, p.raster_m, mt, pt);
  const int64_t p0 = pt * BN;
  int64_t m0 = mt * BM, mend = p.M;
  int grp = 0;
  if (p.goff) {  // whole workgroup leaves together, before any barrier
    if (!st::find_group(p.goff, p.ngroups, BM, mt, p.M, grp, m0, mend)) return;
  }
  const int KT = (int)st::cdiv(p.Q, BK);

  // buffer b: A tile at lds + b*(BM+BN)*RS, B tile right after it
  auto As = [&](int b) { return lds + b * (BM + BN) * RS; };
  auto Bs = [&](int b) { return lds + b * (BM + BN) * RS + BM * RS; };

  // ---- buffer resources: out-of-range loads return zero, so the main loop
  // needs no bounds branches (rows beyond M/P and the contraction tail).
  const auto rsA = make_rsrc(p.A, p.a_bytes);
  const auto rsW = make_rsrc(TL::Q4 ? (const void*)(p.Wq + grp * p.w_gstride)
                                     : (const void*)(p.Wb + grp * p.w_gstride), p.w_bytes);
  const auto rsS = make_rsrc(p.Ws + grp * p.s_gstride, p.s_bytes);
  const float* Lg = p.L + grp * p.l_gstride;

  // A (activations / upstream gradient): 16-byte chunks, row-major, contraction contiguous
  uint32_t a_row[TL::A_IT];
  int a_k[TL::A_IT];
#pragma unroll
  for (int i = 0; i < TL::A_IT; ++i) {
    int id = tid + i * NT, row = id >> 3, c = id & 7;
    int64_t m = m0 + row;
    if (m < mend && p.gather) m = p.gather[m];
    a_row[i] = (m0 + row < mend && m >= 0) ? (uint32_t)((m * p.lda + c * 8) * 2) : kOOB;
    a_k[i] = c * 8;
  }
  // a_row + offset stays at or beyond kOOB for rows outside the tile range;
  // only a contraction tail (Q not a multiple of BK) needs per-chunk checks.
  // Tiles past the last one are loaded (in bounds or zero) but never used.
  auto load_A = [&](int kt, uint4 (&xr)[TL::A_IT]) {
    const bool tail = (int64_t)(kt + 1) * BK > p.Q && kt < KT;
#pragma unroll
    for (int i = 0; i < TL::A_IT; ++i) {
      uint32_t off = a_row[i] + (uint32_t)(kt * BK * 2);
      if (tail && kt * BK + a_k[i] >= p.Q) off = kOOB;
      xr[i] = ld16(rsA, off);
    }
  };
  // LDS addresses of the 256-wide tiles are rebuilt from an opaque copy of
  // tid at each use (a few VALU) rather than kept live across the loop, where
  // they would be the first values the 256x256 tile spills.  The 128x128
  // tile has registers to spare: its addresses stay loop-invariant (rebuilt,
  // the dgrad's transposed-operand addresses alone cost ~160 VALU per k-step).
  auto fresh_tid = [&]() {
    int t = tid;
    if constexpr (BM * BN > 128 * 128) asm volatile("" : "+v"(t));
    return t;
  };
  auto store_A = [&](uint4* as, const uint4 (&xr)[TL::A_IT]) {
    const int ot = fresh_tid();
#pragma unroll
    for (int i = 0; i < TL::A_IT; ++i) {
      int id = ot + i * NT;
      as[pad(id >> 3, id & 7)] = xr[i];
    }
  };

  // B operand source.  FWD_Q4: thread owns EPT consecutive weights of one W row.
  constexpr int TPR = NT / BN;          // threads per W row (1, 2 or 4)
  constexpr int EPT = BK / TPR;         // elements per thread per k-step (64, 32 or 16)
  // DGRAD_Q4 / DGRAD_BF16: the B tile is W[n][k] for BK contraction rows n
  // and BN output columns k, kept in that (natural) orientation; each thread
  // dequantises (or copies) DE consecutive k of one row n, and the MFMA
  // operand is read transposed.
  constexpr int DE = BN * BK / NT;      // dgrad elements per thread per k-step (32 or 16)
  constexpr int DTR = BN / DE;          // dgrad threads per contraction row
  // packed 4-bit words (8 codes each) per thread per k-step
  constexpr int NW = MODE == FWD_Q4 ? EPT / 8 : MODE == DGRAD_Q4 ? DE / 8 : 1;
  static_assert(!TL::Q4 || NW == 2 || NW % 4 == 0, "packed W loads are 8 bytes or whole 16-byte pieces");
  constexpr int WQ = TL::Q4 ? 1 : (TL::DGRAD ? DE / 8 : TL::BF_IT);
  const int brow = tid / TPR, bsub = tid % TPR;       // FWD_Q4 mapping
  const int drow = tid / DTR, dsub = tid % DTR;       // dgrad mapping
  // FWD_Q4 byte offsets at k = 0 of the thread's packed weights and of its
  // row's first scale (kOOB beyond P).  Unless FLAT, K (= ldw) is a multiple
  // of the group, so k-step kt adds kt*BK/2 payload bytes and scale group
  // kt >> (gshift - 6).  FLAT keeps the flat element index w_eo of the
  // thread's first weight.
  uint32_t w_po = kOOB, w_so = kOOB, w_eo = kOOB;
  if constexpr (MODE == FWD_Q4) {
    int64_t n = p0 + brow;
    if (n < p.P) {
      w_eo = (uint32_t)(n * p.ldw + bsub * EPT);
      w_po = w_eo >> 1;
      w_so = (uint32_t)((n * p.ldw) >> p.gshift) * 4;
    }
  }
  const int gstep = p.gshift - 6;  // k-steps per scale group: 1 << gstep
  const bool dcol_ok = p0 + dsub * DE < p.P;
  static_assert(!TL::DGRAD || NT / DTR == BK, "dgrad: one thread row per contraction row");

  static_assert(!FLAT || (TL::Q4 && BM == 128 && BN == 128), "FLAT: 4-bit 128x128 tiles only");
  // DGRAD_Q4 with 128-wide B rows: each thread's 4 words are dequantised and
  // stored in an order rotated by its group dsub, free of LDS bank conflicts
  // with st::trswz<128> (every store instruction of a quarter-wave then
  // writes each 4-chunk group's chunk (ch + group) & 3)
  constexpr bool DROT = MODE == DGRAD_Q4 && BN == 128 && NW == 4 && DTR == 4;
  static_assert(MODE != DGRAD_BF16 || WQ * (NT / (BN / 8)) == BK, "DGRAD_BF16: whole rows per thread block");
  struct WRegs {
    uint4 q[WQ];      // bf16 modes
    uint32_t w[NW];   // 4-bit modes
    float s[FLAT ? NW : 1];  // scale of the tile's group, or of each word (FLAT)
  };
  // NW packed words from byte offset po (kOOB: zeros)
  auto load_words = [&](uint32_t po, uint32_t (&w)[NW]) {
    if constexpr (NW == 2) {
      const uint2 v = st::ld8(rsW, po);
      w[0] = v.x;
      w[1] = v.y;
    } else {
#pragma unroll
      for (int i = 0; i < NW / 4; ++i) {
        const uint4 v = ld16(rsW, po + 16 * i);
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
      }
    }
  };
  auto load_W = [&](int kt, WRegs& w) {
    if constexpr (MODE == FWD_Q4) {
      load_words(w_po + (uint32_t)(kt * (BK / 2)), w.w);
      if constexpr (FLAT) {
#pragma unroll
        for (int j = 0; j < NW; ++j)
          w.s[j] = __builtin_bit_cast(
              float, ld4(rsS, w_eo == kOOB ? kOOB : ((w_eo + (uint32_t)(kt * BK + 8 * j)) >> p.gshift) * 4));
      } else {
        w.s[0] = __builtin_bit_cast(float, ld4(rsS, w_so + (uint32_t)(kt >> gstep) * 4));
      }
    } else if constexpr (MODE == FWD_BF16) {
#pragma unroll
      for (int i = 0; i < WQ; ++i) {
        int id = tid + i * NT, row = id >> 3, c = id & 7;
        int64_t n = p0 + row;
        int k = kt * BK + c * 8;
        w.q[i] = ld16(rsW, (n < p.P && k < p.Q) ? (uint32_t)((n * p.ldw + k) * 2) : kOOB);
      }
    } else if constexpr (MODE == DGRAD_Q4) {
      const int64_t n = (int64_t)kt * BK + drow;
      const bool ok = dcol_ok && n < p.Q;
      // DE-aligned: one scale group unless FLAT
      const int64_t e = n * p.ldw + p0 + dsub * DE;
      load_words(ok ? (uint32_t)(e >> 1) : kOOB, w.w);
#pragma unroll
      for (int j = 0; j < (FLAT ? NW : 1); ++j)
        w.s[j] = __builtin_bit_cast(float, ld4(rsS, ok ? (uint32_t)(((e + 8 * j) >> p.gshift) * 4) : kOOB));
      if constexpr (DROT) {  // stored in rotated order, see store_B_part
        st::rot4(w.w, dsub);
        if constexpr (FLAT) st::rot4(w.s, dsub);
      }
    } else {  // DGRAD_BF16: chunk (row, tid % CPR) for rows tid / CPR + i * NT / CPR
      // (whole 16-byte-chunk rows per load instruction)
      constexpr int CPR = BN / 8;
      const int64_t col = p0 + (tid % CPR) * 8;
#pragma unroll
      for (int i = 0; i < WQ; ++i) {
        const int64_t n = (int64_t)kt * BK + tid / CPR + i * (NT / CPR);
        const bool ok = n < p.Q && col < p.P;
        w.q[i] = ld16(rsW, ok ? (uint32_t)((n * p.ldw + col) * 2) : kOOB);
      }
    }
  };

  // dequantise / stage one quarter (part = 0..3) of the B tile into LDS
  Tbl tbl;
  const uint32_t sh_e = p.hi_first ? 4u : 0u;
  auto store_B_part = [&](uint4* bs, const WRegs& w, int part) {
    if constexpr (TL::Q4) {
      // 8-element chunk ch goes out in quarter ch*4/NW (two chunks per quarter
      // for NW = 8, quarters 0 and 2 for NW = 2)
#pragma unroll
      for (int ch = 0; ch < NW; ++ch) {
        if (ch * 4 / NW != part) continue;
        uint32_t o[4];
        if constexpr (FLAT)
          deq8(w.w[ch], make_tbl(p.lut, w.s[ch]), sh_e, 4u - sh_e, o);
        else
          deq8(w.w[ch], tbl, sh_e, 4u - sh_e, o);
        const int ot = fresh_tid();
        const int idx =
            MODE == FWD_Q4 ? pad(ot / TPR, ((ot % TPR) * EPT) / 8 + ch)
            : DROT         ? dswz(ot / DTR, (ot % DTR) * NW + ((ch + ot % DTR) & 3))
                           : dswz(ot / DTR, (ot % DTR) * NW + ch);
        bs[idx] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    } else if constexpr (MODE == FWD_BF16) {
#pragma unroll
      for (int i = 0; i < WQ; ++i) {
        if (i * 4 / WQ != part) continue;
        int id = tid + i * NT;
        bs[pad(id >> 3, id & 7)] = w.q[i];
      }
    } else {  // DGRAD_BF16: the loaded chunks as they lie, transposed-operand layout
      constexpr int CPR = BN / 8;
      const int ot = fresh_tid();
      if (part < WQ)
        bs[dswz(ot / CPR + part * (NT / CPR), ot % CPR)] = w.q[part < WQ ? part : 0];
    }
  };
  auto prep_B = [&](const WRegs& w) {
    if constexpr (!FLAT && (MODE == FWD_Q4 || MODE == DGRAD_Q4)) tbl = make_tbl(p.lut, w.s[0]);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // MFMA operand fragments of one 16-wide contraction slice s (0..3) of a tile
  auto read_frags = [&](const uint4* as, const uint4* bs, int s, bf16x8 (&a)[FM],
                        bf16x8 (&b)[FN]) {
    const int ln = fresh_tid() & 63;  // rebuilt per call, like the store addresses
    const int c = 2 * s + (ln >> 5);
#pragma unroll
    for (int i = 0; i < FM; ++i)
      a[i] = __builtin_bit_cast(bf16x8, as[pad(wm * WM + i * 32 + (ln & 31), c)]);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      if constexpr (TL::DGRAD)
        b[j] = b_tr(bs, s * 16, wn * WN + j * 32, ln);
      else
        b[j] = __builtin_bit_cast(bf16x8, bs[pad(wn * WN + j * 32 + (ln & 31), c)]);
    }
  };
  auto mfmas = [&](const bf16x8 (&a)[FM], const bf16x8 (&b)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  };

  // One k-step on LDS buffer `cur` (tile kt), staging tile kt+1 into the other
  // buffer and loading tile kt+2 into registers.  Fragments are read one slice
  // ahead of the MFMAs that use them (f0 = slices 0 and 2, f1 = slices 1 and 3),
  // so LDS latency hides behind the previous slice's MFMAs.  The single barrier
  // sits before the last slice: by then every wave has written its part of
  // tile kt+1 and has finished (waitcnt) its reads of tile kt, so slice 3 can
  // already fetch slice 0 of tile kt+1, and the next step may overwrite `cur`.
  uint4 xr[TL::A_IT];
  WRegs w0, w1;
  bf16x8 fa0[FM], fb0[FN], fa1[FM], fb1[FN];
  // new_group: the tile dequantised in this step starts a 128-wide scale group
  // (even tile index), so its decode table must be rebuilt; odd tiles reuse it
  // (with 64-wide groups every tile starts one).
  auto body = [&](int kt, WRegs& wnext, WRegs& wfar, bool new_group) {
    const int cur = kt & 1;
    uint4* as_n = As(cur ^ 1);
    uint4* bs_n = Bs(cur ^ 1);
    const uint4* as = As(cur);
    const uint4* bs = Bs(cur);
    store_A(as_n, xr);
    load_A(kt + 2, xr);
    load_W(kt + 2, wfar);
    if (new_group || MODE == DGRAD_Q4 || gstep == 0) prep_B(wnext);
    read_frags(as, bs, 1, fa1, fb1);
    mfmas(fa0, fb0);
    store_B_part(bs_n, wnext, 0);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(as, bs, 2, fa0, fb0);
    mfmas(fa1, fb1);
    store_B_part(bs_n, wnext, 1);
    __builtin_amdgcn_sched_barrier(0);
    read_frags(as, bs, 3, fa1, fb1);
    mfmas(fa0, fb0);
    store_B_part(bs_n, wnext, 2);
    store_B_part(bs_n, wnext, 3);
    __syncthreads();
    read_frags(as_n, bs_n, 0, fa0, fb0);
    mfmas(fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
  };

  // prologue: tiles 0 (LDS) and 1 (registers), W for tiles 0 and 1
  load_A(0, xr);
  load_W(0, w0);
  load_W(1, w1);
  __syncthreads();
  store_A(As(0), xr);
  prep_B(w0);
#pragma unroll
  for (int s = 0; s < 4; ++s) store_B_part(Bs(0), w0, s);
  load_A(1, xr);
  __syncthreads();
  read_frags(As(0), Bs(0), 0, fa0, fb0);

  // tile kt+1's W sits in w1 (kt even) or w0 (kt odd); W for kt+2 lands in the other
  for (int kt = 0; kt < KT; kt += 2) {
    body(kt, w1, w0, false);
    if (kt + 1 < KT) body(kt + 1, w0, w1, true);
  }
  // the last step's slice-3 reads of the (unused) next buffer must finish
  // before the epilogue reuses LDS
  __syncthreads();

  gemm_epilogue<TL::DGRAD, BM, BN, NT, FM, FN, WM, WN, LG>(p, acc, lds, m0, mend, p0, wm, wn, tid,
                                                       lane, true, Lg);
}

// s_waitcnt for at most VM vector-memory and LGKM LDS/scalar operations in
// flight (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 7 = no wait,
// lgkmcnt in bits 11:8; VM = 63 / LGKM = 15 leave that counter alone)
template <int VM, int LGKM = 15>
__device__ __forceinline__ void wait_cnt() {
  static_assert(VM >= 0 && VM < 64 && LGKM >= 0 && LGKM < 16, "counter range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (LGKM << 8) | ((VM >> 4) << 14));
}
// Workgroup barrier without the fence of __syncthreads (which would also wait
// for every LDS DMA in flight): the caller first waits for exactly the
// operations other waves depend on.  The memory clobber keeps the compiler
// from moving memory accesses across it.
__device__ __forceinline__ void bar() { asm volatile("s_barrier" ::: "memory"); }

// Warp-specialised 256x128 tile, 8 waves in two roles.  Waves 0-3 (one per
// SIMD) only read operand fragments and issue MFMAs on a 2x2 grid of 128x64
// wave tiles; waves 4-7 (the other wave of each SIMD) move data:
//  - A (activations / upstream gradient) goes HBM/L2 -> LDS by buffer DMA
//    (no VGPRs, no ds_write).  Each DMA moves 8 rows x 128 bytes (whole cache
//    lines) into 1 KiB of LDS; chunk c of row r sits at position
//    c ^ ((r >> 1) & 7), chosen through each lane's source address, so the
//    16 rows of a quarter-wave fragment read hit distinct banks.  A ring of
//    WS_DA stages gives each DMA WS_DA-1 k-steps to land.
//  - W streams through a register ring of WS_PW k-steps, is dequantised and
//    written to a double-buffered B tile (forward: fragment-major like A;
//    dgrad: the transposed-operand layout read with ds_read_b64_tr_b16).
// The roles meet at one barrier per k-step; each role's registers are live
// only in its own branch.
constexpr int WS_DA = 4, WS_PW = 4;
template <int MODE>
__global__ __launch_bounds__(512) void gemm_ws_kernel(GemmParams p) {
  static_assert(MODE == FWD_Q4 || MODE == DGRAD_Q4, "4-bit modes only");
  constexpr int BM = 256, BN = 128, NT = 512, NP = 256;  // NP: producer threads
  constexpr int WM = 128, WN = 64, FM = 4, FN = 2;
  constexpr int A_ST = BM * BK / 8;  // 16-byte units per A stage (32 fragments)
  constexpr int B_ST = BN * BK / 8;  // per B buffer
  // separate LDS objects, so the compiler can tell the A DMAs from the B stores
  __shared__ uint4 ldsA[WS_DA * A_ST];
  __shared__ uint4 ldsB[2 * B_ST];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t tiles_p = st::cdiv(p.P, BN);
  int64_t t = st::xcd_remap(blockIdx.x, gridDim.x);
  // split-K: split s covers contraction [q0, q0 + qlen) (q0 a multiple of
  // 4*BK, so ring slots and scale groups keep their phase); the operands'
  // bases move by q0 and every index below stays relative to it
  int64_t q0 = 0, qlen = p.Q;
  int split = 0;
  if (p.splits > 1) {
    const int64_t nt = st::cdiv(p.M, BM) * tiles_p;
    split = (int)(t / nt);
    t -= split * nt;
    q0 = (int64_t)split * p.ks_len * BK;
    qlen = p.Q - q0 < (int64_t)p.ks_len * BK ? p.Q - q0 : (int64_t)p.ks_len * BK;
  }
  int64_t mt, pt;
  st::raster(t, st::cdiv(p.M, BM), tiles_p, p.raster_m, mt, pt);
  const int64_t p0 = pt * BN;
  int64_t m0 = mt * BM, mend = p.M;
  int grp = 0;
  if (p.goff) {  // whole workgroup leaves together, before any barrier
    if (!st::find_group(p.goff, p.ngroups, BM, mt, p.M, grp, m0, mend)) return;
  }
  const int KT = (int)st::cdiv(qlen, BK);
  uint4* const As0 = ldsA;  // stage a at As0 + a*A_ST
  uint4* const Bs0 = ldsB;  // buffer b at Bs0 + b*B_ST
  const float* Lg = p.L + grp * p.l_gstride;
  const int wm = wave >> 1, wn = wave & 1;  // consumer wave grid
  f32x16 acc[FM][FN];

  if (wave >= 4) {
    // ------------------------------------------------------------ producer
    const int pw = wave - 4, ptid = tid - NP;
    // contraction offset of the W operand: along its rows (FWD) or over them
    const int64_t wq0 = MODE == FWD_Q4 ? q0 : q0 * p.ldw;
    const auto rsA = make_rsrc(p.A + q0, p.a_bytes - q0 * 2);
    const auto rsW = make_rsrc(p.Wq + grp * p.w_gstride + wq0 / 2, p.w_bytes - wq0 / 2);
    const auto rsS = make_rsrc(p.Ws + grp * p.s_gstride + (wq0 >> p.gshift),
                               p.s_bytes - (wq0 >> p.gshift) * 4);
    // A: producer wave pw moves rows 64*pw + 8*q + l/8 (q < 8) of each stage;
    // lane l fills position l%8 of its row, i.e. chunk (l%8) ^ ((row>>1) & 7).
    uint32_t a_row[8];
    int a_c[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int row = 64 * pw + 8 * q + (lane >> 3);
      int64_t m = m0 + row;
      if (m < mend && p.gather) m = p.gather[m];
      a_c[q] = (lane & 7) ^ ((row >> 1) & 7);
      a_row[q] = (m0 + row < mend && m >= 0) ? (uint32_t)((m * p.lda + a_c[q] * 8) * 2) : kOOB;
    }
    auto dma_A = [&](int kt) {
      uint4* st_base = As0 + (kt % WS_DA) * A_ST;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const bool ok = a_row[q] != kOOB && kt * BK + a_c[q] * 8 < qlen;
        const uint32_t off = ok ? a_row[q] + (uint32_t)(kt * BK * 2) : kOOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsA, (__attribute__((address_space(3))) void*)(st_base + (8 * pw + q) * 64), 16, off,
            0, 0, 0);
      }
    };
    // W: 32 consecutive weights (16 packed bytes, one scale) per thread per
    // k-step.  FWD: W row n = p0 + ptid%128, k = kt*BK + 32*(ptid/128);
    // DGRAD: contraction row n = kt*BK + ptid/4, columns p0 + 32*(ptid%4).
    const int brow = MODE == FWD_Q4 ? ptid & 127 : ptid >> 2;
    const int bsub = MODE == FWD_Q4 ? ptid >> 7 : ptid & 3;
    uint32_t w_po = kOOB, w_so = kOOB;
    if constexpr (MODE == FWD_Q4) {
      const int64_t n = p0 + brow;
      if (n < p.P) {
        w_po = (uint32_t)((n * p.ldw + bsub * 32) >> 1);
        w_so = (uint32_t)((n * p.ldw) >> p.gshift) * 4;
      }
    }
    const int gstep = p.gshift - 6;  // k-steps per scale group: 1 << gstep
    const bool dcol_ok = p0 + bsub * 32 < p.P;
    struct WR {
      uint4 q;
      float s;
    };
    auto load_W = [&](int kt, WR& w) {
      if constexpr (MODE == FWD_Q4) {
        w.q = ld16(rsW, w_po + (uint32_t)(kt * (BK / 2)));
        w.s = __builtin_bit_cast(float, ld4(rsS, w_so + (uint32_t)(kt >> gstep) * 4));
      } else {
        const int64_t n = (int64_t)kt * BK + brow;
        const bool ok = dcol_ok && n < qlen;
        const int64_t e = n * p.ldw + p0 + bsub * 32;
        w.q = ld16(rsW, ok ? (uint32_t)(e >> 1) : kOOB);
        w.s = __builtin_bit_cast(float, ld4(rsS, ok ? (uint32_t)((e >> p.gshift) * 4) : kOOB));
      }
    };
    Tbl tbl;
    const uint32_t sh_e = p.hi_first ? 4u : 0u;
    auto store_B = [&](uint4* bs, const WR& w) {
      uint32_t words[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
      // dgrad: chunk (ch + bsub) & 3 of the thread's group goes out in store
      // ch, which keeps every store instruction free of bank conflicts
      if constexpr (MODE == DGRAD_Q4) st::rot4(words, bsub);
#pragma unroll
      for (int ch = 0; ch < 4; ++ch) {
        uint32_t o[4];
        deq8(words[ch], tbl, sh_e, 4u - sh_e, o);
        int idx;
        if constexpr (MODE == FWD_Q4) {
          // fragment (n-block brow/32, slice 2*bsub + ch/2), lane brow%32 + 32*(ch&1)
          idx = ((brow >> 5) * 4 + 2 * bsub + (ch >> 1)) * 64 + (brow & 31) + 32 * (ch & 1);
        } else {
          idx = st::trswz<BN>(brow, bsub * 4 + ((ch + bsub) & 3));
        }
        bs[idx] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    };

    // prologue: A stages for tiles 0 .. WS_DA-2, W ring for tiles 0 .. WS_PW-1,
    // B buffer 0 for tile 0.  Each step issues 8 DMAs and 2 W loads.
    WR wr[WS_PW];
#pragma unroll
    for (int j = 0; j < WS_DA - 1; ++j) dma_A(j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < WS_PW; ++j) load_W(j, wr[j]);
    tbl = make_tbl(p.lut, wr[0].s);
    store_B(Bs0, wr[0]);
    load_W(WS_PW, wr[0]);
    __builtin_amdgcn_sched_barrier(0);
    wait_cnt<0, 0>();
    __syncthreads();
    // step kt (between barriers kt-1 and kt): DMA tile kt+WS_DA-1 into the
    // stage tile kt-1 used (free since barrier kt-1), stage tile kt+1's B into
    // buffer (kt+1)&1 (its tile kt-1 was last read before barrier kt-1), and
    // make sure tile kt+1's A has landed before barrier kt.  vmcnt counts in
    // issue order and each step issues 10 operations; tile kt+1's DMAs came
    // WS_DA-2 steps earlier, so at most the 10*(WS_DA-2) operations of the
    // later steps may still be in flight (every load gets WS_DA-2 steps).
    auto step = [&](int kt, int u) {
      dma_A(kt + WS_DA - 1);
      __builtin_amdgcn_sched_barrier(0);
      const int nb = u & 1;
      if (MODE == DGRAD_Q4 || nb == 0 || gstep == 0) tbl = make_tbl(p.lut, wr[u].s);
      store_B(Bs0 + nb * B_ST, wr[u]);
      load_W(kt + 1 + WS_PW, wr[u]);
      __builtin_amdgcn_sched_barrier(0);
      wait_cnt<10 * (WS_DA - 2), 0>();  // tile kt+1's A landed; this step's B stores done
      bar();
    };
    // whole groups of WS_PW steps carry no conditions (static ring slots)
    int kt = 0;
    for (; kt + WS_PW <= KT; kt += WS_PW) {
#pragma unroll
      for (int v = 0; v < WS_PW; ++v) step(kt + v, (v + 1) % WS_PW);
    }
#pragma unroll
    for (int v = 0; v < WS_PW - 1; ++v)
      if (kt + v < KT) step(kt + v, (v + 1) % WS_PW);
    // the DMAs of the last steps (tiles past the end) must land before the
    // epilogue reuses LDS
    wait_cnt<0>();
  } else {
    // ------------------------------------------------------------ consumer
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    // A: row wm*WM + 32i + lane%32, chunk 2s + lane/32 at its swizzled
    // position (the row's bits 1-3 come from lane%32 alone); B fragment-major
    // (forward) or transposed (dgrad)
    const int a_lane = (wm * WM + (lane & 31)) * 8, a_f = ((lane & 31) >> 1) & 7;
    auto read_frags = [&](const uint4* as, const uint4* bs, int s, bf16x8 (&a)[FM],
                          bf16x8 (&b)[FN]) {
      const uint4* ap = as + a_lane + ((2 * s + (lane >> 5)) ^ a_f);
#pragma unroll
      for (int i = 0; i < FM; ++i) a[i] = __builtin_bit_cast(bf16x8, ap[i * 32 * 8]);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if constexpr (MODE == DGRAD_Q4)
          b[j] = st::tr_operand<BN>(bs, s * 16, wn * WN + j * 32, lane);
        else
          b[j] = __builtin_bit_cast(bf16x8, bs[((wn * FN + j) * 4 + s) * 64 + lane]);
      }
    };
    auto mfmas = [&](const bf16x8 (&a)[FM], const bf16x8 (&b)[FN]) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    };
    // Fragments two slices ahead, in three register sets used in rotation
    // (set X holds slice 0 of the step's tile, Y slice 1, Z takes slice 2):
    // the barrier sits after slice 1's MFMAs, once this wave's reads of the
    // tile are done, and slices 0 and 1 of tile kt+1 are read under slices 2
    // and 3 of tile kt.  The rotation repeats every three steps.
    bf16x8 fa[3][FM], fb[3][FN];
    __syncthreads();
    read_frags(As0, Bs0, 0, fa[0], fb[0]);
    read_frags(As0, Bs0, 1, fa[1], fb[1]);
    auto step = [&](int kt, auto rot) {
      constexpr int X = decltype(rot)::value, Y = (X + 1) % 3, Z = (X + 2) % 3;
      const uint4* as = As0 + (kt % WS_DA) * A_ST;
      const uint4* bs = Bs0 + (kt & 1) * B_ST;
      read_frags(as, bs, 2, fa[Z], fb[Z]);
      mfmas(fa[X], fb[X]);
      __builtin_amdgcn_sched_barrier(0);
      read_frags(as, bs, 3, fa[X], fb[X]);
      mfmas(fa[Y], fb[Y]);
      __builtin_amdgcn_sched_barrier(0);
      wait_cnt<63, 0>();  // this tile's fragment reads are done
      bar();
      const uint4* as1 = As0 + ((kt + 1) % WS_DA) * A_ST;
      const uint4* bs1 = Bs0 + ((kt + 1) & 1) * B_ST;
      read_frags(as1, bs1, 0, fa[Y], fb[Y]);
      mfmas(fa[Z], fb[Z]);
      __builtin_amdgcn_sched_barrier(0);
      read_frags(as1, bs1, 1, fa[Z], fb[Z]);
      mfmas(fa[X], fb[X]);
      __builtin_amdgcn_sched_barrier(0);
    };
    using R0 = std::integral_constant<int, 0>;
    using R1 = std::integral_constant<int, 1>;
    using R2 = std::integral_constant<int, 2>;
    int kt = 0;
    for (; kt + 3 <= KT; kt += 3) {
      step(kt, R0{});
      step(kt + 1, R1{});
      step(kt + 2, R2{});
    }
    if (kt < KT) step(kt, R0{});
    if (kt + 1 < KT) step(kt + 1, R1{});
  }
  // every wave's last LDS reads are done before the epilogue reuses LDS
  __syncthreads();
  if (p.splits > 1) {  // raw fp32 sums of this split; splitk_epilogue does the rest
    if (wave < 4) {
      const auto rsP = make_rsrc(p.part + (int64_t)split * p.M * p.P, p.M * p.P * 4);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t col = p0 + wn * WN + j * 32 + (lane & 31);
          const int64_t rb = m0 + wm * WM + i * 32 + (lane >> 5) * 4;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t row = rb + (v >> 2) * 8 + (v & 3);
            const bool ok = row < mend && col < p.P;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][v]), rsP,
                                                  (int)(ok ? (uint32_t)((row * p.P + col) * 4) : kOOB),
                                                  0, 0);
          }
        }
    }
    return;
  }
  gemm_epilogue<MODE == DGRAD_Q4, BM, BN, NT, FM, FN, WM, WN>(p, acc, ldsA, m0, mend, p0, wm, wn,
                                                              tid, lane, wave < 4, Lg);
}

// Split-K epilogue: y[m, n] = the GEMM epilogue of sum_s part[s][m][n], the
// splits summed in ascending order: y = bf16(sum), + the LoRA term
// (forward: bf16(y + scale * sum_j T[m, seg(n)*r + j] B[n, j]); dgrad:
// bf16(y + bf16(sum_j dT[m, j] A[j, n]))), + the residual (bf16(R + y)).
// One thread per 4 consecutive outputs of a row (P % 4 == 0, checked by the
// host), fp32 partials read as 16-byte vectors.
template <bool DGRAD>
__global__ __launch_bounds__(256) void splitk_epilogue(GemmParams p) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per = p.P / 4;
  if (q >= p.M * per) return;
  const int64_t m = q / per, n0 = (q % per) * 4;
  const int64_t mp = p.M * p.P;
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < p.splits; ++s) {
    const float4 v = *(const float4*)(p.part + s * mp + m * p.P + n0);
    a[0] += v.x; a[1] += v.y; a[2] += v.z; a[3] += v.w;
  }
  uint16_t out[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t n = n0 + e;
    float y = st::bf16r(a[e]);
    if (p.T) {
      int coff = 0;
      if (!DGRAD)
        for (int i = 0; i < p.nseg; ++i) coff += p.seg_end[i] <= n ? p.lora_k : 0;
      float la = 0.f;
      for (int j = 0; j < p.lora_k; ++j) {
        const float tv = p.T[m * p.ldt + coff + j];
        const float lv = DGRAD ? p.L[(int64_t)j * p.ldl + n] : p.L[n * p.ldl + j];
        la += tv * lv;
      }
      y = DGRAD ? st::bf16r(y + st::bf16r(la)) : st::bf16r(y + la * p.lora_scale);
    }
    if (p.R) y = st::bf16r(st::bf16_to_f32(p.R[m * p.ldr + n]) + y);
    out[e] = st::f32_to_bf16(y);
  }
  uint16_t* c = p.C + m * p.ldc + n0;
#pragma unroll
  for (int e = 0; e < 4; ++e) c[e] = out[e];
}

// Register-operand forward, 256x256 tile.  In the forward the MFMA B operand
// of a lane is 8 consecutive contraction elements of one W row, i.e. one
// packed 32-bit word, so W goes HBM/L2 -> VGPRs -> dequantised straight into
// B operands with no LDS traffic at all; only A is staged in LDS.  Each wave
// owns 32*FN output columns for all 256 rows (FN = 2: 4 waves, one per SIMD,
// 256 accumulators each; FN = 1: 8 waves), so no two waves dequantise the
// same W element.  Within a k-step of 64 the contraction index is permuted
// alike for both operands: slice s, lane half h takes k = 32h + 8s .. +7, so
// a lane's W for the whole k-step is one 16-byte load (32 codes, one scale)
// and A chunk 4h + s.  Products are the same; only the order of the fp32
// accumulation inside the k-step differs from the LDS-operand kernels.
//  - A: RB_ST stages of 256 rows x 64 by buffer DMA (the swizzled whole-line
//    layout of gemm_ws_kernel); tile kt+RB_ST is issued after the barrier of
//    step kt into the stage tile kt has just released.
//  - W: a ring of RB_ST register sets, also issued RB_ST tiles ahead.
// One barrier per k-step, before the last slice: by then every wave has read
// all of tile kt's fragments, and tile kt+1 has landed.  The k-loop is
// unrolled by RB_ST (even), so ring slots and scale-group parity are static;
// the launcher requires K % (RB_ST * 64) == 0.
constexpr int RB_ST = 4;
// Instruction order of one slice section (sched_group_barrier masks: 0x008
// MFMA, 0x100 LDS read, 0x020 vector-memory read, 0x002 VALU): each MFMA is
// followed by a share of the next slice's LDS reads and dequantisation, so
// the fragment reads are issued early and the VALU co-issues with the MFMAs
// of one wave.  VM adds the section's DMAs and W loads.
#define RB_G(mask, n) __builtin_amdgcn_sched_group_barrier(mask, n, 0)
template <int FN, bool VM, int FM = 8>
__device__ __forceinline__ void rb_order() {
  static_assert(FN == 1 || FN == 2, "one or two B fragments per wave");
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    RB_G(0x008, 1);
    if constexpr (VM) RB_G(0x020, 1);
    RB_G(0x100, 1);
    RB_G(0x002, (FN == 2 ? 3 : 4) * 8 / FM);
    if constexpr (FN == 2) {
      RB_G(0x008, 1);
      if constexpr (VM) RB_G(0x020, 1);
      RB_G(0x002, 4);
    }
  }
}
#undef RB_G
template <int FN, int WAVES, bool HI, int FM = 8>
__global__ __launch_bounds__(64 * WAVES, FM == 4 ? 4 : 1) void gemm_rb_kernel(GemmParams p) {
  constexpr int BM = 32 * FM, NT = 64 * WAVES, WN = 32 * FN, BN = WN * WAVES;
  constexpr int WM = BM;
  constexpr int A_ST = BM * BK / 8;       // 16-byte units per A stage
  constexpr int DMA_W = BM / 8 / WAVES;   // DMAs (8 rows each) per wave per stage
  // vector-memory operations issued per step: the DMAs, FN W loads, and FN
  // scale loads for a tile that starts a scale group (even tiles); two
  // consecutive steps issue RB_PAIR of them
  constexpr int RB_PAIR = 2 * DMA_W + 3 * FN;
  __shared__ uint4 ldsA[RB_ST * A_ST];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t tiles_p = st::cdiv(p.P, BN);
  const int64_t t = st::xcd_remap(blockIdx.x, gridDim.x);
  int64_t mt, pt;
  st::raster(t, st::cdiv(p.M, BM), tiles_p, p.raster_m, mt, pt);
  const int64_t p0 = pt * BN;
  int64_t m0 = mt * BM, mend = p.M;
  int grp = 0;
  if (p.goff) {  // grouped (per-expert) rows: the whole workgroup leaves together
    if (!st::find_group(p.goff, p.ngroups, BM, mt, p.M, grp, m0, mend)) return;
  }
  const int KT = (int)(p.Q / BK);
  const auto rsA = make_rsrc(p.A, p.a_bytes);
  const auto rsW = make_rsrc(p.Wq + grp * p.w_gstride, p.w_bytes);
  const auto rsS = make_rsrc(p.Ws + grp * p.s_gstride, p.s_bytes);

  // A DMA: wave w moves rows 8*(w*DMA_W + q) + lane/8 of each stage; lane l
  // fills position l%8 of its row, i.e. chunk (l%8) ^ ((row>>1) & 7).  Rows
  // beyond M start at kOOB and stay out of range; tiles past the last one
  // (K % 64 == 0) read rows' later bytes or zeros and are never used.
  uint32_t a_row[DMA_W];
#pragma unroll
  for (int q = 0; q < DMA_W; ++q) {
    const int row = 8 * (wave * DMA_W + q) + (lane >> 3);
    const int c = (lane & 7) ^ ((row >> 1) & 7);
    int64_t m = m0 + row;
    if (m < mend && p.gather) m = p.gather[m];  // permuted row -> token row
    a_row[q] = (m0 + row < mend && m >= 0) ? (uint32_t)((m * p.lda + c * 8) * 2) : kOOB;
  }
  auto dma_A = [&](int kt) {
    uint4* st_base = ldsA + (kt % RB_ST) * A_ST;
#pragma unroll
    for (int q = 0; q < DMA_W; ++q) {
      const uint32_t off = a_row[q] + (uint32_t)(kt * BK * 2);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsA, (__attribute__((address_space(3))) void*)(st_base + (wave * DMA_W + q) * 64), 16,
          off, 0, 0, 0);
    }
  };

  // W: column n_j = p0 + wave*WN + 32j + lane%32, contraction half h = lane/32.
  // K (= ldw) is a multiple of 128: k-step kt adds 32 payload bytes, scale
  // group kt/2.  Loads past the end of W read zeros or W's own bytes (unused).
  const int h = lane >> 5;
  uint32_t w_po[FN], w_so[FN];
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int64_t n = p0 + wave * WN + 32 * j + (lane & 31);
    w_po[j] = n < p.P ? (uint32_t)((n * p.ldw + 32 * h) >> 1) : kOOB;
    w_so[j] = n < p.P ? (uint32_t)((n * p.ldw) >> 7) * 4 : kOOB;
  }
  struct WR {
    uint4 q[FN];
    float s[FN];
  };
  // the scale of a group is loaded with its first (even) tile only
  auto load_W = [&](int kt, WR& w, bool group_start) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      w.q[j] = ld16(rsW, w_po[j] + (uint32_t)(kt * (BK / 2)));
      if (group_start)
        w.s[j] = __builtin_bit_cast(float, ld4(rsS, w_so[j] + (uint32_t)(kt >> 1) * 4));
    }
  };
  Tbl tbl[FN];
  auto make_tbls = [&](const WR& w) {
#pragma unroll
    for (int j = 0; j < FN; ++j) tbl[j] = make_tbl(p.lut, w.s[j]);
  };
  auto deq_B = [&](const WR& w, int s, bf16x8 (&b)[FN]) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const uint32_t word = s == 0 ? w.q[j].x : s == 1 ? w.q[j].y : s == 2 ? w.q[j].z : w.q[j].w;
      uint32_t o[4];
      deq8o<HI>(word, tbl[j], o);
      b[j] = __builtin_bit_cast(bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
    }
  };
  // A fragment i of slice s: row 32i + lane%32, chunk 4h + s at its swizzled
  // position (bits 1-3 of the row come from lane%32 alone)
  const int a_lane = (lane & 31) * 8, a_f = ((lane & 31) >> 1) & 7;
  auto read_A = [&](int kt, int s, bf16x8 (&a)[FM]) {
    const uint4* ap = ldsA + (kt % RB_ST) * A_ST + a_lane + ((4 * h + s) ^ a_f);
#pragma unroll
    for (int i = 0; i < FM; ++i) a[i] = __builtin_bit_cast(bf16x8, ap[i * 32 * 8]);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  auto mfmas = [&](const bf16x8 (&a)[FM], const bf16x8 (&b)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  };

  WR wr[RB_ST];
  bf16x8 fa0[FM], fb0[FN], fa1[FM], fb1[FN];
  // prologue: tiles 0..RB_ST-1 issued, tile 0 landed everywhere
#pragma unroll
  for (int j = 0; j < RB_ST; ++j) {
    dma_A(j);
    load_W(j, wr[j], (j & 1) == 0);
  }
  static_assert(RB_ST == 4, "the waits below count two step pairs");
  wait_cnt<RB_PAIR + DMA_W + FN>();  // tiles 1-3 may be in flight
  bar();
  make_tbls(wr[0]);
  read_A(0, 0, fa0);
  deq_B(wr[0], 0, fb0);

  // step kt, W of tile kt in wr[u] (u = kt % RB_ST): slices 0-2 with the next
  // slice's operands read ahead; then wait for tile kt+1 (issued RB_ST-1
  // steps ago; the operations of the RB_ST-2 = 2 later steps, one of each
  // parity, may stay in flight) and for this wave's fragment reads, barrier, refill the
  // released stage and W set with tile kt+RB_ST, and read slice 0 of tile
  // kt+1 under slice 3's MFMAs.
  auto step = [&](int kt, int u) {
    read_A(kt, 1, fa1);
    deq_B(wr[u], 1, fb1);
    mfmas(fa0, fb0);
    rb_order<FN, false, FM>();
    __builtin_amdgcn_sched_barrier(0);
    read_A(kt, 2, fa0);
    deq_B(wr[u], 2, fb0);
    mfmas(fa1, fb1);
    rb_order<FN, false, FM>();
    __builtin_amdgcn_sched_barrier(0);
    read_A(kt, 3, fa1);
    deq_B(wr[u], 3, fb1);
    mfmas(fa0, fb0);
    rb_order<FN, false, FM>();
    __builtin_amdgcn_sched_barrier(0);
    wait_cnt<RB_PAIR, 0>();
    bar();
    dma_A(kt + RB_ST);
    load_W(kt + RB_ST, wr[u], (u & 1) == 0);
    const int un = (u + 1) % RB_ST;
    if ((u & 1) == 1) make_tbls(wr[un]);  // tile kt+1 starts a scale group
    read_A(kt + 1, 0, fa0);
    deq_B(wr[un], 0, fb0);
    mfmas(fa1, fb1);
    rb_order<FN, true, FM>();
    __builtin_amdgcn_sched_barrier(0);
  };
  for (int kt = 0; kt < KT; kt += RB_ST) {
#pragma unroll
    for (int v = 0; v < RB_ST; ++v) step(kt + v, v);
  }
  // the DMAs of tiles past the end must land before the epilogue reuses LDS
  wait_cnt<0>();
  __syncthreads();
  gemm_epilogue<false, BM, BN, NT, FM, FN, WM, WN>(p, acc, ldsA, m0, mend, p0, 0, wave, tid, lane,
                                                   true, p.L + grp * p.l_gstride);
}

// Chooses the epilogue's access width (GemmParams::vec_epi): 16-byte rows
// need C, the residual and gate|up 16-byte aligned with row strides, P and
// the gate|up split multiples of 8, and `waves` staging areas after the LoRA
// operands within the tile's `lds_dwords`.  ST_GEMM_VEC_EPI=0 keeps 2-byte
// accesses where the epilogue has them (every case but the SwiGLU VJP).
template <bool DGRAD, int BM, int BN>
int choose_epilogue(GemmParams& p, int64_t lds_dwords, int waves) {
  auto a16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  bool ok = p.P % 8 == 0 && p.ldc % 8 == 0 && a16(p.C) &&
            epi_stage_offset<DGRAD, BM, BN>(p) + (int64_t)waves * EPI_STG <= lds_dwords;
  if (p.R) ok = ok && p.ldr % 8 == 0 && a16(p.R);
  if (p.swi_gu) {
    ok = ok && p.swi_ld % 8 == 0 && p.swi_I % 8 == 0 && a16(p.swi_gu);
    if (!ok)
      return st::fail(ST_EUNSUPPORTED,
                      "q4gemm: SwiGLU epilogue needs 16-byte aligned gate|up and output rows "
                      "(strides and width multiples of 8) and LDS beside the LoRA operands");
    p.vec_epi = 1;
    return ST_OK;
  }
  const char* env = getenv("ST_GEMM_VEC_EPI");
  p.vec_epi = (ok && !(env && atoi(env) == 0)) ? 1 : 0;
  return ST_OK;
}

// Row tiles per raster group (st::raster) of a dense launch: 4, so each XCD's
// 32 CUs take 4 row panels x 8 column panels at a time and its L2 serves each
// A and W panel to several CUs (with row-major order one A panel and 32 W
// panels: every XCD streamed all of W).  Measured on the Llama-8B layer step:
// 3.84-3.86 ms with 1, 3.76 ms with 2 or 4, 3.78 ms with 8; every fused GEMM
// of the step 1-3% faster.  ST_GEMM_RASTER overrides it; grouped launches
// keep their expert order.
int raster_choice(const GemmParams& p) {
  if (p.goff) return 1;
  const char* env = getenv("ST_GEMM_RASTER");
  const int g = env ? atoi(env) : 4;
  return g > 1 ? g : 1;
}

// Row-tile slots of a launch: grouped launches (per-expert row ranges) take
// sum_g cdiv(rows_g, BM) <= cdiv(rows, BM) + groups; slots past the last
// group's tiles exit at once.
int64_t row_tiles(const GemmParams& p, int BM) {
  return st::cdiv(p.M, BM) + (p.goff ? p.ngroups : 0);
}

// The epilogue addresses C, the residual, T and the LoRA right operand with
// 32-bit byte offsets.
int check_epilogue_extents(const GemmParams& p) {
  const int64_t lim = 1ll << 31;
  bool ok = ((p.M - 1) * p.ldc + p.P) * 2 < lim;
  if (p.R) ok = ok && ((p.M - 1) * p.ldr + p.P) * 2 < lim;
  if (p.swi_gu)
    ok = ok && ((p.M - 1) * p.ldc + 2 * p.swi_I) * 2 < lim &&
         ((p.M - 1) * p.swi_ld + 2 * p.swi_I) * 2 < lim;
  if (p.T) ok = ok && (p.M * p.ldt + p.lora_cols) * 4 < lim &&
                (p.P + p.lora_k) * (p.ldl + 1) * 4 < lim;
  return ok ? ST_OK : st::fail(ST_EUNSUPPORTED, "q4gemm: output, residual or LoRA operand above 2 GiB");
}

template <int MODE, int BM, int BN, int WAVES, int WAVES_M = 2, bool FLAT = false, bool LG = false>
int launch(const GemmParams& p, hipStream_t stream);

template <int MODE>
int launch_ws(const GemmParams& p, hipStream_t stream) {
  constexpr int BM = 256, BN = 128;
  int64_t tiles = row_tiles(p, BM) * st::cdiv(p.P, BN);
  if (tiles > 0x7fffffff) return st::fail(ST_EUNSUPPORTED, "q4gemm: too many tiles");
  if (int rc = check_epilogue_extents(p)) return rc;
  // LoRA operands that do not fit this tile's LDS: the 128x128 kernel
  if (!lora_staged_fits<MODE == DGRAD_Q4, BM, BN>(p, (int64_t)WS_DA * BM * BK / 8 * 4, 4))
    return launch<MODE, 128, 128, 4>(p, stream);
  GemmParams q = p;
  q.raster_m = raster_choice(q);
  if (int rc = choose_epilogue<MODE == DGRAD_Q4, BM, BN>(q, (int64_t)WS_DA * BM * BK / 8 * 4, 4))
    return rc;
  gemm_ws_kernel<MODE><<<(unsigned)tiles, 512, 0, stream>>>(q);
  return st::check_launch("q4gemm");
}

template <int FN, int WAVES, int FM = 8>
int launch_rb(const GemmParams& p, hipStream_t stream) {
  constexpr int BM = 32 * FM, BN = 32 * FN * WAVES, NT = 64 * WAVES;
  constexpr int64_t lds_dwords = (int64_t)RB_ST * BM * BK / 8 * 4;
  const int64_t tiles = row_tiles(p, BM) * st::cdiv(p.P, BN);
  if (tiles > 0x7fffffff) return st::fail(ST_EUNSUPPORTED, "q4gemm: too many tiles");
  if (p.Q % (RB_ST * BK))
    return st::fail(ST_EUNSUPPORTED, "q4gemm: register-operand tile needs K %% %d == 0",
                    RB_ST * BK);
  if (int rc = check_epilogue_extents(p)) return rc;
  if (!lora_staged_fits<false, BM, BN>(p, lds_dwords, NT / 64))
    return launch<FWD_Q4, 128, 128, 4>(p, stream);
  GemmParams q = p;
  q.raster_m = raster_choice(q);
  if (int rc = choose_epilogue<false, BM, BN>(q, lds_dwords, NT / 64)) return rc;
  if (q.hi_first)
    gemm_rb_kernel<FN, WAVES, true, FM><<<(unsigned)tiles, NT, 0, stream>>>(q);
  else
    gemm_rb_kernel<FN, WAVES, false, FM><<<(unsigned)tiles, NT, 0, stream>>>(q);
  return st::check_launch("q4gemm");
}

template <int MODE, int BM, int BN, int WAVES, int WAVES_M, bool FLAT, bool LG>
int launch(const GemmParams& p, hipStream_t stream) {
  constexpr int NT = 64 * WAVES;
  int64_t tiles = row_tiles(p, BM) * st::cdiv(p.P, BN);
  if (tiles > 0x7fffffff) return st::fail(ST_EUNSUPPORTED, "q4gemm: too many tiles");
  if (int rc = check_epilogue_extents(p)) return rc;
  using TL = Tile<MODE, BM, BN, WAVES, WAVES_M>;
  GemmParams q = p;
  q.raster_m = raster_choice(q);
  // the LoRA epilogue stages T and the right operand in the tile's LDS when
  // they fit; otherwise the 128x128 kernel built to read them from global
  // memory runs the GEMM
  if constexpr (LG) {
    q.lora_global = q.T ? 1 : 0;
  } else if constexpr (TL::Q4) {
    if (!lora_staged_fits<TL::DGRAD, BM, BN>(q, (int64_t)TL::LDS_CHUNKS * 4, WAVES))
      return launch<MODE, 128, 128, 4, 2, FLAT, true>(p, stream);
  }
  if (int rc = choose_epilogue<TL::DGRAD, BM, BN>(q, (int64_t)TL::LDS_CHUNKS * 4, WAVES)) return rc;
  gemm_kernel<MODE, BM, BN, WAVES, WAVES_M, FLAT, LG><<<(unsigned)tiles, NT, 0, stream>>>(q);
  return st::check_launch("q4gemm");
}

// 256-row tiles halve the dequant work per MFMA against 128-row ones but need
// enough tiles to cover the 256 CUs.  Forward with >= 192 tiles of 256x256:
// the 256x256 register-operand kernel (the LDS-operand 8-wave kernel with
// ST_GEMM_RB=0); otherwise the warp-specialised 256x128 kernel (2562) where it
// yields >= 192 tiles; else 128x128 (4 waves).  ST_GEMM_TILE forces one, so
// tests can cover every tile the dispatch takes (128, 256, 2562; forward only,
// register-operand: 2566 = 256x256 8 waves, 2567 = 256x128 4 waves (the
// split tail), 2568 = 128x256 8 waves (the grouped forward)).  For the N = 4096 forwards (o,
// down) the 256x128 register-operand and the 128x256 tiles measured no faster
// than the warp-specialised kernel.
int cu_count();

int tile_choice(int mode, int64_t M, int64_t P) {
  const char* env = getenv("ST_GEMM_TILE");
  if (env) return atoi(env);
  // the transposed-operand dgrad runs out of registers at 256x256 (8 waves)
  if (mode == FWD_Q4 && st::cdiv(M, 256) * st::cdiv(P, 256) >= 192) return 256;
  const int64_t t2562 = st::cdiv(M, 256) * st::cdiv(P, 128);
  if (t2562 >= 192) return 2562;
  // a forward whose 256x128 tiles fit one round where 128x128 tiles need a
  // second (the MLA q_a|kv_a projection, 2112 columns at 2048 tokens: 107
  // against 167 us)
  if (mode == FWD_Q4 && t2562 <= cu_count() && st::cdiv(M, 128) * st::cdiv(P, 128) > cu_count())
    return 2562;
  return 128;
}

int cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// Forward output columns [c0, c1) of p as a GEMM of its own (c0 a multiple
// of 128): W rows and LoRA B rows move by c0, the segments (and T columns)
// that end before c0 drop out.
GemmParams column_slice(const GemmParams& p, int64_t c0, int64_t c1) {
  GemmParams q = p;
  q.P = c1 - c0;
  q.C = p.C + c0;
  if (p.R) q.R = p.R + c0;
  q.Wq = p.Wq + c0 * p.ldw / 2;
  q.Ws = p.Ws + ((c0 * p.ldw) >> p.gshift);
  q.w_bytes = p.w_bytes - c0 * p.ldw / 2;
  q.s_bytes = p.s_bytes - ((c0 * p.ldw) >> p.gshift) * 4;
  if (p.T) {
    q.L = p.L + c0 * p.ldl;
    int drop = 0;
    while (drop < p.nseg && p.seg_end[drop] <= c0) ++drop;
    q.nseg = p.nseg - drop;
    for (int i = 0; i < q.nseg; ++i) q.seg_end[i] = p.seg_end[i + drop] - c0;
    q.T = p.T + (int64_t)drop * p.lora_k;
    q.lora_cols = q.nseg * p.lora_k;
  }
  return q;
}

// Tail balancing for the 256x256 forward.  A launch of `tiles` one-per-CU
// tiles takes cdiv(tiles, CUs) rounds; when the last round is partly idle,
// the columns of the whole rounds keep the 256x256 tile and the leftover
// columns run as a second launch of 256x128 warp-specialised tiles (measured
// at ~0.6 of a 256x256 round per round).  Returns the split column (0: no
// split).  ST_GEMM_SPLIT=0 disables it.  (A 256x128 dgrad with a 128x128 tail
// measured no faster, so the dgrad is not split.)
int64_t split_column(int t, int64_t M, int64_t P) {
  const char* env = getenv("ST_GEMM_SPLIT");
  if ((env && !atoi(env)) || t != 256) return 0;
  const int64_t cus = cu_count();
  const int64_t mt = st::cdiv(M, 256), tiles = mt * st::cdiv(P, 256);
  if (tiles <= cus || tiles % cus == 0) return 0;
  const int64_t full = tiles / cus * cus;
  if (full % mt) return 0;
  const int64_t c1 = full / mt * 256;
  if (c1 >= P) return 0;
  const int64_t t2 = mt * st::cdiv(P - c1, 128);
  const double split = (double)(full / cus) + 0.6 * (double)st::cdiv(t2, cus);
  return split < (double)st::cdiv(tiles, cus) ? c1 : 0;
}

// Split-K of a dense 4-bit GEMM whose 256x128 warp-specialised tiles leave
// CUs idle for a long contraction (DeepSeek MLA: kv_b's input gradient, 512
// outputs from 32768; q_b's, 1536 from 24576).  Cost model per CU in k-steps:
// rounds(tiles * splits) * (k-steps per split + 8 for each workgroup's
// prologue and epilogue); splits that cut it below 3/4 of the unsplit cost.
// K-steps per split are a multiple of 4 (the ring phase of gemm_ws_kernel).
// Only GEMMs of 8 GFLOP or more split (smaller ones are latency-bound
// either way), and none while ST_GEMM_TILE pins a tile for the tests.
// ST_GEMM_SPLITK=0 disables, =n asks for n splits.
struct SplitPlan {
  int splits = 1, ks_len = 0;
};
SplitPlan split_plan(int64_t M, int64_t P, int64_t Q) {
  SplitPlan plan;
  const char* env = getenv("ST_GEMM_SPLITK");
  if (env && atoi(env) == 0) return plan;
  const int64_t tiles = st::cdiv(M, 256) * st::cdiv(P, 128), KT = st::cdiv(Q, BK);
  const int64_t cus = cu_count();
  if (KT < 16 || P % 4 || M * P * 4 >= (1ll << 31)) return plan;
  if (!env && (getenv("ST_GEMM_TILE") || 2.0 * (double)M * (double)P * (double)Q < 8e9))
    return plan;
  auto shape = [&](int64_t s, int64_t& len) {
    len = st::cdiv(st::cdiv(KT, s), 4) * 4;
    return st::cdiv(KT, len);
  };
  auto cost = [&](int64_t s) {
    int64_t len;
    const int64_t ns = shape(s, len);
    return st::cdiv(tiles * ns, cus) * (len + 8);
  };
  int64_t best = 1, bc = cost(1);
  if (env) {
    best = atoi(env);
  } else {
    if (tiles >= cus) return plan;
    for (int64_t s = 2; s <= 32; ++s)
      if (cost(s) < bc) bc = cost(s), best = s;
    if (best == 1 || bc * 4 > cost(1) * 3) return plan;
  }
  int64_t len;
  const int64_t ns = shape(best, len);
  if (ns <= 1) return plan;
  plan.splits = (int)ns;
  plan.ks_len = (int)len;
  return plan;
}

int64_t split_workspace(const SplitPlan& plan, int64_t M, int64_t P) {
  return plan.splits > 1 ? (int64_t)plan.splits * M * P * 4 + 256 : 0;
}

// Split-K launch: the warp-specialised kernel writes each split's fp32 sums,
// splitk_epilogue sums them in split order and applies the epilogue.
template <int MODE>
int launch_ws_split(GemmParams p, const SplitPlan& plan, void* workspace, hipStream_t stream) {
  p.part = (float*)(((uintptr_t)workspace + 255) & ~(uintptr_t)255);
  p.splits = plan.splits;
  p.ks_len = plan.ks_len;
  p.raster_m = raster_choice(p);
  const int64_t tiles = st::cdiv(p.M, 256) * st::cdiv(p.P, 128) * plan.splits;
  if (tiles > 0x7fffffff) return st::fail(ST_EUNSUPPORTED, "q4gemm: too many tiles");
  gemm_ws_kernel<MODE><<<(unsigned)tiles, 512, 0, stream>>>(p);
  if (int rc = st::check_launch("q4gemm split-K")) return rc;
  const int64_t threads = p.M * (p.P / 4);
  splitk_epilogue<MODE == DGRAD_Q4><<<(unsigned)st::cdiv(threads, 256), 256, 0, stream>>>(p);
  return st::check_launch("q4gemm split-K epilogue");
}

template <int MODE>
int dispatch(const GemmParams& p, hipStream_t stream) {
  // the dense-W fallbacks (K not a multiple of 128) always use 128x128 tiles
  if constexpr (MODE == FWD_Q4 || MODE == DGRAD_Q4) {
    const int t = tile_choice(MODE, p.M, p.P);
    if constexpr (MODE == FWD_Q4) {
      // 256x256 forward: register-operand kernel (8 waves) unless
      // ST_GEMM_RB=0; its column tail runs on the register-operand 256x128
      // tile, which sums each output in the same order, so a split stays
      // bit-identical to one launch
      const char* rbe = getenv("ST_GEMM_RB");
      const bool rb = (!rbe || atoi(rbe)) && p.Q % (RB_ST * BK) == 0 && p.gshift == 7;
      if (const int64_t c1 = split_column(t, p.M, p.P)) {
        const GemmParams head = column_slice(p, 0, c1), tail = column_slice(p, c1, p.P);
        if (rb) {
          const int rc = launch_rb<1, 8>(head, stream);
          return rc ? rc : launch_rb<1, 4>(tail, stream);
        }
        const int rc = launch<MODE, 256, 256, 8>(head, stream);
        return rc ? rc : launch_ws<MODE>(tail, stream);
      }
      if (t == 256 && rb) return launch_rb<1, 8>(p, stream);
    }
    if (t == 256) return launch<MODE, 256, 256, 8>(p, stream);
    if (t == 2562) return launch_ws<MODE>(p, stream);
    if constexpr (MODE == FWD_Q4) {
      const bool rbk = p.Q % (RB_ST * BK) == 0 && p.gshift == 7;
      if (t == 2566 && rbk) return launch_rb<1, 8>(p, stream);
      if (t == 2567 && rbk) return launch_rb<1, 4>(p, stream);
      if (t == 2568 && rbk) return launch_rb<1, 8, 4>(p, stream);
    }
  }
  return launch<MODE, 128, 128, 4>(p, stream);
}

int run_gemm(int mode, const GemmParams& p, hipStream_t stream) {
  switch (mode) {
    case FWD_Q4: return dispatch<FWD_Q4>(p, stream);
    case DGRAD_Q4: return dispatch<DGRAD_Q4>(p, stream);
    case FWD_BF16: return dispatch<FWD_BF16>(p, stream);
    default: return dispatch<DGRAD_BF16>(p, stream);
  }
}

bool al16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }

}  // namespace

// Every shape runs from the packed weight (K % 128 != 0 on the flat-group
// kernels), so the fused linears take no workspace; the queries stay for
// callers that size one.
extern "C" int64_t st_q4_linear_fwd_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return split_workspace(split_plan(M, N, K), M, N);
}

extern "C" int64_t st_q4_linear_dgrad_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return split_workspace(split_plan(M, K, N), M, K);
}

static int check_lora_common(int64_t rank, int64_t cols) {
  if (rank <= 0 || rank > 65536 || cols > 65536)
    return st::fail(ST_EUNSUPPORTED, "q4 linear: LoRA contraction %lld (%lld columns) out of range",
                    (long long)rank, (long long)cols);
  return ST_OK;
}

extern "C" int st_q4_linear_fwd(const uint16_t* x, int64_t M, int64_t K, int64_t ldx,
                                const uint8_t* payload, const float* scales, int64_t N,
                                const float* lut16, int32_t flags, const float* t, int64_t ldt,
                                const float* lora_b, int32_t rank, float lora_scale, int32_t nseg,
                                const int64_t* seg_end, const uint16_t* residual, int64_t ldr,
                                uint16_t* y, int64_t ldy, void* workspace,
                                int64_t workspace_bytes, st_stream_t stream) {
  ST_CHECK_ARG(M >= 0 && N > 0 && K > 0, "st_q4_linear_fwd: bad shape M=%lld N=%lld K=%lld",
               (long long)M, (long long)N, (long long)K);
  if (M == 0) return ST_OK;
  ST_CHECK_ARG(x && payload && scales && y && lut16, "st_q4_linear_fwd: NULL pointer");
  ST_CHECK_ARG(K % 8 == 0 && ldx % 8 == 0 && ldx >= K && al16(x),
               "st_q4_linear_fwd: x needs K %% 8 == 0, 16-byte rows (K=%lld ldx=%lld)",
               (long long)K, (long long)ldx);
  ST_CHECK_ARG(ldy >= N, "st_q4_linear_fwd: ldy < N");
  GemmParams p{};
  p.A = x; p.lda = ldx; p.M = M; p.P = N; p.Q = K;
  p.C = y; p.ldc = ldy; p.R = residual; p.ldr = ldr;
  p.hi_first = (flags & ST_FLAG_HI_NIBBLE_FIRST) ? 1 : 0;
  p.gshift = (flags & ST_FLAG_GROUP64) ? 6 : 7;
  for (int i = 0; i < 16; ++i) p.lut.v[i] = lut16[i];
  if (residual) ST_CHECK_ARG(ldr >= N, "st_q4_linear_fwd: ldr < N");
  if (t) {
    ST_CHECK_ARG(lora_b != nullptr, "st_q4_linear_fwd: t without lora_b");
    ST_CHECK_ARG(nseg >= 1 && nseg <= 4 && seg_end, "st_q4_linear_fwd: nseg must be 1..4");
    int rc = check_lora_common(rank, (int64_t)rank * nseg);
    if (rc) return rc;
    int64_t prev = 0;
    for (int i = 0; i < nseg; ++i) {
      ST_CHECK_ARG(seg_end[i] > prev && (seg_end[i] % 32 == 0 || seg_end[i] == N),
                   "st_q4_linear_fwd: segment ends must increase and be multiples of 32");
      prev = seg_end[i];
      p.seg_end[i] = seg_end[i];
    }
    ST_CHECK_ARG(prev == N, "st_q4_linear_fwd: last segment end must equal N");
    ST_CHECK_ARG(ldt >= (int64_t)rank * nseg, "st_q4_linear_fwd: ldt too small");
    p.T = t; p.ldt = ldt; p.L = lora_b; p.ldl = rank; p.lora_k = rank;
    p.lora_cols = rank * nseg; p.lora_scale = lora_scale; p.nseg = nseg;
  }
  hipStream_t s = (hipStream_t)stream;
  p.a_bytes = ((M - 1) * ldx + K) * 2;
  ST_CHECK_ARG(p.a_bytes < (1ll << 31) && N * K * 2 < (1ll << 31),
               "st_q4_linear_fwd: operands above 2 GiB are not supported");
  ST_CHECK_ARG(((uintptr_t)payload & 3u) == 0, "st_q4_linear_fwd: payload not 4-byte aligned");
  p.Wq = payload; p.Ws = scales; p.ldw = K;
  p.w_bytes = N * K / 2; p.s_bytes = st::cdiv(N * K, 1ll << p.gshift) * 4;
  if (K % (1 << p.gshift) == 0 && al16(payload)) {
    // split-K when the caller brought the workspace the query asks for
    const SplitPlan plan = split_plan(M, N, K);
    if (plan.splits > 1 && workspace && workspace_bytes >= split_workspace(plan, M, N))
      return launch_ws_split<FWD_Q4>(p, plan, workspace, s);
    return run_gemm(FWD_Q4, p, s);
  }
  // flat scale groups straddle W's rows (or 16-byte loads would be misaligned):
  // per-word scales on the 128x128 tile
  return launch<FWD_Q4, 128, 128, 4, 2, true>(p, s);
}

static int dgrad_impl(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                      const uint8_t* payload, const float* scales, int64_t K, const float* lut16,
                      int32_t flags, const float* dt, int64_t lddt, const float* lora_a,
                      int32_t lora_k, uint16_t* dx, int64_t lddx, const uint16_t* gu,
                      int64_t ldgu, void* workspace, int64_t workspace_bytes,
                      st_stream_t stream) {
  ST_CHECK_ARG(M >= 0 && N > 0 && K > 0, "st_q4_linear_dgrad: bad shape");
  if (M == 0) return ST_OK;
  ST_CHECK_ARG(dy && payload && scales && dx && lut16, "st_q4_linear_dgrad: NULL pointer");
  ST_CHECK_ARG(N % 8 == 0, "st_q4_linear_dgrad: N (contraction) must be a multiple of 8, got %lld",
               (long long)N);
  ST_CHECK_ARG(K % 8 == 0, "st_q4_linear_dgrad: K must be a multiple of 8");
  ST_CHECK_ARG(lddy % 8 == 0 && lddy >= N && al16(dy), "st_q4_linear_dgrad: dy rows not 16-byte");
  ST_CHECK_ARG(lddx >= (gu ? 2 * K : K), "st_q4_linear_dgrad: output row stride too small");
  GemmParams p{};
  p.A = dy; p.lda = lddy; p.M = M; p.P = K; p.Q = N;
  p.C = dx; p.ldc = lddx;
  if (gu) {
    ST_CHECK_ARG(ldgu >= 2 * K, "st_q4_linear_dgrad_swiglu: ldgu < 2 * K");
    p.swi_gu = gu; p.swi_ld = ldgu; p.swi_I = K;
  }
  p.hi_first = (flags & ST_FLAG_HI_NIBBLE_FIRST) ? 1 : 0;
  p.gshift = (flags & ST_FLAG_GROUP64) ? 6 : 7;
  for (int i = 0; i < 16; ++i) p.lut.v[i] = lut16[i];
  if (dt) {
    ST_CHECK_ARG(lora_a != nullptr, "st_q4_linear_dgrad: dt without lora_a");
    int rc = check_lora_common(lora_k, lora_k);
    if (rc) return rc;
    ST_CHECK_ARG(lddt >= lora_k, "st_q4_linear_dgrad: lddt too small");
    p.T = dt; p.ldt = lddt; p.L = lora_a; p.ldl = K; p.lora_k = lora_k; p.lora_cols = lora_k;
    p.lora_scale = 1.0f;
  }
  hipStream_t s = (hipStream_t)stream;
  p.a_bytes = ((M - 1) * lddy + N) * 2;
  ST_CHECK_ARG(p.a_bytes < (1ll << 31) && N * K * 2 < (1ll << 31),
               "st_q4_linear_dgrad: operands above 2 GiB are not supported");
  ST_CHECK_ARG(((uintptr_t)payload & 3u) == 0, "st_q4_linear_dgrad: payload not 4-byte aligned");
  p.Wq = payload; p.Ws = scales; p.ldw = K;
  p.w_bytes = N * K / 2; p.s_bytes = st::cdiv(N * K, 1ll << p.gshift) * 4;
  if (K % (1 << p.gshift) == 0) {
    // split-K (not with the SwiGLU VJP) when the caller brought the workspace
    const SplitPlan plan = split_plan(M, K, N);
    if (!gu && plan.splits > 1 && workspace && workspace_bytes >= split_workspace(plan, M, K))
      return launch_ws_split<DGRAD_Q4>(p, plan, workspace, s);
    return run_gemm(DGRAD_Q4, p, s);
  }
  // flat scale groups straddle W's rows: per-word scales on the 128x128 tile
  return launch<DGRAD_Q4, 128, 128, 4, 2, true>(p, s);
}

extern "C" int st_q4_linear_dgrad(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                                  const uint8_t* payload, const float* scales, int64_t K,
                                  const float* lut16, int32_t flags, const float* dt,
                                  int64_t lddt, const float* lora_a, int32_t lora_k,
                                  uint16_t* dx, int64_t lddx, void* workspace,
                                  int64_t workspace_bytes, st_stream_t stream) {
  return dgrad_impl(dy, M, N, lddy, payload, scales, K, lut16, flags, dt, lddt, lora_a, lora_k,
                    dx, lddx, nullptr, 0, workspace, workspace_bytes, stream);
}

extern "C" int st_q4_linear_dgrad_swiglu(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                                         const uint8_t* payload, const float* scales, int64_t I,
                                         const float* lut16, int32_t flags, const float* dt,
                                         int64_t lddt, const float* lora_a, int32_t lora_k,
                                         const uint16_t* gu, int64_t ldgu, uint16_t* dgu,
                                         int64_t lddgu, void* workspace, int64_t workspace_bytes,
                                         st_stream_t stream) {
  ST_CHECK_ARG(gu != nullptr, "st_q4_linear_dgrad_swiglu: NULL gate|up");
  return dgrad_impl(dy, M, N, lddy, payload, scales, I, lut16, flags, dt, lddt, lora_a, lora_k,
                    dgu, lddgu, gu, ldgu, workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------- grouped (MoE)
namespace {
// Grouped (per-expert) launches take the dense kernels' tiles; ST_GROUPED_TILE
// forces one (128, 2562; forward only: the register-operand 2566 = 256x256,
// 2568 = 128x256).
template <int MODE>
int launch_grouped(const GemmParams& p, hipStream_t stream) {
  // default: register-operand 128x256 tiles for the forward (K % 256 == 0;
  // measured 18-22% faster than 128x128 on expert groups of ~64-256 rows),
  // 128x128 otherwise and for the dgrad
  const char* env = getenv("ST_GROUPED_TILE");
  const int t = env ? atoi(env) : (MODE == FWD_Q4 && p.Q % (RB_ST * BK) == 0) ? 2568 : 128;
  if (t == 2562) return launch_ws<MODE>(p, stream);
  if constexpr (MODE == FWD_Q4) {
    // register-operand tiles (K % 256 == 0)
    if (t == 2566 && p.Q % (RB_ST * BK) == 0) return launch_rb<1, 8>(p, stream);
    if (t == 2568 && p.Q % (RB_ST * BK) == 0) return launch_rb<1, 8, 4>(p, stream);
  }
  return launch<MODE, 128, 128, 4>(p, stream);
}
}  // namespace

extern "C" int st_q4_grouped_fwd(const uint16_t* x, int64_t x_rows, int64_t ldx,
                                 const int32_t* gather, int64_t rows, int64_t K,
                                 const int32_t* offsets, int32_t groups, const uint8_t* payload,
                                 const float* scales, int64_t N, const float* lut16, int32_t flags,
                                 const float* t, int64_t ldt, const float* lora_b, int32_t rank,
                                 float lora_scale, int32_t nseg, const int64_t* seg_end,
                                 uint16_t* y, int64_t ldy, st_stream_t stream) {
  ST_CHECK_ARG(rows >= 0 && N > 0 && K > 0 && groups > 0 && x_rows >= 0,
               "st_q4_grouped_fwd: bad shape");
  if (rows == 0) return ST_OK;
  ST_CHECK_ARG(x && offsets && payload && scales && y && lut16, "st_q4_grouped_fwd: NULL pointer");
  ST_CHECK_ARG(K % 128 == 0, "st_q4_grouped_fwd: K must be a multiple of 128, got %lld",
               (long long)K);
  if (flags & ST_FLAG_GROUP64)
    return st::fail(ST_EUNSUPPORTED, "st_q4_grouped_fwd: expert weights take 128-element groups");
  ST_CHECK_ARG(ldx % 8 == 0 && ldx >= K && al16(x) && al16(payload),
               "st_q4_grouped_fwd: x rows / payload must be 16-byte aligned");
  ST_CHECK_ARG(gather || x_rows >= rows, "st_q4_grouped_fwd: x_rows < rows without gather");
  ST_CHECK_ARG(ldy >= N, "st_q4_grouped_fwd: ldy < N");
  GemmParams p{};
  p.A = x; p.lda = ldx; p.M = rows; p.P = N; p.Q = K;
  p.C = y; p.ldc = ldy;
  p.hi_first = (flags & ST_FLAG_HI_NIBBLE_FIRST) ? 1 : 0;
  for (int i = 0; i < 16; ++i) p.lut.v[i] = lut16[i];
  if (t) {
    ST_CHECK_ARG(lora_b != nullptr, "st_q4_grouped_fwd: t without lora_b");
    ST_CHECK_ARG(nseg >= 1 && nseg <= 4 && seg_end, "st_q4_grouped_fwd: nseg must be 1..4");
    int rc = check_lora_common(rank, (int64_t)rank * nseg);
    if (rc) return rc;
    int64_t prev = 0;
    for (int i = 0; i < nseg; ++i) {
      ST_CHECK_ARG(seg_end[i] > prev && (seg_end[i] % 32 == 0 || seg_end[i] == N),
                   "st_q4_grouped_fwd: segment ends must increase and be multiples of 32");
      prev = seg_end[i];
      p.seg_end[i] = seg_end[i];
    }
    ST_CHECK_ARG(prev == N, "st_q4_grouped_fwd: last segment end must equal N");
    ST_CHECK_ARG(ldt >= (int64_t)rank * nseg, "st_q4_grouped_fwd: ldt too small");
    p.T = t; p.ldt = ldt; p.L = lora_b; p.ldl = rank; p.lora_k = rank;
    p.lora_cols = rank * nseg; p.lora_scale = lora_scale; p.nseg = nseg;
    p.l_gstride = N * rank;
  }
  p.a_bytes = ((x_rows - 1) * ldx + K) * 2;
  ST_CHECK_ARG(x_rows > 0 && p.a_bytes < (1ll << 31) && N * K * 2 < (1ll << 31),
               "st_q4_grouped_fwd: operands above 2 GiB are not supported");
  p.gather = gather; p.goff = offsets; p.ngroups = groups;
  p.gshift = 7;
  p.Wq = payload; p.Ws = scales; p.ldw = K;
  p.w_bytes = N * K / 2; p.s_bytes = N * K / 128 * 4;
  p.w_gstride = N * K / 2; p.s_gstride = N * K / 128;
  return launch_grouped<FWD_Q4>(p, (hipStream_t)stream);
}

static int grouped_dgrad_impl(const uint16_t* dy, int64_t lddy, int64_t rows, int64_t N,
                              const int32_t* offsets, int32_t groups, const uint8_t* payload,
                              const float* scales, int64_t K, const float* lut16, int32_t flags,
                              const float* dt, int64_t lddt, const float* lora_a, int32_t lora_k,
                              uint16_t* dx, int64_t lddx, const uint16_t* gu, int64_t ldgu,
                              st_stream_t stream) {
  ST_CHECK_ARG(rows >= 0 && N > 0 && K > 0 && groups > 0, "st_q4_grouped_dgrad: bad shape");
  if (rows == 0) return ST_OK;
  ST_CHECK_ARG(dy && offsets && payload && scales && dx && lut16,
               "st_q4_grouped_dgrad: NULL pointer");
  ST_CHECK_ARG(K % 128 == 0, "st_q4_grouped_dgrad: K must be a multiple of 128");
  if (flags & ST_FLAG_GROUP64)
    return st::fail(ST_EUNSUPPORTED, "st_q4_grouped_dgrad: expert weights take 128-element groups");
  ST_CHECK_ARG(N % 8 == 0, "st_q4_grouped_dgrad: N (contraction) must be a multiple of 8");
  ST_CHECK_ARG(lddy % 8 == 0 && lddy >= N && al16(dy), "st_q4_grouped_dgrad: dy rows not 16-byte");
  ST_CHECK_ARG(((uintptr_t)payload & 3u) == 0, "st_q4_grouped_dgrad: payload not 4-byte aligned");
  ST_CHECK_ARG(lddx >= (gu ? 2 * K : K), "st_q4_grouped_dgrad: output row stride too small");
  GemmParams p{};
  p.A = dy; p.lda = lddy; p.M = rows; p.P = K; p.Q = N;
  p.C = dx; p.ldc = lddx;
  if (gu) {
    ST_CHECK_ARG(ldgu >= 2 * K, "st_q4_grouped_dgrad_swiglu: ldgu < 2 * I");
    p.swi_gu = gu; p.swi_ld = ldgu; p.swi_I = K;
  }
  p.hi_first = (flags & ST_FLAG_HI_NIBBLE_FIRST) ? 1 : 0;
  for (int i = 0; i < 16; ++i) p.lut.v[i] = lut16[i];
  if (dt) {
    ST_CHECK_ARG(lora_a != nullptr, "st_q4_grouped_dgrad: dt without lora_a");
    int rc = check_lora_common(lora_k, lora_k);
    if (rc) return rc;
    ST_CHECK_ARG(lddt >= lora_k, "st_q4_grouped_dgrad: lddt too small");
    p.T = dt; p.ldt = lddt; p.L = lora_a; p.ldl = K; p.lora_k = lora_k; p.lora_cols = lora_k;
    p.lora_scale = 1.0f;
    p.l_gstride = (int64_t)lora_k * K;
  }
  p.a_bytes = ((rows - 1) * lddy + N) * 2;
  ST_CHECK_ARG(p.a_bytes < (1ll << 31) && N * K * 2 < (1ll << 31),
               "st_q4_grouped_dgrad: operands above 2 GiB are not supported");
  p.goff = offsets; p.ngroups = groups;
  p.gshift = 7;
  p.Wq = payload; p.Ws = scales; p.ldw = K;
  p.w_bytes = N * K / 2; p.s_bytes = N * K / 128 * 4;
  p.w_gstride = N * K / 2; p.s_gstride = N * K / 128;
  return launch_grouped<DGRAD_Q4>(p, (hipStream_t)stream);
}

extern "C" int st_q4_grouped_dgrad(const uint16_t* dy, int64_t lddy, int64_t rows, int64_t N,
                                   const int32_t* offsets, int32_t groups, const uint8_t* payload,
                                   const float* scales, int64_t K, const float* lut16,
                                   int32_t flags, const float* dt, int64_t lddt,
                                   const float* lora_a, int32_t lora_k, uint16_t* dx,
                                   int64_t lddx, st_stream_t stream) {
  return grouped_dgrad_impl(dy, lddy, rows, N, offsets, groups, payload, scales, K, lut16, flags,
                            dt, lddt, lora_a, lora_k, dx, lddx, nullptr, 0, stream);
}

// the experts' down-projection input gradient through SwiGLU: dgate|dup of the
// permuted gate|up rows instead of dX (as st_q4_linear_dgrad_swiglu per expert)
extern "C" int st_q4_grouped_dgrad_swiglu(const uint16_t* dy, int64_t lddy, int64_t rows,
                                          int64_t N, const int32_t* offsets, int32_t groups,
                                          const uint8_t* payload, const float* scales, int64_t I,
                                          const float* lut16, int32_t flags, const float* dt,
                                          int64_t lddt, const float* lora_a, int32_t lora_k,
                                          const uint16_t* gu, int64_t ldgu, uint16_t* dgu,
                                          int64_t lddgu, st_stream_t stream) {
  ST_CHECK_ARG(gu != nullptr, "st_q4_grouped_dgrad_swiglu: NULL gate|up");
  return grouped_dgrad_impl(dy, lddy, rows, N, offsets, groups, payload, scales, I, lut16, flags,
                            dt, lddt, lora_a, lora_k, dgu, lddgu, gu, ldgu, stream);
}

// ---------------------------------------------------------------- plain bf16
extern "C" int st_linear_bf16_fwd(const uint16_t* x, int64_t M, int64_t K, int64_t ldx,
                                  const uint16_t* w, int64_t N, int64_t ldw, uint16_t* y,
                                  int64_t ldy, st_stream_t stream) {
  ST_CHECK_ARG(M >= 0 && N > 0 && K > 0, "st_linear_bf16_fwd: bad shape");
  if (M == 0) return ST_OK;
  ST_CHECK_ARG(x && w && y, "st_linear_bf16_fwd: NULL pointer");
  ST_CHECK_ARG(K % 8 == 0 && ldx % 8 == 0 && ldw % 8 == 0 && ldx >= K && ldw >= K && al16(x) &&
                   al16(w) && ldy >= N,
               "st_linear_bf16_fwd: rows must be 16-byte aligned multiples of 8 elements");
  GemmParams p{};
  p.A = x; p.lda = ldx; p.M = M; p.P = N; p.Q = K;
  p.C = y; p.ldc = ldy;
  p.Wb = w; p.ldw = ldw; p.gshift = 7;
  p.a_bytes = ((M - 1) * ldx + K) * 2;
  p.w_bytes = ((N - 1) * ldw + K) * 2;
  ST_CHECK_ARG(p.a_bytes < (1ll << 31) && p.w_bytes < (1ll << 31),
               "st_linear_bf16_fwd: operands above 2 GiB are not supported");
  // 256x256 tiles where they fill the GPU (the terminal's head GEMM over a
  // whole sequence), 128x128 otherwise
  if (st::cdiv(M, 256) * st::cdiv(N, 256) >= 192)
    return launch<FWD_BF16, 256, 256, 8>(p, (hipStream_t)stream);
  return launch<FWD_BF16, 128, 128, 4>(p, (hipStream_t)stream);
}

extern "C" int st_linear_bf16_dgrad(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                                    const uint16_t* w, int64_t K, int64_t ldw, uint16_t* dx,
                                    int64_t lddx, st_stream_t stream) {
  ST_CHECK_ARG(M >= 0 && N > 0 && K > 0, "st_linear_bf16_dgrad: bad shape");
  if (M == 0) return ST_OK;
  ST_CHECK_ARG(dy && w && dx, "st_linear_bf16_dgrad: NULL pointer");
  ST_CHECK_ARG(N % 8 == 0 && K % 8 == 0 && lddy % 8 == 0 && ldw % 8 == 0 && lddy >= N &&
                   ldw >= K && al16(dy) && al16(w) && lddx >= K,
               "st_linear_bf16_dgrad: rows must be 16-byte aligned multiples of 8 elements");
  GemmParams p{};
  p.A = dy; p.lda = lddy; p.M = M; p.P = K; p.Q = N;
  p.C = dx; p.ldc = lddx;
  p.Wb = w; p.ldw = ldw; p.gshift = 7;
  p.a_bytes = ((M - 1) * lddy + N) * 2;
  p.w_bytes = ((N - 1) * ldw + K) * 2;
  ST_CHECK_ARG(p.a_bytes < (1ll << 31) && p.w_bytes < (1ll << 31),
               "st_linear_bf16_dgrad: operands above 2 GiB are not supported");
  // 256x256 tiles where they fill the GPU (measured on the terminal's
  // [4095, 4096] input gradient over vocab 151936: 256x256 ahead of 256x128,
  // 128x256 and 128x128), 128x128 otherwise
  if (st::cdiv(M, 256) * st::cdiv(K, 256) >= 192)
    return launch<DGRAD_BF16, 256, 256, 8>(p, (hipStream_t)stream);
  return launch<DGRAD_BF16, 128, 128, 4>(p, (hipStream_t)stream);
}
