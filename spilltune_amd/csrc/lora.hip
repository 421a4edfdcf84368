// Rank-r LoRA products with fp32 accumulation (finetune/lora.py:219 and its VJP).
//
//   T  = x_f32 A^T          (Mo = M,    No = r,    Kc = K)
//   dT = s dY_f32 B         (Mo = M,    No = r,    Kc = N)
//   dB = s dY_f32^T T       (Mo = N,    No = r,    Kc = M)
//   dA = dT^T x_f32         (Mo = r,    No = K,    Kc = M)
//
// All four are one strided kernel: out = (acc ? out : 0) + alpha * sum_k a(m,k) b(k,n)
// with a/b either bf16 or fp32.  The contraction is split across blocks into
// fp32 partials in the caller's workspace and summed in a fixed order by a
// second kernel, so results are deterministic run to run.
#include "rank_r.h"

#include <mutex>

namespace {

constexpr int TM = 64, TN = 64, TK = 32, NTH = 256;

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld<uint16_t>(const uint16_t* p, int64_t i) {
  return st::bf16_to_f32(p[i]);
}
template <>
__device__ __forceinline__ float ld<float>(const float* p, int64_t i) {
  return p[i];
}

template <typename TA, typename TB>
__global__ __launch_bounds__(NTH) void lora_partial(int64_t Mo, int64_t No, int64_t Kc,
                                                   const TA* __restrict__ a, int64_t sam,
                                                   int64_t sak, const TB* __restrict__ b,
                                                   int64_t sbk, int64_t sbn, int64_t klen,
                                                   float* __restrict__ part) {
  __shared__ float As[TK][TM + 1];
  __shared__ float Bs[TK][TN + 1];
  const int tid = threadIdx.x, tx = tid % 16, ty = tid / 16;
  const int64_t m0 = (int64_t)blockIdx.x * TM, n0 = (int64_t)blockIdx.y * TN;
  const int64_t kb = (int64_t)blockIdx.z * klen;
  const int64_t ke = kb + klen < Kc ? kb + klen : Kc;
  float acc[4][4] = {};
  for (int64_t k0 = kb; k0 < ke; k0 += TK) {
    for (int e = tid; e < TM * TK; e += NTH) {
      int mm, kk;
      if (sak == 1) { kk = e % TK; mm = e / TK; } else { mm = e % TM; kk = e / TM; }
      int64_t m = m0 + mm, k = k0 + kk;
      As[kk][mm] = (m < Mo && k < ke) ? ld<TA>(a, m * sam + k * sak) : 0.0f;
    }
    for (int e = tid; e < TN * TK; e += NTH) {
      int nn, kk;
      if (sbn == 1) { nn = e % TN; kk = e / TN; } else { kk = e % TK; nn = e / TK; }
      int64_t n = n0 + nn, k = k0 + kk;
      Bs[kk][nn] = (n < No && k < ke) ? ld<TB>(b, k * sbk + n * sbn) : 0.0f;
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < TK; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
  float* dst = part + (int64_t)blockIdx.z * Mo * No;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int64_t m = m0 + ty * 4 + i;
    if (m >= Mo) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int64_t n = n0 + tx * 4 + j;
      if (n < No) dst[m * No + n] = acc[i][j];
    }
  }
}

__global__ __launch_bounds__(NTH) void lora_reduce(int64_t Mo, int64_t No, int ks,
                                                  const float* __restrict__ part, float alpha,
                                                  float* __restrict__ out, int64_t ldo,
                                                  int accumulate) {
  int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= Mo * No) return;
  float s = 0.0f;
  for (int z = 0; z < ks; ++z) s += part[(int64_t)z * Mo * No + e];
  int64_t m = e / No, n = e % No;
  float v = alpha * s;
  if (accumulate) v += out[m * ldo + n];
  out[m * ldo + n] = v;
}

// ---- MFMA path for the LoRA shapes: one bf16 operand G is large, the other
// (S, fp32) has at most 64 columns; st::rk_accumulate (rank_r.h) streams it.
// T = x A^T and dT = dY B are ROW forms (contraction contiguous), dB = dY^T T
// and dA^T = x^T dT COL forms (contraction over G's rows).
using st::RK_BM;
using st::RK_BK;
using st::RK_LD;
using st::RK_RP;
static_assert(st::RK_NTH == NTH, "rank-r tiles run on NTH-thread workgroups");

// One workgroup's share: output rows [tile*RK_BM, +RK_BM) over contraction
// chunk [split*klen, +klen), written to partial slice `split`.
template <bool COL, bool SK1, int NB>
__device__ __forceinline__ void rk_tile(int64_t Mo, int64_t R, int64_t Kc,
                                        const uint16_t* __restrict__ G, int64_t ldg,
                                        int64_t g_bytes, const float* __restrict__ S, int64_t ssk,
                                        int64_t ssj, int64_t s_bytes, int64_t klen,
                                        float* __restrict__ part, int64_t tile, int64_t split,
                                        uint16_t* __restrict__ Gs, uint16_t* __restrict__ Ss) {
  const int64_t m0 = tile * RK_BM;
  const int kb = (int)(split * klen);
  const int ke = (int)(kb + klen < Kc ? kb + klen : Kc);
  f32x16 acc[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.0f;
  st::rk_accumulate<COL, SK1, NB, false>(acc, Mo, R, m0, kb, ke, G, ldg, g_bytes, 0, S, ssk, ssj,
                                         s_bytes, nullptr, 0, nullptr, 0, Gs, Ss);
  float* dst = part + split * Mo * R;
#pragma unroll
  for (int c = 0; c < NB; ++c) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t m = m0 + st::rk_row(v);
      const int j = st::rk_col(c);
      if (m < Mo && j < R) dst[m * R + j] = acc[c][v];
    }
  }
}

// blockIdx.z selects the 64-column chunk [64z, 64z + 64) of the R fp32
// columns; chunk z's partials [ks][Mo][Rz] start at part + z*ks*Mo*64
template <bool COL, bool SK1, int NB>
__global__ __launch_bounds__(NTH) void lora_rk(int64_t Mo, int64_t R, int64_t Kc,
                                              const uint16_t* __restrict__ G, int64_t ldg,
                                              int64_t g_bytes, const float* __restrict__ S,
                                              int64_t ssk, int64_t ssj, int64_t klen, int ks,
                                              float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint16_t Gs[RK_BM * RK_LD];
  __shared__ __attribute__((aligned(16))) uint16_t Ss[st::RK_SS];
  const int64_t c0 = (int64_t)blockIdx.z * RK_RP;
  const int64_t Rc = R - c0 < RK_RP ? R - c0 : RK_RP;
  const int64_t sc_bytes = ((Kc - 1) * ssk + (Rc - 1) * ssj + 1) * 4;
  rk_tile<COL, SK1, NB>(Mo, Rc, Kc, G, ldg, g_bytes, S + c0 * ssj, ssk, ssj, sc_bytes, klen,
                        part + (int64_t)blockIdx.z * ks * Mo * RK_RP, blockIdx.x, blockIdx.y, Gs,
                        Ss);
}

// The whole contraction in one workgroup (no split): output rows
// [blockIdx.x*RK_BM, +RK_BM) and columns [64*blockIdx.z, +64) of
// out[m*so_m + j*so_j] = alpha * sum (+ out when accumulating), written
// directly -- no partials, no reduction launch, every column chunk in the
// same launch.
template <bool COL, bool SK1, int NB>
__global__ __launch_bounds__(NTH) void lora_rk_direct(int64_t Mo, int64_t R, int64_t Kc,
                                                     const uint16_t* __restrict__ G, int64_t ldg,
                                                     int64_t g_bytes, const float* __restrict__ S,
                                                     int64_t ssk, int64_t ssj, float alpha,
                                                     float* __restrict__ out, int64_t so_m,
                                                     int64_t so_j, int accumulate) {
  __shared__ __attribute__((aligned(16))) uint16_t Gs[RK_BM * RK_LD];
  __shared__ __attribute__((aligned(16))) uint16_t Ss[st::RK_SS];
  const int64_t m0 = (int64_t)blockIdx.x * RK_BM, c0 = (int64_t)blockIdx.z * RK_RP;
  const int64_t Rc = R - c0 < RK_RP ? R - c0 : RK_RP;
  const float* Sc = S + c0 * ssj;
  const int64_t sc_bytes = ((Kc - 1) * ssk + (Rc - 1) * ssj + 1) * 4;
  f32x16 acc[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.0f;
  st::rk_accumulate<COL, SK1, NB, false>(acc, Mo, Rc, m0, 0, (int)Kc, G, ldg, g_bytes, 0, Sc, ssk,
                                         ssj, sc_bytes, nullptr, 0, nullptr, 0, Gs, Ss);
#pragma unroll
  for (int c = 0; c < NB; ++c) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t m = m0 + st::rk_row(v);
      const int j = st::rk_col(c);
      if (m < Mo && j < Rc) {
        float* o = out + m * so_m + (c0 + j) * so_j;
        float y = alpha * acc[c][v];
        if (accumulate) y += *o;
        *o = y;
      }
    }
  }
}

// ---- several rank-r products in one launch (the backward of a fused
// projection: dT_s = dY_s B_s and dB_s = dY_s^T T_s for every segment s).
// Each problem is a lora_rk product with its own operands, split count and
// partial slice; workgroup b runs problem p when wg0[p] <= b < wg0[p+1], and
// one reduction launch sums every problem's partials into its output.
constexpr int RK_MAXP = 16;
struct RkProblem {
  const uint16_t* G;
  const float* S;
  float* part;   // [ks][big][R]
  float* out;    // out[m*so_m + j*so_j] (+)= alpha * sum
  int64_t ldg, g_bytes, ssk, ssj, s_bytes, big, R, Kc, klen, so_m, so_j;
  int64_t wg0, e0;  // first workgroup / first reduction element of the problem
  int col, tiles, ks, acc;
  float alpha;
};
struct RkBatch {
  RkProblem p[RK_MAXP];
  int n;
  int64_t wgs, elems;
};

__device__ __forceinline__ int rk_find(const RkBatch& b, int64_t v, bool by_elem) {
  int i = 0;
#pragma unroll
  for (int q = 1; q < RK_MAXP; ++q)
    if (q < b.n && v >= (by_elem ? b.p[q].e0 : b.p[q].wg0)) i = q;
  return i;
}

template <int NB>
__global__ __launch_bounds__(NTH) void lora_rk_batch(const RkBatch b) {
  __shared__ __attribute__((aligned(16))) uint16_t Gs[RK_BM * RK_LD];
  __shared__ __attribute__((aligned(16))) uint16_t Ss[st::RK_SS];
  const int i = rk_find(b, blockIdx.x, false);
  const RkProblem& q = b.p[i];
  const int64_t w = blockIdx.x - q.wg0;
  const int64_t tile = w % q.tiles, split = w / q.tiles;
  if (q.col)
    rk_tile<true, false, NB>(q.big, q.R, q.Kc, q.G, q.ldg, q.g_bytes, q.S, q.ssk, q.ssj,
                             q.s_bytes, q.klen, q.part, tile, split, Gs, Ss);
  else
    rk_tile<false, false, NB>(q.big, q.R, q.Kc, q.G, q.ldg, q.g_bytes, q.S, q.ssk, q.ssj,
                              q.s_bytes, q.klen, q.part, tile, split, Gs, Ss);
}

// p[0] + p[st] + ... + p[(ks-1)*st], summed in ascending split order (a
// fixed order: deterministic); sixteen loads in flight per batch, so the
// usual 16 splits cost one memory round trip
__device__ __forceinline__ float sum_splits(const float* __restrict__ p, int64_t st, int ks) {
  float s = 0.0f;
  int q = 0;
  for (; q + 16 <= ks; q += 16) {
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = p[(q + u) * st];
#pragma unroll
    for (int u = 0; u < 16; ++u) s += v[u];
  }
  if (q + 8 <= ks) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = p[(q + u) * st];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
    q += 8;
  }
  for (; q < ks; ++q) s += p[q * st];
  return s;
}

// sums each problem's partials in ascending split order (as lora_rk_reduce)
__global__ __launch_bounds__(NTH) void lora_rk_reduce_batch(const RkBatch b) {
  const int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= b.elems) return;
  const RkProblem& q = b.p[rk_find(b, e, true)];
  const int64_t le = e - q.e0;
  const float s = sum_splits(q.part + le, q.big * q.R, q.ks);
  const int64_t m = le / q.R, j = le % q.R;
  float v = q.alpha * s;
  float* o = q.out + m * q.so_m + j * q.so_j;
  if (q.acc) v += *o;
  *o = v;
}

// sums the split-K partials into out[m*so_m + j*so_j] (+ out): column j of
// chunk z = j/64 reads [ks][Mo][Rz] at part + z*ks*Mo*64 (Rz = its width)
__global__ __launch_bounds__(NTH) void lora_rk_reduce(int64_t Mo, int64_t R, int ks,
                                                     const float* __restrict__ part, float alpha,
                                                     float* __restrict__ out, int64_t so_m,
                                                     int64_t so_j, int accumulate) {
  int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= Mo * R) return;
  const int64_t m = e / R, j = e % R;
  const int64_t z = j / RK_RP, jz = j % RK_RP;
  const int64_t Rz = R - z * RK_RP < RK_RP ? R - z * RK_RP : RK_RP;
  const float s = sum_splits(part + z * ks * Mo * RK_RP + m * Rz + jz, Mo * Rz, ks);
  float v = alpha * s;
  float* o = out + m * so_m + j * so_j;
  if (accumulate) v += *o;
  *o = v;
}

int rk_ksplit(int64_t Mo, int64_t Kc) {
  // enough workgroups (512) to keep loads in flight on every CU, each
  // streaming at least `chunk` contraction elements
  constexpr int target = 512, chunk = 256;
  int64_t tiles = st::cdiv(Mo, RK_BM);
  int64_t ks = st::cdiv(target, tiles);
  int64_t maxk = st::cdiv(Kc, chunk);
  if (ks > maxk) ks = maxk;
  if (ks < 1) ks = 1;
  return (int)ks;
}

int ksplit_for(int64_t Mo, int64_t No, int64_t Kc) {
  int64_t tiles = st::cdiv(Mo, TM) * st::cdiv(No, TN);
  int64_t ks = st::cdiv(1024, tiles);
  int64_t maxk = st::cdiv(Kc, 256);
  if (ks > maxk) ks = maxk;
  if (ks < 1) ks = 1;
  if (ks > 4096) ks = 4096;
  return (int)ks;
}

template <typename TA, typename TB>
void launch_partial(int64_t Mo, int64_t No, int64_t Kc, const void* a, int64_t sam, int64_t sak,
                    const void* b, int64_t sbk, int64_t sbn, int ks, float* part,
                    hipStream_t s) {
  int64_t klen = st::cdiv(st::cdiv(Kc, ks), TK) * TK;
  dim3 grid((unsigned)st::cdiv(Mo, TM), (unsigned)st::cdiv(No, TN), (unsigned)ks);
  lora_partial<TA, TB><<<grid, NTH, 0, s>>>(Mo, No, Kc, (const TA*)a, sam, sak, (const TB*)b,
                                            sbk, sbn, klen, part);
}

}  // namespace

// Workspace of one st_lora_gemm: the generic kernel's partials or the
// streaming kernel's; `all_chunks` sizes the latter for every 64-column
// chunk in one launch (preferred), else for one chunk at a time (the least
// the call accepts).
static int64_t lora_gemm_workspace(int64_t Mo, int64_t No, int64_t Kc, bool all_chunks) {
  if (Mo <= 0 || No <= 0 || Kc <= 0) return 0;
  int64_t generic = (int64_t)ksplit_for(Mo, No, Kc) * Mo * No * 4;
  int64_t big = Mo > No ? Mo : No, small = Mo > No ? No : Mo;
  int64_t cols = small <= 64 ? small : all_chunks ? st::cdiv(small, 64) * 64 : 64;
  int64_t rk = (int64_t)rk_ksplit(big, Kc) * big * cols * 4;
  return generic > rk ? generic : rk;
}

extern "C" int64_t st_lora_gemm_workspace_bytes(int64_t Mo, int64_t No, int64_t Kc) {
  return lora_gemm_workspace(Mo, No, Kc, true);
}

namespace {

int lora_gemm_impl(int64_t Mo, int64_t No, int64_t Kc, const void* a, int32_t a_dtype,
                   int64_t sam, int64_t sak, const void* b, int32_t b_dtype, int64_t sbk,
                   int64_t sbn, float alpha, float* out, int64_t ldo, int32_t accumulate,
                   void* workspace, int64_t workspace_bytes, st_stream_t stream) {
  ST_CHECK_ARG(Mo >= 0 && No >= 0 && Kc >= 0, "st_lora_gemm: negative shape");
  if (Mo == 0 || No == 0) return ST_OK;
  ST_CHECK_ARG(out && ldo >= No, "st_lora_gemm: bad output");
  ST_CHECK_ARG((a_dtype == ST_DTYPE_BF16 || a_dtype == ST_DTYPE_F32) &&
                   (b_dtype == ST_DTYPE_BF16 || b_dtype == ST_DTYPE_F32),
               "st_lora_gemm: dtype codes must be ST_DTYPE_BF16 or ST_DTYPE_F32");
  hipStream_t s = (hipStream_t)stream;
  if (Kc == 0) {  // empty contraction: out = acc ? out : 0, via the reduce kernel
    lora_reduce<<<(unsigned)st::cdiv(Mo * No, NTH), NTH, 0, s>>>(Mo, No, 0, nullptr, alpha, out,
                                                                 ldo, accumulate);
    return st::check_launch("lora_reduce");
  }
  ST_CHECK_ARG(a && b, "st_lora_gemm: NULL operand");
  // fp32-MFMA path: the bf16 operand is contiguous along one of its dims; the
  // fp32 operand's output columns run 64 at a time (one launch pair each).
  {
    const uint16_t* G = nullptr;
    const float* S = nullptr;
    int64_t ldg = 0, ssk = 0, ssj = 0, big = 0, small = 0, so_m = 0, so_j = 0;
    int col = -1;
    if (a_dtype == ST_DTYPE_BF16 && b_dtype == ST_DTYPE_F32) {
      G = (const uint16_t*)a; S = (const float*)b; ssk = sbk; ssj = sbn;
      big = Mo; small = No; so_m = ldo; so_j = 1;
      if (sak == 1) { col = 0; ldg = sam; } else if (sam == 1) { col = 1; ldg = sak; }
    } else if (a_dtype == ST_DTYPE_F32 && b_dtype == ST_DTYPE_BF16) {
      // out^T[n, m] = sum_k b(k, n) a(m, k)
      G = (const uint16_t*)b; S = (const float*)a; ssk = sak; ssj = sam;
      big = No; small = Mo; so_m = 1; so_j = ldo;
      if (sbk == 1) { col = 0; ldg = sbn; } else if (sbn == 1) { col = 1; ldg = sbk; }
    }
    // the streaming kernel takes 16-byte vector rows and 32-bit buffer offsets
    const int64_t g_bytes = col ? ((Kc - 1) * ldg + big) * 2 : ((big - 1) * ldg + Kc) * 2;
    const int64_t s_bytes = ((Kc - 1) * ssk + (small - 1) * ssj + 1) * 4;
    const bool vec = ((uintptr_t)G & 15u) == 0 && ldg % 8 == 0 && (col ? big : Kc) % 8 == 0 &&
                     ssk >= 0 && ssj >= 0 && g_bytes < (1ll << 31) && s_bytes < (1ll << 31);
    if (col >= 0 && vec) {
      const int ks = rk_ksplit(big, Kc);
      const int64_t nchunk = st::cdiv(small, RK_RP);
      // no split when the contraction is short or the row tiles and column
      // chunks alone give every CU a few workgroups
      if (ks == 1 || st::cdiv(big, RK_BM) * nchunk >= 512) {
        // one workgroup per row tile and column chunk, no partials
        const dim3 grid((unsigned)st::cdiv(big, RK_BM), 1u, (unsigned)st::cdiv(small, RK_RP));
        auto go = [&](auto kern) {
          kern<<<grid, NTH, 0, s>>>(big, small, Kc, G, ldg, g_bytes, S, ssk, ssj, alpha, out,
                                    so_m, so_j, accumulate);
        };
        const bool sk1 = ssk == 1, nb2 = small > 32;
        if (col) {
          if (sk1) nb2 ? go(lora_rk_direct<true, true, 2>) : go(lora_rk_direct<true, true, 1>);
          else nb2 ? go(lora_rk_direct<true, false, 2>) : go(lora_rk_direct<true, false, 1>);
        } else {
          if (sk1) nb2 ? go(lora_rk_direct<false, true, 2>) : go(lora_rk_direct<false, true, 1>);
          else nb2 ? go(lora_rk_direct<false, false, 2>) : go(lora_rk_direct<false, false, 1>);
        }
        return st::check_launch("lora_rk_direct");
      }
      // every 64-column chunk in one launch when the workspace holds all
      // their partials, else chunk by chunk through one chunk's partials
      const int64_t one = (int64_t)ks * big * (small < 64 ? small : 64) * 4;
      const int64_t all = (int64_t)ks * big * nchunk * RK_RP * 4;
      const bool together = nchunk == 1 || (workspace && workspace_bytes >= all);
      if (!workspace || workspace_bytes < one)
        return st::fail(ST_EWORKSPACE, "st_lora_gemm: needs %lld workspace bytes", (long long)one);
      const int64_t klen = st::cdiv(st::cdiv(Kc, ks), RK_BK) * RK_BK;
      float* part = (float*)workspace;
      for (int64_t c0 = 0; c0 < small; c0 += together ? small : 64) {
        const int64_t sc = together ? small : (small - c0 < 64 ? small - c0 : 64);
        const float* Sc = S + c0 * ssj;
        const dim3 grid((unsigned)st::cdiv(big, RK_BM), (unsigned)ks,
                        (unsigned)st::cdiv(sc, RK_RP));
        auto go = [&](auto kern) {
          kern<<<grid, NTH, 0, s>>>(big, sc, Kc, G, ldg, g_bytes, Sc, ssk, ssj, klen, ks, part);
        };
        const bool sk1 = ssk == 1, nb2 = sc > 32;
        if (col) {
          if (sk1) nb2 ? go(lora_rk<true, true, 2>) : go(lora_rk<true, true, 1>);
          else nb2 ? go(lora_rk<true, false, 2>) : go(lora_rk<true, false, 1>);
        } else {
          if (sk1) nb2 ? go(lora_rk<false, true, 2>) : go(lora_rk<false, true, 1>);
          else nb2 ? go(lora_rk<false, false, 2>) : go(lora_rk<false, false, 1>);
        }
        int rc = st::check_launch("lora_rk");
        if (rc) return rc;
        lora_rk_reduce<<<(unsigned)st::cdiv(big * sc, NTH), NTH, 0, s>>>(
            big, sc, ks, part, alpha, out + c0 * so_j, so_m, so_j, accumulate);
        rc = st::check_launch("lora_rk_reduce");
        if (rc) return rc;
      }
      return ST_OK;
    }
  }
  int ks = ksplit_for(Mo, No, Kc);
  int64_t need = (int64_t)ks * Mo * No * 4;
  if (!workspace || workspace_bytes < need)
    return st::fail(ST_EWORKSPACE, "st_lora_gemm: needs %lld workspace bytes", (long long)need);
  float* part = (float*)workspace;
  if (a_dtype == ST_DTYPE_BF16 && b_dtype == ST_DTYPE_F32)
    launch_partial<uint16_t, float>(Mo, No, Kc, a, sam, sak, b, sbk, sbn, ks, part, s);
  else if (a_dtype == ST_DTYPE_F32 && b_dtype == ST_DTYPE_BF16)
    launch_partial<float, uint16_t>(Mo, No, Kc, a, sam, sak, b, sbk, sbn, ks, part, s);
  else if (a_dtype == ST_DTYPE_F32 && b_dtype == ST_DTYPE_F32)
    launch_partial<float, float>(Mo, No, Kc, a, sam, sak, b, sbk, sbn, ks, part, s);
  else
    launch_partial<uint16_t, uint16_t>(Mo, No, Kc, a, sam, sak, b, sbk, sbn, ks, part, s);
  int rc = st::check_launch("lora_partial");
  if (rc) return rc;
  lora_reduce<<<(unsigned)st::cdiv(Mo * No, NTH), NTH, 0, s>>>(Mo, No, ks, part, alpha, out, ldo,
                                                               accumulate);
  return st::check_launch("lora_reduce");
}

// Scratch of the allocation-free variant: the split-K partials live in this
// file-scope device array (one copy per GPU, held until the process ends).
// Host code never passes `scratch` itself to a kernel -- on the host the name
// is only a stand-in -- but the device address hipGetSymbolAddress returns,
// fetched once per device and kept in scratch_ptr.
constexpr int64_t kScratchBytes = 32ll << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) unsigned char scratch[kScratchBytes];
void* scratch_ptr[kMaxDevices];
std::mutex scratch_mu;

int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return st::fail(ST_EDEVICE, "st_lora_gemm_noalloc: hipGetDevice: %s",
                                       hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return st::fail(ST_EUNSUPPORTED, "st_lora_gemm_noalloc: device %d beyond %d", dev,
                    kMaxDevices);
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return st::fail(ST_EDEVICE, "st_lora_gemm_noalloc: hipGetSymbolAddress: %s",
                      hipGetErrorString(e));
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return ST_OK;
}

}  // namespace

extern "C" int st_lora_gemm(int64_t Mo, int64_t No, int64_t Kc, const void* a, int32_t a_dtype,
                            int64_t sam, int64_t sak, const void* b, int32_t b_dtype, int64_t sbk,
                            int64_t sbn, float alpha, float* out, int64_t ldo, int32_t accumulate,
                            void* workspace, int64_t workspace_bytes, st_stream_t stream) {
  return lora_gemm_impl(Mo, No, Kc, a, a_dtype, sam, sak, b, b_dtype, sbk, sbn, alpha, out, ldo,
                        accumulate, workspace, workspace_bytes, stream);
}

extern "C" int st_lora_gemm_noalloc(int64_t Mo, int64_t No, int64_t Kc, const void* a,
                                    int32_t a_dtype, int64_t sam, int64_t sak, const void* b,
                                    int32_t b_dtype, int64_t sbk, int64_t sbn, float alpha,
                                    float* out, int64_t ldo, int32_t accumulate,
                                    st_stream_t stream) {
  ST_CHECK_ARG(Mo >= 0 && No >= 0 && Kc >= 0, "st_lora_gemm_noalloc: negative shape");
  // the least workspace the product accepts (chunk by chunk if need be)
  const int64_t need = lora_gemm_workspace(Mo, No, Kc, false);
  if (need > kScratchBytes)
    return st::fail(ST_EUNSUPPORTED,
                    "st_lora_gemm_noalloc: the product needs %lld scratch bytes, more than the "
                    "%lld-byte static scratch (use st_lora_gemm with a workspace)",
                    (long long)need, (long long)kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_for_current_device(&ws)) return rc;
  }
  return lora_gemm_impl(Mo, No, Kc, a, a_dtype, sam, sak, b, b_dtype, sbk, sbn, alpha, out, ldo,
                        accumulate, ws, kScratchBytes, stream);
}

// ------------------------------------------- backward rank-r products of dY
namespace {

// Problems 2s (dT_s, ROW over dY's segment columns) and 2s+1 (dB_s, COL over
// dY's rows) for segment s; pointers are filled only when `fill` is set.
// Returns the partial floats needed, or -1 when an operand breaks the
// streaming kernel's layout rules (16-byte rows, 32-bit offsets).
int64_t plan_bwd_dy(RkBatch& b, bool fill, const uint16_t* dy, int64_t M, int64_t N,
                    int64_t lddy, const float* B, const float* T, int64_t ldt, int r, int nseg,
                    const int64_t* seg_end, float scale, float* dt, int64_t lddt, float* db,
                    float* part, bool with_db = true) {
  b = RkBatch{};
  const int per = with_db ? 2 : 1;
  b.n = per * nseg;
  int64_t wgs = 0, elems = 0, floats = 0, start = 0;
  for (int s = 0; s < nseg; ++s) {
    const int64_t width = seg_end[s] - start;
    for (int h = 0; h < per; ++h) {
      RkProblem& q = b.p[per * s + h];
      q.col = h;
      q.R = r;
      q.big = h ? width : M;
      q.Kc = h ? M : width;
      q.ldg = lddy;
      q.g_bytes = ((M - 1) * lddy + width) * 2;
      q.ssk = h ? ldt : r;
      q.ssj = 1;
      q.s_bytes = h ? ((M - 1) * ldt + (int64_t)(s + 1) * r - (int64_t)s * r) * 4 : width * r * 4;
      q.so_m = h ? r : lddt;
      q.so_j = 1;
      q.alpha = scale;
      q.tiles = (int)st::cdiv(q.big, RK_BM);
      q.ks = rk_ksplit(q.big, q.Kc);
      q.klen = st::cdiv(st::cdiv(q.Kc, q.ks), RK_BK) * RK_BK;
      q.wg0 = wgs;
      q.e0 = elems;
      const bool vec = (start % 8) == 0 && lddy % 8 == 0 && (h ? width : width) % 8 == 0 &&
                       q.g_bytes < (1ll << 31) && q.s_bytes < (1ll << 31);
      if (!vec) return -1;
      if (fill) {
        q.G = dy + start;
        q.S = h ? T + (int64_t)s * r : B + start * r;
        q.out = h ? db + start * r : dt + (int64_t)s * r;
        q.part = part + floats;
      }
      wgs += (int64_t)q.tiles * q.ks;
      elems += q.big * q.R;
      floats += (int64_t)q.ks * q.big * q.R;
    }
    start = seg_end[s];
  }
  b.wgs = wgs;
  b.elems = elems;
  return floats;
}

int check_segments(int64_t N, int32_t nseg, const int64_t* seg_end) {
  if (nseg < 1 || nseg > RK_MAXP / 2 || !seg_end)
    return st::fail(ST_EINVAL, "st_lora_bwd_dy: nseg must be 1..%d", RK_MAXP / 2);
  int64_t prev = 0;
  for (int i = 0; i < nseg; ++i) {
    if (seg_end[i] <= prev) return st::fail(ST_EINVAL, "st_lora_bwd_dy: segment ends must increase");
    prev = seg_end[i];
  }
  if (prev != N) return st::fail(ST_EINVAL, "st_lora_bwd_dy: last segment end must equal N");
  return ST_OK;
}

}  // namespace

extern "C" int64_t st_lora_bwd_dy_workspace_bytes(int64_t M, int64_t N, int32_t rank,
                                                  int32_t nseg, const int64_t* seg_end) {
  if (M <= 0 || N <= 0 || rank <= 0 || rank > 64 || check_segments(N, nseg, seg_end)) return 0;
  RkBatch b;
  const int64_t floats = plan_bwd_dy(b, false, nullptr, M, N, N, nullptr, nullptr,
                                     (int64_t)nseg * rank, rank, nseg, seg_end, 1.0f, nullptr, 0,
                                     nullptr, nullptr);
  return floats < 0 ? 0 : floats * 4;
}

extern "C" int st_lora_bwd_dy(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                              const float* b, const float* t, int64_t ldt, int32_t rank,
                              int32_t nseg, const int64_t* seg_end, float scale, float* dt,
                              int64_t lddt, float* db, void* workspace, int64_t workspace_bytes,
                              st_stream_t stream) {
  ST_CHECK_ARG(M >= 0 && N > 0, "st_lora_bwd_dy: bad shape");
  ST_CHECK_ARG(rank >= 1 && rank <= 64, "st_lora_bwd_dy: rank must be 1..64");
  if (int rc = check_segments(N, nseg, seg_end)) return rc;
  if (M == 0) return ST_OK;
  ST_CHECK_ARG(dy && b && t && dt, "st_lora_bwd_dy: NULL pointer");
  ST_CHECK_ARG(lddy >= N && ldt >= (int64_t)nseg * rank && lddt >= (int64_t)nseg * rank,
               "st_lora_bwd_dy: leading dimension too small");
  ST_CHECK_ARG(((uintptr_t)dy & 15u) == 0, "st_lora_bwd_dy: dy must be 16-byte aligned");
  RkBatch bt;
  // db == NULL: the dT products only (the caller forms dB elsewhere)
  const int64_t floats = plan_bwd_dy(bt, true, dy, M, N, lddy, b, t, ldt, rank, nseg, seg_end,
                                     scale, dt, lddt, db, (float*)workspace, db != nullptr);
  if (floats < 0)
    return st::fail(ST_EUNSUPPORTED,
                    "st_lora_bwd_dy: segments need 8-element-aligned starts and widths, "
                    "rows a multiple of 8 and operands below 2 GiB");
  if (!workspace || workspace_bytes < floats * 4)
    return st::fail(ST_EWORKSPACE, "st_lora_bwd_dy: needs %lld workspace bytes",
                    (long long)(floats * 4));
  ST_CHECK_ARG(bt.wgs <= 0x7fffffff, "st_lora_bwd_dy: too many workgroups");
  hipStream_t s = (hipStream_t)stream;
  if (rank > 32)
    lora_rk_batch<2><<<(unsigned)bt.wgs, NTH, 0, s>>>(bt);
  else
    lora_rk_batch<1><<<(unsigned)bt.wgs, NTH, 0, s>>>(bt);
  int rc = st::check_launch("lora_rk_batch");
  if (rc) return rc;
  lora_rk_reduce_batch<<<(unsigned)st::cdiv(bt.elems, NTH), NTH, 0, s>>>(bt);
  return st::check_launch("lora_rk_reduce_batch");
}

// ------------------------------------------------ batched independent products
namespace {

// One st_rk_product as a streaming-kernel problem; false when its operands
// break the kernel's layout rules (16-byte G rows, 32-bit offsets, r <= 64).
bool rk_problem(const st_rk_product& x, RkProblem& q) {
  q = RkProblem{};
  if (x.big <= 0 || x.r <= 0 || x.r > 64 || x.Kc <= 0 || !x.G || !x.S || !x.out) return false;
  q.G = x.G;
  q.S = x.S;
  q.out = x.out;
  q.col = x.col ? 1 : 0;
  q.ldg = x.ldg;
  q.ssk = x.ssk;
  q.ssj = x.ssj;
  q.big = x.big;
  q.R = x.r;
  q.Kc = x.Kc;
  q.so_m = x.so_m;
  q.so_j = x.so_j;
  q.alpha = x.alpha;
  q.acc = x.accumulate ? 1 : 0;
  q.g_bytes = q.col ? ((x.Kc - 1) * x.ldg + x.big) * 2 : ((x.big - 1) * x.ldg + x.Kc) * 2;
  q.s_bytes = ((x.Kc - 1) * x.ssk + (x.r - 1) * x.ssj + 1) * 4;
  q.tiles = (int)st::cdiv(x.big, RK_BM);
  q.ks = rk_ksplit(x.big, x.Kc);
  q.klen = st::cdiv(st::cdiv(x.Kc, q.ks), RK_BK) * RK_BK;
  return ((uintptr_t)x.G & 15u) == 0 && x.ldg % 8 == 0 && (q.col ? x.big : x.Kc) % 8 == 0 &&
         x.ssk >= 0 && x.ssj >= 0 && q.g_bytes < (1ll << 31) && q.s_bytes < (1ll << 31);
}

// plans a batch; returns the partial floats needed, or -1 for a bad problem
int64_t plan_batch(RkBatch& b, int32_t n, const st_rk_product* p, float* part) {
  b = RkBatch{};
  b.n = n;
  int64_t wgs = 0, elems = 0, floats = 0;
  for (int i = 0; i < n; ++i) {
    RkProblem& q = b.p[i];
    if (!rk_problem(p[i], q)) return -1;
    q.wg0 = wgs;
    q.e0 = elems;
    q.part = part ? part + floats : nullptr;
    wgs += (int64_t)q.tiles * q.ks;
    elems += q.big * q.R;
    floats += (int64_t)q.ks * q.big * q.R;
  }
  b.wgs = wgs;
  b.elems = elems;
  return floats;
}

}  // namespace

extern "C" int64_t st_rk_batch_workspace_bytes(int32_t n, const st_rk_product* products) {
  if (n <= 0 || n > RK_MAXP || !products) return 0;
  RkBatch b;
  const int64_t floats = plan_batch(b, n, products, nullptr);
  return floats < 0 ? 0 : floats * 4;
}

extern "C" int st_rk_batch(int32_t n, const st_rk_product* products, void* workspace,
                           int64_t workspace_bytes, st_stream_t stream) {
  ST_CHECK_ARG(n >= 0 && n <= RK_MAXP, "st_rk_batch: 0..%d products per call", RK_MAXP);
  if (n == 0) return ST_OK;
  ST_CHECK_ARG(products != nullptr, "st_rk_batch: NULL product list");
  RkBatch b;
  const int64_t floats = plan_batch(b, n, products, (float*)workspace);
  if (floats < 0)
    return st::fail(ST_EUNSUPPORTED,
                    "st_rk_batch: a product breaks the streaming kernel's rules (16-byte "
                    "aligned bf16 rows of multiples of 8, r <= 64, operands below 2 GiB)");
  if (!workspace || workspace_bytes < floats * 4)
    return st::fail(ST_EWORKSPACE, "st_rk_batch: needs %lld workspace bytes",
                    (long long)(floats * 4));
  ST_CHECK_ARG(b.wgs <= 0x7fffffff && b.elems <= 0x7fffffffll * NTH,
               "st_rk_batch: too many workgroups");
  bool wide = false;
  for (int i = 0; i < n; ++i) wide = wide || b.p[i].R > 32;
  hipStream_t s = (hipStream_t)stream;
  if (wide)
    lora_rk_batch<2><<<(unsigned)b.wgs, NTH, 0, s>>>(b);
  else
    lora_rk_batch<1><<<(unsigned)b.wgs, NTH, 0, s>>>(b);
  int rc = st::check_launch("lora_rk_batch");
  if (rc) return rc;
  lora_rk_reduce_batch<<<(unsigned)st::cdiv(b.elems, NTH), NTH, 0, s>>>(b);
  return st::check_launch("lora_rk_reduce_batch");
}
