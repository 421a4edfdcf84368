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
#include "common.h"

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

extern "C" int64_t st_lora_gemm_workspace_bytes(int64_t Mo, int64_t No, int64_t Kc) {
  if (Mo <= 0 || No <= 0 || Kc <= 0) return 0;
  return (int64_t)ksplit_for(Mo, No, Kc) * Mo * No * 4;
}

extern "C" int st_lora_gemm(int64_t Mo, int64_t No, int64_t Kc, const void* a, int32_t a_dtype,
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
