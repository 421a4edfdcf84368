// Fused 4-bit dequant + bf16 MFMA GEMM for the frozen base projections.
//
//   forward  C[M,N]    = X[M,K]  * W[N,K]^T   (+ LoRA, + residual)   lora.py:218-220
//   dgrad    C[M,Kout] = dY[M,N] * W[N,Kout]  (+ LoRA dX term)      autograd of the same
//
// Generic form inside the kernel: C[M,P] = A[M,Q] * B[Q,P], Q = contraction.
// The packed weight is streamed from HBM (0.53 B/element), dequantised in
// registers (codebook in LDS, one fp32 multiply + RNE per element, the exact
// arithmetic of codecs.py:168-170) and written to LDS as bf16, so W never
// exists in HBM as bf16.  Both LDS tiles are stored contraction-contiguous
// (16-byte chunks, XOR swizzled) so one fragment-read path serves both passes:
// the forward dequantises W rows as they lie; the dgrad dequantises 8x8 (or
// 4x8) blocks and writes them transposed.
//
// Tiling: 256 threads = 2x2 waves, BK = 64, LDS double buffered, one barrier
// per k-step.  MFMA v_mfma_f32_32x32x16_bf16 (8 bf16 per lane per operand).
// The LoRA epilogue runs on v_mfma_f32_32x32x2_f32 (fp32 operands and
// accumulation), so the adapter term keeps the reference's fp32 arithmetic.
#include "common.h"

namespace {

constexpr int BK = 64;
constexpr int NT = 256;

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
  float lora_scale;
  int nseg;
  int64_t seg_end[4];
};

// LDS address of 16-byte chunk c (0..7) of tile row `row` (row = 64 bf16).
__device__ __forceinline__ int swz(int row, int c) {
  return row * 8 + (c ^ (row & 7) ^ ((row >> 3) & 7));
}

__device__ __forceinline__ unsigned nib(uint32_t w, int e, int hi_first) {
  return (w >> (4 * (e ^ hi_first))) & 15u;
}

template <int MODE, int BM, int BN>
struct Tile {
  static constexpr int WM = BM / 2, WN = BN / 2;
  static constexpr int FM = WM / 32, FN = WN / 32;
  static constexpr int A_IT = BM * 8 / NT;  // 16-byte chunks per thread
  static constexpr bool Q4 = (MODE == FWD_Q4 || MODE == DGRAD_Q4);
  static constexpr bool DGRAD = (MODE == DGRAD_Q4 || MODE == DGRAD_BF16);
  static constexpr int BF_IT = BN * 8 / NT;  // FWD_BF16 chunks per thread
  static constexpr int BQ_IT = BN * 2 / NT;  // FWD_Q4 16-byte payload loads per thread
  static constexpr int QB = BN / 32;         // dgrad: contraction rows per thread block
  static constexpr int LDS_CHUNKS = 2 * (BM + BN) * 8;
};

template <int MODE, int BM, int BN>
__global__ __launch_bounds__(NT) void gemm_kernel(GemmParams p) {
  using TL = Tile<MODE, BM, BN>;
  constexpr int WM = TL::WM, WN = TL::WN, FM = TL::FM, FN = TL::FN;
  __shared__ uint4 lds[TL::LDS_CHUNKS];
  __shared__ float lut_s[16];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t tiles_p = st::cdiv(p.P, BN);
  const int64_t t = st::xcd_remap(blockIdx.x, gridDim.x);
  const int64_t m0 = (t / tiles_p) * BM, p0 = (t % tiles_p) * BN;
  const int KT = (int)st::cdiv(p.Q, BK);

  if (TL::Q4 && tid < 16) lut_s[tid] = p.lut.v[tid];

  // buffer b: A tile at lds + b*(BM+BN)*8, B tile right after it
  auto As = [&](int b) { return lds + b * (BM + BN) * 8; };
  auto Bs = [&](int b) { return lds + b * (BM + BN) * 8 + BM * 8; };

  // ---- register staging of one k-step ----
  uint4 ra[TL::A_IT];
  uint4 rbw[TL::Q4 ? (TL::DGRAD ? 1 : TL::BQ_IT) : (TL::DGRAD ? TL::QB : TL::BF_IT)];
  uint32_t rqd[TL::DGRAD && TL::Q4 ? TL::QB : 1];
  float rs[TL::Q4 ? (TL::DGRAD ? TL::QB : TL::BQ_IT) : 1];

  auto load_global = [&](int kt) {
    const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < TL::A_IT; ++i) {
      int id = tid + i * NT, row = id >> 3, c = id & 7;
      int64_t m = m0 + row, k = k0 + c * 8;
      ra[i] = (m < p.M && k < p.Q) ? *(const uint4*)(p.A + m * p.lda + k) : make_uint4(0, 0, 0, 0);
    }
    if constexpr (MODE == FWD_Q4) {
#pragma unroll
      for (int i = 0; i < TL::BQ_IT; ++i) {
        int id = tid + i * NT, row = id >> 1, h = id & 1;
        int64_t n = p0 + row, k = k0 + 32 * h;
        if (n < p.P) {
          int64_t e = n * p.ldw + k;
          rbw[i] = *(const uint4*)(p.Wq + (e >> 1));
          rs[i] = p.Ws[e >> 7];
        } else {
          rbw[i] = make_uint4(0x77777777u, 0x77777777u, 0x77777777u, 0x77777777u);
          rs[i] = 0.0f;
        }
      }
    } else if constexpr (MODE == FWD_BF16) {
#pragma unroll
      for (int i = 0; i < TL::BF_IT; ++i) {
        int id = tid + i * NT, row = id >> 3, c = id & 7;
        int64_t n = p0 + row, k = k0 + c * 8;
        rbw[i] = (n < p.P && k < p.Q) ? *(const uint4*)(p.Wb + n * p.ldw + k) : make_uint4(0, 0, 0, 0);
      }
    } else {
      constexpr int PB = BN / 8;
      int pb = tid % PB, qb = tid / PB;
      int64_t pc = p0 + pb * 8;
#pragma unroll
      for (int i = 0; i < TL::QB; ++i) {
        int64_t q = k0 + qb * TL::QB + i;
        bool ok = (pc < p.P) && (q < p.Q);
        if constexpr (MODE == DGRAD_Q4) {
          int64_t e = q * p.ldw + pc;
          rqd[i] = ok ? *(const uint32_t*)(p.Wq + (e >> 1)) : 0x77777777u;
          rs[i] = ok ? p.Ws[e >> 7] : 0.0f;
        } else {
          rbw[i] = ok ? *(const uint4*)(p.Wb + q * p.ldw + pc) : make_uint4(0, 0, 0, 0);
        }
      }
    }
  };

  auto store_lds = [&](int buf) {
    uint4* as = As(buf);
    uint4* bs = Bs(buf);
#pragma unroll
    for (int i = 0; i < TL::A_IT; ++i) {
      int id = tid + i * NT, row = id >> 3, c = id & 7;
      as[swz(row, c)] = ra[i];
    }
    if constexpr (MODE == FWD_Q4) {
#pragma unroll
      for (int i = 0; i < TL::BQ_IT; ++i) {
        int id = tid + i * NT, row = id >> 1, h = id & 1;
        const float s = rs[i];
        uint32_t w4[4] = {rbw[i].x, rbw[i].y, rbw[i].z, rbw[i].w};
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          uint32_t o[4];
#pragma unroll
          for (int e = 0; e < 8; e += 2)
            o[e / 2] = st::pack_bf16x2(lut_s[nib(w4[d], e, p.hi_first)] * s,
                                       lut_s[nib(w4[d], e + 1, p.hi_first)] * s);
          bs[swz(row, 4 * h + d)] = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
    } else if constexpr (MODE == FWD_BF16) {
#pragma unroll
      for (int i = 0; i < TL::BF_IT; ++i) {
        int id = tid + i * NT, row = id >> 3, c = id & 7;
        bs[swz(row, c)] = rbw[i];
      }
    } else {
      constexpr int PB = BN / 8;
      int pb = tid % PB, qb = tid / PB;
      float v[TL::QB][8];
#pragma unroll
      for (int i = 0; i < TL::QB; ++i) {
        if constexpr (MODE == DGRAD_Q4) {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[i][j] = lut_s[nib(rqd[i], j, p.hi_first)] * rs[i];
        } else {
          uint32_t w4[4] = {rbw[i].x, rbw[i].y, rbw[i].z, rbw[i].w};
#pragma unroll
          for (int j = 0; j < 8; ++j)
            v[i][j] = st::bf16_to_f32((uint16_t)(w4[j >> 1] >> (16 * (j & 1))));
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        int prow = pb * 8 + j;
        if constexpr (TL::QB == 8) {
          uint4 o = make_uint4(st::pack_bf16x2(v[0][j], v[1][j]), st::pack_bf16x2(v[2][j], v[3][j]),
                               st::pack_bf16x2(v[4][j], v[5][j]), st::pack_bf16x2(v[6][j], v[7][j]));
          bs[swz(prow, qb)] = o;
        } else {
          uint2 o = make_uint2(st::pack_bf16x2(v[0][j], v[1][j]), st::pack_bf16x2(v[2][j], v[3][j]));
          ((uint2*)&bs[swz(prow, qb >> 1)])[qb & 1] = o;
        }
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  load_global(0);
  __syncthreads();  // lut_s visible before the first dequant
  store_lds(0);
  __syncthreads();

  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_global(kt + 1);
    const uint4* as = As(cur);
    const uint4* bs = Bs(cur);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int c = 2 * s + (lane >> 5);
      bf16x8 a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        a[i] = __builtin_bit_cast(bf16x8, as[swz(wm * WM + i * 32 + (lane & 31), c)]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        b[j] = __builtin_bit_cast(bf16x8, bs[swz(wn * WN + j * 32 + (lane & 31), c)]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) store_lds(cur ^ 1);
    __syncthreads();
  }

  // ---------------- epilogue ----------------
  const bool lora = p.T != nullptr;
  float* Ts = (float*)lds;
  const int tstride = p.lora_cols + 1;
  float* Ls = Ts + BM * tstride;
  const int lstride = TL::DGRAD ? BN : (p.lora_k + 1);
  if (lora) {
    // stage T rows [m0, m0+BM) x [0, lora_cols) and the LoRA right operand
    for (int e = tid; e < BM * p.lora_cols; e += NT) {
      int r = e / p.lora_cols, c = e % p.lora_cols;
      int64_t m = m0 + r;
      Ts[r * tstride + c] = m < p.M ? p.T[m * p.ldt + c] : 0.0f;
    }
    if (TL::DGRAD) {  // L = A_cat [lora_k, P]
      for (int e = tid; e < p.lora_k * BN; e += NT) {
        int r = e / BN, c = e % BN;
        int64_t pc = p0 + c;
        Ls[r * lstride + c] = pc < p.P ? p.L[r * p.ldl + pc] : 0.0f;
      }
    } else {  // L = B_lora [P, rank]
      for (int e = tid; e < BN * p.lora_k; e += NT) {
        int r = e / p.lora_k, c = e % p.lora_k;
        int64_t pc = p0 + r;
        Ls[r * lstride + c] = pc < p.P ? p.L[pc * p.ldl + c] : 0.0f;
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int cl = wn * WN + j * 32;  // tile-local first column of this block
    const int64_t pcol = p0 + cl + (lane & 31);
    int coff = 0;
    if (lora && !TL::DGRAD) {
      int64_t pblk = p0 + cl;
      int s = 0;
      for (int q = 0; q < p.nseg; ++q) s += (p.seg_end[q] <= pblk) ? 1 : 0;
      coff = s * p.lora_k;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int rl = wm * WM + i * 32;
      f32x16 la;
      if (lora) {
#pragma unroll
        for (int v = 0; v < 16; ++v) la[v] = 0.0f;
        for (int kk = 0; kk < p.lora_k; kk += 2) {
          int kx = kk + (lane >> 5);
          float av = Ts[(rl + (lane & 31)) * tstride + coff + kx];
          float bv = TL::DGRAD ? Ls[kx * lstride + cl + (lane & 31)]
                               : Ls[(cl + (lane & 31)) * lstride + kx];
          la = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, la, 0, 0, 0);
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t m = m0 + rl + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
        if (m < p.M && pcol < p.P) {
          float y = st::bf16r(acc[i][j][v]);
          if (lora) {
            if (TL::DGRAD)
              y = st::bf16r(y + st::bf16r(la[v]));
            else
              y = st::bf16r(y + la[v] * p.lora_scale);
          }
          if (p.R) y = st::bf16r(st::bf16_to_f32(p.R[m * p.ldr + pcol]) + y);
          p.C[m * p.ldc + pcol] = st::f32_to_bf16(y);
        }
      }
    }
  }
}

template <int MODE, int BM, int BN>
int launch(const GemmParams& p, hipStream_t stream) {
  int64_t tiles = st::cdiv(p.M, BM) * st::cdiv(p.P, BN);
  if (tiles > 0x7fffffff) return st::fail(ST_EUNSUPPORTED, "q4gemm: too many tiles");
  if (p.T) {  // the LoRA epilogue stages T and the right operand in the tile's LDS
    using TL = Tile<MODE, BM, BN>;
    int64_t need = (int64_t)BM * (p.lora_cols + 1) +
                   (TL::DGRAD ? (int64_t)p.lora_k * BN : (int64_t)BN * (p.lora_k + 1));
    if (need > (int64_t)TL::LDS_CHUNKS * 4)
      return st::fail(ST_EUNSUPPORTED, "q4gemm: LoRA epilogue (%d columns) exceeds tile LDS",
                      p.lora_cols);
  }
  gemm_kernel<MODE, BM, BN><<<(unsigned)tiles, NT, 0, stream>>>(p);
  return st::check_launch("q4gemm");
}

int tile_choice(int64_t M, int64_t P) {
  // 256x256 needs enough tiles to cover the 256 CUs; otherwise 128x128.
  const char* env = getenv("ST_GEMM_TILE");
  if (env) return atoi(env);
  int64_t big = st::cdiv(M, 256) * st::cdiv(P, 256);
  return big >= 256 ? 256 : 128;
}

template <int MODE>
int dispatch(const GemmParams& p, hipStream_t stream) {
  if (tile_choice(p.M, p.P) == 256) return launch<MODE, 256, 256>(p, stream);
  return launch<MODE, 128, 128>(p, stream);
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

namespace st {
int launch_dequant4(const uint8_t* payload, const float* scales, int64_t numel, int32_t group,
                    const float* lut16, int32_t flags, uint16_t* out, hipStream_t stream);
}

extern "C" int64_t st_q4_linear_fwd_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  (void)M;
  return (K % 128 == 0) ? 0 : N * K * 2;
}

extern "C" int64_t st_q4_linear_dgrad_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  (void)M;
  return (K % 128 == 0) ? 0 : N * K * 2;
}

static int check_lora_common(int64_t rank, int64_t cols) {
  if (rank <= 0 || rank % 2 || rank > 64)
    return st::fail(ST_EUNSUPPORTED, "q4 linear: LoRA contraction %lld must be even and <= 64",
                    (long long)rank);
  if (cols > 64)
    return st::fail(ST_EUNSUPPORTED, "q4 linear: %lld LoRA columns exceed 64", (long long)cols);
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
  if (K % 128 == 0 && al16(payload)) {
    p.Wq = payload; p.Ws = scales; p.ldw = K;
    return run_gemm(FWD_Q4, p, s);
  }
  // flat groups straddle rows: decode W once into the workspace, bf16 GEMM
  int64_t need = N * K * 2;
  if (!workspace || workspace_bytes < need)
    return st::fail(ST_EWORKSPACE, "st_q4_linear_fwd: K=%lld needs %lld workspace bytes",
                    (long long)K, (long long)need);
  ST_CHECK_ARG(al16(workspace), "st_q4_linear_fwd: workspace not 16-byte aligned");
  int rc = st::launch_dequant4(payload, scales, N * K, 128, lut16, flags, (uint16_t*)workspace, s);
  if (rc) return rc;
  p.Wb = (const uint16_t*)workspace; p.ldw = K;
  return run_gemm(FWD_BF16, p, s);
}

extern "C" int st_q4_linear_dgrad(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                                  const uint8_t* payload, const float* scales, int64_t K,
                                  const float* lut16, int32_t flags, const float* dt,
                                  int64_t lddt, const float* lora_a, int32_t lora_k,
                                  uint16_t* dx, int64_t lddx, void* workspace,
                                  int64_t workspace_bytes, st_stream_t stream) {
  ST_CHECK_ARG(M >= 0 && N > 0 && K > 0, "st_q4_linear_dgrad: bad shape");
  if (M == 0) return ST_OK;
  ST_CHECK_ARG(dy && payload && scales && dx && lut16, "st_q4_linear_dgrad: NULL pointer");
  ST_CHECK_ARG(N % 8 == 0, "st_q4_linear_dgrad: N (contraction) must be a multiple of 8, got %lld",
               (long long)N);
  ST_CHECK_ARG(K % 8 == 0, "st_q4_linear_dgrad: K must be a multiple of 8");
  ST_CHECK_ARG(lddy % 8 == 0 && lddy >= N && al16(dy), "st_q4_linear_dgrad: dy rows not 16-byte");
  ST_CHECK_ARG(lddx >= K, "st_q4_linear_dgrad: lddx < K");
  GemmParams p{};
  p.A = dy; p.lda = lddy; p.M = M; p.P = K; p.Q = N;
  p.C = dx; p.ldc = lddx;
  p.hi_first = (flags & ST_FLAG_HI_NIBBLE_FIRST) ? 1 : 0;
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
  if (K % 128 == 0) {
    p.Wq = payload; p.Ws = scales; p.ldw = K;
    return run_gemm(DGRAD_Q4, p, s);
  }
  int64_t need = N * K * 2;
  if (!workspace || workspace_bytes < need)
    return st::fail(ST_EWORKSPACE, "st_q4_linear_dgrad: K=%lld needs %lld workspace bytes",
                    (long long)K, (long long)need);
  ST_CHECK_ARG(al16(workspace), "st_q4_linear_dgrad: workspace not 16-byte aligned");
  int rc = st::launch_dequant4(payload, scales, N * K, 128, lut16, flags, (uint16_t*)workspace, s);
  if (rc) return rc;
  p.Wb = (const uint16_t*)workspace; p.ldw = K;
  return run_gemm(DGRAD_BF16, p, s);
}
