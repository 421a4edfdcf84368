// Shared device/host helpers for the SpillTune MI355X (gfx950) kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/spilltune_hip.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// 16-entry fp32 codebook passed by value as a kernel argument.
struct Lut16 {
  float v[16];
};

namespace st {

// ---- error reporting (thread-local, read through st_last_error) ----
void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int check_launch(const char* what);

// ---- bf16 helpers ----
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, (uint32_t)h << 16);
}
// Two fp32 -> packed bf16x2 (v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
  return (uint16_t)(pack_bf16x2(x, 0.0f) & 0xffffu);
}
// round an fp32 value through bf16 and back (models a bf16 tensor op result)
__device__ __forceinline__ float bf16r(float x) { return bf16_to_f32(f32_to_bf16(x)); }

// SwiGLU VJP of one element of a = silu(g) * u (bf16 tensors) for the
// upstream value y, with autograd's roundings through bf16 tensors: the silu
// output and the silu-gradient input dsv = y * u are bf16, dg and du are
// returned in fp32 for the caller to round.  The sigmoid uses the hardware
// 2^x and reciprocal (a few fp32 ulp, far below the bf16 resolution of every
// result) instead of a libm exp and two IEEE divisions: the backward runs it
// in GEMM epilogues, where those took most of the VALU time.  Infinite g
// gives torch's NaN/inf results.
__device__ __forceinline__ void swiglu_vjp(float g, float u, float y, float& dg, float& du) {
  const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.44269504088896341f));
  const float sv = bf16r(g * sg);
  const float dsv = bf16r(y * u);
  du = y * sv;
  dg = dsv * (sg * (1.0f + g * (1.0f - sg)));
}

__host__ __device__ __forceinline__ int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Buffer-resource loads: 32-bit byte offsets into a buffer of `bytes` bytes
// (below 2 GiB); an offset at or beyond the extent (kOOB is beyond every one)
// reads as zero, so tiles need no bounds branches.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr uint32_t kOOB = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* ptr, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(ptr), (short)0, (int)bytes,
                                           0x00020000);
}
__device__ __forceinline__ uint4 ld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// Transposed-operand tile: rows n (the contraction) of BN bf16 held as BN/8
// 16-byte chunks, chunk c of row n at n*(BN/8) + (c ^ x(n)).  For BN = 128
// (rows of 256 bytes, each starting at bank 0) x(n) = ((n & 3) << 2) |
// ((n >> 2) & 3), a permutation of n & 15; wider tiles use x(n) = 5*(n & 3).
// The transposing reads below (4 rows x 4 consecutive chunks per half-wave)
// and the 16-byte stores of the dgrad kernels (each lane writes the 4 chunks
// of its 32-column group in an order rotated by that group's index, see
// rot4) are free of bank conflicts with the BN = 128 form (measured with
// SQ_LDS_BANK_CONFLICT; the earlier 5*(n & 3) form cost 8 conflict cycles
// per store instruction).  Index in 16-byte units; BN >= 128.
template <int BN>
__device__ __forceinline__ int trswz(int n, int c) {
  if constexpr (BN == 128)
    return n * 16 + (c ^ (((n & 3) << 2) | ((n >> 2) & 3)));
  else
    return n * (BN / 8) + (c ^ (5 * (n & 3)));
}
// Rotates four words left by r (0..3): w[i] <- w[(i + r) & 3], with selects
// (no dynamic register indexing).
template <typename T>
__device__ __forceinline__ void rot4(T (&w)[4], int r) {
  const bool r2 = r & 2, r1 = r & 1;
  const T a0 = r2 ? w[2] : w[0], a1 = r2 ? w[3] : w[1], a2 = r2 ? w[0] : w[2],
          a3 = r2 ? w[1] : w[3];
  w[0] = r1 ? a1 : a0;
  w[1] = r1 ? a2 : a1;
  w[2] = r1 ? a3 : a2;
  w[3] = r1 ? a0 : a3;
}
// MFMA 32x32x16 operand from such a tile: lane (column kc + lane%32, half
// g = lane/32) gets rows n0 + 8g + s, s = 0..7.  ds_read_b64_tr_b16: within
// 16 lanes, lane i receives element (i % 4) of the 4-element rows supplied
// by lanes 4j + i/4, j = 0..3.
template <int BN>
__device__ __forceinline__ bf16x8 tr_operand(const uint4* bs, int n0, int kc, int lane) {
  typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
  const int G = lane >> 4, i = lane & 15, g = lane >> 5;
  const int col = kc + 16 * (G & 1) + 4 * (i & 3);
  v4bf r[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int n = n0 + 8 * g + 4 * h + (i >> 2);
    const uint16_t* e = (const uint16_t*)(bs + trswz<BN>(n, col >> 3)) + (col & 7);
    r[h] = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) v4bf*)e);
  }
  return __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7);
}

// XCD-aware block remap: consecutive logical tiles land on the same XCD so they
// share that XCD's L2 (blocks are dispatched round-robin over the 8 XCDs).
__device__ __forceinline__ int64_t xcd_remap(int64_t b, int64_t nb) {
  if (nb % 8 != 0) return b;
  return (b % 8) * (nb / 8) + b / 8;
}

// Tile (row tile mt, column tile pt) of logical tile t in a grouped raster:
// logical tiles walk `gm` row tiles for each column tile before the next
// column tile, group after group of gm row tiles (gm <= 1: row-major, the
// column tile fastest).  With xcd_remap, an XCD's consecutive logical tiles
// then cover gm row panels x (its share / gm) column panels, so its L2 serves
// each A panel and each W panel to several of its CUs.
__device__ __forceinline__ void raster(int64_t t, int64_t tiles_m, int64_t tiles_p, int gm,
                                       int64_t& mt, int64_t& pt) {
  if (gm <= 1) {
    mt = t / tiles_p;
    pt = t % tiles_p;
    return;
  }
  const int64_t per = (int64_t)gm * tiles_p;
  const int64_t m0 = t / per * gm, r = t % per;
  const int64_t h = tiles_m - m0 < gm ? tiles_m - m0 : gm;  // rows of a short last group
  mt = m0 + r % h;
  pt = r / h;
}

// Grouped (per-expert) row tiles: group g owns rows [off[g], off[g+1]) and
// cdiv(rows_g, BM) tiles, numbered consecutively over the groups.  Maps tile
// `slot` to its group, first row and the group's row end (clamped to `rows`).
// Every lane of the calling wave gets the same answer; false when `slot` lies
// beyond the last tile.  Offsets are read as given: rows outside [0, rows)
// are clamped, so bad offsets cannot move a tile out of bounds.
__device__ __forceinline__ bool find_group(const int32_t* off, int groups, int BM, int64_t slot,
                                           int64_t rows, int& grp, int64_t& m0, int64_t& mend) {
  const int lane = threadIdx.x & 63;
  int64_t base = 0;
  for (int c = 0; c < groups; c += 64) {
    const int e = c + lane;
    int start = 0, cnt = 0;
    if (e < groups) {
      start = off[e];
      cnt = off[e + 1] - start;
      if (cnt < 0) cnt = 0;
    }
    const int tiles = (cnt + BM - 1) / BM;
    int inc = tiles;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(inc, d);
      if (lane >= d) inc += v;
    }
    const int exc = inc - tiles;
    const bool hit = tiles > 0 && slot >= base + exc && slot < base + inc;
    const unsigned long long b = __ballot(hit);
    if (b) {
      const int src = __ffsll((long long)b) - 1;
      const int64_t s0 = __shfl(start, src), n0 = __shfl(cnt, src), x0 = __shfl(exc, src);
      grp = c + src;
      m0 = s0 + (slot - base - x0) * BM;
      mend = s0 + n0 < rows ? s0 + n0 : rows;
      if (m0 < 0) m0 = 0;
      return true;
    }
    base += __shfl(inc, 63);
  }
  return false;
}

}  // namespace st

#define ST_CHECK_ARG(cond, ...)                           \
  do {                                                    \
    if (!(cond)) return st::fail(ST_EINVAL, __VA_ARGS__); \
  } while (0)
