// Standalone 4-bit -> bf16 dequantisation (HBM-bound).
//
// Replaces the chunked torch decode of codecs.py:158-170 (int4-sym-g128) and
// the NF4 decode inside bitsandbytes (nf4_backend.py:312).  One fp32 multiply
// then RNE to bf16 per element: bit-identical to codecs.py:168-170.
//
// Default kernel (dequant4_word): one packed word = 8 consecutive elements per
// lane per step (a word never straddles a group of 64/128), decoded through
// the per-scale v_perm table of decode4.h and written as one 16-byte store, so
// each store instruction of a wave writes 1 KiB of whole cache lines.  A
// payload that is not 4-byte aligned or an output that is not 16-byte aligned
// takes the element-wise kernel.
// Per element: 0.5 B read + 2 B written (+4/group B scale).
#include <algorithm>

#include "common.h"
#include "decode4.h"

namespace {

constexpr int kThreads = 256;

// Register-table form, one packed word (8 codes) per lane per step: every
// 4-byte load instruction of a wave reads 256 contiguous bytes and every
// 16-byte store writes 1 KiB in one piece (whole cache lines, where the
// 64-byte-per-lane form leaves each store instruction 16 bytes per 64).
// Each lane builds the v_perm table of its word's scale (decode4.h): the
// same bf16_rne(codebook[c] * s) as the reference.  A workgroup covers
// RW consecutive words per lane (4 KiB of payload per 256 threads at RW=4).
constexpr int RW = 4;
template <bool HI>
__global__ __launch_bounds__(kThreads) void dequant4_word(const uint32_t* __restrict__ payload,
                                                         const float* __restrict__ scales,
                                                         int64_t nwords, int group_shift,
                                                         Lut16 lut, uint4* __restrict__ out) {
  const int64_t w0 = (int64_t)blockIdx.x * (RW * kThreads) + threadIdx.x;
  uint32_t p[RW];
  float s[RW];
#pragma unroll
  for (int j = 0; j < RW; ++j) {
    const int64_t w = w0 + j * kThreads;
    p[j] = w < nwords ? payload[w] : 0u;
    s[j] = w < nwords ? scales[(w * 8) >> group_shift] : 0.0f;
  }
#pragma unroll
  for (int j = 0; j < RW; ++j) {
    const int64_t w = w0 + j * kThreads;
    if (w >= nwords) continue;
    uint32_t o[4];
    st::deq8o<HI>(p[j], st::make_tbl(lut, s[j]), o);
    out[w] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// element-wise tail / unaligned path: one element per thread
__global__ __launch_bounds__(kThreads) void dequant4_scalar(const uint8_t* __restrict__ payload,
                                                           const float* __restrict__ scales,
                                                           int64_t begin, int64_t numel,
                                                           int group, Lut16 lut, int hi_first,
                                                           uint16_t* __restrict__ out) {
  int64_t i = begin + (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= numel) return;
  unsigned b = payload[i >> 1];
  unsigned code = (b >> (4 * ((unsigned)(i & 1) ^ (unsigned)hi_first))) & 15u;
  out[i] = st::f32_to_bf16(lut.v[code] * scales[i / group]);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// bitsandbytes' double-quantised NF4 statistics (quantize_4bit(blocksize=64,
// compress_statistics=True), nf4_backend.py:292-298; state layout
// nf4_backend.py:219-240): the absmax of 64-element block j is a uint8 code
// into a 256-entry fp32 map, with one fp32 scale per `nested_block` (256)
// codes and one fp32 offset, and decodes to
//   absmax_j = fp32( fp32(map[q_j] * nested[j / nested_block]) + offset )
// -- the product rounded to fp32 before the offset is added (the library's
// blockwise dequantize followed by its `absmax += offset`).  The fused GEMMs
// then read these as their fp32 per-64 scales (ST_FLAG_GROUP64).
__global__ __launch_bounds__(kThreads) void nf4_dq_scales_kernel(
    const uint8_t* __restrict__ q, const float* __restrict__ nested,
    const float* __restrict__ map256, float offset, int64_t blocks, int nested_block,
    float* __restrict__ out) {
  static_assert(kThreads == 256, "one map entry per thread");
  __shared__ float map[256];
  map[threadIdx.x] = map256[threadIdx.x];
  __syncthreads();
  for (int64_t j = (int64_t)blockIdx.x * kThreads + threadIdx.x; j < blocks;
       j += (int64_t)gridDim.x * kThreads) {
    const float prod = map[q[j]] * nested[j / nested_block];
    out[j] = prod + offset;
  }
}

}  // namespace

namespace st {
int launch_dequant4(const uint8_t* payload, const float* scales, int64_t numel, int32_t group,
                    const float* lut16, int32_t flags, uint16_t* out, hipStream_t stream) {
  Lut16 lut;
  for (int i = 0; i < 16; ++i) lut.v[i] = lut16[i];
  int hi = (flags & ST_FLAG_HI_NIBBLE_FIRST) ? 1 : 0;
  int64_t vec_elems = 0;
  const int shift = group == 128 ? 7 : 6;
  if (((uintptr_t)payload & 3u) == 0 && aligned16(out)) {
    const int64_t nwords = numel / 8;
    if (nwords > 0) {
      const unsigned blocks = (unsigned)cdiv(nwords, RW * kThreads);
      if (hi)
        dequant4_word<true><<<blocks, kThreads, 0, stream>>>((const uint32_t*)payload, scales,
                                                             nwords, shift, lut, (uint4*)out);
      else
        dequant4_word<false><<<blocks, kThreads, 0, stream>>>((const uint32_t*)payload, scales,
                                                              nwords, shift, lut, (uint4*)out);
      vec_elems = nwords * 8;
    }
  }
  if (vec_elems < numel) {
    int64_t rest = numel - vec_elems;
    dequant4_scalar<<<(unsigned)cdiv(rest, kThreads), kThreads, 0, stream>>>(
        payload, scales, vec_elems, numel, group, lut, hi, out);
  }
  return check_launch("dequant4");
}
}  // namespace st

extern "C" int st_dequant4(const uint8_t* payload, const float* scales, int64_t numel,
                           int32_t group, const float* lut16, int32_t flags, uint16_t* out,
                           st_stream_t stream) {
  ST_CHECK_ARG(numel >= 0, "st_dequant4: negative numel");
  ST_CHECK_ARG(group == 64 || group == 128, "st_dequant4: group must be 64 or 128, got %d", group);
  ST_CHECK_ARG(lut16 != nullptr, "st_dequant4: lut16 is NULL");
  if (numel == 0) return ST_OK;
  ST_CHECK_ARG(payload && scales && out, "st_dequant4: NULL device pointer");
  return st::launch_dequant4(payload, scales, numel, group, lut16, flags, out,
                             (hipStream_t)stream);
}


extern "C" int st_nf4_dq_scales(const uint8_t* absmax_q, const float* nested_absmax,
                                const float* nested_map, float offset, int64_t blocks,
                                int32_t nested_block, float* scales, st_stream_t stream) {
  ST_CHECK_ARG(blocks >= 0 && nested_block > 0, "st_nf4_dq_scales: bad sizes");
  if (blocks == 0) return ST_OK;
  ST_CHECK_ARG(absmax_q && nested_absmax && nested_map && scales,
               "st_nf4_dq_scales: NULL device pointer");
  const int64_t grid = std::min<int64_t>(st::cdiv(blocks, kThreads), 4096);
  nf4_dq_scales_kernel<<<(unsigned)grid, kThreads, 0, (hipStream_t)stream>>>(
      absmax_q, nested_absmax, nested_map, offset, blocks, nested_block, scales);
  return st::check_launch("nf4_dq_scales");
}
