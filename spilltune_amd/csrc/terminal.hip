// Causal-LM terminal: row-wise cross-entropy and its logit gradient on bf16
// logits, in place (training/engine.py:58-75, quantization/native_terminal.py:
// 11-32 of the reference: logits.float() -> cross_entropy(sum, ignore -100),
// gradient of value/normalization cast back to bf16 by the .float() VJP).
//
//   loss[r]   = logsumexp(x_r) - x_r[y_r]                       (0 when y_r == ignore)
//   x_r[c]   <- bf16((softmax(x_r)[c] - [c == y_r]) * grad_scale)   (0 when ignored)
//
// x_r is the fp32 value of the bf16 logits of row r.  One workgroup per row
// streams it twice (online max/sum, then gradient), 16 bytes per thread per
// access, so the kernel runs at HBM speed; fp32 logits never exist in memory.
#include "common.h"

namespace {

constexpr int NT = 512;

struct MS {  // running (max, sum of exp(x - max))
  float m, s;
};
__device__ __forceinline__ MS ms_merge(MS a, MS b) {
  const float m = fmaxf(a.m, b.m);
  if (m == -INFINITY) return {m, 0.0f};
  return {m, a.s * expf(a.m - m) + b.s * expf(b.m - m)};
}
__device__ __forceinline__ void ms_add(MS& a, float x) {
  if (x > a.m) {
    a.s = a.s * expf(a.m - x) + 1.0f;
    a.m = x;
  } else {
    a.s += expf(x - a.m);
  }
}

__global__ __launch_bounds__(NT) void ce_rows(uint16_t* __restrict__ logits, int64_t ld,
                                              int64_t V, const int64_t* __restrict__ labels,
                                              int64_t ignore, float grad_scale, int vec,
                                              float* __restrict__ loss) {
  __shared__ MS red[NT / 64];
  __shared__ float xy;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t r = blockIdx.x;
  uint16_t* row = logits + r * ld;
  const int64_t y = labels[r];
  const int64_t vend = vec ? V / 8 * 8 : 0;  // vector part [0, vend), scalar tail after

  if (y == ignore) {
    for (int64_t c = (int64_t)tid * 8; c < vend; c += NT * 8) *(uint4*)(row + c) = make_uint4(0, 0, 0, 0);
    for (int64_t c = vend + tid; c < V; c += NT) row[c] = 0;
    if (tid == 0) loss[r] = 0.0f;
    return;
  }
  // labels are validated by the host; an out-of-range one reads nothing and
  // yields a NaN loss rather than touching memory outside the row
  if (tid == 0) xy = (y >= 0 && y < V) ? st::bf16_to_f32(row[y]) : __uint_as_float(0x7fc00000u);

  // pass 1: max and sum of exp
  MS a = {-INFINITY, 0.0f};
  for (int64_t c = (int64_t)tid * 8; c < vend; c += NT * 8) {
    const uint4 q = *(const uint4*)(row + c);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      ms_add(a, __uint_as_float(w[e] << 16));
      ms_add(a, __uint_as_float(w[e] & 0xffff0000u));
    }
  }
  for (int64_t c = vend + tid; c < V; c += NT) ms_add(a, st::bf16_to_f32(row[c]));
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    MS b = {__shfl_xor(a.m, off), __shfl_xor(a.s, off)};
    a = ms_merge(a, b);
  }
  if (lane == 0) red[wave] = a;
  __syncthreads();
  MS t = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) t = ms_merge(t, red[i]);
  const float lse = t.m + logf(t.s);
  if (tid == 0) loss[r] = lse - xy;

  // pass 2: gradient, written over the logits
  auto grad = [&](float x, int64_t c) {
    const float p = expf(x - lse);
    return (p - (c == y ? 1.0f : 0.0f)) * grad_scale;
  };
  for (int64_t c = (int64_t)tid * 8; c < vend; c += NT * 8) {
    const uint4 q = *(const uint4*)(row + c);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = st::pack_bf16x2(grad(__uint_as_float(w[e] << 16), c + 2 * e),
                             grad(__uint_as_float(w[e] & 0xffff0000u), c + 2 * e + 1));
    *(uint4*)(row + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
  for (int64_t c = vend + tid; c < V; c += NT) row[c] = st::f32_to_bf16(grad(st::bf16_to_f32(row[c]), c));
}

}  // namespace

extern "C" int st_cross_entropy_rows(uint16_t* logits, int64_t rows, int64_t vocab, int64_t ld,
                                     const int64_t* labels, int64_t ignore_index,
                                     float grad_scale, float* loss_rows, st_stream_t stream) {
  ST_CHECK_ARG(rows >= 0 && vocab > 0 && ld >= vocab, "st_cross_entropy_rows: bad shape");
  if (rows == 0) return ST_OK;
  ST_CHECK_ARG(logits && labels && loss_rows, "st_cross_entropy_rows: NULL pointer");
  ST_CHECK_ARG(rows <= 0x7fffffff, "st_cross_entropy_rows: too many rows");
  const int vec = (((uintptr_t)logits & 15u) == 0 && ld % 8 == 0) ? 1 : 0;
  ce_rows<<<(unsigned)rows, NT, 0, (hipStream_t)stream>>>(logits, ld, vocab, labels, ignore_index,
                                                          grad_scale, vec, loss_rows);
  return st::check_launch("st_cross_entropy_rows");
}
