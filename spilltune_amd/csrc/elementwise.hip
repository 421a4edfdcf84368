// Decoder-layer elementwise kernels (HBM-bound): RMSNorm, rotary embedding
// with the head relayout and SwiGLU.
//
// Each forward reproduces the reference's bf16 rounding points
// (adapters/dense.py:115-153); each backward reproduces the roundings that
// PyTorch autograd applies to the same graph (bf16 gradients of bf16 ops,
// fp32 inside the fp32 regions).
#include <cmath>

#include "common.h"

namespace {

constexpr int NTH = 256;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = 0.0f;
  for (int i = 0; i < NTH / 64; ++i) s += red[i];
  return s;
}

// ------------------------------------------------------------------ RMSNorm
// 8 bf16 in a 16-byte vector <-> fp32 values
__device__ __forceinline__ void unpack8(uint4 q, float (&f)[8]) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(w[e] << 16);
    f[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  return make_uint4(st::pack_bf16x2(f[0], f[1]), st::pack_bf16x2(f[2], f[3]),
                    st::pack_bf16x2(f[4], f[5]), st::pack_bf16x2(f[6], f[7]));
}

// Vector forms (H % 8 == 0, 16-byte aligned rows): 8 elements per thread per
// access, same per-element rounding as the scalar kernels below.
__global__ __launch_bounds__(NTH) void rmsnorm_fwd_vec(const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w, int64_t H,
                                                      float eps, uint16_t* __restrict__ y,
                                                      float* __restrict__ rstd) {
  __shared__ float red[NTH / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * H;
  float ss = 0.0f;
  for (int64_t i = threadIdx.x * 8; i < H; i += NTH * 8) {
    float v[8];
    unpack8(*(const uint4*)(xr + i), v);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
  }
  ss = block_sum(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)H + eps);
  if (threadIdx.x == 0) rstd[row] = r;
  for (int64_t i = threadIdx.x * 8; i < H; i += NTH * 8) {
    float v[8], g[8], o[8];
    unpack8(*(const uint4*)(xr + i), v);
    unpack8(*(const uint4*)(w + i), g);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = g[e] * st::bf16r(v[e] * r);
    *(uint4*)(y + row * H + i) = pack8(o);
  }
}

__global__ __launch_bounds__(NTH) void rmsnorm_bwd_vec(const uint16_t* __restrict__ dy,
                                                      const uint16_t* __restrict__ x,
                                                      const uint16_t* __restrict__ w,
                                                      const float* __restrict__ rstd,
                                                      const uint16_t* __restrict__ dres, int64_t H,
                                                      uint16_t* __restrict__ dx) {
  __shared__ float red[NTH / 64];
  const int64_t row = blockIdx.x;
  const float r = rstd[row];
  float dot = 0.0f;
  for (int64_t i = threadIdx.x * 8; i < H; i += NTH * 8) {
    float d[8], v[8], g[8];
    unpack8(*(const uint4*)(dy + row * H + i), d);
    unpack8(*(const uint4*)(x + row * H + i), v);
    unpack8(*(const uint4*)(w + i), g);
#pragma unroll
    for (int e = 0; e < 8; ++e) dot += st::bf16r(d[e] * g[e]) * v[e];
  }
  dot = block_sum(dot, red);
  const float c = r * r * r * dot / (float)H;
  for (int64_t i = threadIdx.x * 8; i < H; i += NTH * 8) {
    float d[8], v[8], g[8], o[8], rs[8];
    unpack8(*(const uint4*)(dy + row * H + i), d);
    unpack8(*(const uint4*)(x + row * H + i), v);
    unpack8(*(const uint4*)(w + i), g);
    if (dres) unpack8(*(const uint4*)(dres + row * H + i), rs);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = st::bf16r(r * st::bf16r(d[e] * g[e]) - v[e] * c);
      if (dres) o[e] = rs[e] + o[e];
    }
    *(uint4*)(dx + row * H + i) = pack8(o);
  }
}

__global__ __launch_bounds__(NTH) void rmsnorm_fwd(const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w, int64_t H,
                                                  float eps, uint16_t* __restrict__ y,
                                                  float* __restrict__ rstd) {
  __shared__ float red[NTH / 64];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * H;
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < H; i += NTH) {
    float v = st::bf16_to_f32(xr[i]);
    ss += v * v;
  }
  ss = block_sum(ss, red);
  const float r = 1.0f / sqrtf(ss / (float)H + eps);
  if (threadIdx.x == 0) rstd[row] = r;
  for (int64_t i = threadIdx.x; i < H; i += NTH) {
    float n = st::bf16r(st::bf16_to_f32(xr[i]) * r);
    y[row * H + i] = st::f32_to_bf16(st::bf16_to_f32(w[i]) * n);
  }
}

__global__ __launch_bounds__(NTH) void rmsnorm_bwd(const uint16_t* __restrict__ dy,
                                                  const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w,
                                                  const float* __restrict__ rstd,
                                                  const uint16_t* __restrict__ dres, int64_t H,
                                                  uint16_t* __restrict__ dx) {
  __shared__ float red[NTH / 64];
  const int64_t row = blockIdx.x;
  const float r = rstd[row];
  float dot = 0.0f;
  for (int64_t i = threadIdx.x; i < H; i += NTH) {
    float dn = st::bf16r(st::bf16_to_f32(dy[row * H + i]) * st::bf16_to_f32(w[i]));
    dot += dn * st::bf16_to_f32(x[row * H + i]);
  }
  dot = block_sum(dot, red);
  const float c = r * r * r * dot / (float)H;
  for (int64_t i = threadIdx.x; i < H; i += NTH) {
    float dn = st::bf16r(st::bf16_to_f32(dy[row * H + i]) * st::bf16_to_f32(w[i]));
    float g = st::bf16r(r * dn - st::bf16_to_f32(x[row * H + i]) * c);
    if (dres) g = st::bf16r(st::bf16_to_f32(dres[row * H + i]) + g);
    dx[row * H + i] = st::f32_to_bf16(g);
  }
}

// ------------------------------------------------------------------ RoPE
// one thread per (b, s, h, d) element; grid over B*S*heads*D
__global__ __launch_bounds__(NTH) void rope_fwd(const uint16_t* __restrict__ x, int64_t ldx,
                                               const uint16_t* __restrict__ cs,
                                               const uint16_t* __restrict__ sn, int64_t S,
                                               int64_t heads, int64_t D, int rotate, int64_t total,
                                               uint16_t* __restrict__ out) {
  int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= total) return;
  int64_t d = e % D, t = e / D;
  int64_t h = t % heads;
  t /= heads;
  int64_t s = t % S, b = t / S;
  const uint16_t* xr = x + (b * S + s) * ldx + h * D;
  float v = st::bf16_to_f32(xr[d]);
  float o = v;
  if (rotate) {
    int64_t half = D / 2;
    float rot = d < half ? -st::bf16_to_f32(xr[d + half]) : st::bf16_to_f32(xr[d - half]);
    int64_t ci = (b * S + s) * D + d;
    o = st::bf16r(v * st::bf16_to_f32(cs[ci])) + st::bf16r(rot * st::bf16_to_f32(sn[ci]));
  }
  out[((b * heads + h) * S + s) * D + d] = st::f32_to_bf16(o);
}

__global__ __launch_bounds__(NTH) void rope_bwd(const uint16_t* __restrict__ g,
                                               const uint16_t* __restrict__ cs,
                                               const uint16_t* __restrict__ sn, int64_t S,
                                               int64_t heads, int64_t D, int rotate, int64_t total,
                                               uint16_t* __restrict__ dx, int64_t lddx) {
  int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= total) return;
  int64_t d = e % D, t = e / D;
  int64_t h = t % heads;
  t /= heads;
  int64_t s = t % S, b = t / S;
  const uint16_t* gr = g + ((b * heads + h) * S + s) * D;
  float gv = st::bf16_to_f32(gr[d]);
  float o = gv;
  if (rotate) {
    int64_t half = D / 2;
    int64_t cb = (b * S + s) * D;
    float a = st::bf16r(gv * st::bf16_to_f32(cs[cb + d]));
    // r[d] = gs[d + half] (d < half), -gs[d - half] (d >= half), gs = bf16(g * sin)
    int64_t dd = d < half ? d + half : d - half;
    float gs = st::bf16r(st::bf16_to_f32(gr[dd]) * st::bf16_to_f32(sn[cb + dd]));
    o = a + (d < half ? gs : -gs);
  }
  dx[(b * S + s) * lddx + h * D + d] = st::f32_to_bf16(o);
}

// Vector forms: one workgroup per token (b, s); a thread handles 8 consecutive
// elements (16 bytes) of one head and reads the partner chunk half a head
// away, so there is no per-element index arithmetic.  Same rounding points as
// rope_fwd / rope_bwd.  Needs D % 16 == 0 and 16-byte aligned rows.
// One 8-element chunk c of a head row xr (D elements) rotated with the token's
// cos/sin rows: o = bf16(x*cos) + bf16(rotate_half(x)*sin) (dense.py:141),
// or copied when !rotate; written to dst.
__device__ __forceinline__ void rope_chunk_fwd(const uint16_t* xr, const uint16_t* csr,
                                               const uint16_t* snr, int c, int half, int rotate,
                                               uint16_t* dst) {
  float v[8], o[8];
  unpack8(*(const uint4*)(xr + c * 8), v);
  if (rotate) {
    float p[8], cv[8], sv[8];
    unpack8(*(const uint4*)(xr + (c < half ? c + half : c - half) * 8), p);
    unpack8(*(const uint4*)(csr + c * 8), cv);
    unpack8(*(const uint4*)(snr + c * 8), sv);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float rot = c < half ? -p[e] : p[e];
      o[e] = st::bf16r(v[e] * cv[e]) + st::bf16r(rot * sv[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = v[e];
  }
  *(uint4*)dst = pack8(o);
}

// VJP of rope_chunk_fwd for chunk c of a head-major gradient row gr.
__device__ __forceinline__ void rope_chunk_bwd(const uint16_t* gr, const uint16_t* csr,
                                               const uint16_t* snr, int c, int half, int rotate,
                                               uint16_t* dst) {
  float gv[8], o[8];
  unpack8(*(const uint4*)(gr + c * 8), gv);
  if (rotate) {
    const int pc = c < half ? c + half : c - half;
    float gp[8], cv[8], sp[8];
    unpack8(*(const uint4*)(gr + pc * 8), gp);
    unpack8(*(const uint4*)(csr + c * 8), cv);
    unpack8(*(const uint4*)(snr + pc * 8), sp);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a = st::bf16r(gv[e] * cv[e]);
      const float gs = st::bf16r(gp[e] * sp[e]);
      o[e] = a + (c < half ? gs : -gs);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = gv[e];
  }
  *(uint4*)dst = pack8(o);
}

__global__ __launch_bounds__(NTH) void rope_fwd_vec(const uint16_t* __restrict__ x, int64_t ldx,
                                                   const uint16_t* __restrict__ cs,
                                                   const uint16_t* __restrict__ sn, int S,
                                                   int heads, int D, int rotate,
                                                   uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.x;  // token b*S + s
  const int64_t b = t / S, s = t % S;
  const int CH = D / 8, half = CH / 2;
  for (int i = threadIdx.x; i < heads * CH; i += NTH) {
    const int h = i / CH, c = i % CH;
    rope_chunk_fwd(x + t * ldx + h * D, cs + t * D, sn + t * D, c, half, rotate,
                   out + ((b * heads + h) * S + s) * D + c * 8);
  }
}

__global__ __launch_bounds__(NTH) void rope_bwd_vec(const uint16_t* __restrict__ g,
                                                   const uint16_t* __restrict__ cs,
                                                   const uint16_t* __restrict__ sn, int S,
                                                   int heads, int D, int rotate,
                                                   uint16_t* __restrict__ dx, int64_t lddx) {
  const int64_t t = blockIdx.x;
  const int64_t b = t / S, s = t % S;
  const int CH = D / 8, half = CH / 2;
  for (int i = threadIdx.x; i < heads * CH; i += NTH) {
    const int h = i / CH, c = i % CH;
    rope_chunk_bwd(g + ((b * heads + h) * S + s) * D, cs + t * D, sn + t * D, c, half, rotate,
                   dx + t * lddx + h * D + c * 8);
  }
}

// q, k and v of one fused q|k|v row in one launch: segment 0 = the Hq query
// heads (rotated), 1 = the Hkv key heads (rotated), 2 = the Hkv value heads
// (copied), each to its own head-major tensor [B, heads, S, D].
struct QkvHeads {
  const uint16_t* g[3];  // backward: head-major gradients of q, k, v
  uint16_t* o[3];        // forward: head-major q, k, v
  int h[3];
};
__global__ __launch_bounds__(NTH) void rope_qkv_fwd_vec(const uint16_t* __restrict__ x,
                                                       int64_t ldx,
                                                       const uint16_t* __restrict__ cs,
                                                       const uint16_t* __restrict__ sn, int S,
                                                       int D, QkvHeads qh) {
  const int64_t t = blockIdx.x;
  const int64_t b = t / S, s = t % S;
  const int CH = D / 8, half = CH / 2;
  const int n0 = qh.h[0] * CH, n1 = n0 + qh.h[1] * CH, n2 = n1 + qh.h[2] * CH;
  for (int i = threadIdx.x; i < n2; i += NTH) {
    const int seg = i < n0 ? 0 : i < n1 ? 1 : 2;
    const int j = i - (seg == 0 ? 0 : seg == 1 ? n0 : n1);
    const int h = j / CH, c = j % CH;
    const int heads = seg == 0 ? qh.h[0] : seg == 1 ? qh.h[1] : qh.h[2];
    uint16_t* out = seg == 0 ? qh.o[0] : seg == 1 ? qh.o[1] : qh.o[2];
    const int col = (seg == 0 ? 0 : seg == 1 ? n0 : n1) * 8 + h * D;  // column of the head in x
    rope_chunk_fwd(x + t * ldx + col, cs + t * D, sn + t * D, c, half, seg < 2,
                   out + ((b * heads + h) * S + s) * D + c * 8);
  }
}
__global__ __launch_bounds__(NTH) void rope_qkv_bwd_vec(const uint16_t* __restrict__ cs,
                                                       const uint16_t* __restrict__ sn, int S,
                                                       int D, QkvHeads qh,
                                                       uint16_t* __restrict__ dx, int64_t lddx) {
  const int64_t t = blockIdx.x;
  const int64_t b = t / S, s = t % S;
  const int CH = D / 8, half = CH / 2;
  const int n0 = qh.h[0] * CH, n1 = n0 + qh.h[1] * CH, n2 = n1 + qh.h[2] * CH;
  for (int i = threadIdx.x; i < n2; i += NTH) {
    const int seg = i < n0 ? 0 : i < n1 ? 1 : 2;
    const int j = i - (seg == 0 ? 0 : seg == 1 ? n0 : n1);
    const int h = j / CH, c = j % CH;
    const int heads = seg == 0 ? qh.h[0] : seg == 1 ? qh.h[1] : qh.h[2];
    const uint16_t* g = seg == 0 ? qh.g[0] : seg == 1 ? qh.g[1] : qh.g[2];
    const int col = (seg == 0 ? 0 : seg == 1 ? n0 : n1) * 8 + h * D;
    rope_chunk_bwd(g + ((b * heads + h) * S + s) * D, cs + t * D, sn + t * D, c, half, seg < 2,
                   dx + t * lddx + col + c * 8);
  }
}

__global__ __launch_bounds__(NTH) void relayout(const uint16_t* __restrict__ x, int64_t S,
                                               int64_t heads, int64_t D, int64_t total,
                                               int to_tokens, uint16_t* __restrict__ out) {
  int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= total) return;
  int64_t d = e % D, t = e / D;
  int64_t h = t % heads;
  t /= heads;
  int64_t s = t % S, b = t / S;
  int64_t tok = ((b * S + s) * heads + h) * D + d;
  int64_t hd = ((b * heads + h) * S + s) * D + d;
  if (to_tokens)
    out[tok] = x[hd];
  else
    out[hd] = x[tok];
}

// ------------------------------------------------------------------ SwiGLU
__global__ __launch_bounds__(NTH) void swiglu_fwd(const uint16_t* __restrict__ g, int64_t ldg,
                                                 const uint16_t* __restrict__ u, int64_t ldu,
                                                 int64_t I, int64_t total,
                                                 uint16_t* __restrict__ a, int64_t lda) {
  int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= total) return;
  int64_t r = e / I, c = e % I;
  float gv = st::bf16_to_f32(g[r * ldg + c]);
  float s = st::bf16r(gv / (1.0f + expf(-gv)));
  a[r * lda + c] = st::f32_to_bf16(s * st::bf16_to_f32(u[r * ldu + c]));
}

__global__ __launch_bounds__(NTH) void swiglu_bwd(const uint16_t* __restrict__ da, int64_t ldda,
                                                 const uint16_t* __restrict__ g, int64_t ldg,
                                                 const uint16_t* __restrict__ u, int64_t ldu,
                                                 int64_t I, int64_t total,
                                                 uint16_t* __restrict__ dg, int64_t lddg,
                                                 uint16_t* __restrict__ du, int64_t lddu) {
  int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= total) return;
  int64_t r = e / I, c = e % I;
  float gv = st::bf16_to_f32(g[r * ldg + c]);
  float uv = st::bf16_to_f32(u[r * ldu + c]);
  float dav = st::bf16_to_f32(da[r * ldda + c]);
  float dgv, duv;
  st::swiglu_vjp(gv, uv, dav, dgv, duv);
  du[r * lddu + c] = st::f32_to_bf16(duv);
  dg[r * lddg + c] = st::f32_to_bf16(dgv);
}





// 8 elements per thread; all rows/strides multiples of 8 elements
__global__ __launch_bounds__(NTH) void swiglu_fwd_vec(const uint16_t* __restrict__ g, int64_t ldg,
                                                     const uint16_t* __restrict__ u, int64_t ldu,
                                                     int64_t I, int64_t total8,
                                                     uint16_t* __restrict__ a, int64_t lda) {
  int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= total8) return;
  const int64_t per = I / 8, r = e / per, c = (e % per) * 8;
  uint4 gq = *(const uint4*)(g + r * ldg + c), uq = *(const uint4*)(u + r * ldu + c);
  uint32_t gw[4] = {gq.x, gq.y, gq.z, gq.w}, uw[4] = {uq.x, uq.y, uq.z, uq.w}, o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float r2[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float gv = st::bf16_to_f32((uint16_t)(gw[k] >> (16 * h)));
      float uv = st::bf16_to_f32((uint16_t)(uw[k] >> (16 * h)));
      r2[h] = st::bf16r(gv / (1.0f + expf(-gv))) * uv;
    }
    o[k] = st::pack_bf16x2(r2[0], r2[1]);
  }
  *(uint4*)(a + r * lda + c) = make_uint4(o[0], o[1], o[2], o[3]);
}

__global__ __launch_bounds__(NTH) void swiglu_bwd_vec(const uint16_t* __restrict__ da, int64_t ldda,
                                                     const uint16_t* __restrict__ g, int64_t ldg,
                                                     const uint16_t* __restrict__ u, int64_t ldu,
                                                     int64_t I, int64_t total8,
                                                     uint16_t* __restrict__ dg, int64_t lddg,
                                                     uint16_t* __restrict__ du, int64_t lddu) {
  int64_t e = (int64_t)blockIdx.x * NTH + threadIdx.x;
  if (e >= total8) return;
  const int64_t per = I / 8, r = e / per, c = (e % per) * 8;
  uint4 aq = *(const uint4*)(da + r * ldda + c), gq = *(const uint4*)(g + r * ldg + c),
        uq = *(const uint4*)(u + r * ldu + c);
  uint32_t aw[4] = {aq.x, aq.y, aq.z, aq.w}, gw[4] = {gq.x, gq.y, gq.z, gq.w},
           uw[4] = {uq.x, uq.y, uq.z, uq.w}, og[4], ou[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float rg[2], ru[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float gv = st::bf16_to_f32((uint16_t)(gw[k] >> (16 * h)));
      float uv = st::bf16_to_f32((uint16_t)(uw[k] >> (16 * h)));
      float dav = st::bf16_to_f32((uint16_t)(aw[k] >> (16 * h)));
      st::swiglu_vjp(gv, uv, dav, rg[h], ru[h]);
    }
    og[k] = st::pack_bf16x2(rg[0], rg[1]);
    ou[k] = st::pack_bf16x2(ru[0], ru[1]);
  }
  *(uint4*)(dg + r * lddg + c) = make_uint4(og[0], og[1], og[2], og[3]);
  *(uint4*)(du + r * lddu + c) = make_uint4(ou[0], ou[1], ou[2], ou[3]);
}

bool vec8(const void* p) { return ((uintptr_t)p & 15u) == 0; }

unsigned nblk(int64_t total) { return (unsigned)st::cdiv(total, NTH); }


// Qwen3's per-head q/k RMSNorm fused with the rotation (dense.py:128-141):
// every query and key head of a fused q|k|v row is normalised over its D
// elements (weights wq / wk, the rounding of rmsnorm_fwd: w * bf16(x * r)) and
// then rotated (rope_chunk_fwd's rounding); value heads are copied.  One
// workgroup per token; CH = D/8 consecutive lanes hold one head (lane c has
// chunk c), so the head's sum of squares is a CH-lane xor reduction and the
// rotation's partner chunk c ^ CH/2 comes from a lane of the same group.  The
// loop runs the same number of steps on every wave; groups past the last head
// only skip their loads and stores.
template <int D>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = D / 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ void shfl8(const float (&v)[8], int o, float (&p)[8]) {
  const uint4 q = pack8(v);
  uint4 r;
  r.x = __shfl_xor(q.x, o, 64);
  r.y = __shfl_xor(q.y, o, 64);
  r.z = __shfl_xor(q.z, o, 64);
  r.w = __shfl_xor(q.w, o, 64);
  unpack8(r, p);
}
template <int D>
__global__ __launch_bounds__(NTH) void rope_qkv_norm_fwd(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ cs,
    const uint16_t* __restrict__ sn, int S, QkvHeads qh, const uint16_t* __restrict__ wq,
    const uint16_t* __restrict__ wk, float eps, float* __restrict__ rstd) {
  constexpr int CH = D / 8, HALF = CH / 2, GPB = NTH / CH;  // lanes per head, heads per pass
  const int64_t t = blockIdx.x;
  const int64_t b = t / S, s = t % S;
  const int nn = qh.h[0] + qh.h[1], nh = nn + qh.h[2];
  const int c = threadIdx.x % CH;
  for (int h0 = 0; h0 < nh; h0 += GPB) {
    const int hh = h0 + threadIdx.x / CH;
    const bool ok = hh < nh;
    const int seg = hh < qh.h[0] ? 0 : hh < nn ? 1 : 2;
    const int hl = hh - (seg == 0 ? 0 : seg == 1 ? qh.h[0] : nn);
    float v[8];
    unpack8(ok ? *(const uint4*)(x + t * ldx + (int64_t)hh * D + c * 8) : make_uint4(0, 0, 0, 0), v);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
    ss = group_sum<D>(ss);
    const float r = 1.0f / sqrtf(ss / (float)D + eps);
    float n[8], p[8], o[8];
    if (seg < 2) {
      float g[8];
      unpack8(*(const uint4*)((seg == 0 ? wq : wk) + c * 8), g);
#pragma unroll
      for (int e = 0; e < 8; ++e) n[e] = st::bf16r(g[e] * st::bf16r(v[e] * r));
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) n[e] = v[e];
    }
    shfl8(n, HALF, p);
    if (!ok) continue;
    if (seg < 2) {
      float cv[8], sv[8];
      unpack8(*(const uint4*)(cs + t * D + c * 8), cv);
      unpack8(*(const uint4*)(sn + t * D + c * 8), sv);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float rot = c < HALF ? -p[e] : p[e];
        o[e] = st::bf16r(n[e] * cv[e]) + st::bf16r(rot * sv[e]);
      }
      if (c == 0) rstd[t * nn + hh] = r;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = n[e];
    }
    *(uint4*)(qh.o[seg] + ((b * qh.h[seg] + hl) * S + s) * D + c * 8) = pack8(o);
  }
}

// VJP of rope_qkv_norm_fwd: rope_chunk_bwd's rotation VJP (rounded to bf16),
// then rmsnorm_bwd's VJP of the head norm with the saved rstd; value heads
// are copied.  dx rows of stride lddx.
template <int D>
__global__ __launch_bounds__(NTH) void rope_qkv_norm_bwd(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ cs,
    const uint16_t* __restrict__ sn, int S, QkvHeads qh, const uint16_t* __restrict__ wq,
    const uint16_t* __restrict__ wk, const float* __restrict__ rstd, uint16_t* __restrict__ dx,
    int64_t lddx) {
  constexpr int CH = D / 8, HALF = CH / 2, GPB = NTH / CH;
  const int64_t t = blockIdx.x;
  const int64_t b = t / S, s = t % S;
  const int nn = qh.h[0] + qh.h[1], nh = nn + qh.h[2];
  const int c = threadIdx.x % CH;
  for (int h0 = 0; h0 < nh; h0 += GPB) {
    const int hh = h0 + threadIdx.x / CH;
    const bool ok = hh < nh;
    const int seg = hh < qh.h[0] ? 0 : hh < nn ? 1 : 2;
    const int hl = hh - (seg == 0 ? 0 : seg == 1 ? qh.h[0] : nn);
    float gv[8], gp[8];
    unpack8(ok ? *(const uint4*)(qh.g[seg] + ((b * qh.h[seg] + hl) * S + s) * D + c * 8)
               : make_uint4(0, 0, 0, 0), gv);
    shfl8(gv, HALF, gp);
    float d[8], xv[8], g[8], dn[8];
    float dot = 0.0f, r = 0.0f;
    if (seg < 2) {
      float cv[8], sp[8];
      unpack8(*(const uint4*)(cs + t * D + c * 8), cv);
      unpack8(*(const uint4*)(sn + t * D + (c ^ HALF) * 8), sp);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float a = st::bf16r(gv[e] * cv[e]);
        const float gs = st::bf16r(gp[e] * sp[e]);
        d[e] = st::bf16r(a + (c < HALF ? gs : -gs));
      }
      unpack8(ok ? *(const uint4*)(x + t * ldx + (int64_t)hh * D + c * 8) : make_uint4(0, 0, 0, 0),
              xv);
      unpack8(*(const uint4*)((seg == 0 ? wq : wk) + c * 8), g);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dn[e] = st::bf16r(d[e] * g[e]);
        dot += dn[e] * xv[e];
      }
      r = ok ? rstd[t * nn + hh] : 0.0f;
    }
    dot = group_sum<D>(dot);
    if (!ok) continue;
    float o[8];
    if (seg < 2) {
      const float cc = r * r * r * dot / (float)D;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = st::bf16r(r * dn[e] - xv[e] * cc);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = gv[e];
    }
    *(uint4*)(dx + t * lddx + (int64_t)hh * D + c * 8) = pack8(o);
  }
}

}  // namespace

extern "C" int st_rmsnorm_fwd(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t H,
                              float eps, uint16_t* y, float* rstd, st_stream_t stream) {
  ST_CHECK_ARG(rows >= 0 && H > 0, "st_rmsnorm_fwd: bad shape");
  if (rows == 0) return ST_OK;
  ST_CHECK_ARG(x && w && y && rstd, "st_rmsnorm_fwd: NULL pointer");
  if (H % 8 == 0 && H >= NTH * 8 / 4 && (((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) & 15u) == 0)
    rmsnorm_fwd_vec<<<(unsigned)rows, NTH, 0, (hipStream_t)stream>>>(x, w, H, eps, y, rstd);
  else
    rmsnorm_fwd<<<(unsigned)rows, NTH, 0, (hipStream_t)stream>>>(x, w, H, eps, y, rstd);
  return st::check_launch("rmsnorm_fwd");
}

extern "C" int st_rmsnorm_bwd(const uint16_t* dy, const uint16_t* x, const uint16_t* w,
                              const float* rstd, const uint16_t* dres, int64_t rows, int64_t H,
                              uint16_t* dx, st_stream_t stream) {
  ST_CHECK_ARG(rows >= 0 && H > 0, "st_rmsnorm_bwd: bad shape");
  if (rows == 0) return ST_OK;
  ST_CHECK_ARG(dy && x && w && rstd && dx, "st_rmsnorm_bwd: NULL pointer");
  if (H % 8 == 0 && H >= NTH * 8 / 4 &&
      (((uintptr_t)dy | (uintptr_t)x | (uintptr_t)w | (uintptr_t)dres | (uintptr_t)dx) & 15u) == 0)
    rmsnorm_bwd_vec<<<(unsigned)rows, NTH, 0, (hipStream_t)stream>>>(dy, x, w, rstd, dres, H, dx);
  else
    rmsnorm_bwd<<<(unsigned)rows, NTH, 0, (hipStream_t)stream>>>(dy, x, w, rstd, dres, H, dx);
  return st::check_launch("rmsnorm_bwd");
}

extern "C" int st_rope_fwd(const uint16_t* x, int64_t ldx, const uint16_t* cos,
                           const uint16_t* sin, int64_t B, int64_t S, int64_t heads, int64_t D,
                           int32_t rotate, uint16_t* out, st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && heads > 0 && D > 0 && D % 2 == 0, "st_rope_fwd: bad shape");
  int64_t total = B * S * heads * D;
  if (total == 0) return ST_OK;
  ST_CHECK_ARG(x && out && (!rotate || (cos && sin)), "st_rope_fwd: NULL pointer");
  ST_CHECK_ARG(ldx >= heads * D, "st_rope_fwd: ldx < heads*D");
  const bool vec = D % 16 == 0 && ldx % 8 == 0 && S <= 0x7fffffff && heads * D <= 0x7fffffff &&
                   (((uintptr_t)x | (uintptr_t)out | (uintptr_t)cos | (uintptr_t)sin) & 15u) == 0;
  if (vec && B * S <= 0x7fffffff)
    rope_fwd_vec<<<(unsigned)(B * S), NTH, 0, (hipStream_t)stream>>>(x, ldx, cos, sin, (int)S,
                                                                     (int)heads, (int)D, rotate, out);
  else
    rope_fwd<<<nblk(total), NTH, 0, (hipStream_t)stream>>>(x, ldx, cos, sin, S, heads, D, rotate,
                                                           total, out);
  return st::check_launch("rope_fwd");
}

extern "C" int st_rope_bwd(const uint16_t* dout, const uint16_t* cos, const uint16_t* sin,
                           int64_t B, int64_t S, int64_t heads, int64_t D, int32_t rotate,
                           uint16_t* dx, int64_t lddx, st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && heads > 0 && D > 0 && D % 2 == 0, "st_rope_bwd: bad shape");
  int64_t total = B * S * heads * D;
  if (total == 0) return ST_OK;
  ST_CHECK_ARG(dout && dx && (!rotate || (cos && sin)), "st_rope_bwd: NULL pointer");
  ST_CHECK_ARG(lddx >= heads * D, "st_rope_bwd: lddx < heads*D");
  const bool vec = D % 16 == 0 && lddx % 8 == 0 && S <= 0x7fffffff && heads * D <= 0x7fffffff &&
                   (((uintptr_t)dout | (uintptr_t)dx | (uintptr_t)cos | (uintptr_t)sin) & 15u) == 0;
  if (vec && B * S <= 0x7fffffff)
    rope_bwd_vec<<<(unsigned)(B * S), NTH, 0, (hipStream_t)stream>>>(dout, cos, sin, (int)S,
                                                                     (int)heads, (int)D, rotate,
                                                                     dx, lddx);
  else
    rope_bwd<<<nblk(total), NTH, 0, (hipStream_t)stream>>>(dout, cos, sin, S, heads, D, rotate,
                                                           total, dx, lddx);
  return st::check_launch("rope_bwd");
}

extern "C" int st_rope_qkv_fwd(const uint16_t* x, int64_t ldx, const uint16_t* cos,
                               const uint16_t* sin, int64_t B, int64_t S, int64_t heads,
                               int64_t kv_heads, int64_t D, uint16_t* q, uint16_t* k,
                               uint16_t* v, st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && heads > 0 && kv_heads > 0 && D > 0 && D % 2 == 0,
               "st_rope_qkv_fwd: bad shape");
  if (B * S == 0) return ST_OK;
  ST_CHECK_ARG(x && cos && sin && q && k && v, "st_rope_qkv_fwd: NULL pointer");
  const int64_t width = (heads + 2 * kv_heads) * D;
  ST_CHECK_ARG(ldx >= width, "st_rope_qkv_fwd: ldx < (heads + 2*kv_heads)*D");
  const bool vec = D % 16 == 0 && ldx % 8 == 0 && B * S <= 0x7fffffff && width <= 0x7fffffff &&
                   (((uintptr_t)x | (uintptr_t)cos | (uintptr_t)sin | (uintptr_t)q |
                     (uintptr_t)k | (uintptr_t)v) & 15u) == 0;
  if (!vec) {  // one launch per segment
    int rc = st_rope_fwd(x, ldx, cos, sin, B, S, heads, D, 1, q, stream);
    if (!rc) rc = st_rope_fwd(x + heads * D, ldx, cos, sin, B, S, kv_heads, D, 1, k, stream);
    if (!rc)
      rc = st_rope_fwd(x + (heads + kv_heads) * D, ldx, cos, sin, B, S, kv_heads, D, 0, v, stream);
    return rc;
  }
  QkvHeads qh{};
  qh.o[0] = q; qh.o[1] = k; qh.o[2] = v;
  qh.h[0] = (int)heads; qh.h[1] = (int)kv_heads; qh.h[2] = (int)kv_heads;
  rope_qkv_fwd_vec<<<(unsigned)(B * S), NTH, 0, (hipStream_t)stream>>>(x, ldx, cos, sin, (int)S,
                                                                      (int)D, qh);
  return st::check_launch("rope_qkv_fwd");
}

extern "C" int st_rope_qkv_bwd(const uint16_t* dq, const uint16_t* dk, const uint16_t* dv,
                               const uint16_t* cos, const uint16_t* sin, int64_t B, int64_t S,
                               int64_t heads, int64_t kv_heads, int64_t D, uint16_t* dx,
                               int64_t lddx, st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && heads > 0 && kv_heads > 0 && D > 0 && D % 2 == 0,
               "st_rope_qkv_bwd: bad shape");
  if (B * S == 0) return ST_OK;
  ST_CHECK_ARG(dq && dk && dv && cos && sin && dx, "st_rope_qkv_bwd: NULL pointer");
  const int64_t width = (heads + 2 * kv_heads) * D;
  ST_CHECK_ARG(lddx >= width, "st_rope_qkv_bwd: lddx < (heads + 2*kv_heads)*D");
  const bool vec = D % 16 == 0 && lddx % 8 == 0 && B * S <= 0x7fffffff && width <= 0x7fffffff &&
                   (((uintptr_t)dq | (uintptr_t)dk | (uintptr_t)dv | (uintptr_t)cos |
                     (uintptr_t)sin | (uintptr_t)dx) & 15u) == 0;
  if (!vec) {
    int rc = st_rope_bwd(dq, cos, sin, B, S, heads, D, 1, dx, lddx, stream);
    if (!rc) rc = st_rope_bwd(dk, cos, sin, B, S, kv_heads, D, 1, dx + heads * D, lddx, stream);
    if (!rc)
      rc = st_rope_bwd(dv, cos, sin, B, S, kv_heads, D, 0, dx + (heads + kv_heads) * D, lddx,
                       stream);
    return rc;
  }
  QkvHeads qh{};
  qh.g[0] = dq; qh.g[1] = dk; qh.g[2] = dv;
  qh.h[0] = (int)heads; qh.h[1] = (int)kv_heads; qh.h[2] = (int)kv_heads;
  rope_qkv_bwd_vec<<<(unsigned)(B * S), NTH, 0, (hipStream_t)stream>>>(cos, sin, (int)S, (int)D,
                                                                      qh, dx, lddx);
  return st::check_launch("rope_qkv_bwd");
}

// Per-head q/k RMSNorm + rotation of a fused q|k|v row (Qwen3 qk_norm), one launch
extern "C" int st_rope_qkv_norm_fwd(const uint16_t* x, int64_t ldx, const uint16_t* cos,
                                    const uint16_t* sin, int64_t B, int64_t S, int64_t heads,
                                    int64_t kv_heads, int64_t D, const uint16_t* wq,
                                    const uint16_t* wk, float eps, uint16_t* q, uint16_t* k,
                                    uint16_t* v, float* rstd, st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && heads > 0 && kv_heads > 0 && (D == 64 || D == 128),
               "st_rope_qkv_norm_fwd: bad shape (D must be 64 or 128)");
  if (B * S == 0) return ST_OK;
  ST_CHECK_ARG(x && cos && sin && wq && wk && q && k && v && rstd,
               "st_rope_qkv_norm_fwd: NULL pointer");
  ST_CHECK_ARG(ldx >= (heads + 2 * kv_heads) * D && ldx % 8 == 0 && B * S <= 0x7fffffff,
               "st_rope_qkv_norm_fwd: ldx must be >= (heads + 2*kv_heads)*D and a multiple of 8");
  ST_CHECK_ARG(((((uintptr_t)x | (uintptr_t)cos | (uintptr_t)sin | (uintptr_t)wq |
                  (uintptr_t)wk | (uintptr_t)q | (uintptr_t)k | (uintptr_t)v) & 15u) == 0),
               "st_rope_qkv_norm_fwd: operands must be 16-byte aligned");
  QkvHeads qh{};
  qh.o[0] = q; qh.o[1] = k; qh.o[2] = v;
  qh.h[0] = (int)heads; qh.h[1] = (int)kv_heads; qh.h[2] = (int)kv_heads;
  if (D == 128)
    rope_qkv_norm_fwd<128><<<(unsigned)(B * S), NTH, 0, (hipStream_t)stream>>>(
        x, ldx, cos, sin, (int)S, qh, wq, wk, eps, rstd);
  else
    rope_qkv_norm_fwd<64><<<(unsigned)(B * S), NTH, 0, (hipStream_t)stream>>>(
        x, ldx, cos, sin, (int)S, qh, wq, wk, eps, rstd);
  return st::check_launch("rope_qkv_norm_fwd");
}

extern "C" int st_rope_qkv_norm_bwd(const uint16_t* dq, const uint16_t* dk, const uint16_t* dv,
                                    const uint16_t* x, int64_t ldx, const uint16_t* cos,
                                    const uint16_t* sin, const uint16_t* wq, const uint16_t* wk,
                                    const float* rstd, int64_t B, int64_t S, int64_t heads,
                                    int64_t kv_heads, int64_t D, uint16_t* dx, int64_t lddx,
                                    st_stream_t stream) {
  ST_CHECK_ARG(B >= 0 && S >= 0 && heads > 0 && kv_heads > 0 && (D == 64 || D == 128),
               "st_rope_qkv_norm_bwd: bad shape (D must be 64 or 128)");
  if (B * S == 0) return ST_OK;
  ST_CHECK_ARG(dq && dk && dv && x && cos && sin && wq && wk && rstd && dx,
               "st_rope_qkv_norm_bwd: NULL pointer");
  const int64_t width = (heads + 2 * kv_heads) * D;
  ST_CHECK_ARG(ldx >= width && lddx >= width && ldx % 8 == 0 && lddx % 8 == 0 &&
                   B * S <= 0x7fffffff,
               "st_rope_qkv_norm_bwd: row strides must be >= (heads + 2*kv_heads)*D, multiples of 8");
  ST_CHECK_ARG(((((uintptr_t)dq | (uintptr_t)dk | (uintptr_t)dv | (uintptr_t)x |
                  (uintptr_t)cos | (uintptr_t)sin | (uintptr_t)wq | (uintptr_t)wk |
                  (uintptr_t)dx) & 15u) == 0),
               "st_rope_qkv_norm_bwd: operands must be 16-byte aligned");
  QkvHeads qh{};
  qh.g[0] = dq; qh.g[1] = dk; qh.g[2] = dv;
  qh.h[0] = (int)heads; qh.h[1] = (int)kv_heads; qh.h[2] = (int)kv_heads;
  if (D == 128)
    rope_qkv_norm_bwd<128><<<(unsigned)(B * S), NTH, 0, (hipStream_t)stream>>>(
        x, ldx, cos, sin, (int)S, qh, wq, wk, rstd, dx, lddx);
  else
    rope_qkv_norm_bwd<64><<<(unsigned)(B * S), NTH, 0, (hipStream_t)stream>>>(
        x, ldx, cos, sin, (int)S, qh, wq, wk, rstd, dx, lddx);
  return st::check_launch("rope_qkv_norm_bwd");
}

extern "C" int st_heads_to_tokens(const uint16_t* x, int64_t B, int64_t S, int64_t heads,
                                  int64_t D, uint16_t* out, st_stream_t stream) {
  int64_t total = B * S * heads * D;
  ST_CHECK_ARG(B >= 0 && S >= 0 && heads >= 0 && D >= 0, "st_heads_to_tokens: bad shape");
  if (total == 0) return ST_OK;
  ST_CHECK_ARG(x && out, "st_heads_to_tokens: NULL pointer");
  relayout<<<nblk(total), NTH, 0, (hipStream_t)stream>>>(x, S, heads, D, total, 1, out);
  return st::check_launch("heads_to_tokens");
}

extern "C" int st_tokens_to_heads(const uint16_t* x, int64_t B, int64_t S, int64_t heads,
                                  int64_t D, uint16_t* out, st_stream_t stream) {
  int64_t total = B * S * heads * D;
  ST_CHECK_ARG(B >= 0 && S >= 0 && heads >= 0 && D >= 0, "st_tokens_to_heads: bad shape");
  if (total == 0) return ST_OK;
  ST_CHECK_ARG(x && out, "st_tokens_to_heads: NULL pointer");
  relayout<<<nblk(total), NTH, 0, (hipStream_t)stream>>>(x, S, heads, D, total, 0, out);
  return st::check_launch("tokens_to_heads");
}

extern "C" int st_swiglu_fwd(const uint16_t* g, int64_t ldg, const uint16_t* u, int64_t ldu,
                             int64_t rows, int64_t I, uint16_t* a, int64_t lda,
                             st_stream_t stream) {
  ST_CHECK_ARG(rows >= 0 && I > 0, "st_swiglu_fwd: bad shape");
  int64_t total = rows * I;
  if (total == 0) return ST_OK;
  ST_CHECK_ARG(g && u && a, "st_swiglu_fwd: NULL pointer");
  if (I % 8 == 0 && ldg % 8 == 0 && ldu % 8 == 0 && lda % 8 == 0 && vec8(g) && vec8(u) && vec8(a)) {
    swiglu_fwd_vec<<<nblk(total / 8), NTH, 0, (hipStream_t)stream>>>(g, ldg, u, ldu, I, total / 8,
                                                                       a, lda);
    return st::check_launch("swiglu_fwd");
  }
  swiglu_fwd<<<nblk(total), NTH, 0, (hipStream_t)stream>>>(g, ldg, u, ldu, I, total, a, lda);
  return st::check_launch("swiglu_fwd");
}

extern "C" int st_swiglu_bwd(const uint16_t* da, int64_t ldda, const uint16_t* g, int64_t ldg,
                             const uint16_t* u, int64_t ldu, int64_t rows, int64_t I,
                             uint16_t* dg, int64_t lddg, uint16_t* du, int64_t lddu,
                             st_stream_t stream) {
  ST_CHECK_ARG(rows >= 0 && I > 0, "st_swiglu_bwd: bad shape");
  int64_t total = rows * I;
  if (total == 0) return ST_OK;
  ST_CHECK_ARG(da && g && u && dg && du, "st_swiglu_bwd: NULL pointer");
  if (I % 8 == 0 && ldda % 8 == 0 && ldg % 8 == 0 && ldu % 8 == 0 && lddg % 8 == 0 &&
      lddu % 8 == 0 && vec8(da) && vec8(g) && vec8(u) && vec8(dg) && vec8(du)) {
    swiglu_bwd_vec<<<nblk(total / 8), NTH, 0, (hipStream_t)stream>>>(
        da, ldda, g, ldg, u, ldu, I, total / 8, dg, lddg, du, lddu);
    return st::check_launch("swiglu_bwd");
  }
  swiglu_bwd<<<nblk(total), NTH, 0, (hipStream_t)stream>>>(da, ldda, g, ldg, u, ldu, I, total, dg,
                                                           lddg, du, lddu);
  return st::check_launch("swiglu_bwd");
}
