// Mixture-of-experts pieces around the grouped 4-bit GEMM (gfx950):
// routers (softmax top-k; sigmoid group-limited top-k) and their VJPs, the
// token permutation, the weighted combine in the reference's bf16 order and
// its VJP, the gather-sum of permuted input gradients, and the grouped
// low-rank (LoRA) products over permuted rows.
#include "rank_r.h"

namespace {

constexpr int NTH = 256;
constexpr int MAXE = 512;  // experts per router (8 per lane of one wave)

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
  return v;
}
// larger value wins, equal values -> lower index
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const float ov = __shfl_xor(v, d);
    const int oi = __shfl_xor(i, d);
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
  }
}

// ---------------------------------------------------------------- softmax router
// One wave per token: fp32 softmax of bf16 logits, k-fold arg-max (ties to the
// lower expert), optional renormalisation, optional bf16 rounding.
__global__ __launch_bounds__(NTH) void route_softmax(const uint16_t* __restrict__ logits,
                                                     int64_t T, int E, int k, int norm,
                                                     int round_bf16, float* __restrict__ w_out,
                                                     int32_t* __restrict__ idx_out) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * (NTH / 64) + (threadIdx.x >> 6);
  if (t >= T) return;  // no barriers below
  float v[MAXE / 64];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < MAXE / 64; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? st::bf16_to_f32(logits[t * E + e]) : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
  mx = wave_max(mx);
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXE / 64; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? expf(v[i] - mx) : 0.0f;
    sum += v[i];
  }
  sum = wave_sum(sum);
  unsigned taken = 0;
#pragma unroll
  for (int i = 0; i < MAXE / 64; ++i) v[i] = v[i] / sum;
  float mine = 0.0f;
  int mine_i = 0;
  for (int j = 0; j < k; ++j) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < MAXE / 64; ++i) {
      const int e = lane + 64 * i;
      if (e < E && !((taken >> i) & 1u) && (v[i] > bv || (v[i] == bv && e < bi))) {
        bv = v[i];
        bi = e;
      }
    }
    wave_argmax(bv, bi);
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    if (lane == j) { mine = bv; mine_i = bi; }
  }
  if (norm) {
    const float s = wave_sum(lane < k ? mine : 0.0f);
    mine = mine / s;
  }
  if (round_bf16) mine = st::bf16r(mine);
  if (lane < k) {
    w_out[t * k + lane] = mine;
    idx_out[t * k + lane] = mine_i;
  }
}

// VJP of the softmax router w.r.t. the logits (selection has no gradient):
// dp[idx_j] = dw_j (through the renormalisation when enabled), then the
// softmax VJP p * (dp - sum p dp); result rounded to bf16 (bf16 logits).
__global__ __launch_bounds__(NTH) void route_softmax_bwd(const uint16_t* __restrict__ logits,
                                                         const int32_t* __restrict__ idx,
                                                         const float* __restrict__ dw,
                                                         int64_t T, int E, int k, int norm,
                                                         uint16_t* __restrict__ dlogits) {
  __shared__ float ps[NTH / 64][MAXE];
  __shared__ float dps[NTH / 64][MAXE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * (NTH / 64) + wave;
  const bool live = t < T;
  float v[MAXE / 64];
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < MAXE / 64; ++i) {
    const int e = lane + 64 * i;
    v[i] = (live && e < E) ? st::bf16_to_f32(logits[t * E + e]) : -INFINITY;
    mx = fmaxf(mx, v[i]);
  }
  mx = wave_max(mx);
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < MAXE / 64; ++i) {
    const int e = lane + 64 * i;
    v[i] = (live && e < E) ? expf(v[i] - mx) : 0.0f;
    sum += v[i];
  }
  sum = wave_sum(sum);
#pragma unroll
  for (int i = 0; i < MAXE / 64; ++i) {
    const int e = lane + 64 * i;
    v[i] = live ? v[i] / sum : 0.0f;
    if (e < E) { ps[wave][e] = v[i]; dps[wave][e] = 0.0f; }
  }
  __syncthreads();
  int ie = -1;
  float w = 0.0f, g = 0.0f;
  if (live && lane < k) {
    ie = idx[t * k + lane];
    if (ie < 0 || ie >= E) ie = -1;
    w = ie >= 0 ? ps[wave][ie] : 0.0f;
    g = dw[t * k + lane];
  }
  float dr = g;
  if (norm) {
    const float S = wave_sum(w);
    const float dot = wave_sum(g * w);
    dr = g / S - dot / (S * S);
  }
  const float gs = wave_sum(ie >= 0 ? w * dr : 0.0f);
  if (ie >= 0) dps[wave][ie] = dr;
  __syncthreads();
  if (live) {
#pragma unroll
    for (int i = 0; i < MAXE / 64; ++i) {
      const int e = lane + 64 * i;
      if (e < E) dlogits[t * E + e] = st::f32_to_bf16(v[i] * (dps[wave][e] - gs));
    }
  }
}

// ---------------------------------------------------------------- sigmoid router
// Group-limited routing: scores = sigmoid(logits); choice = scores + bias;
// group score = sum of the two largest choices in the group; keep the best
// group_k groups; top-k experts by choice among them (ties to the lower
// index); weights = scores at the picks, renormalised (+1e-20) and scaled.
__global__ __launch_bounds__(NTH) void route_sigmoid(const float* __restrict__ logits,
                                                     const float* __restrict__ bias, int64_t T,
                                                     int E, int groups, int group_k, int k,
                                                     int normalize, float scale,
                                                     float* __restrict__ w_out,
                                                     int32_t* __restrict__ idx_out) {
  __shared__ float cs[NTH / 64][MAXE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * (NTH / 64) + wave;
  const bool live = t < T;
  const int gs = E / groups;
  float sc[MAXE / 64], ch[MAXE / 64];
#pragma unroll
  for (int i = 0; i < MAXE / 64; ++i) {
    const int e = lane + 64 * i;
    const float x = (live && e < E) ? logits[t * E + e] : 0.0f;
    sc[i] = 1.0f / (1.0f + expf(-x));
    ch[i] = sc[i] + ((live && e < E) ? bias[e] : 0.0f);
    if (e < E) cs[wave][e] = ch[i];
  }
  __syncthreads();
  // lane g scores group g
  float gscore = -INFINITY;
  if (lane < groups) {
    float a = -INFINITY, b = -INFINITY;
    for (int q = 0; q < gs; ++q) {
      const float c = cs[wave][lane * gs + q];
      if (c > a) { b = a; a = c; } else if (c > b) { b = c; }
    }
    gscore = a + b;
  }
  unsigned long long allowed = 0;
  for (int j = 0; j < group_k; ++j) {
    float bv = (lane < groups && !((allowed >> lane) & 1ull)) ? gscore : -INFINITY;
    int bi = lane < groups && !((allowed >> lane) & 1ull) ? lane : 0x7fffffff;
    wave_argmax(bv, bi);
    if (bi < groups) allowed |= 1ull << bi;
  }
  unsigned taken = 0;
  float mine = 0.0f;
  int mine_i = 0;
  for (int j = 0; j < k; ++j) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < MAXE / 64; ++i) {
      const int e = lane + 64 * i;
      if (e < E && ((allowed >> (e / gs)) & 1ull) && !((taken >> i) & 1u) &&
          (ch[i] > bv || (ch[i] == bv && e < bi))) {
        bv = ch[i];
        bi = e;
      }
    }
    float sel = -INFINITY;  // score (not choice) of the pick
#pragma unroll
    for (int i = 0; i < MAXE / 64; ++i)
      if (lane + 64 * i == bi) sel = sc[i];
    wave_argmax(bv, bi);
    sel = __shfl(sel, bi & 63);
    if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    if (lane == j) { mine = sel; mine_i = bi; }
  }
  if (normalize) {
    const float s = wave_sum(lane < k ? mine : 0.0f);
    mine = mine / (s + 1e-20f);
  }
  mine = mine * scale;
  if (live && lane < k) {
    w_out[t * k + lane] = mine;
    idx_out[t * k + lane] = mine_i;
  }
}

// VJP of the sigmoid router w.r.t. its fp32 logits; unselected experts get 0.
__global__ __launch_bounds__(NTH) void route_sigmoid_bwd(const float* __restrict__ logits,
                                                         const int32_t* __restrict__ idx,
                                                         const float* __restrict__ dw,
                                                         int64_t T, int E, int k, int normalize,
                                                         float scale,
                                                         float* __restrict__ dlogits) {
  __shared__ float ds[NTH / 64][MAXE];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * (NTH / 64) + wave;
  const bool live = t < T;
  for (int e = lane; e < E; e += 64) ds[wave][e] = 0.0f;
  __syncthreads();
  int ie = -1;
  float s = 0.0f, g = 0.0f;
  if (live && lane < k) {
    ie = idx[t * k + lane];
    if (ie < 0 || ie >= E) ie = -1;
    s = ie >= 0 ? 1.0f / (1.0f + expf(-logits[t * E + ie])) : 0.0f;
    g = dw[t * k + lane];
  }
  float dsc = scale * g;
  if (normalize) {
    const float den = wave_sum(s) + 1e-20f;
    const float dot = wave_sum(g * s);
    dsc = scale * (g / den - dot / (den * den));
  }
  if (ie >= 0) ds[wave][ie] = dsc * (1.0f - s) * s;
  __syncthreads();
  if (live)
    for (int e = lane; e < E; e += 64) dlogits[t * E + e] = ds[wave][e];
}

// ---------------------------------------------------------------- permutation
// One workgroup per expert: every workgroup builds the expert histogram of
// all (token, slot) picks, takes its offset from the prefix, then places its
// picks in ascending (token, slot) order: row_token[row] = token of the pick,
// pick_row[token * k + slot] = its permuted row (-1 for an out-of-range
// expert).  Deterministic, no global atomics.  Wave w owns a contiguous block
// of picks and walks it in 64-pick rounds (coalesced loads, lane order = pick
// order, ballot ranks within a round); the waves' match counts are scanned
// once, so the placement needs no workgroup barrier per round.
constexpr int NTHP = 1024;
__global__ __launch_bounds__(NTHP) void permute(const int32_t* __restrict__ idx, int64_t n, int k,
                                                int E, int32_t* __restrict__ offsets,
                                                int32_t* __restrict__ row_token,
                                                int32_t* __restrict__ pick_row) {
  constexpr int NTH = NTHP, NW = NTH / 64;
  __shared__ int hist[1024];
  __shared__ int wsum[NW];
  __shared__ int base_s;
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < E; i += NTH) hist[i] = 0;
  __syncthreads();
  const int64_t blk = (n + NTH - 1) / NTH * 64;  // picks per wave, whole rounds
  const int64_t b0 = min(n, wave * blk), b1 = min(n, b0 + blk);
  const uint64_t below = (1ull << lane) - 1ull;
  // eight rounds of loads in flight at a time
  constexpr int U = 8;
  auto load = [&](int64_t c, int (&xs)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = c + u * 64 + lane;
      xs[u] = i < b1 ? idx[i] : -1;
    }
  };
  int cnt = 0;
  for (int64_t c = b0; c < b1; c += U * 64) {
    int xs[U];
    load(c, xs);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (xs[u] >= 0 && xs[u] < E) atomicAdd(&hist[xs[u]], 1);
      cnt += __popcll(__ballot(xs[u] == e));
    }
  }
  if (lane == 0) wsum[wave] = cnt;
  __syncthreads();  // the histogram and the wave counts are complete
  if (tid == 0) {
    int acc = 0;
    for (int i = 0; i < e; ++i) acc += hist[i];
    base_s = acc;
    if (e == 0) {
      int run = 0;
      for (int i = 0; i < E; ++i) {
        offsets[i] = run;
        run += hist[i];
      }
      offsets[E] = run;
    }
  }
  __syncthreads();
  int r = base_s;
  for (int w = 0; w < wave; ++w) r += wsum[w];
  for (int64_t c = b0; c < b1; c += U * 64) {
    int xs[U];
    load(c, xs);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = c + u * 64 + lane;
      const int x = xs[u];
      const uint64_t b = __ballot(x == e);
      if (x == e) {
        const int rr = r + __popcll(b & below);
        row_token[rr] = (int32_t)(i / k);
        pick_row[i] = rr;
      } else if (e == 0 && i < b1 && (x < 0 || x >= E)) {
        pick_row[i] = -1;
      }
      r += __popcll(b);
    }
  }
}

// ---------------------------------------------------------------- combine
// out[t] = bf16 running sum, in ascending expert order, of bf16(v[row] * w)
// over the token's picks: the order and roundings of the reference's per-expert
// index_add_ into a bf16 output.  One workgroup per token, 8 columns a thread.
constexpr int MAXK = 32;

__global__ __launch_bounds__(NTH) void combine(const uint16_t* __restrict__ v,
                                               const float* __restrict__ w,
                                               const int32_t* __restrict__ idx,
                                               const int32_t* __restrict__ pick_row, int64_t T,
                                               int k, int64_t H, int64_t R,
                                               uint16_t* __restrict__ out) {
  __shared__ int rows[MAXK];
  __shared__ float ws[MAXK];
  const int64_t t = blockIdx.x;
  if (threadIdx.x == 0) {  // insertion sort of the token's picks by expert
    int ex[MAXK];
    for (int j = 0; j < k; ++j) {
      int b = j - 1;
      const int ke = idx[t * k + j];
      while (b >= 0 && ex[b] > ke) {
        ex[b + 1] = ex[b]; rows[b + 1] = rows[b]; ws[b + 1] = ws[b];
        --b;
      }
      ex[b + 1] = ke;
      rows[b + 1] = pick_row[t * k + j];
      ws[b + 1] = w[t * k + j];
    }
  }
  __syncthreads();
  for (int64_t c = threadIdx.x * 8; c < H; c += NTH * 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int j = 0; j < k; ++j) {
      const int r = rows[j];
      if (r < 0 || r >= R) continue;
      const float wj = ws[j];
      const uint4 q = *(const uint4*)(v + (int64_t)r * H + c);
      const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = st::bf16_to_f32((uint16_t)(qw[e >> 1] >> (16 * (e & 1))));
        acc[e] = st::bf16r(acc[e] + st::bf16r(x * wj));
      }
    }
    *(uint4*)(out + t * H + c) =
        make_uint4(st::pack_bf16x2(acc[0], acc[1]), st::pack_bf16x2(acc[2], acc[3]),
                   st::pack_bf16x2(acc[4], acc[5]), st::pack_bf16x2(acc[6], acc[7]));
  }
}

// VJP of combine: dv[row] = bf16(dout[t] * w); dw = sum_h dout * v, with each
// product rounded to bf16 and the sum rounded to bf16 when the weights are
// bf16 (Qwen3), plain fp32 otherwise (fp32 weights, DeepSeek).
__global__ __launch_bounds__(NTH) void combine_bwd(const uint16_t* __restrict__ dout,
                                                   const uint16_t* __restrict__ v,
                                                   const float* __restrict__ w,
                                                   const int32_t* __restrict__ pick_row,
                                                   int64_t T, int k, int64_t H, int64_t R,
                                                   int bf16_weights, uint16_t* __restrict__ dv,
                                                   float* __restrict__ dw) {
  __shared__ float red[NTH / 64][MAXK];
  const int64_t t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int j = 0; j < k; ++j) {
    const int r = pick_row[t * k + j];
    const bool ok = r >= 0 && r < R;
    const float wj = w[t * k + j];
    float part = 0.0f;
    for (int64_t c = tid * 8; ok && c < H; c += NTH * 8) {
      const uint4 g = *(const uint4*)(dout + t * H + c);
      const uint4 q = *(const uint4*)(v + (int64_t)r * H + c);
      const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
      const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
      float gf[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        gf[e] = st::bf16_to_f32((uint16_t)(gw[e >> 1] >> (16 * (e & 1))));
        const float x = st::bf16_to_f32((uint16_t)(qw[e >> 1] >> (16 * (e & 1))));
        const float pr = gf[e] * x;
        part += bf16_weights ? st::bf16r(pr) : pr;
      }
      *(uint4*)(dv + (int64_t)r * H + c) =
          make_uint4(st::pack_bf16x2(gf[0] * wj, gf[1] * wj), st::pack_bf16x2(gf[2] * wj, gf[3] * wj),
                     st::pack_bf16x2(gf[4] * wj, gf[5] * wj), st::pack_bf16x2(gf[6] * wj, gf[7] * wj));
    }
    part = wave_sum(part);
    if (lane == 0) red[wave][j] = part;
  }
  __syncthreads();
  if (tid < k) {
    float s = 0.0f;
    for (int q = 0; q < NTH / 64; ++q) s += red[q][tid];
    dw[t * k + tid] = bf16_weights ? st::bf16r(s) : s;
  }
}

// out[t] = bf16( sum_j rows[pick_row[t, j]] + extra[t] ), fp32 accumulation.
__global__ __launch_bounds__(NTH) void gather_sum(const uint16_t* __restrict__ rows_in,
                                                  const int32_t* __restrict__ pick_row,
                                                  int64_t T, int k, int64_t H, int64_t R,
                                                  const void* __restrict__ extra, int extra_dtype,
                                                  uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.x;
  for (int64_t c = threadIdx.x * 8; c < H; c += NTH * 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (extra) {
      if (extra_dtype == ST_DTYPE_BF16) {
        const uint4 q = *(const uint4*)((const uint16_t*)extra + t * H + c);
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = st::bf16_to_f32((uint16_t)(qw[e >> 1] >> (16 * (e & 1))));
      } else {
        const float* x = (const float*)extra + t * H + c;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = x[e];
      }
    }
    for (int j = 0; j < k; ++j) {
      const int r = pick_row[t * k + j];
      if (r < 0 || r >= R) continue;
      const uint4 q = *(const uint4*)(rows_in + (int64_t)r * H + c);
      const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += st::bf16_to_f32((uint16_t)(qw[e >> 1] >> (16 * (e & 1))));
    }
    *(uint4*)(out + t * H + c) =
        make_uint4(st::pack_bf16x2(acc[0], acc[1]), st::pack_bf16x2(acc[2], acc[3]),
                   st::pack_bf16x2(acc[4], acc[5]), st::pack_bf16x2(acc[6], acc[7]));
  }
}

// ---------------------------------------------------------------- grouped low-rank
// out[m, j] = alpha * sum_k G[row(m), k] S_g[k, j]       (ROW: rows of one group per tile)
// out_g[m, j] = alpha * sum_{r in g} G[row(r), m] S[r, j] (COL: contraction over a group)
// G is bf16 (row gather optional), S fp32 split into three bf16 parts for the
// MFMA (st::split3: the exact fp32 products); grid.z selects a segment (LoRA
// of gate | up side by side).
constexpr int GK_BM = 128, GK_BK = 64, GK_RP = 64;
constexpr int GK_LD = GK_BK + 8;

struct GroupedRk {
  int64_t rows;     // permuted rows
  int64_t R;        // output columns of this launch (<= 64)
  int64_t Rseg;     // output columns per segment (segment z starts at z * Rseg)
  int64_t seg_len;  // ROW: contraction per segment; COL: G columns per segment
  const uint16_t* G;
  int64_t ldg, g_rows;
  const int32_t* gather;
  const float* S;
  int64_t ssk, ssj, s_gstride;
  const int32_t* offsets;
  int groups;
  float* out;
  int64_t o_gstride, so_m, so_j;
  float alpha;
  int accumulate;
  int vec;
};

template <bool COL>
__global__ __launch_bounds__(NTH) void grouped_rk(GroupedRk a) {
  __shared__ __attribute__((aligned(16))) uint16_t Gs[GK_BM * GK_LD];
  __shared__ __attribute__((aligned(16))) uint16_t Ss[st::RK_SPLIT * GK_RP * GK_LD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int z = blockIdx.z;
  int grp = 0;
  int64_t m0, mend, kb, ke;  // output-row tile and contraction range
  int64_t gcol0;             // first G column of this segment
  const float* S = a.S;
  if (!COL) {
    if (!st::find_group(a.offsets, a.groups, GK_BM, blockIdx.x, a.rows, grp, m0, mend)) return;
    kb = 0;
    ke = a.seg_len;
    gcol0 = (int64_t)z * a.seg_len;
    S += grp * a.s_gstride + (int64_t)z * a.seg_len * a.ssk;
  } else {
    grp = blockIdx.y;
    m0 = (int64_t)blockIdx.x * GK_BM;
    mend = a.seg_len;
    kb = a.offsets[grp];
    ke = a.offsets[grp + 1];
    if (kb < 0) kb = 0;
    if (ke > a.rows) ke = a.rows;
    gcol0 = (int64_t)z * a.seg_len;
    S += (int64_t)z * a.Rseg * a.ssj;
  }
  const int nb = a.R > 32 ? 2 : 1;
  const int RP = nb * 32;
  const int SIT = GK_BK * RP / NTH;
  auto grow = [&](int64_t r) -> int64_t {  // source row of permuted row r, -1 if invalid
    int64_t s = a.gather ? (int64_t)a.gather[r] : r;
    return (s >= 0 && s < a.g_rows) ? s : -1;
  };
  f32x16 acc[2];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.0f;

  // ROW: each thread owns 16-byte chunks of 4 tile rows, with their source rows
  int64_t srow[4];
  if (!COL) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t m = m0 + ((tid + i * NTH) >> 3);
      srow[i] = m < mend ? grow(m) : -1;
    }
  }
  uint4 gr[4];
  float sr[16];
  auto load = [&](int64_t k0) {
    if (!COL) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = (tid + i * NTH) & 7;
        const int64_t k = k0 + c * 8;
        const int64_t sm = srow[i];
        const uint16_t* src = a.G + sm * a.ldg + gcol0 + k;
        if (a.vec && sm >= 0 && k + 8 <= ke) {
          gr[i] = *(const uint4*)src;
        } else {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint32_t lo = (sm >= 0 && k + 2 * e < ke) ? src[2 * e] : 0u;
            uint32_t hi = (sm >= 0 && k + 2 * e + 1 < ke) ? src[2 * e + 1] : 0u;
            w[e] = lo | (hi << 16);
          }
          gr[i] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    } else {
      const int kg = tid >> 4, mg = tid & 15;
      const int64_t m = m0 + mg * 8;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const int64_t k = k0 + kg * 4 + h;
        const int64_t sr_ = k < ke ? grow(k) : -1;
        const uint16_t* src = a.G + sr_ * a.ldg + gcol0 + m;
        if (a.vec && sr_ >= 0 && m + 8 <= mend) {
          gr[h] = *(const uint4*)src;
        } else {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint32_t lo = (sr_ >= 0 && m + 2 * e < mend) ? src[2 * e] : 0u;
            uint32_t hi = (sr_ >= 0 && m + 2 * e + 1 < mend) ? src[2 * e + 1] : 0u;
            w[e] = lo | (hi << 16);
          }
          gr[h] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i >= SIT) break;
      const int e = tid + i * NTH;
      int kk, j;
      if (a.ssk == 1) { kk = e % GK_BK; j = e / GK_BK; } else { kk = e / RP; j = e % RP; }
      const int64_t k = k0 + kk;
      sr[i] = (k < ke && j < a.R) ? S[k * a.ssk + j * a.ssj] : 0.0f;
    }
  };
  auto store = [&]() {
    if (!COL) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int id = tid + i * NTH, row = id >> 3, c = id & 7;
        *(uint4*)&Gs[row * GK_LD + c * 8] = gr[i];
      }
    } else {  // [contraction][column] as loaded; the MFMA operand is read transposed
      const int kg = tid >> 4, mg = tid & 15;
#pragma unroll
      for (int h = 0; h < 4; ++h) ((uint4*)Gs)[st::trswz<GK_BM>(kg * 4 + h, mg)] = gr[h];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i >= SIT) break;
      const int e = tid + i * NTH;
      int kk, j;
      if (a.ssk == 1) { kk = e % GK_BK; j = e / GK_BK; } else { kk = e / RP; j = e % RP; }
      uint16_t hb, mb, lb;
      st::split3(sr[i], hb, mb, lb);
      Ss[j * GK_LD + kk] = hb;
      Ss[(GK_RP + j) * GK_LD + kk] = mb;
      Ss[(2 * GK_RP + j) * GK_LD + kk] = lb;
    }
  };

  if (kb < ke) load(kb);
  for (int64_t k0 = kb; k0 < ke; k0 += GK_BK) {
    store();
    __syncthreads();
    if (k0 + GK_BK < ke) load(k0 + GK_BK);
#pragma unroll
    for (int s = 0; s < GK_BK / 16; ++s) {
      const int ko = s * 16 + (lane >> 5) * 8;
      const bf16x8 av =
          COL ? st::tr_operand<GK_BM>((const uint4*)Gs, s * 16, wave * 32, lane)
              : *(const bf16x8*)&Gs[(wave * 32 + (lane & 31)) * GK_LD + ko];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        if (c >= nb) break;
#pragma unroll
        for (int h = 0; h < st::RK_SPLIT; ++h) {
          const bf16x8 bv = *(const bf16x8*)&Ss[(h * GK_RP + c * 32 + (lane & 31)) * GK_LD + ko];
          acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc[c], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }
  float* dst = a.out;
  int64_t om, oj;
  if (!COL) {
    om = a.so_m; oj = a.so_j;
    dst += (int64_t)z * a.Rseg * a.so_j;
  } else {
    om = a.so_m; oj = a.so_j;
    dst += grp * a.o_gstride + (int64_t)z * a.seg_len * a.so_m;
  }
  for (int c = 0; c < nb; ++c) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t m = m0 + wave * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
      const int j = c * 32 + (lane & 31);
      if (m < mend && j < a.R) {
        float* o = dst + m * om + j * oj;
        const float val = a.alpha * acc[c][v];
        *o = a.accumulate ? *o + val : val;
      }
    }
  }
}

// Streaming version of grouped_rk for 16-byte-aligned G rows (multiples of 8
// elements) below 2 GiB: st::rk_accumulate's prefetch ring and buffer loads.
// COL forms with a gather stage the group's source rows in LDS, GK_IDX at a
// time.  Same outputs, roundings and summation order per output as
// grouped_rk (ascending contraction in 64-wide MFMA steps).
constexpr int GK_IDX = 2048;

template <bool COL, bool SK1, int NB, bool GATHER>
__global__ __launch_bounds__(st::RK_NTH) void grouped_rk_stream(GroupedRk a, int64_t g_bytes) {
  __shared__ __attribute__((aligned(16))) uint16_t Gs[st::RK_BM * st::RK_LD];
  __shared__ __attribute__((aligned(16))) uint16_t Ss[st::RK_SS];
  __shared__ int idx[COL && GATHER ? GK_IDX : 1];
  const int tid = threadIdx.x;
  const int z = blockIdx.z;
  int grp = 0;
  int64_t m0, mend, kb, ke, gcol0 = (int64_t)z * a.seg_len;
  const float* S = a.S;
  if (!COL) {
    if (!st::find_group(a.offsets, a.groups, st::RK_BM, blockIdx.x, a.rows, grp, m0, mend)) return;
    kb = 0;
    ke = a.seg_len;
    S += grp * a.s_gstride + (int64_t)z * a.seg_len * a.ssk;
  } else {
    grp = blockIdx.y;
    m0 = (int64_t)blockIdx.x * st::RK_BM;
    mend = a.seg_len;
    kb = a.offsets[grp];
    ke = a.offsets[grp + 1];
    if (kb < 0) kb = 0;
    if (ke > a.rows) ke = a.rows;
    S += (int64_t)z * a.Rseg * a.ssj;
  }
  f32x16 acc[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[c][v] = 0.0f;
  if constexpr (COL && GATHER) {
    for (int64_t s0 = kb; s0 < ke; s0 += GK_IDX) {
      const int64_t s1 = s0 + GK_IDX < ke ? s0 + GK_IDX : ke;
      __syncthreads();  // the previous range's loads have read idx
      for (int64_t i = tid; i < s1 - s0; i += st::RK_NTH) idx[i] = a.gather[s0 + i];
      __syncthreads();
      st::rk_accumulate<true, SK1, NB, true>(acc, mend, a.R, m0, (int)s0, (int)s1, a.G, a.ldg,
                                             g_bytes, gcol0, S, a.ssk, a.ssj, 0x7fffffff,
                                             nullptr, a.g_rows, idx, (int)s0, Gs, Ss);
    }
  } else {
    // the valid mask of the contraction / rows is exact: S reads use an
    // open extent, every offset they form is in range
    st::rk_accumulate<COL, SK1, NB, GATHER>(acc, mend, a.R, m0, (int)kb, (int)ke, a.G, a.ldg,
                                            g_bytes, gcol0, S, a.ssk, a.ssj, 0x7fffffff,
                                            a.gather, a.g_rows, nullptr, 0, Gs, Ss);
  }
  float* dst = a.out;
  if (!COL)
    dst += (int64_t)z * a.Rseg * a.so_j;
  else
    dst += grp * a.o_gstride + (int64_t)z * a.seg_len * a.so_m;
#pragma unroll
  for (int c = 0; c < NB; ++c) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t m = m0 + st::rk_row(v);
      const int j = st::rk_col(c);
      if (m < mend && j < a.R) {
        float* o = dst + m * a.so_m + j * a.so_j;
        const float val = a.alpha * acc[c][v];
        *o = a.accumulate ? *o + val : val;
      }
    }
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Launches the streaming kernel when G qualifies; returns false otherwise.
template <bool COL>
bool launch_grouped_stream(const GroupedRk& a, dim3 grid, hipStream_t stream) {
  const int64_t g_bytes = a.g_rows * a.ldg * 2;
  if (!a.vec || g_bytes >= (1ll << 31)) return false;
  const bool sk1 = a.ssk == 1, nb2 = a.R > 32, gat = a.gather != nullptr;
  auto go = [&](auto kern) { kern<<<grid, st::RK_NTH, 0, stream>>>(a, g_bytes); };
  if (nb2) {
    if (gat) sk1 ? go(grouped_rk_stream<COL, true, 2, true>) : go(grouped_rk_stream<COL, false, 2, true>);
    else sk1 ? go(grouped_rk_stream<COL, true, 2, false>) : go(grouped_rk_stream<COL, false, 2, false>);
  } else {
    if (gat) sk1 ? go(grouped_rk_stream<COL, true, 1, true>) : go(grouped_rk_stream<COL, false, 1, true>);
    else sk1 ? go(grouped_rk_stream<COL, true, 1, false>) : go(grouped_rk_stream<COL, false, 1, false>);
  }
  return true;
}

}  // namespace

// ================================================================ C ABI
extern "C" int st_moe_route_softmax(const uint16_t* logits, int64_t tokens, int32_t experts,
                                    int32_t top_k, int32_t normalize, int32_t round_bf16,
                                    float* weights, int32_t* indices, st_stream_t stream) {
  ST_CHECK_ARG(tokens >= 0 && experts > 0 && experts <= MAXE && top_k > 0 && top_k <= MAXK &&
                   top_k <= experts,
               "st_moe_route_softmax: need 0 < top_k <= min(experts, %d), experts <= %d", MAXK,
               MAXE);
  if (tokens == 0) return ST_OK;
  ST_CHECK_ARG(logits && weights && indices, "st_moe_route_softmax: NULL pointer");
  route_softmax<<<(unsigned)st::cdiv(tokens, NTH / 64), NTH, 0, (hipStream_t)stream>>>(
      logits, tokens, experts, top_k, normalize, round_bf16, weights, indices);
  return st::check_launch("route_softmax");
}

extern "C" int st_moe_route_softmax_bwd(const uint16_t* logits, const int32_t* indices,
                                        const float* dweights, int64_t tokens, int32_t experts,
                                        int32_t top_k, int32_t normalize, uint16_t* dlogits,
                                        st_stream_t stream) {
  ST_CHECK_ARG(tokens >= 0 && experts > 0 && experts <= MAXE && top_k > 0 && top_k <= 64 &&
                   top_k <= experts,
               "st_moe_route_softmax_bwd: bad shape");
  if (tokens == 0) return ST_OK;
  ST_CHECK_ARG(logits && indices && dweights && dlogits, "st_moe_route_softmax_bwd: NULL pointer");
  route_softmax_bwd<<<(unsigned)st::cdiv(tokens, NTH / 64), NTH, 0, (hipStream_t)stream>>>(
      logits, indices, dweights, tokens, experts, top_k, normalize, dlogits);
  return st::check_launch("route_softmax_bwd");
}

extern "C" int st_moe_route_sigmoid(const float* logits, const float* bias, int64_t tokens,
                                    int32_t experts, int32_t groups, int32_t group_k,
                                    int32_t top_k, int32_t normalize, float scale, float* weights,
                                    int32_t* indices, st_stream_t stream) {
  ST_CHECK_ARG(tokens >= 0 && experts > 0 && experts <= MAXE && groups > 0 && groups <= 64 &&
                   experts % groups == 0 && experts / groups >= 2 && group_k > 0 &&
                   group_k <= groups && top_k > 0 && top_k <= MAXK &&
                   top_k <= group_k * (experts / groups),
               "st_moe_route_sigmoid: bad routing shape");
  if (tokens == 0) return ST_OK;
  ST_CHECK_ARG(logits && bias && weights && indices, "st_moe_route_sigmoid: NULL pointer");
  route_sigmoid<<<(unsigned)st::cdiv(tokens, NTH / 64), NTH, 0, (hipStream_t)stream>>>(
      logits, bias, tokens, experts, groups, group_k, top_k, normalize, scale, weights, indices);
  return st::check_launch("route_sigmoid");
}

extern "C" int st_moe_route_sigmoid_bwd(const float* logits, const int32_t* indices,
                                        const float* dweights, int64_t tokens, int32_t experts,
                                        int32_t top_k, int32_t normalize, float scale,
                                        float* dlogits, st_stream_t stream) {
  ST_CHECK_ARG(tokens >= 0 && experts > 0 && experts <= MAXE && top_k > 0 && top_k <= 64 &&
                   top_k <= experts,
               "st_moe_route_sigmoid_bwd: bad shape");
  if (tokens == 0) return ST_OK;
  ST_CHECK_ARG(logits && indices && dweights && dlogits, "st_moe_route_sigmoid_bwd: NULL pointer");
  route_sigmoid_bwd<<<(unsigned)st::cdiv(tokens, NTH / 64), NTH, 0, (hipStream_t)stream>>>(
      logits, indices, dweights, tokens, experts, top_k, normalize, scale, dlogits);
  return st::check_launch("route_sigmoid_bwd");
}

extern "C" int st_moe_permute(const int32_t* indices, int64_t tokens, int32_t top_k,
                              int32_t experts, int32_t* offsets, int32_t* row_token,
                              int32_t* pick_row, st_stream_t stream) {
  ST_CHECK_ARG(tokens >= 0 && top_k > 0 && experts > 0 && experts <= 1024,
               "st_moe_permute: need 0 < experts <= 1024");
  ST_CHECK_ARG(tokens * top_k < (1ll << 31), "st_moe_permute: too many picks");
  ST_CHECK_ARG(offsets && (tokens == 0 || (indices && row_token && pick_row)),
               "st_moe_permute: NULL pointer");
  permute<<<(unsigned)experts, NTHP, 0, (hipStream_t)stream>>>(
      indices, tokens * top_k, top_k, experts, offsets, row_token, pick_row);
  return st::check_launch("permute");
}

extern "C" int st_moe_combine(const uint16_t* values, int64_t rows, const float* weights,
                              const int32_t* indices, const int32_t* pick_row, int64_t tokens,
                              int32_t top_k, int64_t hidden, uint16_t* out, st_stream_t stream) {
  ST_CHECK_ARG(tokens >= 0 && top_k > 0 && top_k <= MAXK && hidden > 0 && rows >= 0,
               "st_moe_combine: need 0 < top_k <= %d", MAXK);
  if (tokens == 0) return ST_OK;
  ST_CHECK_ARG(values && weights && indices && pick_row && out, "st_moe_combine: NULL pointer");
  ST_CHECK_ARG(hidden % 8 == 0 && al16(values) && al16(out),
               "st_moe_combine: hidden must be a multiple of 8 with 16-byte aligned rows");
  combine<<<(unsigned)tokens, NTH, 0, (hipStream_t)stream>>>(values, weights, indices, pick_row,
                                                            tokens, top_k, hidden, rows, out);
  return st::check_launch("combine");
}

extern "C" int st_moe_combine_bwd(const uint16_t* dout, const uint16_t* values, int64_t rows,
                                  const float* weights, const int32_t* pick_row, int64_t tokens,
                                  int32_t top_k, int64_t hidden, int32_t bf16_weights,
                                  uint16_t* dvalues, float* dweights, st_stream_t stream) {
  ST_CHECK_ARG(tokens >= 0 && top_k > 0 && top_k <= MAXK && hidden > 0 && rows >= 0,
               "st_moe_combine_bwd: need 0 < top_k <= %d", MAXK);
  if (tokens == 0) return ST_OK;
  ST_CHECK_ARG(dout && values && weights && pick_row && dvalues && dweights,
               "st_moe_combine_bwd: NULL pointer");
  ST_CHECK_ARG(hidden % 8 == 0 && al16(dout) && al16(values) && al16(dvalues),
               "st_moe_combine_bwd: hidden must be a multiple of 8 with 16-byte aligned rows");
  combine_bwd<<<(unsigned)tokens, NTH, 0, (hipStream_t)stream>>>(
      dout, values, weights, pick_row, tokens, top_k, hidden, rows, bf16_weights, dvalues,
      dweights);
  return st::check_launch("combine_bwd");
}

extern "C" int st_moe_gather_sum(const uint16_t* rows_in, int64_t rows, const int32_t* pick_row,
                                 int64_t tokens, int32_t top_k, int64_t hidden, const void* extra,
                                 int32_t extra_dtype, uint16_t* out, st_stream_t stream) {
  ST_CHECK_ARG(tokens >= 0 && top_k > 0 && hidden > 0 && rows >= 0, "st_moe_gather_sum: bad shape");
  if (tokens == 0) return ST_OK;
  ST_CHECK_ARG(rows_in && pick_row && out, "st_moe_gather_sum: NULL pointer");
  ST_CHECK_ARG(!extra || extra_dtype == ST_DTYPE_BF16 || extra_dtype == ST_DTYPE_F32,
               "st_moe_gather_sum: extra dtype must be ST_DTYPE_BF16 or ST_DTYPE_F32");
  ST_CHECK_ARG(hidden % 8 == 0 && al16(rows_in) && al16(out) && (!extra || al16(extra)),
               "st_moe_gather_sum: hidden must be a multiple of 8 with 16-byte aligned rows");
  gather_sum<<<(unsigned)tokens, NTH, 0, (hipStream_t)stream>>>(rows_in, pick_row, tokens, top_k,
                                                               hidden, rows, extra, extra_dtype,
                                                               out);
  return st::check_launch("gather_sum");
}

extern "C" int st_moe_lora_rows(int64_t rows, int32_t R, int64_t seg_len, int32_t nseg,
                                const uint16_t* g, int64_t ldg, int64_t g_rows,
                                const int32_t* gather, const float* s, int64_t ssk, int64_t ssj,
                                int64_t s_gstride, const int32_t* offsets, int32_t groups,
                                float alpha, float* out, int64_t ldo, st_stream_t stream) {
  ST_CHECK_ARG(rows >= 0 && R > 0 && seg_len > 0 && nseg > 0 && groups > 0,
               "st_moe_lora_rows: need 0 < R");
  if (rows == 0) return ST_OK;
  ST_CHECK_ARG(g && s && offsets && out && ldo >= (int64_t)R * nseg,
               "st_moe_lora_rows: NULL pointer or ldo too small");
  ST_CHECK_ARG(ldg >= seg_len * nseg && (!gather || g_rows > 0),
               "st_moe_lora_rows: ldg < nseg * seg_len");
  GroupedRk a{};
  a.rows = rows; a.Rseg = R; a.seg_len = seg_len;
  a.G = g; a.ldg = ldg; a.g_rows = gather ? g_rows : rows; a.gather = gather;
  a.ssk = ssk; a.ssj = ssj; a.s_gstride = s_gstride;
  a.offsets = offsets; a.groups = groups;
  a.so_m = ldo; a.so_j = 1; a.alpha = alpha; a.accumulate = 0;
  a.vec = (al16(g) && ldg % 8 == 0 && seg_len % 8 == 0) ? 1 : 0;
  dim3 grid((unsigned)(st::cdiv(rows, GK_BM) + groups), 1, (unsigned)nseg);
  // output columns 64 at a time (one launch each)
  for (int32_t c0 = 0; c0 < R; c0 += 64) {
    a.R = R - c0 < 64 ? R - c0 : 64;
    a.S = s + c0 * ssj;
    a.out = out + c0;
    if (!launch_grouped_stream<false>(a, grid, (hipStream_t)stream))
      grouped_rk<false><<<grid, NTH, 0, (hipStream_t)stream>>>(a);
    if (int rc = st::check_launch("grouped_rk rows")) return rc;
  }
  return ST_OK;
}

extern "C" int st_moe_lora_grads(int64_t rows, int32_t R, int64_t seg_len, int32_t nseg,
                                 const uint16_t* g, int64_t ldg, int64_t g_rows,
                                 const int32_t* gather, const float* s, int64_t ssk, int64_t ssj,
                                 const int32_t* offsets, int32_t groups, float alpha, float* out,
                                 int64_t o_gstride, int64_t so_m, int64_t so_j,
                                 int32_t accumulate, st_stream_t stream) {
  ST_CHECK_ARG(rows >= 0 && R > 0 && seg_len > 0 && nseg > 0 && groups > 0,
               "st_moe_lora_grads: need 0 < R");
  ST_CHECK_ARG(offsets && out && (rows == 0 || (g && s)), "st_moe_lora_grads: NULL pointer");
  ST_CHECK_ARG(ldg >= seg_len * nseg, "st_moe_lora_grads: ldg < nseg * seg_len");
  GroupedRk a{};
  a.rows = rows; a.Rseg = R; a.seg_len = seg_len;
  a.G = g; a.ldg = ldg; a.g_rows = gather ? g_rows : rows; a.gather = gather;
  a.ssk = ssk; a.ssj = ssj;
  a.offsets = offsets; a.groups = groups;
  a.o_gstride = o_gstride; a.so_m = so_m; a.so_j = so_j;
  a.alpha = alpha; a.accumulate = accumulate;
  a.vec = (al16(g) && ldg % 8 == 0 && seg_len % 8 == 0) ? 1 : 0;
  dim3 grid((unsigned)st::cdiv(seg_len, GK_BM), (unsigned)groups, (unsigned)nseg);
  // output columns 64 at a time (one launch each)
  for (int32_t c0 = 0; c0 < R; c0 += 64) {
    a.R = R - c0 < 64 ? R - c0 : 64;
    a.S = s ? s + c0 * ssj : nullptr;
    a.out = out + c0 * so_j;
    if (!launch_grouped_stream<true>(a, grid, (hipStream_t)stream))
      grouped_rk<true><<<grid, NTH, 0, (hipStream_t)stream>>>(a);
    if (int rc = st::check_launch("grouped_rk grads")) return rc;
  }
  return ST_OK;
}
