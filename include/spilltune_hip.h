/*
 * spilltune_hip.h -- C ABI of the MI355X (gfx950) per-layer NF4 LoRA training
 * kernels (libspilltune_hip.so).
 *
 * Conventions
 *  - Every pointer is a device pointer owned by the caller (PyTorch tensors in
 *    the Python host), except `lut16` and `seg_end`, which are host arrays read
 *    during the call.  bf16 data is passed as uint16_t bit patterns.
 *  - Matrices are row-major; `ld*` arguments are row strides in elements.
 *  - Every call is asynchronous on `stream` (a hipStream_t) and stateless, so
 *    it may be issued from the autograd worker thread.  Nothing allocates:
 *    scratch comes in through `workspace`/`workspace_bytes`; the matching
 *    *_workspace_bytes() query says how much a call needs (0 = none).
 *  - Return value: ST_OK (0) or an ST_E* code; st_last_error() then returns a
 *    thread-local message.  The Python host maps ST_EINVAL/ST_EUNSUPPORTED to
 *    ValueError('unsupported_capability: ...') and ST_EDEVICE to RuntimeError,
 *    as the reference does for its own failures (config.py:34-62).
 *
 * Reference interfaces replaced (paths relative to /root/reference/src/
 * ram_vram_finetune):
 *  - quantization/codecs.py:158-170 decode_into and the bitsandbytes
 *    dequantize_4bit call at quantization/nf4_backend.py:312   -> st_dequant4*
 *  - finetune/lora.py:205-220 LoRAProjection.forward (base F.linear + fp32
 *    LoRA) and quantization/nf4_backend_cuda.py:888-917 linear_cuda
 *    (bnb.matmul_4bit)                                      -> st_q4_linear_fwd
 *  - the autograd VJP of the same projection inside training/recompute.py:
 *    102-105 (dX = dY W, dA, dB)           -> st_q4_linear_dgrad, st_lora_*
 *  - adapters/dense.py:115-117 rms, :137-141 rotate, :153 silu(gate)*up
 *                                          -> st_rmsnorm_*, st_rope_*, st_swiglu_*
 *  - adapters/dense.py:142-148 eager GQA attention -> st_flash_attn_*
 *  - adapters/deepseek.py:129-157 MLA attention (q/kv latent projections,
 *    shared rope key, qk 192 against v 128)   -> st_mla_*
 *  - adapters/qwen3_moe.py:95-113 and adapters/deepseek.py:115-176 (routers
 *    and the routed-expert loop)          -> st_moe_*, st_q4_grouped_*,
 *                                             st_linear_bf16_*
 */
#ifndef SPILLTUNE_HIP_H
#define SPILLTUNE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* st_stream_t; /* == hipStream_t */

enum {
  ST_OK = 0,
  ST_EINVAL = 1,       /* bad shape / pointer / alignment                */
  ST_EUNSUPPORTED = 2, /* valid request outside what the kernels support  */
  ST_EDEVICE = 3,      /* HIP runtime / launch failure                    */
  ST_EWORKSPACE = 4    /* workspace missing or too small                  */
};

/* storage flags */
#define ST_FLAG_HI_NIBBLE_FIRST 1 /* element 2i in the high nibble (bitsandbytes) */
#define ST_FLAG_GROUP64 2         /* fused GEMMs: one fp32 scale per 64 flat elements
                                     (bitsandbytes' blocksize) instead of 128 */

/* dtype codes for st_lora_gemm operands */
#define ST_DTYPE_BF16 0
#define ST_DTYPE_F32 1

int st_abi_version(void);
const char* st_last_error(void);

/* ---------------------------------------------------------------- dequant */
/*
 * out[i] = bf16_rne(lut16[code_i] * scales[i / group]) for i < numel, codes
 * packed two per byte (low nibble first unless ST_FLAG_HI_NIBBLE_FIRST),
 * groups over the FLATTENED tensor (they straddle rows when K % group != 0).
 * group is 64 or 128.  Replaces codecs.py:158-170 (lut16[c] = c - 8 for
 * int4-sym-g128) and the NF4 decode of nf4_backend.py:312.
 */
int st_dequant4(const uint8_t* payload, const float* scales, int64_t numel, int32_t group,
                const float* lut16, int32_t flags, uint16_t* out, st_stream_t stream);

/*
 * Block scales of bitsandbytes' double-quantised NF4 state (blocksize 64,
 * nested blocksize 256; nf4_backend.py:200-240 state layout, :292-298
 * quantize_4bit(blocksize=64, compress_statistics=True); staged on the device
 * by nf4_backend_cuda.py:748-837 and consumed by linear_cuda -> matmul_4bit,
 * nf4_backend_cuda.py:888-917):
 *   scales[j] = fp32( fp32(nested_map[absmax_q[j]] * nested_absmax[j / nested_block])
 *                     + offset )                      for j < blocks
 * (no fused multiply-add).  The result is the fp32 per-64 scale array the
 * fused GEMMs and st_dequant4 (group 64) take with the high-nibble-first
 * payload as it lies.  nested_map has 256 entries.
 */
int st_nf4_dq_scales(const uint8_t* absmax_q, const float* nested_absmax, const float* nested_map,
                     float offset, int64_t blocks, int32_t nested_block, float* scales,
                     st_stream_t stream);

/* ------------------------------------------------- fused projection GEMMs */
/*
 * Forward of a frozen 4-bit projection with LoRA (lora.py:218-220):
 *   base[m,n] = bf16( sum_k x[m,k] * W[n,k] )            (W = dequant, bf16)
 *   y[m,n]    = bf16( base + lora_scale * sum_j t[m, seg(n)*rank + j] * lora_b[n,j] )
 *   y[m,n]    = bf16( residual[m,n] + y[m,n] )            (if residual)
 * W [N,K] is payload/scales in flat groups of 128 (64 with ST_FLAG_GROUP64:
 * bitsandbytes' NF4 blocksize, scales from st_nf4_dq_scales), dequantised
 * inside the GEMM and never written to HBM as bf16 (K % group != 0, where
 * the groups straddle W's rows: each packed word reads its own group's
 * scale).  K % 8 == 0.  `workspace`: split-K partials for shapes whose
 * 256x128 tiles leave CUs idle on a long contraction (fp32 [splits, M, N],
 * summed in split order by a second kernel before the epilogue); the query
 * returns the bytes it takes, 0 when the shape runs unsplit.  Without that
 * workspace the call runs unsplit (same epilogue, another fp32 order).
 * `t` = x_f32 A_cat^T from st_lora_gemm ([M, nseg*rank] fp32) or NULL for no
 * LoRA; any rank >= 1 (up to 65536 T columns).  The epilogue stages t and
 * lora_b in the tile's LDS; when they do not fit (more than 64 T columns on
 * the 256-wide tiles), the GEMM runs on 128x128 tiles whose epilogue reads
 * them from global memory (L2), with the same products in the same order.
 * nseg/seg_end describe N-concatenated projections (fused q|k|v, gate|up):
 * column n belongs to segment s = #{seg_end[i] <= n}; segment ends must be
 * multiples of 32.  nseg = 1 with seg_end[0] = N for a single projection.
 */
int64_t st_q4_linear_fwd_workspace_bytes(int64_t M, int64_t N, int64_t K);
int st_q4_linear_fwd(const uint16_t* x, int64_t M, int64_t K, int64_t ldx,
                     const uint8_t* payload, const float* scales, int64_t N,
                     const float* lut16, int32_t flags,
                     const float* t, int64_t ldt, const float* lora_b, int32_t rank,
                     float lora_scale, int32_t nseg, const int64_t* seg_end,
                     const uint16_t* residual, int64_t ldr,
                     uint16_t* y, int64_t ldy,
                     void* workspace, int64_t workspace_bytes, st_stream_t stream);

/*
 * Input gradient of the same projection (autograd of lora.py:218-220):
 *   dx[m,k] = bf16( bf16(sum_n dy[m,n] W[n,k]) + bf16(sum_j dt[m,j] lora_a[j,k]) )
 * with dt = lora_scale * dy_f32 B ([M, lora_k] fp32, from st_lora_bwd_dy;
 * N-concatenated projections stack their dt columns and lora_a rows) or
 * dt == NULL for no LoRA term; 1 <= lora_k <= 65536 (operands beyond the
 * tile's LDS as in the forward).  W [N,K] as above,
 * dequantised into LDS in its natural orientation and read transposed.
 * `workspace` as in the forward (the split runs over N).
 */
int64_t st_q4_linear_dgrad_workspace_bytes(int64_t M, int64_t N, int64_t K);
int st_q4_linear_dgrad(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                       const uint8_t* payload, const float* scales, int64_t K,
                       const float* lut16, int32_t flags,
                       const float* dt, int64_t lddt, const float* lora_a, int32_t lora_k,
                       uint16_t* dx, int64_t lddx,
                       void* workspace, int64_t workspace_bytes, st_stream_t stream);

/*
 * The same input gradient for a projection that reads silu(gate) * up of a
 * fused gate|up pre-activation gu [M, 2I] (row stride ldgu): instead of dx,
 * the epilogue applies the SwiGLU VJP of dense.py:153 to each bf16 dx value
 * (the roundings of st_swiglu_bwd) and writes dgu[m, i] = dgate and
 * dgu[m, I + i] = dup (row stride lddgu).  I is this projection's in_features.
 * gu and dgu must be 16-byte aligned with ldgu, lddgu and I multiples of 8
 * (ST_EUNSUPPORTED otherwise).
 */
int st_q4_linear_dgrad_swiglu(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                              const uint8_t* payload, const float* scales, int64_t I,
                              const float* lut16, int32_t flags,
                              const float* dt, int64_t lddt, const float* lora_a, int32_t lora_k,
                              const uint16_t* gu, int64_t ldgu, uint16_t* dgu, int64_t lddgu,
                              void* workspace, int64_t workspace_bytes, st_stream_t stream);

/* ------------------------------------------------------- LoRA rank-r work */
/*
 * Generic skinny fp32-accumulating product used by the LoRA terms:
 *   out[m,n] = (accumulate ? out[m,n] : 0) + alpha * sum_k a(m,k) * b(k,n)
 * a(m,k) = a[m*sam + k*sak], b(k,n) = b[k*sbk + n*sbn], each bf16 or fp32.
 * With one bf16 and one fp32 operand the product streams the bf16 one and
 * takes the fp32 one 64 columns at a time.  st_lora_gemm_workspace_bytes is
 * the size that runs every 64-column chunk in one launch; a workspace down to
 * one chunk's split-K partials runs the chunks in turn, with the same bits.
 * Products whose row tiles and column chunks fill the GPU by themselves run
 * without a split and use no workspace.
 */
int64_t st_lora_gemm_workspace_bytes(int64_t Mo, int64_t No, int64_t Kc);
int st_lora_gemm(int64_t Mo, int64_t No, int64_t Kc,
                 const void* a, int32_t a_dtype, int64_t sam, int64_t sak,
                 const void* b, int32_t b_dtype, int64_t sbk, int64_t sbn,
                 float alpha, float* out, int64_t ldo, int32_t accumulate,
                 void* workspace, int64_t workspace_bytes, st_stream_t stream);

/*
 * st_lora_gemm without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The split-K partials live in
 * a static 32 MiB device array of the library (one per GPU, held until the
 * process ends); a product whose partials need more even one 64-column chunk
 * at a time is rejected with ST_EUNSUPPORTED.  Nothing is allocated or freed.
 * Every call on one GPU shares that array: calls that overlap in time on one
 * GPU (two streams, two threads) race and must be ordered by the caller.
 * Results equal st_lora_gemm's bit for bit (same kernels, same order).
 */
int st_lora_gemm_noalloc(int64_t Mo, int64_t No, int64_t Kc,
                         const void* a, int32_t a_dtype, int64_t sam, int64_t sak,
                         const void* b, int32_t b_dtype, int64_t sbk, int64_t sbn,
                         float alpha, float* out, int64_t ldo, int32_t accumulate,
                         st_stream_t stream);

/*
 * The two products of the LoRA VJP that read dY (the autograd of
 * finetune/lora.py:219 inside training/recompute.py:102-105), for a
 * projection of nseg N-concatenated segments (ends seg_end[], rank r each):
 *   dt[m, s*r + j] = scale * sum_{n in seg s} dy_f32[m, n] * b[n, j]
 *   db[n, j]       = scale * sum_m dy_f32[m, n] * t[m, s*r + j]   (n in seg s)
 * dy [M, N] bf16 (lddy), b [N, r] fp32 (the segments' B stacked), t [M, nseg*r]
 * fp32 (ldt; the forward's x_f32 A_cat^T), dt [M, nseg*r] (lddt), db [N, r].
 * All 2*nseg products run in one launch, their split-K sums in one more (fixed
 * order).  nseg <= 8, r <= 64; segment starts and widths must be multiples of
 * 8 (the workspace query returns 0 otherwise, a rank above 64 included: use
 * st_lora_gemm per product).
 * db == NULL runs the dt products only (db formed later, e.g. by st_rk_batch).
 */
int64_t st_lora_bwd_dy_workspace_bytes(int64_t M, int64_t N, int32_t rank, int32_t nseg,
                                       const int64_t* seg_end);
int st_lora_bwd_dy(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                   const float* b, const float* t, int64_t ldt, int32_t rank,
                   int32_t nseg, const int64_t* seg_end, float scale,
                   float* dt, int64_t lddt, float* db,
                   void* workspace, int64_t workspace_bytes, st_stream_t stream);

/*
 * Independent rank-r products in one launch (+ one fixed-order reduction):
 * the deferred adapter gradients of a layer's backward (dB_s = s*dY_s^T*T_s and
 * dA_s = dT_s^T*x for every projection of the layer, training/recompute.py:
 * 102-133 / finetune/lora.py:219), written straight into the adapters' gradient
 * buffers (accumulate: add, as across microbatches of an accumulation window).
 * Each product: out[m*so_m + j*so_j] (+)= alpha * sum_{k<Kc} g(m,k) * S[k*ssk + j*ssj]
 * for m < big, j < r (r <= 64), with g(m,k) = G[m*ldg + k] (col = 0) or
 * G[k*ldg + m] (col = 1), G bf16 with 16-byte aligned rows of multiples of 8.
 * n <= 16 products per call.
 */
typedef struct st_rk_product {
  const uint16_t* G;
  int64_t ldg;
  int32_t col;
  const float* S;
  int64_t ssk, ssj;
  int64_t big, r, Kc;
  float alpha;
  float* out;
  int64_t so_m, so_j;
  int32_t accumulate;
} st_rk_product;
int64_t st_rk_batch_workspace_bytes(int32_t n, const st_rk_product* products);
int st_rk_batch(int32_t n, const st_rk_product* products, void* workspace,
                int64_t workspace_bytes, st_stream_t stream);

/* ------------------------------------------------------- layer elementwise */
/* y = w * bf16(x * rsqrt(mean(x^2) + eps)) (dense.py:115-117); rstd[row] saved. */
int st_rmsnorm_fwd(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t H, float eps,
                   uint16_t* y, float* rstd, st_stream_t stream);
/* dx = bf16(VJP of the above) [+ dres, added in bf16 like autograd's sum]. */
int st_rmsnorm_bwd(const uint16_t* dy, const uint16_t* x, const uint16_t* w, const float* rstd,
                   const uint16_t* dres, int64_t rows, int64_t H, uint16_t* dx,
                   st_stream_t stream);

/*
 * Rotary embedding (dense.py:137-141) fused with the [B,S,heads,D] ->
 * [B,heads,S,D] relayout: out = bf16(bf16(x*cos) + bf16(rot(x)*sin)), rot(x) =
 * cat(-x[D/2:], x[:D/2]); cos/sin are [B,S,D] bf16.  rotate = 0 copies only
 * (the value projection).  x rows have stride ldx elements.
 */
int st_rope_fwd(const uint16_t* x, int64_t ldx, const uint16_t* cos, const uint16_t* sin,
                int64_t B, int64_t S, int64_t heads, int64_t D, int32_t rotate,
                uint16_t* out, st_stream_t stream);
/* VJP of st_rope_fwd: dout [B,heads,S,D] -> dx rows of stride lddx. */
int st_rope_bwd(const uint16_t* dout, const uint16_t* cos, const uint16_t* sin,
                int64_t B, int64_t S, int64_t heads, int64_t D, int32_t rotate,
                uint16_t* dx, int64_t lddx, st_stream_t stream);
/* st_rope_fwd of a fused q|k|v projection output in one launch (dense.py:135-141
 * for q and k, the plain view/transpose for v): x rows of stride ldx hold the
 * heads*D query, kv_heads*D key and kv_heads*D value columns; q [B,heads,S,D],
 * k and v [B,kv_heads,S,D].  Same results as three st_rope_fwd calls. */
int st_rope_qkv_fwd(const uint16_t* x, int64_t ldx, const uint16_t* cos, const uint16_t* sin,
                    int64_t B, int64_t S, int64_t heads, int64_t kv_heads, int64_t D,
                    uint16_t* q, uint16_t* k, uint16_t* v, st_stream_t stream);
/* VJP of st_rope_qkv_fwd: dq, dk, dv head-major -> dx rows of stride lddx. */
int st_rope_qkv_bwd(const uint16_t* dq, const uint16_t* dk, const uint16_t* dv,
                    const uint16_t* cos, const uint16_t* sin, int64_t B, int64_t S,
                    int64_t heads, int64_t kv_heads, int64_t D, uint16_t* dx, int64_t lddx,
                    st_stream_t stream);
/* Qwen3 qk_norm fused with st_rope_qkv_fwd (dense.py:128-141 with qk_norm):
 * every query head and key head of the fused q|k|v rows is RMS-normalised over
 * its D elements (weights wq / wk [D], eps; rounding of st_rmsnorm_fwd) and
 * then rotated; value heads are copied.  rstd [B*S, heads+kv_heads] fp32 is
 * kept for the backward.  D = 64 or 128, 16-byte aligned operands. */
int st_rope_qkv_norm_fwd(const uint16_t* x, int64_t ldx, const uint16_t* cos, const uint16_t* sin,
                         int64_t B, int64_t S, int64_t heads, int64_t kv_heads, int64_t D,
                         const uint16_t* wq, const uint16_t* wk, float eps, uint16_t* q,
                         uint16_t* k, uint16_t* v, float* rstd, st_stream_t stream);
/* VJP of st_rope_qkv_norm_fwd (x: the forward's input rows): the rotation's
 * VJP then the norm's (rounding of st_rope_qkv_bwd, st_rmsnorm_bwd); dx rows
 * of stride lddx. */
int st_rope_qkv_norm_bwd(const uint16_t* dq, const uint16_t* dk, const uint16_t* dv,
                         const uint16_t* x, int64_t ldx, const uint16_t* cos, const uint16_t* sin,
                         const uint16_t* wq, const uint16_t* wk, const float* rstd, int64_t B,
                         int64_t S, int64_t heads, int64_t kv_heads, int64_t D, uint16_t* dx,
                         int64_t lddx, st_stream_t stream);
/* [B,heads,S,D] -> [B,S,heads*D] copy (attention output relayout). */
int st_heads_to_tokens(const uint16_t* x, int64_t B, int64_t S, int64_t heads, int64_t D,
                       uint16_t* out, st_stream_t stream);
int st_tokens_to_heads(const uint16_t* x, int64_t B, int64_t S, int64_t heads, int64_t D,
                       uint16_t* out, st_stream_t stream);

/* a = bf16(bf16(silu(g)) * u) (dense.py:153); g/u rows of stride ldg/ldu. */
int st_swiglu_fwd(const uint16_t* g, int64_t ldg, const uint16_t* u, int64_t ldu,
                  int64_t rows, int64_t I, uint16_t* a, int64_t lda, st_stream_t stream);
int st_swiglu_bwd(const uint16_t* da, int64_t ldda, const uint16_t* g, int64_t ldg,
                  const uint16_t* u, int64_t ldu, int64_t rows, int64_t I,
                  uint16_t* dg, int64_t lddg, uint16_t* du, int64_t lddu, st_stream_t stream);

/* ---------------------------------------------------------------------
 * Causal GQA flash attention, replacing the eager chain of
 * adapters/dense.py:142-148 (repeat k/v over the group, scores = q k^T *
 * scale + causal mask, fp32 softmax, probabilities @ v, relayout to tokens).
 * q [B,H,S,D], k/v [B,Hkv,S,D] head-major bf16; D in {64, 128}; any S >= 0.
 * kv_len: NULL (every key valid) or a device int32 [B] of valid key counts
 * for right-padded rows (dense.py:237-246): keys >= kv_len[b] are masked for
 * every query of row b, padded queries included, as the reference's additive
 * finfo.min mask does; values are clamped to [1, S].
 * out is token-major [B,S,H*D] bf16; lse [B,H,S] fp32 is the base-2
 * log-sum-exp of scale*log2(e)*q.k per query (the backward's statistics).
 * Probabilities are kept in fp32 until the bf16 P.V product (the reference
 * rounds the normalised probabilities to bf16 first; within bf16 tolerance).
 * --------------------------------------------------------------------- */
int64_t st_flash_attn_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t Hkv, int64_t D,
                                      int32_t backward);
int st_flash_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t B,
                      int64_t S, int64_t H, int64_t Hkv, int64_t D, float scale,
                      const int32_t* kv_len, uint16_t* out, float* lse, void* workspace,
                      int64_t workspace_bytes, st_stream_t stream);
/* VJP of st_flash_attn_fwd (autograd of dense.py:142-148): from dout
 * (token-major [B,S,H*D]), the forward's out and lse, writes dq [B,H,S,D]
 * and dk, dv [B,Hkv,S,D] head-major bf16 (GQA group sums in fp32, one
 * rounding; with H == Hkv the dK/dV pass writes them directly and the
 * workspace holds no fp32 partials).  Deterministic: no atomics.  kv_len as
 * in the forward (masked keys get zero dk, dv). */
int st_flash_attn_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                      const uint16_t* out, const float* lse, const uint16_t* dout, int64_t B,
                      int64_t S, int64_t H, int64_t Hkv, int64_t D, float scale,
                      const int32_t* kv_len, uint16_t* dq, uint16_t* dk, uint16_t* dv,
                      void* workspace, int64_t workspace_bytes, st_stream_t stream);

/* ---------------------------------------------------------------------
 * Causal multi-head latent attention of DeepSeek-V3 (adapters/deepseek.py:
 * 150-153: query = cat(q_nope, rotate(q_rope)), key = cat(k_nope,
 * rotate(k_rope) shared by every head), scores * attention_scale + causal
 * mask, fp32 softmax, probabilities @ value), the same flash kernels with
 * query/key heads of DQ and value heads of DV: q, k [B,H,S,DQ], v [B,H,S,DV]
 * head-major bf16 (no grouping: every head has its own key); out token-major
 * [B,S,H*DV]; lse [B,H,S] and kv_len as st_flash_attn_fwd.  (DQ, DV) =
 * (192, 128), the V3 shape (qk_nope 128 + qk_rope 64, v 128), or 64/64,
 * 128/128.
 * --------------------------------------------------------------------- */
/* Query/key/value assembly of deepseek.py:137-150 (and its VJP): from q
 * [M, H*(nope+rope)] (row stride ldq; per head q_nope | q_rope), kv
 * [M, H*(nope+v_dim)] (ldkv; per head k_nope | value) and the shared rope key
 * kr [M, rope] (ldkr; the last rope columns of kv_a_proj_with_mqa), M = B*S
 * token rows, writes Q = cat(q_nope, rotate(q_rope)) and K = cat(k_nope,
 * rotate(kr)) [B,H,S,nope+rope] and V [B,H,S,v_dim].  rotate is the default
 * (t*cos + cat(-t2, t1)*sin) or, with interleave, the pairwise form of
 * deepseek.py:146-148; cos/sin [B,S,rope] bf16; every product and sum rounds to
 * bf16 as the reference's bf16 ops do.  nope, v_dim % 8 == 0; rope % 16 == 0,
 * rope <= 128 and dividing 256. */
int st_mla_rope_fwd(const uint16_t* q, int64_t ldq, const uint16_t* kv, int64_t ldkv,
                    const uint16_t* kr, int64_t ldkr, const uint16_t* cos, const uint16_t* sin,
                    int64_t B, int64_t S, int64_t H, int64_t nope, int64_t rope, int64_t v_dim,
                    int32_t interleave, uint16_t* Q, uint16_t* K, uint16_t* V,
                    st_stream_t stream);
/* VJP: dq [M, H*(nope+rope)], dkv [M, H*(nope+v_dim)] and dkr [M, rope] (the
 * rope key's gradient: the sum over heads of dK's rope part, rounded once to
 * bf16, through the VJP of rotate). */
int st_mla_rope_bwd(const uint16_t* dQ, const uint16_t* dK, const uint16_t* dV,
                    const uint16_t* cos, const uint16_t* sin, int64_t B, int64_t S, int64_t H,
                    int64_t nope, int64_t rope, int64_t v_dim, int32_t interleave, uint16_t* dq,
                    int64_t lddq, uint16_t* dkv, int64_t lddkv, uint16_t* dkr, int64_t lddkr,
                    st_stream_t stream);
int64_t st_mla_attn_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t DQ, int64_t DV,
                                    int32_t backward);
int st_mla_attn_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t B,
                    int64_t S, int64_t H, int64_t DQ, int64_t DV, float scale,
                    const int32_t* kv_len, uint16_t* out, float* lse, void* workspace,
                    int64_t workspace_bytes, st_stream_t stream);
/* VJP of st_mla_attn_fwd: dq, dk [B,H,S,DQ], dv [B,H,S,DV]. */
int st_mla_attn_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                    const uint16_t* out, const float* lse, const uint16_t* dout, int64_t B,
                    int64_t S, int64_t H, int64_t DQ, int64_t DV, float scale,
                    const int32_t* kv_len, uint16_t* dq, uint16_t* dk, uint16_t* dv,
                    void* workspace, int64_t workspace_bytes, st_stream_t stream);

/* ---------------------------------------------------------------------
 * Plain bf16 linear (router logits and their input gradient).
 * y[M,N] = bf16(x[M,K] . w[N,K]^T);  dx[M,K] = bf16(dy[M,N] . w[N,K]).
 * Replaces F.linear(flat, weights['mlp.gate.weight']) in
 * adapters/qwen3_moe.py:97 and its autograd input gradient.
 * Rows must be 16-byte aligned multiples of 8 elements.
 * --------------------------------------------------------------------- */
int st_linear_bf16_fwd(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, const uint16_t* w,
                       int64_t N, int64_t ldw, uint16_t* y, int64_t ldy, st_stream_t stream);
int st_linear_bf16_dgrad(const uint16_t* dy, int64_t M, int64_t N, int64_t lddy,
                         const uint16_t* w, int64_t K, int64_t ldw, uint16_t* dx, int64_t lddx,
                         st_stream_t stream);

/* Causal-LM terminal, one row of logits per workgroup, in place
 * (training/engine.py:58-75; quantization/native_terminal.py:11-32 replace
 * logits.float() -> F.cross_entropy(sum, ignore_index) and its VJP):
 *   loss_rows[r] = logsumexp(x_r) - x_r[labels[r]]   (0 for ignore_index rows)
 *   logits[r][c] <- bf16((softmax(x_r)[c] - [c == labels[r]]) * grad_scale)
 * with x_r the fp32 values of the bf16 row (row stride ld >= vocab).  Labels
 * must be ignore_index or in [0, vocab) (checked by the caller); grad_scale is
 * 1/normalization.  Pair with st_linear_bf16_fwd (logits = h head^T) before
 * and st_linear_bf16_dgrad (dh = dlogits head) after. */
int st_cross_entropy_rows(uint16_t* logits, int64_t rows, int64_t vocab, int64_t ld,
                          const int64_t* labels, int64_t ignore_index, float grad_scale,
                          float* loss_rows, st_stream_t stream);

/* ---------------------------------------------------------------------
 * Mixture of experts (adapters/qwen3_moe.py:95-113; adapters/deepseek.py:
 * 115-176).  Tokens T, picks per token k, experts E; a "pick" is (token t,
 * slot j) at flat index t*k + j; permuted rows list the picks grouped by
 * expert (ascending), inside an expert in ascending pick order.
 * --------------------------------------------------------------------- */

/* Softmax router, qwen3_moe.py:97-100: p = softmax_fp32(logits); top-k by
 * value (descending; equal values -> lower expert, torch leaves tie order
 * unspecified); if normalize, w /= sum(w); if round_bf16, w is rounded to
 * bf16 (the reference's routing.to(logits.dtype)).  logits bf16 [T,E],
 * E <= 512, k <= 32; weights fp32 [T,k], indices int32 [T,k]. */
int st_moe_route_softmax(const uint16_t* logits, int64_t tokens, int32_t experts, int32_t top_k,
                         int32_t normalize, int32_t round_bf16, float* weights, int32_t* indices,
                         st_stream_t stream);
/* VJP of the above w.r.t. logits for given picks: dweights fp32 [T,k]
 * -> dlogits bf16 [T,E] (the autograd of topk/renormalise/softmax). */
int st_moe_route_softmax_bwd(const uint16_t* logits, const int32_t* indices,
                             const float* dweights, int64_t tokens, int32_t experts,
                             int32_t top_k, int32_t normalize, uint16_t* dlogits,
                             st_stream_t stream);
/* Sigmoid group-limited router, deepseek.py:115-126 (fp32 logits [T,E],
 * selection bias [E]); weights = scale * s / (sum s + 1e-20) when normalize. */
int st_moe_route_sigmoid(const float* logits, const float* bias, int64_t tokens,
                         int32_t experts, int32_t groups, int32_t group_k, int32_t top_k,
                         int32_t normalize, float scale, float* weights, int32_t* indices,
                         st_stream_t stream);
/* VJP of the sigmoid router weights w.r.t. fp32 logits (selection: none). */
int st_moe_route_sigmoid_bwd(const float* logits, const int32_t* indices, const float* dweights,
                             int64_t tokens, int32_t experts, int32_t top_k, int32_t normalize,
                             float scale, float* dlogits, st_stream_t stream);
/* Token permutation, the one_hot/where of qwen3_moe.py:101-106:
 * offsets int32 [E+1] (expert e owns rows [offsets[e], offsets[e+1])),
 * row_token int32 [T*k] (token of each permuted row), pick_row int32 [T*k]
 * (permuted row of each pick, -1 for an index outside [0, E)). E <= 1024. */
int st_moe_permute(const int32_t* indices, int64_t tokens, int32_t top_k, int32_t experts,
                   int32_t* offsets, int32_t* row_token, int32_t* pick_row, st_stream_t stream);
/* Weighted combine, qwen3_moe.py:110-111: out[t] = bf16 running sum, in
 * ascending expert order, of bf16(values[row] * w) over the token's picks
 * (the roundings of index_add_ into a bf16 output).  values bf16 [rows,H],
 * weights fp32 [T,k] (bf16-valued for Qwen3), out bf16 [T,H]; H % 8 == 0. */
int st_moe_combine(const uint16_t* values, int64_t rows, const float* weights,
                   const int32_t* indices, const int32_t* pick_row, int64_t tokens,
                   int32_t top_k, int64_t hidden, uint16_t* out, st_stream_t stream);
/* VJP of combine: dvalues[row] = bf16(dout[t] * w); dweights = sum_h
 * dout * values (products and sum rounded to bf16 when bf16_weights). */
int st_moe_combine_bwd(const uint16_t* dout, const uint16_t* values, int64_t rows,
                       const float* weights, const int32_t* pick_row, int64_t tokens,
                       int32_t top_k, int64_t hidden, int32_t bf16_weights, uint16_t* dvalues,
                       float* dweights, st_stream_t stream);
/* Input gradient of flat[tokens] over all experts: out[t] = bf16(sum_j
 * rows_in[pick_row[t,j]] + extra[t]) with fp32 accumulation; extra (bf16 or
 * fp32 [T,H], may be NULL) carries the router's input gradient. */
int st_moe_gather_sum(const uint16_t* rows_in, int64_t rows, const int32_t* pick_row,
                      int64_t tokens, int32_t top_k, int64_t hidden, const void* extra,
                      int32_t extra_dtype, uint16_t* out, st_stream_t stream);
/* Grouped 4-bit GEMMs (the per-expert F.linear calls of qwen3_moe.py:107-108
 * with LoRAProjection.forward, finetune/lora.py:205-220, per expert).
 * Expert e's weight is payload/scales block e ([N,K] each, K % 128 == 0,
 * contiguous experts); permuted row r of x is x[gather[r]] (gather NULL:
 * row r).  LoRA: t fp32 [rows, nseg*rank] in permuted order, lora_b fp32
 * [E, N, rank] (segments stacked along N), lora_a fp32 [E, lora_k, K]. */
int st_q4_grouped_fwd(const uint16_t* x, int64_t x_rows, int64_t ldx, const int32_t* gather,
                      int64_t rows, int64_t K, const int32_t* offsets, int32_t groups,
                      const uint8_t* payload, const float* scales, int64_t N,
                      const float* lut16, int32_t flags, const float* t, int64_t ldt,
                      const float* lora_b, int32_t rank, float lora_scale, int32_t nseg,
                      const int64_t* seg_end, uint16_t* y, int64_t ldy, st_stream_t stream);
int st_q4_grouped_dgrad(const uint16_t* dy, int64_t lddy, int64_t rows, int64_t N,
                        const int32_t* offsets, int32_t groups, const uint8_t* payload,
                        const float* scales, int64_t K, const float* lut16, int32_t flags,
                        const float* dt, int64_t lddt, const float* lora_a, int32_t lora_k,
                        uint16_t* dx, int64_t lddx, st_stream_t stream);
/* st_q4_grouped_dgrad of the experts' down projection through the SwiGLU of
 * qwen3_moe.py:108 (silu(gate) * up per expert): with gu the permuted
 * gate|up pre-activation [rows, 2I] (row stride ldgu), writes dgate|dup
 * [rows, 2I] (lddgu) from the dX values instead of dX, with the rounding of
 * st_swiglu_bwd.  I = the down projection's in_features; gu, dgu 16-byte
 * aligned with row strides that are multiples of 8. */
int st_q4_grouped_dgrad_swiglu(const uint16_t* dy, int64_t lddy, int64_t rows, int64_t N,
                               const int32_t* offsets, int32_t groups, const uint8_t* payload,
                               const float* scales, int64_t I, const float* lut16, int32_t flags,
                               const float* dt, int64_t lddt, const float* lora_a,
                               int32_t lora_k, const uint16_t* gu, int64_t ldgu, uint16_t* dgu,
                               int64_t lddgu, st_stream_t stream);
/* Grouped low-rank products over permuted rows (per-expert LoRA), fp32 out.
 * rows form: out[r, z*R + j] = alpha * sum_{k < seg_len} g[row(r), z*seg_len + k]
 *            * s[e(r)*s_gstride + (z*seg_len + k)*ssk + j*ssj]
 * grads form: out[e*o_gstride + (z*seg_len + m)*so_m + j*so_j] (+)= alpha *
 *            sum_{r in e} g[row(r), z*seg_len + m] * s[r*ssk + (z*R + j)*ssj]
 * for segments z < nseg, any R >= 1 (64 output columns per launch); row(r) =
 * gather[r] (NULL: r), bounded by
 * g_rows.  The grads form writes every expert (zero rows -> 0). */
int st_moe_lora_rows(int64_t rows, int32_t R, int64_t seg_len, int32_t nseg, const uint16_t* g,
                     int64_t ldg, int64_t g_rows, const int32_t* gather, const float* s,
                     int64_t ssk, int64_t ssj, int64_t s_gstride, const int32_t* offsets,
                     int32_t groups, float alpha, float* out, int64_t ldo, st_stream_t stream);
int st_moe_lora_grads(int64_t rows, int32_t R, int64_t seg_len, int32_t nseg,
                      const uint16_t* g, int64_t ldg, int64_t g_rows, const int32_t* gather,
                      const float* s, int64_t ssk, int64_t ssj, const int32_t* offsets,
                      int32_t groups, float alpha, float* out, int64_t o_gstride, int64_t so_m,
                      int64_t so_j, int32_t accumulate, st_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* SPILLTUNE_HIP_H */
