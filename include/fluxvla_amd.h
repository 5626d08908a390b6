/*
 * fluxvla_amd.h -- C ABI of libfluxvla_amd.so, the MI355X (gfx950) kernels of
 * FluxVLA's PI0 / PI0.5 fused inference path.
 *
 * Conventions shared by every entry point:
 *   - All tensors are device pointers (HIP), row-major, 16-byte aligned.
 *     bf16 storage is raw 16-bit (torch.bfloat16 bit pattern).
 *   - Weight matrices are [out_features, in_features] (the nn.Linear layout):
 *     the reduction dimension is contiguous, which is what the MFMA operand
 *     fetch wants.  The reference's prepare hooks emit [in, out] instead
 *     (fluxvla/models/backbones/llms/condition_gemma_inference.py:91-105).
 *   - `stream` is a hipStream_t (0 = legacy default stream).  Nothing here
 *     synchronizes, allocates or frees: every entry point is safe inside HIP
 *     graph capture and only enqueues kernels.
 *   - Every entry point returns 0 on success or a negative fvx_status code
 *     without launching anything; fvx_last_error() then describes the
 *     problem (thread-local).  Nothing aborts the process.
 *   - Split-K GEMMs and split-KV attention need a device workspace for
 *     their fp32 partials (size from fvx_gemm_workspace_bytes /
 *     fvx_attention_workspace_bytes).  A GEMM workspace holds per-tile
 *     arrival counters in its first 4 KiB, an attention workspace per-row-
 *     group arrival counters in its first 64 KiB: zero them once before the
 *     first call that uses the buffer; every call leaves them zero again.
 *     Keep GEMM and attention workspaces apart.  Calls on one stream may share a workspace; calls
 *     overlapping on different streams must not.  A NULL or too small
 *     workspace is an error (FVX_ERR_WORKSPACE) whenever the problem needs a
 *     split.
 */
#ifndef FLUXVLA_AMD_H_
#define FLUXVLA_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fvx_status {
  FVX_OK = 0,
  FVX_ERR_NULL = -1,      /* a required pointer is NULL */
  FVX_ERR_SHAPE = -2,     /* a size is out of the supported range */
  FVX_ERR_ALIGN = -3,     /* pointer / leading dimension not 16B aligned */
  FVX_ERR_LAUNCH = -4,    /* the HIP launch itself failed */
  FVX_ERR_ARG = -5,       /* an enum / flag argument is invalid */
  FVX_ERR_WORKSPACE = -6, /* workspace too small for the requested split */
  FVX_ERR_MERGE = -7,     /* an in-launch merge stopped waiting (fvx_attention_check) */
};

/* GEMM epilogue modes. */
enum fvx_gemm_mode {
  FVX_GEMM_PLAIN = 0, /* out = epilogue(A @ B^T) */
  FVX_GEMM_GEGLU = 1, /* out = gelu_tanh(A @ B^T) * (A @ B2^T) */
  FVX_GEMM_QKV_ROPE = 2, /* split into Q/K/V, rotate Q and K pairs */
  FVX_GEMM_EULER = 3, /* v = A @ B^T + bias; xt += dt * v (fp32) */
};

enum fvx_act { FVX_ACT_NONE = 0, FVX_ACT_SILU = 1, FVX_ACT_GELU_TANH = 2 };

/*
 * One GEMM launch: acc[m][n] = sum_k A[m][k] * B[n][k] (fp32 accumulate),
 * followed by the fused epilogue, applied in this order:
 *   v = acc
 *   v *= rsqrt(mean_k(A[m][k]^2) + rownorm_eps)      if rownorm
 *   v += bias[n] (bf16) ; v += bias_f32[n] (fp32)    if given (locked RTC
 *        rows: bias_f32_locked[n], see below)
 *   v = act(v)
 *   v *= gate[(m / gate_group) * ldg + n]            if gate
 *   v += residual[orow(m) * ldr + n]                 if residual (may alias c)
 *   v += pos[(m % pos_period) * ldp + n]             if pos
 *   c[orow(m) * ldc + n] = bf16(v)  (fp32 if out_f32)
 * where orow(m) = (m / row_group) * row_group_stride + m % row_group
 * (identity when row_group == 0).  m, row_group, gate_group, pos_period and
 * rtc_period must be below 2^31 (FVX_ERR_SHAPE otherwise): the epilogue
 * divides by them in 32 bits.
 */
typedef struct fvx_gemm_desc {
  const void* a; int64_t lda;      /* [M, K] bf16 */
  const void* b; int64_t ldb;      /* [N, K] bf16 */
  const void* b2;                  /* GEGLU: up weight, same shape as b */
  void* c; int64_t ldc;            /* [M, N] output */
  int64_t m, n, k;
  const void* bias;                /* [N] bf16 or NULL */
  const float* bias_f32;           /* [N] fp32 or NULL */
  const void* residual; int64_t ldr;
  const void* gate; int64_t ldg; int64_t gate_group;
  const void* pos; int64_t ldp; int64_t pos_period;
  int32_t act;                     /* fvx_act */
  int32_t mode;                    /* fvx_gemm_mode */
  int32_t rownorm;                 /* 1: apply the per-row RMS factor of A */
  int32_t out_f32;                 /* 1: c is fp32 */
  float rownorm_eps;
  float dt;                        /* EULER step */
  int64_t row_group, row_group_stride;
  /* QKV_ROPE: columns [0, nq*hd) -> q, [nq*hd, nq*hd+hd) -> k, next hd -> v
   * (n_q_heads may be 0: K/V only, e.g. the last prefix layer).
   * Q and K columns are in pair-interleaved order (2i, 2i+1) = (x_i,
   * x_{i+hd/2}); rope[(pos * hd/2 + i) * 2 + {0,1}] = {cos, sin}. */
  const float* rope;
  const int32_t* positions;        /* [M] rope position per row */
  void* q_out; int64_t ldq;
  void* k_out; int64_t ldk;        /* rows remapped by orow() */
  void* v_out; int64_t ldv;        /* rows remapped by orow(), or V^T: */
  int32_t n_q_heads, head_dim;
  /* EULER: xt[m*ldx + n] += dt * v ; xt_bf16 mirrors it in bf16 */
  float* xt; int64_t ldx;
  void* xt_bf16; int64_t ldxb;
  /* split-K workspace (may be NULL) */
  void* workspace; int64_t workspace_bytes;
  int32_t split_k;                 /* 0 = choose automatically */
  /* QKV_ROPE with v_transposed: V is written transposed, element (m, d) at
   * v_out[((m / row_group) * head_dim + d) * ldv + m % row_group] (the
   * [batch][head_dim][tokens] value-cache layout the attention reads). */
  int32_t v_transposed;
  /* Fragment-major operands (M <= 64, K % 32 == 0; one MFMA operand step
   * per contiguous 1 KiB block, so every wave load is fully coalesced):
   *   a_frag: element (m, k) of A at ((k/32 * 4 + m/16) * 64
   *           + (k%32)/8 * 16 + m%16) * 8 + k%8  (rows >= M are ignored)
   *   b_frag: element (n, k) of B (and b2) at (((n/16) * (K/32) + k/32) * 64
   *           + (k%32)/8 * 16 + n%16) * 8 + k%8  (needs N % 16 == 0)
   *   c_frag: PLAIN / GEGLU with M <= 64 and N % 32 == 0: the bf16 output
   *           is also written there in the a_frag layout (K' = N), ready
   *           as the A operand of the next skinny GEMM. */
  int32_t a_frag, b_frag;
  void* c_frag;
  /* fp8 weights (PI0.5 quantized variant; no counterpart in the reference,
   * which has no fp8 path): b (and b2) hold OCP e4m3fn bytes with one fp32
   * scale per output channel, W[n][k] = b_scale[n] * e4m3(b[n][k]).
   * ldb counts bytes.  K % 128 == 0.  The arithmetic follows fp8_act:
   *   0 (W8A16, the default): A stays bf16; the kernels convert the e4m3
   *     bytes to bf16 in registers (exact: every e4m3 value is a bf16
   *     value), run the bf16 MFMA with fp32 accumulation and scale the
   *     accumulator by b_scale[n] in the epilogue, i.e. exactly
   *     A @ dequant(W)^T up to fp32 summation order;
   *   1 (W8A8): each row of A is quantized to e4m3 on the fly with one
   *     power-of-two (E8M0) scale per row and k step -- 64 wide in the
   *     tiled and wide kernels, 128 wide in the M <= 64 kernel -- and the
   *     block-scaled fp8 MFMA runs; a8 (below) can hand the copy over.
   *   b_frag with b_fp8: element (n, k) at byte
   *     ((n/16) * (K/128) + k/128) * 2048 + ((k%128)/8 % 4 * 16 + n%16) * 32
   *     + (k%128)/32 * 8 + k%8
   *   (one 16x128 MFMA operand per contiguous 2 KiB; lane (n%16, g) holds
   *   k = 32t + 8g + j, t = 0..3, j = 0..7, the k positions the fragment-major
   *   A gives that lane). */
  int32_t b_fp8;
  const float* b_scale;            /* [N] */
  const float* b2_scale;           /* [N], GEGLU up weight */
  /* Row sums of squares handed from one GEMM to the next (no counterpart in
   * the reference; it lets the fused RMSNorm of a rownorm GEMM skip its pass
   * over A when A is the output of the previous GEMM):
   *   ss_out (PLAIN, M > 64): ss_out[(n / 64) * ss_ld + m] = sum over the
   *           64-column block of n of bf16(c[m][n'])^2 (ceil(N / 64) parts);
   *   ss_in  (rownorm): the sum of squares of row m of A is taken as
   *           ss_in[0 * ss_ld + m] + ... + ss_in[(ss_parts - 1) * ss_ld + m],
   *           added in that order (deterministic). */
  float* ss_out;
  const float* ss_in;
  int64_t ss_ld;
  int32_t ss_parts;
  /* e4m3 activations handed from one GEMM to the next (fp8-weight variant;
   * no counterpart in the reference):
   *   a8_out / a8_out_scale (PLAIN or GEGLU, bf16 output, M > 64): an e4m3
   *     copy of the stored output, a8_out[m * a8_out_ld + n] =
   *     e4m3(c[m][n] / 2^(e - 127)) with one E8M0 exponent e per row and
   *     64-column block at a8_out_scale[(n / 64) * a8_out_sld + m]: the
   *     smallest power of two that keeps the block's largest magnitude
   *     within 448 (the rule the fp8 GEMMs quantize A with);
   *   a8 / a8_scale (same layout, strides a8_ld / a8_sld): such a copy of
   *     A.  The W8A8 fp8-weight wide kernel then reads it instead of
   *     quantizing A (same values, same result); every other path ignores
   *     it, and so does a rownorm GEMM without ss_in.  a8_sld % 4 == 0. */
  void* a8_out; void* a8_out_scale; int64_t a8_out_ld, a8_out_sld;
  const void* a8; const void* a8_scale; int64_t a8_ld, a8_sld;
  /* with b_fp8: 0 = bf16 activations (W8A16), 1 = e4m3 activations (W8A8);
   * see b_fp8 above.  a8 is read only by W8A8 GEMMs. */
  int32_t fp8_act;
  /* Real-time chunking (RTC) of the Euler loop.  Replaces the per-step
   * tensor updates of PI0FlowMatching._predict_action_prefix_rtc and
   * _predict_action_guidance_rtc (fluxvla/models/vlas/pi0_flowmatching.py:
   * 651-700) and apply_rtc_guidance without VJP
   * (fluxvla/engines/utils/rtc_guidance.py:107-155).
   * Row m is "locked" when rtc_lock is given and (m % rtc_period) <
   * *rtc_lock (a device int32, so one captured graph serves every prefix
   * length):
   *   PLAIN, EULER: locked rows add bias_f32_locked instead of bias_f32
   *     (the prefix method gives locked positions time 0);
   *   EULER with rtc_prev: locked rows store rtc_prev[m * ld_prev + n].
   * EULER with rtc_cw (guidance method): every row stores
   *     xt + dt * v + rtc_cw[m % rtc_period]
   *                   * (rtc_prev[m * ld_prev + n] - xt + rtc_omt * v)
   *   (rtc_cw[r] = -dt * guidance weight * prefix weight of row r, 0 for rows
   *   without guidance; rtc_prev then needs all m rows).
   * rtc_period > 0 is required with any of these.  All zero / NULL: the
   * plain epilogues above. */
  const int32_t* rtc_lock;
  int64_t rtc_period;
  const float* bias_f32_locked;    /* [n] fp32 */
  const float* rtc_prev;           /* fp32, row stride ld_prev */
  int64_t ld_prev;
  const float* rtc_cw;             /* [rtc_period] fp32 */
  float rtc_omt;
  /* Adaptive RMSNorm folded into the GEMM (PI0.5 action expert at M <= 64).
   * a_scale (bf16 [K]): A's column k is multiplied by (1 + a_scale[k]) in
   * fp32 as it is loaded, then rounded to bf16 for the MFMA (the rownorm sums
   * use A as given): the adaptive scale of GemmaRMSNorm
   * (condition_gemma.py:126-145) applied to the raw residual stream, whose
   * RMS factor the rownorm applies to the product; the shift becomes a bias
   * (shift @ B^T, precomputed by the caller).
   * With it, QKV_ROPE and GEGLU take fp32 biases too, after the rownorm
   * scaling: QKV_ROPE adds bias_f32[n] before the rotation; GEGLU adds
   * bias_f32[n] to the gate half and bias2_f32[n] to the up half before
   * gelu_tanh(gate) * up.  M <= 64 (skinny) GEMMs with bf16 or W8A16
   * weights only; NULL: unused. */
  const void* a_scale;
  const float* bias2_f32;          /* [N] fp32, GEGLU up half */
  /* LayerNorm folded into the GEMM (no counterpart in the reference; it
   * replaces the LayerNorm launches in front of SigLIP's Q|K|V, fc1 and the
   * projector, siglip_vit.py via HF SiglipEncoderLayer).  With ln_csum
   * ([N] fp32) a rownorm GEMM sums A's values (sum_m) and squares (ss_m)
   * per row in its K loop and computes, before bias and activation,
   *   v = (acc - mean_m * ln_csum[n]) * rsqrt(var_m + rownorm_eps),
   *   mean_m = sum_m / K,  var_m = max(ss_m / K - mean_m^2, 0),
   * which is LayerNorm(A) @ B^T when B is the layer's weight scaled by the
   * norm's gain along k and ln_csum[n] = sum_k B[n][k] (the norm's shift
   * enters as bias_f32).  PLAIN, M > 64, one K range (the tile kernel),
   * bf16 weights, no ss_in, no hand-over outputs; NULL: unused. */
  const float* ln_csum;
  /* A's rows in groups (no counterpart in the reference; one launch for the
   * action rows of a whole batch, which sit behind each sample's state row
   * in the suffix stream): with a_row_group > 0, row m of the product reads
   * row (m / a_row_group) * a_row_group_stride + m % a_row_group of a, rows
   * lda elements apart (a_row_group_stride >= a_row_group, both < 2^31).
   * A call with m > a_row_group takes the tile kernel (not with a_frag or
   * a8); 0: rows m of a. */
  int64_t a_row_group;
  int64_t a_row_group_stride;
  /* GEGLU pre-activations (no counterpart in the reference; for the
   * GeGLU backward of guidance RTC with use_vjp, which autograd feeds from
   * the same two values): gu_out (may be NULL) receives per output row the
   * bf16 gate values (columns n) and up values (columns N + n) that the
   * product gelu_tanh(gate) * up is taken from, row stride ld_gu >= 2 N.
   * GEGLU mode on the skinny and tile kernels (the wide kernel is not used
   * with it). */
  void* gu_out;
  int64_t ld_gu;
  /* QKV_ROPE with v_transposed, copies in the other layouts (no
   * counterpart in the reference; the operands of the attention backward of
   * guidance RTC with use_vjp): k_t_out (may be NULL) receives the rotated
   * keys transposed like v_out, element (m, d) at k_t_out[((m / row_group)
   * * head_dim + d) * ld_kt + m % row_group]; v_rows_out (may be NULL) the
   * values row-major with k_out's row map and row stride ld_vr. */
  void* k_t_out;
  int64_t ld_kt;
  void* v_rows_out;
  int64_t ld_vr;
} fvx_gemm_desc;

/* Library identity / diagnostics. */
int fvx_version(void);
const char* fvx_last_error(void);
/* Workspace bytes fvx_gemm needs for the given problem (0 if it runs in
 * one pass).  M <= 64 problems split K in ranges of at most 256; split_k > 0
 * requests a range length of ceil(K / split_k) (still capped at 256). */
int64_t fvx_gemm_workspace_bytes(const fvx_gemm_desc* d);

/* General GEMM with fused epilogue.  Replaces the reference's
 * matmul_bias_cuda (fluxvla/ops/cuda/matmul_bias/matmul_bias.py:19-60,
 * matmul_bias_forward.cpp:21-51) and the Triton GEMMs behind
 * fluxvla/ops/atomic_ops.py:34-378 (matmul_bias_res, matmul_res,
 * matmul_bias_silu, matmul_bias_small, rms_matmul_gate / matmul_gate,
 * rms_matmul_qkv_rope / matmul_qkv_rope, matmul_res_gate, ...): one
 * descriptor covers every epilogue those entry points fuse. */
int fvx_gemm(const fvx_gemm_desc* d, void* stream);

/*
 * fvx_gemm without a caller-passed workspace: the split-K scratch (arrival
 * counters + fp32 partials) lives in a library-owned static device array of
 * FVX_GEMM_NOALLOC_SCRATCH_BYTES per GPU, set up on the first call on a
 * device (its address fetched once, its counters cleared by a small kernel
 * on `stream`).  d->workspace and d->workspace_bytes are ignored.  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Nothing here allocates or frees.
 * Limit: a problem whose fvx_gemm_workspace_bytes() exceeds the scratch
 * returns FVX_ERR_WORKSPACE without launching.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (other streams or
 * threads) race; calls on one stream do not.  The stream's device must be
 * reachable with hipSetDevice from the calling thread.
 */
#define FVX_GEMM_NOALLOC_SCRATCH_BYTES (32ll << 20)
int fvx_gemm_noalloc(const fvx_gemm_desc* d, void* stream);

/*
 * Fused residual-add + RMSNorm.  Replaces GemmaRMSNorm.forward followed by
 * the residual add (fluxvla/models/backbones/llms/condition_gemma.py:75-116,
 * :319-337) and the weight-less rms_norm_kernel
 * (fluxvla/ops/triton/norm_triton_ops.py:317-332).
 *   h = x (+ residual, fp32 add)            residual may be NULL
 *   residual_out = bf16(h)                  residual_out may be NULL
 *   out = bf16(h * rsqrt(mean(h^2) + eps) * weight)   weight may be NULL (=1)
 * The Gemma (1 + w) scale is passed pre-folded in `weight`.
 */
int fvx_rms_norm_residual(const void* x, const void* residual,
                          const void* weight, void* out, void* residual_out,
                          int64_t rows, int64_t cols, float eps, void* stream);

/* LayerNorm with affine (SigLIP).  Replaces layer_norm_small_kernel
 * (fluxvla/ops/triton/norm_triton_ops.py:90-125). */
int fvx_layer_norm(const void* x, const void* weight, const void* bias,
                   void* out, int64_t rows, int64_t cols, float eps,
                   void* stream);

/* Adaptive RMSNorm (PI0.5).  Replaces adarms_norm_kernel
 * (fluxvla/ops/triton/norm_triton_ops.py:355-395):
 *   style row s = row / rows_per_style holds [scale | shift | gate] (bf16)
 *   out = bf16(rms(x) * (1 + scale) + shift);  gate_out = gate (may be NULL) */
int fvx_adarms_norm(const void* x, const void* style, void* out,
                    void* gate_out, int64_t rows, int64_t cols,
                    int64_t rows_per_style, int64_t style_stride, float eps,
                    void* stream);

/* fvx_adarms_norm with per-position conditioning for the prefix method of
 * real-time chunking: rows with (row % lock_period) < *lock (device int32)
 * take their [scale | shift | gate] from the single row style_locked (the
 * conditioning at time 0) instead of style.  Replaces the per-position
 * adarms_cond of PI05FlowMatching.embed_suffix with a [B, T] timestep
 * (fluxvla/models/vlas/pi05_flowmatching.py:68-127,
 * condition_gemma.py:126-145) under _predict_action_prefix_rtc
 * (pi0_flowmatching.py:651-669). */
int fvx_adarms_norm_locked(const void* x, const void* style,
                           const void* style_locked, const int32_t* lock,
                           int64_t lock_period, void* out, void* gate_out,
                           int64_t rows, int64_t cols, int64_t rows_per_style,
                           int64_t style_stride, float eps, void* stream);

/*
 * Fused multi-query attention: softmax(Q K^T * scale + mask) V, flash-style
 * (online softmax, fp32 statistics).  Replaces matmul_abT_scale +
 * softmax_kernel_masklen / softmax_kernel_prefix_suffix + matmul_small
 * (fluxvla/ops/triton/attention_triton_ops.py:5-146,
 * fluxvla/ops/atomic_ops.py:209-221) and the SigLIP SDPA call
 * (fluxvla/ops/atomic_ops.py:65-76).
 *
 * One problem z (z < n_problems) has sq query tokens x heads query rows and
 * sk keys; query row r is token r / heads, head r % heads (all heads share
 * the problem's single K/V head).  Pointer offsets of problem z are
 * (z / zdiv) * zs1 + (z % zdiv) * zs2 elements, per tensor.
 * Mask: key j is visible to query token t iff kgrp[j] <= qgrp[t]; NULL
 * kgrp/qgrp means no mask.  This encodes make_att_2d_masks
 * (fluxvla/engines/utils/model_utils.py:77-95): kgrp = pad ? cumsum(att) :
 * INT32_MAX, qgrp = cumsum(att).  Rows that see no key produce zeros.
 * kv_splits > 1 splits the key range across workgroups (needs workspace);
 * the split partials are merged by a second kernel on the same stream, or,
 * for key ranges of fewer than 4 tiles (the bs=1 action expert) with
 * sq * heads % 8 == 0, by merging workgroups of the same launch: each
 * 64-row group's ranges and mergers run on one XCD and meet through its L2;
 * a merger waits (bounded) only for ranges that precede it in dispatch
 * order and wait on nothing.
 * Problems with a transposed value cache (v_d_stride > 0), head_dim 256 and
 * operand offsets below 2^30 elements run the decode kernels: a workgroup
 * owns 64 or 128 query rows and a key range of whole 64-key tiles staged
 * through LDS (about 128 64-row groups x ranges by default, or kv_splits
 * ranges).  Key ranges of 4 tiles or more (the prefix) run a transposed-
 * score kernel (128 rows per workgroup); shorter ranges (the bs=1 action
 * expert) a 4-wave kernel with lower fixed cost.
 */
typedef struct fvx_attn_desc {
  const void* q; int64_t q_tok_stride, q_head_stride, q_zs1, q_zs2;
  const void* k; int64_t k_tok_stride, k_zs1, k_zs2;
  const void* v; int64_t v_tok_stride, v_zs1, v_zs2;
  /* v_d_stride > 0: V is stored transposed (the value cache), element
   * (key j, dim d) at v[d * v_d_stride + j]; v_tok_stride is then unused.
   * Needs sk <= v_d_stride and v_d_stride % 8 == 0. */
  int64_t v_d_stride;
  void* o; int64_t o_tok_stride, o_head_stride, o_zs1, o_zs2;
  const int32_t* kgrp; int64_t kgrp_zs1;
  const int32_t* qgrp; int64_t qgrp_zs1;
  int64_t sq, sk, heads, head_dim, n_problems, zdiv;
  float scale;
  int32_t kv_splits;
  void* workspace; int64_t workspace_bytes;
  /* Decode path only (transposed V, head_dim 256, n_problems * sq <= 64):
   * if non-NULL, the output is also written in the fragment-major A layout
   * of fvx_gemm_desc.a_frag, row z * sq + token, column head * 256 + d --
   * the A operand of the o-projection. */
  void* o_frag;
  /* Prefetch (no counterpart in the reference).  Decode path with key
   * ranges of fewer than 4 tiles (the bs=1 action expert) only: extra
   * workgroups of the attention launch read the device ranges
   * [prefetch[i], prefetch[i] + prefetch_bytes[i]) (into LDS, discarded)
   * while the attention runs on the CUs it leaves idle, so that the next
   * kernels' operands -- the expert layer's O / gate / up / down weights,
   * the next layer's Q|K|V weights -- are cached when those kernels start.
   * prefetch_tile_bytes[i] > 0: the range is a sequence of tiles of that
   * size, tile j read by a workgroup the hardware places on XCD j % 8 (the
   * fragment-major weights of the M <= 64 GEMM); each tile is then read
   * from a CU of that XCD, into that XCD's L2.  0: no placement (the
   * memory-side cache).  NULL entries are skipped; pointers 16-byte
   * aligned; bytes (and tile bytes) multiples of 1024.  prefetch_wgs > 0:
   * that many extra workgroups; 0: as many as leave one workgroup per CU.
   * Ignored on other paths. */
  const void* prefetch[8];
  int64_t prefetch_bytes[8];
  int64_t prefetch_tile_bytes[8];
  int32_t prefetch_wgs;
  /* Test hook, 0 in every real call: nonzero makes the in-launch merge of
   * the decode path stop waiting for its key ranges at once, as if its
   * bounded wait had run out (see fvx_attention_check). */
  int32_t merge_no_wait;
} fvx_attn_desc;

int64_t fvx_attention_workspace_bytes(const fvx_attn_desc* d);
int fvx_attention(const fvx_attn_desc* d, void* stream);

/*
 * Status of the decode path's in-launch merge (no counterpart in the
 * reference, whose attention has no in-launch merge).  The merging
 * workgroups wait for the key ranges of their row group with a bounded
 * poll; a workgroup whose poll runs out merges what has arrived, so the
 * output of that call is wrong, and it counts itself in a status word of
 * the workspace's counter region.  This call waits for `stream`, reads the
 * word and, when it is non-zero, clears the whole counter region (so the
 * next call starts from zero counts) and returns FVX_ERR_MERGE.  It
 * synchronizes: call it after a call or a chunk, outside graph capture.
 */
int fvx_attention_check(void* workspace, int64_t workspace_bytes,
                        void* stream);

/*
 * SigLIP patch im2col: images [n_img, 3, H, W] (or [n_img, H, W, 3] with
 * channels_last; bf16 or fp32 per `in_f32`) -> patches
 * [n_img * (H/p) * (W/p), k_pad] bf16, column order (channel, ky, kx) (the
 * Conv2d weight flattening), zero-filled from 3*p*p up to k_pad.  Optional
 * affine: value * in_scale + in_shift.  Replaces the patch gather of
 * conv2d_embed_res (fluxvla/ops/atomic_ops.py:34-53).
 */
int fvx_im2col_patches(const void* images, int in_f32, int channels_last,
                       void* patches, int64_t n_img, int64_t height,
                       int64_t width, int64_t patch, int64_t k_pad,
                       float in_scale, float in_shift, void* stream);

/* Token embedding gather: out[orow(i)] = bf16(table[ids[i]] * scale). */
int fvx_embed_tokens(const void* table, const int64_t* ids, void* out,
                     int64_t n_tokens, int64_t dim, int64_t vocab,
                     float scale, int64_t row_group, int64_t row_group_stride,
                     void* stream);

/* Row copy of bf16 rows of `cols` elements: dst row orow(i) = src row i,
 * orow(i) = (i / row_group) * dst_group_stride + i % row_group (identity
 * when row_group == 0).  Used to place the per-chunk state token in front of
 * each sample's action tokens. */
int fvx_copy_rows(const void* src, int64_t src_ld, void* dst, int64_t dst_ld,
                  int64_t rows, int64_t cols, int64_t row_group,
                  int64_t dst_group_stride, void* stream);

/*
 * Row-major [rows <= 64, cols] bf16 -> the fragment-major A layout of
 * fvx_gemm_desc.a_frag (cols % 32 == 0).  No counterpart in the reference:
 * it re-lays an activation that no fused epilogue wrote in that layout.
 */
int fvx_pack_frag(const void* src, int64_t src_ld, void* dst, int64_t rows,
                  int64_t cols, void* stream);

/*
 * Camera-frame preprocessing: resize + pad + normalize + channel reorder of n
 * RGB images into fp32 CHW planes (the patch embedding's input).  Replaces the
 * host transforms ResizeImages (cv2 INTER_LINEAR), ResizeImagesWithPad,
 * NormalizeImages and TransformImage (PIL BILINEAR)
 * (fluxvla/transforms/transform_images.py:80-200, 313-390, 414-560) and
 * resize_with_pad (fluxvla/engines/utils/model_utils.py:98-120).
 *
 * dst pixel (y, x) of image i, channel c:
 *   inside [off_y, off_y + rh) x [off_x, off_x + rw): the source resized to
 *     rh x rw, sampled at (y - off_y, x - off_x), source channel c (2 - c
 *     with swap_rb);
 *   elsewhere: pad_value;
 *   out = (v / pre_div - mean[c]) / den[c]   (fp32 division, as numpy does)
 * Filters: LINEAR -- two-tap bilinear, half-pixel centres, edge clamp, fp32
 *   (torch's bilinear interpolate with align_corners=False; OpenCV's
 *   INTER_LINEAR up to its 11-bit weight rounding); round_u8 rounds the
 *   resized value to uint8 as a uint8 resize returns it.
 *   PIL_BILINEAR -- Pillow's antialiased BILINEAR resample (uint8 sources):
 *   triangle filter widened by the downscale factor, 22-bit fixed-point
 *   weights, horizontal then vertical pass, each rounded to uint8.
 * Sources: uint8 or fp32 (LINEAR without rounding), interleaved [h][w][3]
 * (src_hwc) or planar [3][h][w]; image i at src + i * src_img_stride
 * elements, dst planes at dst + i * dst_img_stride elements.
 */
enum fvx_resize_filter { FVX_RESIZE_LINEAR = 0, FVX_RESIZE_PIL_BILINEAR = 1 };

typedef struct fvx_image_desc {
  const void* src;
  int32_t src_u8, src_hwc;
  int64_t n, src_h, src_w, src_img_stride;
  float* dst;
  int64_t dst_h, dst_w, dst_img_stride;
  int64_t rh, rw, off_y, off_x;
  float pad_value;
  int32_t filter, round_u8, swap_rb;
  float pre_div;
  float mean[3], den[3];
  /* pad_per_channel != 0: the pad is pad_rgb[c] for output channel c (a
   * raw pixel value, normalized like the picture) instead of pad_value --
   * TransformImage's letterbox fill colour. */
  int32_t pad_per_channel;
  float pad_rgb[3];
} fvx_image_desc;

int fvx_resize_normalize(const fvx_image_desc* desc, void* stream);

/*
 * Backward ops of the action expert for guidance real-time chunking with
 * use_vjp: the correction J^T e that apply_rtc_guidance takes from torch
 * autograd through the denoiser (fluxvla/engines/utils/rtc_guidance.py:
 * 142-150).  The reference has no fused counterparts (autograd runs the
 * backward of each torch op); the products with weights and attention
 * operands go through fvx_gemm on transposed copies, these ops sit between
 * them.  All fp32 arithmetic; bf16 outputs are the next GEMM's A operand.
 */

/* RMSNorm backward (GemmaRMSNorm, condition_gemma.py:75-80, with its
 * (1 + w) gain folded into the next GEMM's weights; adaRMS (:126-145) with
 * its (1 + scale) as `scale`):  g = dy * (1 + scale) (scale bf16 [cols] or
 * NULL), r = rsqrt(mean(x^2) + eps),
 *   dx = dres + r g - (r^3 / cols) (x . g) x.
 * out (fp32, may be NULL) = dx; out_bf16 (may be NULL) = bf16(dx * gate)
 * (gate bf16 [cols] or NULL: 1).  Rows of x, dres, out and out_bf16 follow
 * the row-group map (m / row_group) * row_group_stride + m % row_group
 * (identity for row_group 0); dy rows are compact.  cols % 8 == 0,
 * cols <= 4096, leading dims multiples of 8, pointers 16-byte aligned.
 * out_frag (may be NULL): out_bf16's values in the fragment-major A layout
 * of fvx_gemm_desc.a_frag (mapped rows < 64, cols % 32 == 0), for the
 * M <= 64 GEMM that reads them. */
int fvx_rms_norm_backward(const void* x, int64_t ldx, const float* dy,
                          int64_t ldy, const float* dres, int64_t ldr,
                          const void* scale, const void* gate, float* out,
                          int64_t ldo, void* out_bf16, int64_t ldob,
                          void* out_frag, int64_t rows, int64_t cols,
                          int64_t row_group, int64_t row_group_stride,
                          float eps, void* stream);

/* Activation backward, bf16 in and out (GemmaMLP's GeGLU,
 * condition_gemma.py:156-192; the PI0 action-time MLP's SiLU,
 * pi0_flowmatching.py:300-310):
 *   FVX_ACT_BWD_GEGLU: in = [gate | up] ([rows, 2 cols]), dy = dh ->
 *     out = [dh * up * gelu_tanh'(gate) | dh * gelu_tanh(gate)]
 *   FVX_ACT_BWD_SILU: in = z ([rows, cols]) -> out = dy * silu'(z)
 * cols % 8 == 0, leading dims multiples of 8, pointers 16-byte aligned.
 * out and out_frag (the fragment-major A layout, rows <= 64, widths % 32
 * == 0) may each be NULL, not both. */
#define FVX_ACT_BWD_GEGLU 0
#define FVX_ACT_BWD_SILU 1
int fvx_act_backward(int act, const void* in, int64_t ldi, const void* dy,
                     int64_t ldy, void* out, int64_t ldo, void* out_frag,
                     int64_t rows, int64_t cols, void* stream);

/* GeGLU product row by row: out[r][c] = bf16(gelu_tanh(gu[r][c]) *
 * gu[r][cols + c]) -- GemmaMLP's act(gate) * up (condition_gemma.py:
 * 156-192) from a stored [gate | up] GEMM output, which the backward then
 * reuses (the fused GEGLU GEMM keeps neither).  Same layout rules as
 * fvx_act_backward. */
int fvx_geglu_rows(const void* gu, int64_t ldgu, void* out, int64_t ldo,
                   void* out_frag, int64_t rows, int64_t cols, void* stream);

/* Masked-softmax backward of one attention problem
 * (condition_gemma.py:340-535's eager attention, softmax over
 * scale * q k^T with the make_att_2d_masks rule of model_utils.py:77-95):
 * row r is query token r / heads; s = q . k and dp = dO . v (fp32
 * [rows, lds / lddp]); key j visible iff kgrp[j] <= qgrp[r / heads] (both
 * NULL: all visible).  P = softmax of the visible logits, D = sum P dp,
 *   ds[r][j] = bf16(scale P (dp - D))  for j < n_cols (0 past n_keys and
 *   on masked keys).
 * ds_t / p_t (bf16 [n_suffix, ldt], may be NULL): column r receives ds and
 * P of keys key0 .. key0 + n_suffix - 1 (the A operands of dK = ds^T Q and
 * dV = P^T dO). */
int fvx_attention_rows_backward(const float* s, int64_t lds, const float* dp,
                                int64_t lddp, const int32_t* kgrp,
                                const int32_t* qgrp, void* ds, int64_t ldds,
                                void* ds_t, void* p_t, int64_t ldt,
                                int64_t key0, int64_t n_suffix, int64_t rows,
                                int64_t heads, int64_t n_keys, int64_t n_cols,
                                float scale, void* stream);

/* Gradients of the suffix keys and values of one attention problem
 * (the eager attention's backward, condition_gemma.py:340-535): with ds_t /
 * p_t as fvx_attention_rows_backward writes them ([n_suffix, ldt] bf16,
 * column r = query row r),
 *   dk[j][c] = sum_r ds_t[j][r] q[r][c],  dv[j][c] = sum_r p_t[j][r] dout[r][c]
 * for j < n_suffix, c < cols, r < rows (q, dout bf16 [rows, ld], 16-byte
 * aligned, cols and the leading dims multiples of 8; dk, dv fp32).  The
 * heads of a key/value head are rows of the same sums. */
int fvx_attention_suffix_kv_backward(const void* ds_t, const void* p_t,
                                     int64_t ldt, const void* q, int64_t ldq,
                                     const void* dout, int64_t ldo, float* dk,
                                     int64_t ldk, float* dv, int64_t ldv,
                                     int64_t n_suffix, int64_t rows,
                                     int64_t cols, void* stream);

/* Fused attention backward of the decode shape (the action expert's
 * suffix rows against its cached prefix and suffix keys; the eager
 * attention's backward under autograd, condition_gemma.py:340-535), on bf16
 * MFMA in 32-row x 64-key tiles.  Per problem z: rows r = token * heads +
 * head of q / o / dout ([rows][256] bf16, o the attention output), keys j <
 * n_keys of k and v ([n_keys][256] bf16 rows) and kt (the keys transposed,
 * [256][kt_ld] bf16, zero past n_keys), visibility kgrp[j] <= qgrp[r /
 * heads] (both NULL: all).  With P = softmax(scale q k^T) over the visible
 * keys, D = dout . o per row and dS = scale P (dout v^T - D):
 *   dq  (fp32 [dq_parts][n_problems * rows][256]): key tile t's share of
 *       dS k (dq_parts = fvx_attention_backward_parts(n_keys); their sum is
 *       dq, which fvx_rope_backward adds up);
 *   ds_t / p_t (may be NULL; bf16 [n_problems][n_suffix][ldt], problem
 *       stride t_zs): dS and P of keys key0 .. key0 + n_suffix - 1,
 *       column r = row r (fvx_attention_suffix_kv_backward's operands);
 *   stats: fp32 scratch of 2 * n_problems * dq_parts * rows floats.
 * vt (may be NULL): the values transposed ([256][vt_ld] bf16 per problem,
 * the value cache); with it the call first rewrites, for keys
 * refresh_key0 .. refresh_key0 + refresh_n - 1, kt's columns from k and
 * v's rows from vt (the keys a step has just written into the caches), so
 * kt and v are then written as well as read.
 * Strides (*_zs) in elements; head_dim must be 256. */
typedef struct fvx_attn_bwd_desc {
  const void* q; int64_t q_zs;
  const void* o; int64_t o_zs;
  const void* dout; int64_t do_zs;
  const void* k; int64_t k_zs;
  const void* v; int64_t v_zs;
  const void* kt; int64_t kt_ld, kt_zs;
  const void* vt; int64_t vt_ld, vt_zs;
  int64_t refresh_key0, refresh_n;
  const int32_t* kgrp; int64_t kgrp_zs;
  const int32_t* qgrp; int64_t qgrp_zs;
  float* stats;
  float* dq; int64_t dq_parts;
  void* ds_t; void* p_t; int64_t ldt, t_zs;
  int64_t rows, heads, head_dim, n_keys, key0, n_suffix, n_problems;
  float scale;
} fvx_attn_bwd_desc;

int fvx_attention_backward(const fvx_attn_bwd_desc* d, void* stream);
int64_t fvx_attention_backward_parts(int64_t n_keys);

/* bf16 transpose: dst[b][c][r] = src[b][r][c] for b < batch, r < rows,
 * c < cols (element offsets b * batch_stride + row * ld). */
int fvx_transpose_bf16(const void* src, int64_t ld_src,
                       int64_t src_batch_stride, void* dst, int64_t ld_dst,
                       int64_t dst_batch_stride, int64_t rows, int64_t cols,
                       int64_t batch, void* stream);

/* RoPE backward packed into the Q|K|V GEMM's dY: row m of out (bf16) =
 * [dq (n_q_heads heads) | dk | dv], each head's column pair (2i, 2i+1)
 * of dq and dk rotated by the transpose of the forward rotation at
 * rope[positions[m]][i] (fp32 (cos, sin) pairs, the fvx_gemm QKV_ROPE
 * table): (ga, gb) -> (ga cos + gb sin, gb cos - ga sin).  dq is the sum of
 * dq_parts partials dq_part_stride elements apart (fvx_attention_backward's
 * key tiles; 1 for a plain dq).  out_frag (may be NULL; out may be NULL
 * with it): the same rows in the fragment-major A layout (rows <= 64). */
int fvx_rope_backward(const float* dq, int64_t ldq, int64_t dq_parts,
                      int64_t dq_part_stride, const float* dk,
                      int64_t ldk, const float* dv, int64_t ldv,
                      const float* rope, const int32_t* positions, void* out,
                      int64_t ldo, void* out_frag, int64_t rows,
                      int64_t n_q_heads, int64_t head_dim, void* stream);

/* Guidance error and corrected update of one Euler step with use_vjp
 * (apply_rtc_guidance, rtc_guidance.py:107-155, under
 * _predict_action_guidance_rtc, pi0_flowmatching.py:671-700, whose
 * denoiser is -u for the model velocity u; omt = 1 - t of the step).
 * Row m is action step m % period of its sample, w fp32 [period] the
 * prefix weights (zero past the previous chunk):
 *   fvx_rtc_vjp_error:  e = bf16(w (prev - x + omt u))
 *   fvx_rtc_vjp_update: x <- x + dt u - dt gw e + dt gw omt g, with e in
 *                       fp32 as above, g = J_u^T e, gw = *gw (device, the
 *                       step's guidance weight); x_bf16 (may be NULL)
 *                       receives the bf16 copy. */
int fvx_rtc_vjp_error(const float* x, int64_t ldx, const float* u,
                      int64_t ldu, const float* prev, int64_t ldp,
                      const float* w, void* e, int64_t lde, int64_t rows,
                      int64_t cols, int64_t period, float omt, void* stream);
int fvx_rtc_vjp_update(float* x, int64_t ldx, void* x_bf16, int64_t ldxb,
                       const float* u, int64_t ldu, const float* prev,
                       int64_t ldp, const float* w, const float* g,
                       int64_t ldg, const float* gw, int64_t rows,
                       int64_t cols, int64_t period, float omt, float dt,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLUXVLA_AMD_H_ */
