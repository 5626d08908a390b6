// Backward kernels of the action expert: the vector-Jacobian product J^T e
// of one denoising step that guidance real-time chunking with use_vjp adds
// to the velocity (fluxvla/engines/utils/rtc_guidance.py:142-150, which
// takes it from torch autograd through the whole denoiser).
//
// The products with weights (dY @ W for every linear layer, and the
// attention's Q K^T, dO V^T, dS K, dS^T Q, P^T dO) run through fvx_gemm on
// transposed operand copies; this file holds what lies between them:
//   rms_backward_kernel      RMSNorm (and adaRMS scale) backward + residual
//   act_backward_kernel      GeGLU and SiLU backward, elementwise
//   attn_rows_backward_kernel  masked softmax backward per query row
//   transpose_kernel         bf16 [rows, cols] -> [cols, rows] (batched)
//   rope_backward_kernel     RoPE backward of dq / dk, packed with dv
//   rtc_vjp_*_kernel         the guidance error and the corrected update
// Every kernel reads and writes in fp32 except where a bf16 operand of the
// next GEMM is produced; one thread or one wavefront per independent item,
// every access bounds-checked against the sizes the host validated.
#include "capi_util.h"
#include "common.h"

namespace fvx {

namespace {

constexpr int kBwdRows = 4;  // rows (wavefronts) per 256-thread workgroup

__device__ __forceinline__ void ld_f8(const float* p, float* f) {
  const f32x4_t a = *reinterpret_cast<const f32x4_t*>(p);
  const f32x4_t b = *reinterpret_cast<const f32x4_t*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[e] = a[e];
    f[4 + e] = b[e];
  }
}

__device__ __forceinline__ void st_f8(float* p, const float* f) {
  *reinterpret_cast<f32x4_t*>(p) = f32x4_t{f[0], f[1], f[2], f[3]};
  *reinterpret_cast<f32x4_t*>(p + 4) = f32x4_t{f[4], f[5], f[6], f[7]};
}

__device__ __forceinline__ int64_t grouped_row(int64_t m, int64_t g, int64_t gs) {
  return g > 0 ? (m / g) * gs + m % g : m;
}

// ---------------------------------------------------------------------------
// RMSNorm backward.  Forward (GemmaRMSNorm with the (1 + w) gain folded into
// the next GEMM's weights, condition_gemma.py:75-80; adaRMS keeps its
// per-style (1 + scale), :126-145):  y = x r (1 + scale),
// r = rsqrt(mean(x^2) + eps).  With g = dy (1 + scale):
//   dx = dres + r g - (r^3 / n) (x . g) x.
// One wavefront per row; vector v (8 columns) of the row is lane v % 64's
// (v / 64)-th.  x, dres, out and out_b rows follow the row-group map
// (m / g) * gs + m % g (identity for g = 0); dy rows are compact.
// out_b = bf16(dx * gate): the A operand of the next backward GEMM; out_f
// the same values in the fragment-major A layout (row pr, M <= 64 GEMMs).
// ---------------------------------------------------------------------------
template <int NV>
__global__ __launch_bounds__(256) void rms_backward_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const float* __restrict__ dy,
    int64_t ldy, const float* __restrict__ dres, int64_t ldr,
    const bf16_t* __restrict__ scale, const bf16_t* __restrict__ gate,
    float* __restrict__ out, int64_t ldo, bf16_t* __restrict__ out_b,
    int64_t ldob, bf16_t* __restrict__ out_f, int64_t rows, int cols,
    int64_t grp, int64_t grp_stride, float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t m = (int64_t)blockIdx.x * kBwdRows + (threadIdx.x >> 6);
  if (m >= rows) return;
  const int64_t pr = grouped_row(m, grp, grp_stride);
  const int nvec = cols >> 3;
  float xv[NV][8], g[NV][8];
  float ss = 0.f, dot = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    if (v < nvec) {
      unpack8(ld8(x + pr * ldx + v * 8), xv[i]);
      ld_f8(dy + m * ldy + v * 8, g[i]);
      if (scale) {
        float sc[8];
        unpack8(ld8(scale + v * 8), sc);
#pragma unroll
        for (int e = 0; e < 8; ++e) g[i][e] *= 1.f + sc[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[i][e] = g[i][e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      ss += xv[i][e] * xv[i][e];
      dot += xv[i][e] * g[i][e];
    }
  }
  ss = wave_sum(ss);
  dot = wave_sum(dot);
  const float r = rsqrtf(ss / (float)cols + eps);
  const float c = r * r * r * dot / (float)cols;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    if (v >= nvec) continue;
    float d[8], rd[8];
    if (dres) {
      ld_f8(dres + pr * ldr + v * 8, rd);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) rd[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = rd[e] + r * g[i][e] - c * xv[i][e];
    if (out) st_f8(out + pr * ldo + v * 8, d);
    if (out_b || out_f) {
      if (gate) {
        float gf[8];
        unpack8(ld8(gate + v * 8), gf);
#pragma unroll
        for (int e = 0; e < 8; ++e) d[e] *= gf[e];
      }
      const bf16x8 b = pack8(d);
      if (out_b) st8(out_b + pr * ldob + v * 8, b);
      if (out_f) st8(out_f + frag_offset(pr, v * 8), b);
    }
  }
}

// ---------------------------------------------------------------------------
// Activation backward, 8 columns per thread.
//   GEGLU (GemmaMLP, condition_gemma.py:156-192: h = gelu_tanh(gg) * uu):
//     in = [gg | uu] (cols each), dy = dh ->
//     out = [dh uu gelu'(gg) | dh gelu(gg)]
//   SILU (the PI0 action-time MLP, pi0_flowmatching.py:300-310): in = z,
//     out = dy silu'(z)
// gelu_tanh(x) = x s, s = 1 / (1 + exp(-2u)), u = sqrt(2/pi) (x + 0.044715
// x^3) (the forward's own formula, common.h), so gelu' = s + x s (1 - s)
// 2 sqrt(2/pi) (1 + 3 * 0.044715 x^2);  silu'(z) = sig (1 + z (1 - sig)).
// ---------------------------------------------------------------------------
constexpr int kActGeglu = 0, kActSilu = 1, kGegluFwd = 2;

template <int ACT>
__global__ __launch_bounds__(256) void act_backward_kernel(
    const bf16_t* __restrict__ in, int64_t ldi, const bf16_t* __restrict__ dy,
    int64_t ldy, bf16_t* __restrict__ out, int64_t ldo, bf16_t* __restrict__ out_f,
    int64_t rows, int cols) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nv = cols >> 3;
  if (t >= rows * nv) return;
  const int64_t m = t / nv;
  const int c = (int)(t - m * nv) * 8;
  float a[8], d[8], o[8];
  unpack8(ld8(in + m * ldi + c), a);
  if (ACT == kGegluFwd) {
    // the forward product itself: out = gelu_tanh(gate) * up (dy unused)
    unpack8(ld8(in + m * ldi + cols + c), d);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = gelu_tanh(a[e]) * d[e];
    const bf16x8 b = pack8(o);
    if (out) st8(out + m * ldo + c, b);
    if (out_f) st8(out_f + frag_offset(m, c), b);
    return;
  }
  unpack8(ld8(dy + m * ldy + c), d);
  if (ACT == kActGeglu) {
    float u[8], o2[8];
    unpack8(ld8(in + m * ldi + cols + c), u);
#pragma unroll
    for (int e = 0; e < 8; ++e) geglu_grad(d[e], a[e], u[e], o[e], o2[e]);
    const bf16x8 b = pack8(o), b2 = pack8(o2);
    if (out) {
      st8(out + m * ldo + c, b);
      st8(out + m * ldo + cols + c, b2);
    }
    if (out_f) {
      st8(out_f + frag_offset(m, c), b);
      st8(out_f + frag_offset(m, cols + c), b2);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float z = a[e];
      const float sg = 1.f / (1.f + expf(-z));
      o[e] = d[e] * sg * (1.f + z * (1.f - sg));
    }
    const bf16x8 b = pack8(o);
    if (out) st8(out + m * ldo + c, b);
    if (out_f) st8(out_f + frag_offset(m, c), b);
  }
}

// ---------------------------------------------------------------------------
// Masked softmax backward of one attention problem, one wavefront per query
// row (row r = query token r / heads, head r % heads).  s: raw scores q . k
// (fp32), dp: dO . v (fp32), both [rows, ld]; key j is visible to the row
// iff kgrp[j] <= qgrp[token] (the make_att_2d_masks rule,
// model_utils.py:77-95).  With logits l = scale s and P = softmax over the
// visible keys:
//   D = sum_j P_j dp_j,  ds_j = scale P_j (dp_j - D)   (d of the raw score)
// ds is written for columns [0, n_cols) (zero past n_keys and on masked
// keys); for the n_suffix keys from key0 the row also goes into column r of
// ds_t and p_t ([n_suffix, ldt], bf16): the A operands of dK = ds^T Q and
// dV = P^T dO.  Four passes over the row (max, sum, D, write) re-read s and
// dp from the cache instead of holding a row of any length in registers.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attn_rows_backward_kernel(
    const float* __restrict__ s, int64_t lds, const float* __restrict__ dp,
    int64_t lddp, const int32_t* __restrict__ kgrp,
    const int32_t* __restrict__ qgrp, bf16_t* __restrict__ ds, int64_t ldds,
    bf16_t* __restrict__ ds_t, bf16_t* __restrict__ p_t, int64_t ldt,
    int64_t key0, int n_suffix, int64_t rows, int heads, int n_keys,
    int n_cols, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * kBwdRows + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int32_t qg = qgrp ? qgrp[r / heads] : 0;
  const float* sr = s + r * lds;
  const float* dr = dp + r * lddp;
  constexpr float kLog2e = 1.4426950408889634f;
  float mx = -INFINITY;
  for (int j = lane; j < n_keys; j += 64)
    if (!kgrp || kgrp[j] <= qg) mx = fmaxf(mx, sr[j] * scale);
  mx = wave_max(mx);
  float l = 0.f;
  if (mx != -INFINITY)
    for (int j = lane; j < n_keys; j += 64)
      if (!kgrp || kgrp[j] <= qg) l += exp2f((sr[j] * scale - mx) * kLog2e);
  l = wave_sum(l);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float dsum = 0.f;
  for (int j = lane; j < n_keys; j += 64)
    if (!kgrp || kgrp[j] <= qg)
      dsum += exp2f((sr[j] * scale - mx) * kLog2e) * inv * dr[j];
  dsum = wave_sum(dsum);
  for (int j = lane; j < n_cols; j += 64) {
    float p = 0.f, d = 0.f;
    if (j < n_keys && (!kgrp || kgrp[j] <= qg) && l > 0.f) {
      p = exp2f((sr[j] * scale - mx) * kLog2e) * inv;
      d = scale * p * (dr[j] - dsum);
    }
    ds[r * ldds + j] = f2bf(d);
    const int64_t js = j - key0;
    if (js >= 0 && js < n_suffix) {
      if (ds_t) ds_t[js * ldt + r] = f2bf(d);
      if (p_t) p_t[js * ldt + r] = f2bf(p);
    }
  }
}

// The same with the row held in registers (NK keys per lane, up to 64 NK
// keys): every load of the row is issued at once, one memory round trip
// instead of four passes' worth.
template <int NK>
__global__ __launch_bounds__(256) void attn_rows_backward_reg_kernel(
    const float* __restrict__ s, int64_t lds, const float* __restrict__ dp,
    int64_t lddp, const int32_t* __restrict__ kgrp,
    const int32_t* __restrict__ qgrp, bf16_t* __restrict__ ds, int64_t ldds,
    bf16_t* __restrict__ ds_t, bf16_t* __restrict__ p_t, int64_t ldt,
    int64_t key0, int n_suffix, int64_t rows, int heads, int n_keys,
    int n_cols, float scale) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * kBwdRows + (threadIdx.x >> 6);
  if (r >= rows) return;
  const int32_t qg = qgrp ? qgrp[r / heads] : 0;
  const float* sr = s + r * lds;
  const float* dr = dp + r * lddp;
  constexpr float kLog2e = 1.4426950408889634f;
  float lg[NK], dv[NK];
  bool vis[NK];
#pragma unroll
  for (int c = 0; c < NK; ++c) {
    const int j = lane + 64 * c;
    const bool in = j < n_keys;
    lg[c] = in ? sr[j] : 0.f;
    dv[c] = in ? dr[j] : 0.f;
    vis[c] = in && (!kgrp || kgrp[j] <= qg);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < NK; ++c) {
    lg[c] *= scale;
    if (vis[c]) mx = fmaxf(mx, lg[c]);
  }
  mx = wave_max(mx);
  float l = 0.f;
#pragma unroll
  for (int c = 0; c < NK; ++c) {
    lg[c] = vis[c] ? exp2f((lg[c] - mx) * kLog2e) : 0.f;
    l += lg[c];
  }
  l = wave_sum(l);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  float dsum = 0.f;
#pragma unroll
  for (int c = 0; c < NK; ++c) {
    lg[c] *= inv;  // P
    dsum += lg[c] * dv[c];
  }
  dsum = wave_sum(dsum);
#pragma unroll
  for (int c = 0; c < NK; ++c) {
    const int j = lane + 64 * c;
    if (j < n_cols) {
      const float d = scale * lg[c] * (dv[c] - dsum);  // 0 where P is 0
      ds[r * ldds + j] = f2bf(d);
      const int64_t js = j - key0;
      if (js >= 0 && js < n_suffix) {
        if (ds_t) ds_t[js * ldt + r] = f2bf(d);
        if (p_t) p_t[js * ldt + r] = f2bf(lg[c]);
      }
    }
  }
  for (int j = lane + 64 * NK; j < n_cols; j += 64) ds[r * ldds + j] = 0;
}

// ---------------------------------------------------------------------------
// Suffix keys' gradients of one attention problem: dk[j] = sum_r ds_t[j][r]
// q[r] and dv[j] = sum_r p_t[j][r] dO[r] (ds already carries the softmax
// scale), the sums over every query row r = (token, head) -- the heads
// share the one key/value head.  Workgroup (j, 64-column block): thread t
// owns 8 columns (t % 8) of every 32nd row from t / 8, loading 16 bytes of
// q and dO per row, four rows in flight; the 32 row groups' sums then add
// through LDS in row-group order.  fp32 out.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void attn_suffix_kv_backward_kernel(
    const bf16_t* __restrict__ ds_t, const bf16_t* __restrict__ p_t,
    int64_t ldt, const bf16_t* __restrict__ q, int64_t ldq,
    const bf16_t* __restrict__ dout, int64_t ldo, float* __restrict__ dk,
    int64_t ldk, float* __restrict__ dv, int64_t ldv, int rows, int cols) {
  __shared__ float red[2][32][65];
  const int t = threadIdx.x;
  const int cg = t & 7, rg = t >> 3;
  const int64_t j = blockIdx.x;
  const int c0 = blockIdx.y * 64 + cg * 8;
  const bool live = c0 < cols;  // cols % 8 == 0
  float ak[8], av[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) ak[e] = av[e] = 0.f;
  const bf16_t* dsr = ds_t + j * ldt;
  const bf16_t* ptr = p_t + j * ldt;
  int r = rg;
  for (; r + 96 < rows; r += 128) {
    float a[4], b[4];
    bf16x8 qv[4], ov[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int rr = r + 32 * u;
      a[u] = bf2f(dsr[rr]);
      b[u] = bf2f(ptr[rr]);
      qv[u] = live ? ld8(q + (int64_t)rr * ldq + c0) : zero8();
      ov[u] = live ? ld8(dout + (int64_t)rr * ldo + c0) : zero8();
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float qf[8], of[8];
      unpack8(qv[u], qf);
      unpack8(ov[u], of);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ak[e] += a[u] * qf[e];
        av[e] += b[u] * of[e];
      }
    }
  }
  for (; r < rows; r += 32) {
    const float a = bf2f(dsr[r]), b = bf2f(ptr[r]);
    if (live) {
      float qf[8], of[8];
      unpack8(ld8(q + (int64_t)r * ldq + c0), qf);
      unpack8(ld8(dout + (int64_t)r * ldo + c0), of);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ak[e] += a * qf[e];
        av[e] += b * of[e];
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[0][rg][cg * 8 + e] = ak[e];
    red[1][rg][cg * 8 + e] = av[e];
  }
  __syncthreads();
  if (t < 128) {
    const int which = t >> 6, c = t & 63;
    float sum = 0.f;
    for (int g = 0; g < 32; ++g) sum += red[which][g][c];
    const int col = blockIdx.y * 64 + c;
    if (col < cols) {
      if (which == 0) dk[j * ldk + col] = sum;
      else dv[j * ldv + col] = sum;
    }
  }
}

// ---------------------------------------------------------------------------
// Fused attention backward of the decode shape (rows r = (token, head) of
// one problem against all its keys, head_dim 256, one key/value head), on
// bf16 MFMA.  Tiles of 32 rows x 64 keys, one workgroup each (grid: row
// block, key tile, problem):
//   attn_bwd_stats_kernel  S = Q K^T for the tile, the masked row maximum
//                          and sum of exp2 over its keys (log2 domain);
//   attn_bwd_main_kernel   the row's log-sum-exp from every tile's pair,
//                          D = dO . O per row, S again (bitwise the same
//                          MFMA sequence), P, dP = dO V^T, dS = scale P (dP -
//                          D), the suffix keys' dS and P transposed into
//                          ds_t / p_t, and dQ's share of the tile, dS K, as
//                          an fp32 partial per key tile (summed by the RoPE
//                          backward).
// MFMA 32x32x16 (common.h mfma32x32x16): lane l supplies row / column
// l % 32 with the 8 k-values 8 (l / 32) .. of each 16-k step; accumulator i
// of lane l is (row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32).
// Operands come straight from global memory through buffer views whose
// bounds make rows past R and keys past the problem's read as zero.
// ---------------------------------------------------------------------------
constexpr int kBwdD = 256;       // head_dim of this path
constexpr int kBwdRB = 32;       // rows per tile
constexpr int kBwdKT = 64;       // keys per tile

struct AttnBwdArgs {
  const bf16_t* q; int64_t q_zs;     // [R][256] per problem (rows contiguous)
  const bf16_t* o; int64_t o_zs;     // attention output, same layout
  const bf16_t* dout; int64_t do_zs; // its gradient, same layout
  const bf16_t* k; int64_t k_zs;     // key rows [nk][256]
  const bf16_t* v; int64_t v_zs;     // value rows [nk][256]
  const bf16_t* kt; int64_t kt_ld, kt_zs;  // keys transposed [256][kt_ld]
  const bf16_t* vt; int64_t vt_ld, vt_zs;  // values transposed [256][vt_ld] (refresh)
  int rk0, rn;                        // keys whose kt columns / v rows are refreshed
  const int32_t* kgrp; int64_t kgrp_zs;
  const int32_t* qgrp; int64_t qgrp_zs;
  float* pm; float* pl;              // [problem][key tile][R]
  float* dq; int64_t dq_part_stride; // [key tile][problems * R][256]
  bf16_t* ds_t; bf16_t* p_t; int64_t ldt, t_zs;  // [problem][n_suffix][ldt]
  int rows, heads, n_keys, key0, n_suffix, n_kt;
  float scale;
};

// Visibility inputs of a tile, read once: each lane's key group (INT_MAX
// past the keys) and the tile rows' query groups in LDS (INT_MIN past the
// rows, so that nothing is visible there).  A load per (row, key) behind
// the mask test would make every test wait for its own round trip.
__device__ __forceinline__ int32_t bwd_key_group(const AttnBwdArgs& a, const int32_t* kg,
                                                 int j) {
  return j < a.n_keys ? (kg ? kg[j] : 0) : INT32_MAX;
}

__device__ __forceinline__ void bwd_stage_qgrp(const AttnBwdArgs& a, const int32_t* qg,
                                               int r0, int32_t* sQG) {
  const int t = threadIdx.x;
  if (t < kBwdRB) {
    const int r = r0 + t;
    sQG[t] = r < a.rows ? (qg ? qg[r / a.heads] : 0) : INT32_MIN;
  }
}

// S (or dP) block of 32 rows x 32 keys: A rows from `ra` (row r0 + l % 32),
// B rows from `rb` (key kb + l % 32), 16 steps over the 256 dims.  All 32
// loads are issued before the first MFMA (the scheduling barrier keeps the
// compiler from interleaving them with the MFMAs, which would make every
// step wait for its own round trip).
__device__ __forceinline__ f32x16_t bwd_block(__amdgpu_buffer_rsrc_t ra, int r0,
                                              __amdgpu_buffer_rsrc_t rb, int kb, int lane) {
  f32x16_t acc = {};
  const uint32_t ao = (uint32_t)((r0 + (lane & 31)) * kBwdD + 8 * (lane >> 5)) * 2;
  const uint32_t bo = (uint32_t)((kb + (lane & 31)) * kBwdD + 8 * (lane >> 5)) * 2;
  bf16x8 av[16], bv[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    av[t] = bload8(ra, ao + (uint32_t)(16 * t) * 2);
    bv[t] = bload8(rb, bo + (uint32_t)(16 * t) * 2);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < 16; ++t) acc = mfma32x32x16(av[t], bv[t], acc);
  return acc;
}

__device__ __forceinline__ int acc_row(int i, int lane) {
  return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
}

__global__ __launch_bounds__(128) void attn_bwd_stats_kernel(AttnBwdArgs a) {
  // the tile's masked logits (log2 domain), [row][key], then reduced per row
  // by 4 threads of 16 keys each (LDS instead of 2 x 5 cross-lane steps per
  // accumulator row)
  __shared__ float sX[kBwdRB][kBwdKT + 1];
  __shared__ int32_t sQG[kBwdRB];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int z = blockIdx.z, kt = blockIdx.y, r0 = blockIdx.x * kBwdRB;
  const int kb = kt * kBwdKT + 32 * w;
  const int32_t* kg = a.kgrp ? a.kgrp + z * a.kgrp_zs : nullptr;
  const int32_t* qg = a.qgrp ? a.qgrp + z * a.qgrp_zs : nullptr;
  const int j = kb + (lane & 31);
  // the mask groups' loads go out first and are consumed after the MFMAs
  const int32_t kgv = bwd_key_group(a, kg, j);
  const int32_t qgv = (t < kBwdRB && r0 + t < a.rows) ? (qg ? qg[(r0 + t) / a.heads] : 0)
                                                      : INT32_MIN;
  const uint32_t rbytes = (uint32_t)a.rows * kBwdD * 2, kbytes = (uint32_t)a.n_keys * kBwdD * 2;
  const f32x16_t s = bwd_block(make_rsrc(a.q + z * a.q_zs, rbytes), r0,
                               make_rsrc(a.k + z * a.k_zs, kbytes), kb, lane);
  if (t < kBwdRB) sQG[t] = qgv;
  __syncthreads();
  const float c = a.scale * 1.4426950408889634f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rr = acc_row(i, lane);
    sX[rr][32 * w + (lane & 31)] = kgv <= sQG[rr] ? s[i] * c : -INFINITY;
  }
  __syncthreads();
  const int rr = t >> 2, part = t & 3;
  float x[16], m = -INFINITY;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    x[u] = sX[rr][16 * part + u];
    m = fmaxf(m, x[u]);
  }
  m = fmaxf(m, __shfl_xor(m, 1, 64));
  m = fmaxf(m, __shfl_xor(m, 2, 64));
  float e = 0.f;
  if (m != -INFINITY)
#pragma unroll
    for (int u = 0; u < 16; ++u) e += x[u] == -INFINITY ? 0.f : exp2f(x[u] - m);
  e += __shfl_xor(e, 1, 64);
  e += __shfl_xor(e, 2, 64);
  if (part == 0 && r0 + rr < a.rows) {
    const int64_t at = ((int64_t)z * a.n_kt + kt) * a.rows + r0 + rr;
    a.pm[at] = m;
    a.pl[at] = e;
  }
  // Refresh of the main pass's operand copies for keys [rk0, rk0 + rn) of
  // this tile (the keys this step wrote into the caches): kt's columns from
  // the key rows and v's rows from the transposed values.  The tile's row
  // blocks split the 256 dims between them (8 at a time), so the few
  // elements each writes cost no more than a short tail.  Only the main
  // pass reads kt and v.
  if (a.vt) {
    const int j0 = max(kt * kBwdKT, a.rk0), j1 = min(kt * kBwdKT + kBwdKT, a.rk0 + a.rn);
    const int dch = ((kBwdD / 8 + (int)gridDim.x - 1) / (int)gridDim.x) * 8;
    const int d0 = blockIdx.x * dch, d1 = min(kBwdD, d0 + dch);
    if (j0 < j1 && d0 < d1) {
      const int nj = j1 - j0, nd = d1 - d0;
      const bf16_t* kz = a.k + z * a.k_zs;
      const bf16_t* vtz = a.vt + z * a.vt_zs;
      bf16_t* ktz = const_cast<bf16_t*>(a.kt) + z * a.kt_zs;
      bf16_t* vz = const_cast<bf16_t*>(a.v) + z * a.v_zs;
      // 16 elements per thread and pass: all loads first, then the stores
      // (a store ahead of the next load would make every element wait for
      // its own round trip: the compiler cannot move a load above a store
      // that may alias it)
      const int total = nj * nd;
      for (int base = t; base < total; base += 128 * 16) {  // writes along keys
        bf16_t vals[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int idx = base + 128 * u;
          const int d = d0 + idx / nj, jj = idx % nj;
          vals[u] = idx < total ? kz[(int64_t)(j0 + jj) * kBwdD + d] : (bf16_t)0;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int idx = base + 128 * u;
          const int d = d0 + idx / nj, jj = idx % nj;
          if (idx < total) ktz[(int64_t)d * a.kt_ld + j0 + jj] = vals[u];
        }
      }
      for (int base = t; base < total; base += 128 * 16) {  // writes along dims
        bf16_t vals[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int idx = base + 128 * u;
          const int jj = idx / nd, d = d0 + idx % nd;
          vals[u] = idx < total ? vtz[(int64_t)d * a.vt_ld + j0 + jj] : (bf16_t)0;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int idx = base + 128 * u;
          const int jj = idx / nd, d = d0 + idx % nd;
          if (idx < total) vz[(int64_t)(j0 + jj) * kBwdD + d] = vals[u];
        }
      }
    }
  }
}

__global__ __launch_bounds__(256) void attn_bwd_main_kernel(AttnBwdArgs a) {
  __shared__ float sD[kBwdRB], sLse[kBwdRB];
  __shared__ int32_t sQG[kBwdRB];
  __shared__ float sdP[2][16][64];
  __shared__ __align__(16) bf16_t sDS[kBwdRB][kBwdKT + 8];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int z = blockIdx.z, kt = blockIdx.y, r0 = blockIdx.x * kBwdRB;
  const int k0 = kt * kBwdKT;
  const uint32_t rbytes = (uint32_t)a.rows * kBwdD * 2, kbytes = (uint32_t)a.n_keys * kBwdD * 2;
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q + z * a.q_zs, rbytes);
  const __amdgpu_buffer_rsrc_t rdo = make_rsrc(a.dout + z * a.do_zs, rbytes);
  // D = dO . O of the tile's rows: thread t takes 32 dims of row t / 8
  {
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.o + z * a.o_zs, rbytes);
    const int rr = t >> 3;
    const uint32_t off = (uint32_t)((r0 + rr) * kBwdD + 32 * (t & 7)) * 2;
    float d = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float fo[8], fd[8];
      unpack8(bload8(ro, off + 16 * u), fo);
      unpack8(bload8(rdo, off + 16 * u), fd);
#pragma unroll
      for (int e = 0; e < 8; ++e) d += fo[e] * fd[e];
    }
    d += __shfl_xor(d, 1, 64);
    d += __shfl_xor(d, 2, 64);
    d += __shfl_xor(d, 4, 64);
    if ((t & 7) == 0) sD[rr] = d;
  }
  // log-sum-exp (log2 domain) of each row over every key tile's pair: 16
  // tiles' pairs loaded at once per pass (unconditional buffer loads; the
  // tiles past n_kt are masked after), a running rescale between passes
  if (t < kBwdRB) {
    float M = -INFINITY, L = 0.f;
    if (r0 + t < a.rows) {
      // views of this problem's pairs (workgroup-uniform: a per-lane view
      // would make every load a loop over the lanes)
      const int64_t base = (int64_t)z * a.n_kt * a.rows;
      const uint32_t bytes = (uint32_t)((int64_t)a.n_kt * a.rows * 4);
      const __amdgpu_buffer_rsrc_t rm = make_rsrc(a.pm + base, bytes);
      const __amdgpu_buffer_rsrc_t rl = make_rsrc(a.pl + base, bytes);
      for (int u0 = 0; u0 < a.n_kt; u0 += 16) {
        float mv[16], lv[16], mn = M;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const uint32_t off = (uint32_t)(((int64_t)(u0 + u) * a.rows + r0 + t) * 4);
          mv[u] = bload1f(rm, off);
          lv[u] = bload1f(rl, off);
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          if (u0 + u >= a.n_kt) mv[u] = -INFINITY;
          mn = fmaxf(mn, mv[u]);
        }
        if (mn != -INFINITY) {
          L *= exp2f(M - mn);  // 0 on the first pass (M = -inf)
#pragma unroll
          for (int u = 0; u < 16; ++u)
            if (mv[u] != -INFINITY) L += lv[u] * exp2f(mv[u] - mn);
          M = mn;
        }
      }
    }
    sLse[t] = L > 0.f ? M + log2f(L) : INFINITY;
  }
  const int32_t* kg = a.kgrp ? a.kgrp + z * a.kgrp_zs : nullptr;
  const int32_t* qg = a.qgrp ? a.qgrp + z * a.qgrp_zs : nullptr;
  const int kh = w & 1, kb = k0 + 32 * kh, j = kb + (lane & 31);
  const int32_t kgv = bwd_key_group(a, kg, j);
  // loaded now, stored after the MFMAs (no wait ahead of the operand loads)
  const int rq_t = t - 128;
  const int32_t qgv = (rq_t >= 0 && rq_t < kBwdRB && r0 + rq_t < a.rows)
                          ? (qg ? qg[(r0 + rq_t) / a.heads] : 0)
                          : INT32_MIN;
  f32x16_t acc;
  if (w < 2) {
    acc = bwd_block(rq, r0, make_rsrc(a.k + z * a.k_zs, kbytes), kb, lane);
  } else {
    acc = bwd_block(rdo, r0, make_rsrc(a.v + z * a.v_zs, kbytes), kb, lane);
  }
  // the dQ product's K^T fragments (wave w: dims 64 w .. 64 w + 63), loaded
  // now so that they are in flight during the softmax and ahead of the
  // stores below (a load after a possibly aliasing store waits for it)
  const __amdgpu_buffer_rsrc_t rkt =
      make_rsrc(a.kt + z * a.kt_zs, (uint32_t)(kBwdD * a.kt_ld * 2));
  bf16x8 kv[4][2];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int key = k0 + 16 * ks + 8 * (lane >> 5);  // 8 keys wholly below kt_ld or not
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int d = 64 * w + 32 * nb + (lane & 31);
      kv[ks][nb] = bload8(rkt, key < a.kt_ld ? (uint32_t)(d * a.kt_ld + key) * 2 : kOOB);
    }
  }
  if (w >= 2) {
#pragma unroll
    for (int i = 0; i < 16; ++i) sdP[kh][i][lane] = acc[i];
    if (rq_t >= 0 && rq_t < kBwdRB) sQG[rq_t] = qgv;
  }
  __syncthreads();
  if (w < 2) {
    const float c = a.scale * 1.4426950408889634f;
    bf16_t* dst = a.ds_t ? a.ds_t + z * a.t_zs : nullptr;
    bf16_t* pst = a.p_t ? a.p_t + z * a.t_zs : nullptr;
    const int js = j - a.key0;
    const bool suf = js >= 0 && js < a.n_suffix;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rr = acc_row(i, lane), r = r0 + rr;
      float p = 0.f, ds = 0.f;
      if (kgv <= sQG[rr]) {
        p = exp2f(acc[i] * c - sLse[rr]);
        ds = a.scale * p * (sdP[kh][i][lane] - sD[rr]);
      }
      sDS[rr][32 * kh + (lane & 31)] = f2bf(ds);
      if (suf && r < a.rows) {
        if (dst) dst[(int64_t)js * a.ldt + r] = f2bf(ds);
        if (pst) pst[(int64_t)js * a.ldt + r] = f2bf(p);
      }
    }
  }
  __syncthreads();
  // dQ share of this key tile: [32 rows][256 dims] = dS [32][64] K [64][256];
  // wave w takes the dims 64 w .. 64 w + 63 (two 32-column blocks)
  f32x16_t dq[2] = {};
  bf16x8 av[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    av[ks] = *reinterpret_cast<const bf16x8*>(&sDS[lane & 31][16 * ks + 8 * (lane >> 5)]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) dq[nb] = mfma32x32x16(av[ks], kv[ks][nb], dq[nb]);
  float* out = a.dq + (int64_t)kt * a.dq_part_stride + ((int64_t)z * a.rows + r0) * kBwdD;
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int d = 64 * w + 32 * nb + (lane & 31);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rr = acc_row(i, lane);
      if (r0 + rr < a.rows) out[(int64_t)rr * kBwdD + d] = dq[nb][i];
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 transpose, 32 x 32 tiles through LDS (one padding column keeps the
// column reads conflict-free): dst[b][c][r] = src[b][r][c].
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void transpose_kernel(
    const bf16_t* __restrict__ src, int64_t ld_src, int64_t src_bs,
    bf16_t* __restrict__ dst, int64_t ld_dst, int64_t dst_bs, int64_t rows,
    int64_t cols) {
  __shared__ bf16_t tile[32][33];
  const int64_t b = blockIdx.z;
  const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
  const bf16_t* sb = src + b * src_bs;
  bf16_t* db = dst + b * dst_bs;
#pragma unroll
  for (int i = 0; i < 32; i += 8) {
    const int64_t r = r0 + ty + i, c = c0 + tx;
    if (r < rows && c < cols) tile[ty + i][tx] = sb[r * ld_src + c];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 32; i += 8) {
    const int64_t c = c0 + ty + i, r = r0 + tx;
    if (r < rows && c < cols) db[c * ld_dst + r] = tile[tx][ty + i];
  }
}

// ---------------------------------------------------------------------------
// RoPE backward, packed: row m of out = [dq rotated back (n_q_heads heads) |
// dk rotated back | dv], bf16 -- the dY of the Q|K|V GEMM.  The forward
// rotates pair (2i, 2i+1) of each head (pair-interleaved columns) by
// (cos, sin) = rope[pos][i]: (a, b) -> (a c - b s, b c + a s); its
// transpose takes (ga, gb) -> (ga c + gb s, gb c - ga s).  One thread per
// column pair.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rope_backward_kernel(
    const float* __restrict__ dq, int64_t ldq, int dq_parts, int64_t dq_part_stride,
    const float* __restrict__ dk,
    int64_t ldk, const float* __restrict__ dv, int64_t ldv,
    const float* __restrict__ rope, const int32_t* __restrict__ positions,
    bf16_t* __restrict__ out, int64_t ldo, bf16_t* __restrict__ out_f, int64_t rows,
    int n_q_heads, int head_dim) {
  const int half = head_dim >> 1;
  const int pairs = (n_q_heads + 2) * half;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * pairs) return;
  const int64_t m = t / pairs;
  const int p = (int)(t - m * pairs);
  const int qpairs = n_q_heads * half;
  float a, b;
  bool rot = true;
  if (p < qpairs) {
    // dq: the sum of dq_parts partials (key tiles), in part order, eight
    // partials' loads in flight at a time (one round trip per eight)
    a = b = 0.f;
    const float* src = dq + m * ldq + 2 * p;
    for (int u0 = 0; u0 < dq_parts; u0 += 8) {
      float2 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = u0 + u < dq_parts
                   ? *reinterpret_cast<const float2*>(src + (int64_t)(u0 + u) * dq_part_stride)
                   : float2{0.f, 0.f};
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        a += v[u].x;
        b += v[u].y;
      }
    }
  } else if (p < qpairs + half) {
    const int i = p - qpairs;
    a = dk[m * ldk + 2 * i];
    b = dk[m * ldk + 2 * i + 1];
  } else {
    const int i = p - qpairs - half;
    a = dv[m * ldv + 2 * i];
    b = dv[m * ldv + 2 * i + 1];
    rot = false;
  }
  if (rot) {
    const int i = p % half;
    const float* cs = rope + ((int64_t)positions[m] * half + i) * 2;
    const float c = cs[0], s = cs[1];
    const float ga = a * c + b * s, gb = b * c - a * s;
    a = ga;
    b = gb;
  }
  const uint32_t v = f2bf2(a, b);
  if (out) *reinterpret_cast<uint32_t*>(out + m * ldo + 2 * p) = v;
  if (out_f) *reinterpret_cast<uint32_t*>(out_f + frag_offset(m, 2 * p)) = v;
}

// ---------------------------------------------------------------------------
// Guidance error and corrected Euler update (rtc_guidance.py:107-155 with
// use_vjp, under _predict_action_guidance_rtc, pi0_flowmatching.py:671-700,
// whose denoiser is -u for the model velocity u).  Row m is action step
// m % period of its sample; w: per-step prefix weights (zero past the
// previous chunk), omt = 1 - t of the step.
//   e = w (prev - x + omt u)                  (the error at x_1 = x - omt u)
//   x <- x + dt u - dt gw e + dt gw omt g      (g = J_u^T e)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rtc_vjp_error_kernel(
    const float* __restrict__ x, int64_t ldx, const float* __restrict__ u,
    int64_t ldu, const float* __restrict__ prev, int64_t ldp,
    const float* __restrict__ w, bf16_t* __restrict__ e, int64_t lde,
    int64_t rows, int cols, int64_t period, float omt) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * cols) return;
  const int64_t m = t / cols;
  const int c = (int)(t - m * cols);
  const float ev = w[m % period] * (prev[m * ldp + c] - x[m * ldx + c] + omt * u[m * ldu + c]);
  e[m * lde + c] = f2bf(ev);
}

__global__ __launch_bounds__(256) void rtc_vjp_update_kernel(
    float* __restrict__ x, int64_t ldx, bf16_t* __restrict__ xb, int64_t ldxb,
    const float* __restrict__ u, int64_t ldu, const float* __restrict__ prev,
    int64_t ldp, const float* __restrict__ w, const float* __restrict__ g,
    int64_t ldg, const float* __restrict__ gw, int64_t rows, int cols,
    int64_t period, float omt, float dt) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= rows * cols) return;
  const int64_t m = t / cols;
  const int c = (int)(t - m * cols);
  const float xv = x[m * ldx + c], uv = u[m * ldu + c];
  const float ev = w[m % period] * (prev[m * ldp + c] - xv + omt * uv);
  const float k = dt * gw[0];
  const float xn = xv + dt * uv - k * ev + k * omt * g[m * ldg + c];
  x[m * ldx + c] = xn;
  if (xb) xb[m * ldxb + c] = f2bf(xn);
}

inline unsigned blocks(int64_t items, int64_t per) {
  return (unsigned)((items + per - 1) / per);
}

inline bool al16(const void* p) { return aligned16(p); }

}  // namespace

}  // namespace fvx

using namespace fvx;

// A fragment-major output holds rows < 64 and 32-column steps.
static bool frag_fits(int64_t last_row, int64_t cols) {
  return last_row < 64 && cols % 32 == 0 && cols < (1 << 24);
}

extern "C" int fvx_rms_norm_backward(const void* x, int64_t ldx, const float* dy,
                                     int64_t ldy, const float* dres, int64_t ldr,
                                     const void* scale, const void* gate, float* out,
                                     int64_t ldo, void* out_bf16, int64_t ldob,
                                     void* out_frag, int64_t rows, int64_t cols,
                                     int64_t row_group, int64_t row_group_stride,
                                     float eps, void* stream) {
  clear_error();
  FVX_REQUIRE(x && dy && (out || out_bf16 || out_frag), FVX_ERR_NULL,
              "rms_norm_backward: x, dy and an output are required");
  {
    const int64_t last = rows <= 0 ? 0
                         : row_group > 0
                             ? ((rows - 1) / row_group) * row_group_stride + (rows - 1) % row_group
                             : rows - 1;
    FVX_REQUIRE(!out_frag || (frag_fits(last, cols) && al16(out_frag)), FVX_ERR_ARG,
                "rms_norm_backward: out_frag needs mapped rows < 64, cols %% 32 == 0 and a "
                "16-byte aligned buffer");
  }
  FVX_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 4096, FVX_ERR_SHAPE,
              "rms_norm_backward: cols must be a positive multiple of 8 <= 4096");
  FVX_REQUIRE(ldx >= cols && ldy >= cols && ldx % 8 == 0 && ldy % 8 == 0 &&
                  (!dres || (ldr >= cols && ldr % 8 == 0)) &&
                  (!out || (ldo >= cols && ldo % 8 == 0)) &&
                  (!out_bf16 || (ldob >= cols && ldob % 8 == 0)),
              FVX_ERR_SHAPE, "rms_norm_backward: leading dims must be >= cols, multiples of 8");
  FVX_REQUIRE(al16(x) && al16(dy) && al16(dres) && al16(out) && al16(out_bf16) &&
                  al16(scale) && al16(gate),
              FVX_ERR_ALIGN, "rms_norm_backward: pointers must be 16-byte aligned");
  FVX_REQUIRE(row_group >= 0 && (row_group == 0 || row_group_stride >= row_group),
              FVX_ERR_ARG, "rms_norm_backward: bad row group");
  FVX_REQUIRE(eps >= 0.f, FVX_ERR_ARG, "rms_norm_backward: eps must be >= 0");
  if (rows == 0) return FVX_OK;
  hipStream_t s = (hipStream_t)stream;
  const int nv = (int)((cols / 8 + 63) / 64);
  const dim3 grid(blocks(rows, kBwdRows));
#define L(NV)                                                                          \
  hipLaunchKernelGGL(rms_backward_kernel<NV>, grid, dim3(256), 0, s, (const bf16_t*)x, \
                     ldx, dy, ldy, dres, ldr, (const bf16_t*)scale,                    \
                     (const bf16_t*)gate, out, ldo, (bf16_t*)out_bf16, ldob,           \
                     (bf16_t*)out_frag, rows, (int)cols, row_group, row_group_stride, eps)
  switch (nv) {
    case 1: L(1); break;
    case 2: L(2); break;
    case 3: L(3); break;
    case 4: L(4); break;
    case 5: L(5); break;
    case 6: L(6); break;
    case 7: L(7); break;
    default: L(8); break;
  }
#undef L
  return launch_status("rms_norm_backward");
}

extern "C" int fvx_act_backward(int act, const void* in, int64_t ldi, const void* dy,
                                int64_t ldy, void* out, int64_t ldo, void* out_frag,
                                int64_t rows, int64_t cols, void* stream) {
  clear_error();
  FVX_REQUIRE(in && dy && (out || out_frag), FVX_ERR_NULL,
              "act_backward: in, dy and an output are required");
  FVX_REQUIRE(!out_frag || (frag_fits(rows - 1, act == FVX_ACT_BWD_GEGLU ? 2 * cols : cols) &&
                            al16(out_frag)),
              FVX_ERR_ARG, "act_backward: out_frag needs rows <= 64, 32-column steps and a "
                           "16-byte aligned buffer");
  FVX_REQUIRE(act == FVX_ACT_BWD_GEGLU || act == FVX_ACT_BWD_SILU, FVX_ERR_ARG,
              "act_backward: bad act %d", act);
  const int64_t w = act == FVX_ACT_BWD_GEGLU ? 2 * cols : cols;
  FVX_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols < (1 << 30), FVX_ERR_SHAPE,
              "act_backward: cols must be a positive multiple of 8");
  FVX_REQUIRE(ldi >= w && (!out || ldo >= w) && ldy >= cols && ldi % 8 == 0 &&
                  ldo % 8 == 0 && ldy % 8 == 0,
              FVX_ERR_SHAPE, "act_backward: leading dims too small or not multiples of 8");
  FVX_REQUIRE(al16(in) && al16(dy) && al16(out), FVX_ERR_ALIGN,
              "act_backward: pointers must be 16-byte aligned");
  if (rows == 0) return FVX_OK;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(blocks(rows * (cols / 8), 256));
  if (act == FVX_ACT_BWD_GEGLU)
    hipLaunchKernelGGL(act_backward_kernel<kActGeglu>, grid, dim3(256), 0, s,
                       (const bf16_t*)in, ldi, (const bf16_t*)dy, ldy, (bf16_t*)out, ldo,
                       (bf16_t*)out_frag, rows, (int)cols);
  else
    hipLaunchKernelGGL(act_backward_kernel<kActSilu>, grid, dim3(256), 0, s,
                       (const bf16_t*)in, ldi, (const bf16_t*)dy, ldy, (bf16_t*)out, ldo,
                       (bf16_t*)out_frag, rows, (int)cols);
  return launch_status("act_backward");
}

extern "C" int fvx_geglu_rows(const void* gu, int64_t ldgu, void* out, int64_t ldo,
                              void* out_frag, int64_t rows, int64_t cols, void* stream) {
  clear_error();
  FVX_REQUIRE(gu && (out || out_frag), FVX_ERR_NULL,
              "geglu_rows: gu and an output are required");
  FVX_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols < (1 << 30) &&
                  ldgu >= 2 * cols && (!out || ldo >= cols) && ldgu % 8 == 0 && ldo % 8 == 0,
              FVX_ERR_SHAPE, "geglu_rows: bad sizes");
  FVX_REQUIRE(al16(gu) && al16(out) && al16(out_frag), FVX_ERR_ALIGN,
              "geglu_rows: pointers must be 16-byte aligned");
  FVX_REQUIRE(!out_frag || frag_fits(rows - 1, cols), FVX_ERR_ARG,
              "geglu_rows: out_frag needs rows <= 64 and cols %% 32 == 0");
  if (rows == 0) return FVX_OK;
  hipLaunchKernelGGL(act_backward_kernel<kGegluFwd>, dim3(blocks(rows * (cols / 8), 256)),
                     dim3(256), 0, (hipStream_t)stream, (const bf16_t*)gu, ldgu,
                     (const bf16_t*)gu, ldgu, (bf16_t*)out, ldo, (bf16_t*)out_frag, rows,
                     (int)cols);
  return launch_status("geglu_rows");
}

extern "C" int fvx_attention_rows_backward(
    const float* s, int64_t lds, const float* dp, int64_t lddp, const int32_t* kgrp,
    const int32_t* qgrp, void* ds, int64_t ldds, void* ds_t, void* p_t, int64_t ldt,
    int64_t key0, int64_t n_suffix, int64_t rows, int64_t heads, int64_t n_keys,
    int64_t n_cols, float scale, void* stream) {
  clear_error();
  FVX_REQUIRE(s && dp && ds, FVX_ERR_NULL, "attention_rows_backward: s, dp, ds are required");
  FVX_REQUIRE((kgrp == nullptr) == (qgrp == nullptr), FVX_ERR_ARG,
              "attention_rows_backward: kgrp and qgrp must both be given or both be NULL");
  FVX_REQUIRE(rows >= 0 && heads > 0 && n_keys > 0 && n_cols >= n_keys &&
                  n_cols < (1 << 30) && lds >= n_keys && lddp >= n_keys && ldds >= n_cols,
              FVX_ERR_SHAPE, "attention_rows_backward: bad sizes");
  FVX_REQUIRE((!ds_t && !p_t) ||
                  (n_suffix > 0 && key0 >= 0 && key0 + n_suffix <= n_keys && ldt >= rows),
              FVX_ERR_SHAPE, "attention_rows_backward: bad suffix columns");
  if (rows == 0) return FVX_OK;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid(blocks(rows, kBwdRows));
  const int nk = (int)((n_keys + 63) / 64);
#define L(KERNEL)                                                                         \
  hipLaunchKernelGGL(KERNEL, grid, dim3(256), 0, st, s, lds, dp, lddp, kgrp, qgrp,        \
                     (bf16_t*)ds, ldds, (bf16_t*)ds_t, (bf16_t*)p_t, ldt, key0,           \
                     (int)n_suffix, rows, (int)heads, (int)n_keys, (int)n_cols, scale)
  if (nk <= 4) L(attn_rows_backward_reg_kernel<4>);
  else if (nk <= 8) L(attn_rows_backward_reg_kernel<8>);
  else if (nk <= 12) L(attn_rows_backward_reg_kernel<12>);
  else if (nk <= 16) L(attn_rows_backward_reg_kernel<16>);
  else L(attn_rows_backward_kernel);
#undef L
  return launch_status("attention_rows_backward");
}

extern "C" int fvx_attention_suffix_kv_backward(const void* ds_t, const void* p_t,
                                                int64_t ldt, const void* q, int64_t ldq,
                                                const void* dout, int64_t ldo, float* dk,
                                                int64_t ldk, float* dv, int64_t ldv,
                                                int64_t n_suffix, int64_t rows,
                                                int64_t cols, void* stream) {
  clear_error();
  FVX_REQUIRE(ds_t && p_t && q && dout && dk && dv, FVX_ERR_NULL,
              "attention_suffix_kv_backward: every operand is required");
  FVX_REQUIRE(n_suffix >= 0 && n_suffix < 65536 && rows > 0 && rows < (1 << 30) &&
                  cols > 0 && cols % 8 == 0 && cols < (1 << 22) && ldt >= rows &&
                  ldq >= cols && ldo >= cols && ldq % 8 == 0 && ldo % 8 == 0 &&
                  ldk >= cols && ldv >= cols,
              FVX_ERR_SHAPE, "attention_suffix_kv_backward: bad sizes");
  FVX_REQUIRE(al16(q) && al16(dout), FVX_ERR_ALIGN,
              "attention_suffix_kv_backward: q and dout must be 16-byte aligned");
  if (n_suffix == 0) return FVX_OK;
  hipLaunchKernelGGL(attn_suffix_kv_backward_kernel,
                     dim3((unsigned)n_suffix, blocks(cols, 64)), dim3(256), 0,
                     (hipStream_t)stream, (const bf16_t*)ds_t, (const bf16_t*)p_t, ldt,
                     (const bf16_t*)q, ldq, (const bf16_t*)dout, ldo, dk, ldk, dv, ldv,
                     (int)rows, (int)cols);
  return launch_status("attention_suffix_kv_backward");
}

extern "C" int fvx_transpose_bf16(const void* src, int64_t ld_src, int64_t src_batch_stride,
                                  void* dst, int64_t ld_dst, int64_t dst_batch_stride,
                                  int64_t rows, int64_t cols, int64_t batch, void* stream) {
  clear_error();
  FVX_REQUIRE(src && dst, FVX_ERR_NULL, "transpose_bf16: src and dst are required");
  FVX_REQUIRE(rows >= 0 && cols >= 0 && batch >= 0 && batch < 65536 && ld_src >= cols &&
                  ld_dst >= rows && rows < ((int64_t)1 << 31) / 32 * 32 &&
                  cols < ((int64_t)1 << 31) / 32 * 32,
              FVX_ERR_SHAPE, "transpose_bf16: bad sizes");
  if (rows == 0 || cols == 0 || batch == 0) return FVX_OK;
  const dim3 grid(blocks(cols, 32), blocks(rows, 32), (unsigned)batch);
  FVX_REQUIRE(grid.y < 65536, FVX_ERR_SHAPE, "transpose_bf16: too many rows");
  hipLaunchKernelGGL(transpose_kernel, grid, dim3(256), 0, (hipStream_t)stream,
                     (const bf16_t*)src, ld_src, src_batch_stride, (bf16_t*)dst, ld_dst,
                     dst_batch_stride, rows, cols);
  return launch_status("transpose_bf16");
}

extern "C" int fvx_rope_backward(const float* dq, int64_t ldq, int64_t dq_parts,
                                 int64_t dq_part_stride, const float* dk, int64_t ldk,
                                 const float* dv, int64_t ldv, const float* rope,
                                 const int32_t* positions, void* out, int64_t ldo,
                                 void* out_frag, int64_t rows, int64_t n_q_heads,
                                 int64_t head_dim, void* stream) {
  clear_error();
  FVX_REQUIRE(!out_frag || (frag_fits(rows - 1, (n_q_heads + 2) * head_dim) &&
                            ((uintptr_t)out_frag & 3) == 0),
              FVX_ERR_ARG, "rope_backward: out_frag needs rows <= 64 and 32-column steps");
  FVX_REQUIRE(dq_parts >= 1 && dq_parts < 4096 && (dq_parts == 1 || dq_part_stride % 2 == 0),
              FVX_ERR_ARG, "rope_backward: bad dq parts");
  FVX_REQUIRE(dq && dk && dv && rope && positions && (out || out_frag), FVX_ERR_NULL,
              "rope_backward: every operand and an output are required");
  FVX_REQUIRE(rows >= 0 && n_q_heads > 0 && head_dim > 0 && head_dim % 2 == 0 &&
                  ldq >= n_q_heads * head_dim && ldk >= head_dim && ldv >= head_dim &&
                  ldq % 2 == 0 && ldk % 2 == 0 && ldv % 2 == 0 && ldo % 2 == 0 &&
                  (!out || ldo >= (n_q_heads + 2) * head_dim),
              FVX_ERR_SHAPE, "rope_backward: bad sizes");
  FVX_REQUIRE(((uintptr_t)out & 3) == 0 && ((uintptr_t)dq & 7) == 0 &&
                  ((uintptr_t)dk & 7) == 0 && ((uintptr_t)dv & 7) == 0,
              FVX_ERR_ALIGN, "rope_backward: misaligned operand");
  if (rows == 0) return FVX_OK;
  const int64_t pairs = (n_q_heads + 2) * head_dim / 2;
  hipLaunchKernelGGL(rope_backward_kernel, dim3(blocks(rows * pairs, 256)), dim3(256), 0,
                     (hipStream_t)stream, dq, ldq, (int)dq_parts, dq_part_stride, dk, ldk,
                     dv, ldv, rope, positions, (bf16_t*)out, ldo, (bf16_t*)out_frag, rows,
                     (int)n_q_heads, (int)head_dim);
  return launch_status("rope_backward");
}

extern "C" int fvx_rtc_vjp_error(const float* x, int64_t ldx, const float* u, int64_t ldu,
                                 const float* prev, int64_t ldp, const float* w, void* e,
                                 int64_t lde, int64_t rows, int64_t cols, int64_t period,
                                 float omt, void* stream) {
  clear_error();
  FVX_REQUIRE(x && u && prev && w && e, FVX_ERR_NULL, "rtc_vjp_error: every operand is required");
  FVX_REQUIRE(rows >= 0 && cols > 0 && period > 0 && ldx >= cols && ldu >= cols &&
                  ldp >= cols && lde >= cols && cols < (1 << 30),
              FVX_ERR_SHAPE, "rtc_vjp_error: bad sizes");
  if (rows == 0) return FVX_OK;
  hipLaunchKernelGGL(rtc_vjp_error_kernel, dim3(blocks(rows * cols, 256)), dim3(256), 0,
                     (hipStream_t)stream, x, ldx, u, ldu, prev, ldp, w, (bf16_t*)e, lde,
                     rows, (int)cols, period, omt);
  return launch_status("rtc_vjp_error");
}

extern "C" int fvx_rtc_vjp_update(float* x, int64_t ldx, void* x_bf16, int64_t ldxb,
                                  const float* u, int64_t ldu, const float* prev, int64_t ldp,
                                  const float* w, const float* g, int64_t ldg,
                                  const float* gw, int64_t rows, int64_t cols,
                                  int64_t period, float omt, float dt, void* stream) {
  clear_error();
  FVX_REQUIRE(x && u && prev && w && g && gw, FVX_ERR_NULL,
              "rtc_vjp_update: x, u, prev, w, g and gw are required");
  FVX_REQUIRE(rows >= 0 && cols > 0 && period > 0 && ldx >= cols && ldu >= cols &&
                  ldp >= cols && ldg >= cols && (!x_bf16 || ldxb >= cols) && cols < (1 << 30),
              FVX_ERR_SHAPE, "rtc_vjp_update: bad sizes");
  if (rows == 0) return FVX_OK;
  hipLaunchKernelGGL(rtc_vjp_update_kernel, dim3(blocks(rows * cols, 256)), dim3(256), 0,
                     (hipStream_t)stream, x, ldx, (bf16_t*)x_bf16, ldxb, u, ldu, prev, ldp, w,
                     g, ldg, gw, rows, (int)cols, period, omt, dt);
  return launch_status("rtc_vjp_update");
}

extern "C" int fvx_attention_backward(const fvx_attn_bwd_desc* d, void* stream) {
  clear_error();
  FVX_REQUIRE(d, FVX_ERR_NULL, "attention_backward: descriptor is NULL");
  FVX_REQUIRE(d->q && d->o && d->dout && d->k && d->v && d->kt && d->stats && d->dq,
              FVX_ERR_NULL, "attention_backward: q, o, dout, k, v, kt, stats, dq required");
  FVX_REQUIRE(d->head_dim == kBwdD, FVX_ERR_SHAPE,
              "attention_backward: head_dim must be 256 (got %lld)", (long long)d->head_dim);
  FVX_REQUIRE((d->kgrp == nullptr) == (d->qgrp == nullptr), FVX_ERR_ARG,
              "attention_backward: kgrp and qgrp must both be given or both be NULL");
  FVX_REQUIRE(d->n_problems > 0 && d->n_problems < 65536 && d->heads > 0 && d->rows > 0 &&
                  d->rows % d->heads == 0 && d->n_keys > 0 && d->kt_ld >= d->n_keys &&
                  d->kt_ld % 8 == 0 && (int64_t)d->rows * kBwdD * 2 < ((int64_t)1 << 31) &&
                  (int64_t)d->kt_ld * kBwdD * 2 < ((int64_t)1 << 31),
              FVX_ERR_SHAPE, "attention_backward: bad sizes");
  FVX_REQUIRE(!d->vt || (d->refresh_key0 >= 0 && d->refresh_n >= 0 &&
                          d->refresh_key0 + d->refresh_n <= d->n_keys &&
                          d->vt_ld >= d->n_keys && al16(d->vt)),
              FVX_ERR_SHAPE, "attention_backward: bad refresh range or vt");
  FVX_REQUIRE((!d->ds_t && !d->p_t) ||
                  (d->n_suffix > 0 && d->key0 >= 0 && d->key0 + d->n_suffix <= d->n_keys &&
                   d->ldt >= d->rows),
              FVX_ERR_SHAPE, "attention_backward: bad suffix columns");
  FVX_REQUIRE(al16(d->q) && al16(d->o) && al16(d->dout) && al16(d->k) && al16(d->v) &&
                  al16(d->kt) && d->q_zs % 8 == 0 && d->o_zs % 8 == 0 && d->do_zs % 8 == 0 &&
                  d->k_zs % 8 == 0 && d->v_zs % 8 == 0 && d->kt_zs % 8 == 0,
              FVX_ERR_ALIGN, "attention_backward: operands must be 16-byte aligned");
  const int n_rb = (int)((d->rows + kBwdRB - 1) / kBwdRB);
  const int n_kt = (int)((d->n_keys + kBwdKT - 1) / kBwdKT);
  FVX_REQUIRE(d->dq_parts == n_kt, FVX_ERR_ARG,
              "attention_backward: dq must hold %d key-tile partials (dq_parts = %lld)", n_kt,
              (long long)d->dq_parts);
  AttnBwdArgs a;
  a.q = (const bf16_t*)d->q; a.q_zs = d->q_zs;
  a.o = (const bf16_t*)d->o; a.o_zs = d->o_zs;
  a.dout = (const bf16_t*)d->dout; a.do_zs = d->do_zs;
  a.k = (const bf16_t*)d->k; a.k_zs = d->k_zs;
  a.v = (const bf16_t*)d->v; a.v_zs = d->v_zs;
  a.kt = (const bf16_t*)d->kt; a.kt_ld = d->kt_ld; a.kt_zs = d->kt_zs;
  a.vt = (const bf16_t*)d->vt; a.vt_ld = d->vt_ld; a.vt_zs = d->vt_zs;
  a.rk0 = (int)d->refresh_key0; a.rn = (int)d->refresh_n;
  a.kgrp = d->kgrp; a.kgrp_zs = d->kgrp_zs;
  a.qgrp = d->qgrp; a.qgrp_zs = d->qgrp_zs;
  a.pm = d->stats;
  a.pl = d->stats + d->n_problems * n_kt * d->rows;
  a.dq = d->dq; a.dq_part_stride = d->n_problems * d->rows * kBwdD;
  a.ds_t = (bf16_t*)d->ds_t; a.p_t = (bf16_t*)d->p_t; a.ldt = d->ldt; a.t_zs = d->t_zs;
  a.rows = (int)d->rows; a.heads = (int)d->heads; a.n_keys = (int)d->n_keys;
  a.key0 = (int)d->key0; a.n_suffix = (int)d->n_suffix; a.n_kt = n_kt;
  a.scale = d->scale;
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid(n_rb, n_kt, (unsigned)d->n_problems);
  hipLaunchKernelGGL(attn_bwd_stats_kernel, grid, dim3(128), 0, s, a);
  hipLaunchKernelGGL(attn_bwd_main_kernel, grid, dim3(256), 0, s, a);
  return launch_status("attention_backward");
}

extern "C" int64_t fvx_attention_backward_parts(int64_t n_keys) {
  return n_keys > 0 ? (n_keys + kBwdKT - 1) / kBwdKT : 0;
}
