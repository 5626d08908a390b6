// Fused multi-query attention (gfx950): softmax(Q K^T * scale + mask) V.
//
// One workgroup = 4 waves x 16 query rows.  For MQA every query head of a
// token shares the single K/V head, so query rows are (token, head) pairs
// and one K/V tile in LDS feeds all of them (8 heads x 8 tokens per block for
// Gemma).  Keys stream in tiles of 32:
//
//   S^T(16 keys x 16 rows) = K_tile(16 x d) . Q^T(d x 16)     (MFMA, Q in VGPRs)
//
// computing S transposed leaves each lane with 8 scores of ONE query row, so
// the online-softmax statistics need only in-lane math plus two cross-lane
// shuffles, and the probabilities are already in the A-operand layout of
//
//   O(16 rows x 16 d) += P(16 x 32 keys) . V(32 keys x 16 d)
//
// for which V is stored transposed in LDS (keys contiguous) as it is copied
// in.  K/V rows past the key range are zero-filled; masked scores are -inf
// and never produce NaN (a row that has seen no visible key yet keeps a zero
// reference).  With kv_splits > 1 each split writes (O, m, l) partials to a
// workspace and the last workgroup of a row block merges them in split
// order (deterministic) -- used for the decode-shaped action-expert
// attention (408 query rows against the 867-key prefix+suffix cache).
#include <math.h>

#include "capi_util.h"
#include "common.h"

namespace fvx {

constexpr int kKeyTile = 32;
constexpr int kAttnCounterBytes = 4096 * 4;
constexpr float kLog2e = 1.4426950408889634f;

template <int HDP, int HDV>
__host__ __device__ constexpr int64_t attn_part_floats() {
  // per row block per split: 4 waves * (HDV/16 frags * 64 lanes * 4) + m,l
  return (int64_t)4 * (HDV / 16) * 64 * 4 + 2 * 64;
}

template <int HDP, int HDV>
__global__ __launch_bounds__(256) void attn_kernel(fvx_attn_desc p,
                                                   int n_row_blocks,
                                                   int splits, int64_t kps) {
  constexpr int LDK = HDP + 8;
  constexpr int LDV = kKeyTile + 8;
  constexpr int NS = HDP / 32;   // 32-wide d chunks of the QK^T product
  constexpr int ND = HDV / 16;   // 16-wide d chunks of the output
  __shared__ __align__(16) bf16_t sK[kKeyTile * LDK];
  __shared__ __align__(16) bf16_t sVt[HDV * LDV];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;
  const int rb = blockIdx.x, split = blockIdx.y, z = blockIdx.z;
  const int HD = (int)p.head_dim;
  const int64_t heads = p.heads;
  const int64_t R = p.sq * heads;

  const int64_t zb = z / p.zdiv, zh = z % p.zdiv;
  const bf16_t* Q = (const bf16_t*)p.q + zb * p.q_zs1 + zh * p.q_zs2;
  const bf16_t* K = (const bf16_t*)p.k + zb * p.k_zs1 + zh * p.k_zs2;
  const bf16_t* V = (const bf16_t*)p.v + zb * p.v_zs1 + zh * p.v_zs2;
  bf16_t* O = (bf16_t*)p.o + zb * p.o_zs1 + zh * p.o_zs2;
  const int32_t* kgrp = p.kgrp ? p.kgrp + zb * p.kgrp_zs1 : nullptr;
  const int32_t* qgrp = p.qgrp ? p.qgrp + zb * p.qgrp_zs1 : nullptr;

  // Zero the padded d-columns of the K tile once (HD < HDP).
  if (HD < HDP) {
    for (int i = tid; i < kKeyTile * (HDP - HD); i += 256) {
      const int key = i / (HDP - HD), d = HD + i % (HDP - HD);
      sK[key * LDK + d] = 0;
    }
  }

  // This lane's query row (B operand / softmax row).
  const int64_t qrow = (int64_t)rb * 64 + wave * 16 + fr;
  const bool qval = qrow < R;
  const int64_t qtok = qval ? qrow / heads : 0;
  const int64_t qhead = qval ? qrow % heads : 0;
  const int32_t qg = (qgrp && qval) ? qgrp[qtok] : 0;
  bf16x8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int d = 32 * s + 8 * g;
    qf[s] = (qval && d < HD)
                ? ld8(Q + qtok * p.q_tok_stride + qhead * p.q_head_stride + d)
                : zero8();
  }

  const float sc = p.scale * kLog2e;
  float m_run = -INFINITY, l_run = 0.f;  // per query row (lanes fr)
  f32x4_t o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int64_t kbeg = (int64_t)split * kps;
  const int64_t kend = (kbeg + kps < p.sk) ? kbeg + kps : p.sk;
  const int kchunks = HD / 8;

  for (int64_t t0 = kbeg; t0 < kend; t0 += kKeyTile) {
    __syncthreads();  // previous tile fully consumed
    // K tile -> sK (row-major, d contiguous)
    for (int i = tid; i < kKeyTile * kchunks; i += 256) {
      const int key = i / kchunks, c = i % kchunks;
      const int64_t j = t0 + key;
      st8(&sK[key * LDK + c * 8],
          j < kend ? ld8(K + j * p.k_tok_stride + c * 8) : zero8());
    }
    // V tile -> sVt (transposed, keys contiguous)
    for (int i = tid; i < kKeyTile * kchunks; i += 256) {
      const int key = i % kKeyTile, c = i / kKeyTile;
      const int64_t j = t0 + key;
      const bf16x8 vv = j < kend ? ld8(V + j * p.v_tok_stride + c * 8) : zero8();
      const bf16_t* ve = (const bf16_t*)&vv;
#pragma unroll
      for (int e = 0; e < 8; ++e) sVt[(c * 8 + e) * LDV + key] = ve[e];
    }
    __syncthreads();

    // Scores: lane holds keys t0 + kf*16 + 4g + e for its query row.
    float s[2][4];
#pragma unroll
    for (int kf = 0; kf < 2; ++kf) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ss = 0; ss < NS; ++ss)
        acc = mfma16x16x32(ld8(&sK[(kf * 16 + fr) * LDK + ss * 32 + 8 * g]),
                           qf[ss], acc);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t j = t0 + kf * 16 + 4 * g + e;
        bool vis = j < kend;
        if (vis && kgrp) vis = kgrp[j] <= qg;
        s[kf][e] = vis ? acc[e] * sc : -INFINITY;
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kf = 0; kf < 2; ++kf)
#pragma unroll
      for (int e = 0; e < 4; ++e) tmax = fmaxf(tmax, s[kf][e]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float m_ref = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_ref);
    float psum = 0.f;
    float pr[2][4];
#pragma unroll
    for (int kf = 0; kf < 2; ++kf)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pr[kf][e] = exp2f(s[kf][e] - m_ref);
        psum += pr[kf][e];
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // P as A operand: keys {4g+e} (e<4) and {16+4g+e} (e>=4).
    float pf[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pf[e] = pr[0][e];
      pf[4 + e] = pr[1][e];
    }
    const bf16x8 pa = pack8(pf);
    // Rescale O rows 4g+j by alpha of that row (held by lane 4g+j).
    float al[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) al[j] = __shfl(alpha, 4 * g + j, 64);
#pragma unroll
    for (int df = 0; df < ND; ++df) {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[df][j] *= al[j];
      const bf16_t* vt = &sVt[(df * 16 + fr) * LDV];
      bf16x8 vb;
      const uint2 lo = *(const uint2*)(vt + 4 * g);
      const uint2 hi = *(const uint2*)(vt + 16 + 4 * g);
      vb.w[0] = lo.x;
      vb.w[1] = lo.y;
      vb.w[2] = hi.x;
      vb.w[3] = hi.y;
      o[df] = mfma16x16x32(pa, vb, o[df]);
    }
  }

  // Rows of this lane's O fragment: rb*64 + wave*16 + 4g + j.
  const int64_t orow0 = (int64_t)rb * 64 + wave * 16 + 4 * g;
  if (splits > 1) {
    float* ws = (float*)((char*)p.workspace + kAttnCounterBytes);
    unsigned* counters = (unsigned*)p.workspace;
    const int64_t blk = (int64_t)z * n_row_blocks + rb;
    constexpr int64_t PF = attn_part_floats<HDP, HDV>();
    float* part = ws + (blk * splits + split) * PF;
#pragma unroll
    for (int df = 0; df < ND; ++df)
      *(f32x4_t*)(part + ((wave * ND + df) * 64 + lane) * 4) = o[df];
    if (g == 0) {
      part[4 * ND * 64 * 4 + wave * 16 + fr] = m_run;
      part[4 * ND * 64 * 4 + 64 + wave * 16 + fr] = l_run;
    }
    __threadfence();
    __syncthreads();
    __shared__ unsigned s_last;
    if (tid == 0) {
      const unsigned prev = atomicAdd(&counters[blk], 1u);
      s_last = (prev == (unsigned)(splits - 1)) ? 1u : 0u;
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    float mx = -INFINITY;
    for (int s2 = 0; s2 < splits; ++s2) {
      const float* q = ws + (blk * splits + s2) * PF;
      mx = fmaxf(mx, __builtin_nontemporal_load(q + 4 * ND * 64 * 4 + wave * 16 + fr));
    }
    const float mref = (mx == -INFINITY) ? 0.f : mx;
#pragma unroll
    for (int df = 0; df < ND; ++df) o[df] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    l_run = 0.f;
    for (int s2 = 0; s2 < splits; ++s2) {
      const float* q = ws + (blk * splits + s2) * PF;
      const float ms = __builtin_nontemporal_load(q + 4 * ND * 64 * 4 + wave * 16 + fr);
      const float ls = __builtin_nontemporal_load(q + 4 * ND * 64 * 4 + 64 + wave * 16 + fr);
      const float w = exp2f(ms - mref);
      l_run += ls * w;
      float wj[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) wj[j] = __shfl(w, 4 * g + j, 64);
#pragma unroll
      for (int df = 0; df < ND; ++df) {
        const f32x4_t t = __builtin_nontemporal_load(
            (const f32x4_t*)(q + ((wave * ND + df) * 64 + lane) * 4));
#pragma unroll
        for (int j = 0; j < 4; ++j) o[df][j] += t[j] * wj[j];
      }
    }
    if (tid == 0) counters[blk] = 0u;
  }

  float inv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float l = __shfl(l_run, 4 * g + j, 64);
    inv[j] = l > 0.f ? 1.f / l : 0.f;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t r = orow0 + j;
    if (r >= R) break;
    const int64_t tok = r / heads, h = r % heads;
    bf16_t* orow = O + tok * p.o_tok_stride + h * p.o_head_stride;
#pragma unroll
    for (int df = 0; df < ND; ++df) {
      const int d = df * 16 + fr;
      if (d < HD) orow[d] = f2bf(o[df][j] * inv[j]);
    }
  }
}

struct AttnPlan {
  int n_row_blocks, splits, hdp;
  int64_t kps, ws_bytes;
};

static AttnPlan plan_attn(const fvx_attn_desc& d) {
  AttnPlan a;
  const int64_t R = d.sq * d.heads;
  a.n_row_blocks = (int)((R + 63) / 64);
  a.hdp = d.head_dim > 96 ? 256 : 96;
  int splits = d.kv_splits;
  const int64_t blocks = (int64_t)a.n_row_blocks * d.n_problems;
  if (splits <= 0) {
    splits = (int)((256 + blocks - 1) / blocks);
    const int64_t max_split = (d.sk + 63) / 64;  // >= 2 key tiles per split
    if (splits > max_split) splits = (int)max_split;
    if (splits > 32) splits = 32;
    if (splits < 1) splits = 1;
  }
  int64_t kps = (d.sk + splits - 1) / splits;
  kps = (kps + kKeyTile - 1) / kKeyTile * kKeyTile;
  if (kps < kKeyTile) kps = kKeyTile;
  splits = (int)((d.sk + kps - 1) / kps);
  if (splits < 1) splits = 1;
  a.splits = splits;
  a.kps = splits == 1 ? ((d.sk + kKeyTile - 1) / kKeyTile) * kKeyTile : kps;
  const int64_t pf = a.hdp == 256 ? attn_part_floats<256, 256>()
                                  : attn_part_floats<96, 80>();
  a.ws_bytes = splits > 1 ? kAttnCounterBytes + blocks * splits * pf * 4 : 0;
  return a;
}

}  // namespace fvx

using namespace fvx;

extern "C" int64_t fvx_attention_workspace_bytes(const fvx_attn_desc* d) {
  if (!d || d->sq <= 0 || d->sk <= 0 || d->heads <= 0 || d->n_problems <= 0)
    return 0;
  return plan_attn(*d).ws_bytes;
}

extern "C" int fvx_attention(const fvx_attn_desc* dp, void* stream) {
  clear_error();
  FVX_REQUIRE(dp, FVX_ERR_NULL, "attention: descriptor is NULL");
  const fvx_attn_desc& d = *dp;
  FVX_REQUIRE(d.q && d.k && d.v && d.o, FVX_ERR_NULL,
              "attention: q, k, v, o required");
  FVX_REQUIRE(d.sq >= 0 && d.sk >= 0 && d.heads > 0 && d.n_problems >= 0 &&
                  d.zdiv > 0,
              FVX_ERR_SHAPE, "attention: bad sizes");
  FVX_REQUIRE(d.head_dim > 0 && d.head_dim % 8 == 0 &&
                  (d.head_dim <= 80 || d.head_dim == 256),
              FVX_ERR_SHAPE,
              "attention: head_dim must be a multiple of 8 and <= 80, or 256 "
              "(got %lld)",
              (long long)d.head_dim);
  FVX_REQUIRE(aligned16(d.q) && aligned16(d.k) && aligned16(d.v) &&
                  d.q_tok_stride % 8 == 0 && d.q_head_stride % 8 == 0 &&
                  d.k_tok_stride % 8 == 0 && d.v_tok_stride % 8 == 0 &&
                  d.q_zs1 % 8 == 0 && d.q_zs2 % 8 == 0 && d.k_zs1 % 8 == 0 &&
                  d.k_zs2 % 8 == 0 && d.v_zs1 % 8 == 0 && d.v_zs2 % 8 == 0,
              FVX_ERR_ALIGN,
              "attention: q/k/v pointers and strides must be 16B aligned");
  FVX_REQUIRE((d.kgrp == nullptr) == (d.qgrp == nullptr), FVX_ERR_ARG,
              "attention: kgrp and qgrp must both be given or both be NULL");
  if (d.sq == 0 || d.n_problems == 0) return FVX_OK;
  FVX_REQUIRE(d.sk > 0, FVX_ERR_SHAPE, "attention: sk must be > 0");
  AttnPlan a = plan_attn(d);
  if (a.splits > 1 && (!d.workspace || d.workspace_bytes < a.ws_bytes ||
                       (int64_t)a.n_row_blocks * d.n_problems > 4096)) {
    FVX_REQUIRE(d.kv_splits <= 1, FVX_ERR_WORKSPACE,
                "attention: kv_splits=%d needs %lld workspace bytes, got %lld",
                d.kv_splits, (long long)a.ws_bytes,
                (long long)d.workspace_bytes);
    a.splits = 1;
    a.kps = ((d.sk + kKeyTile - 1) / kKeyTile) * kKeyTile;
  }
  FVX_REQUIRE(aligned16(d.workspace), FVX_ERR_ALIGN,
              "attention: workspace must be 16B aligned");
  dim3 grid((unsigned)a.n_row_blocks, (unsigned)a.splits,
            (unsigned)d.n_problems);
  hipStream_t s = (hipStream_t)stream;
  if (a.hdp == 256)
    hipLaunchKernelGGL((attn_kernel<256, 256>), grid, dim3(256), 0, s, d,
                       a.n_row_blocks, a.splits, a.kps);
  else
    hipLaunchKernelGGL((attn_kernel<96, 80>), grid, dim3(256), 0, s, d,
                       a.n_row_blocks, a.splits, a.kps);
  return launch_status("attention");
}
