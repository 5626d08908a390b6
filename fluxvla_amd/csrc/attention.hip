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
// workspace and a merge kernel, the next kernel on the stream, combines them
// in split order (deterministic).  The decode-shaped action-expert attention
// (408 query rows against the 867-key prefix+suffix cache) runs the
// barrier-free attn_decode_kernel further below.
#include <math.h>

#include "capi_util.h"
#include "common.h"

namespace fvx {

constexpr int kKeyTile = 32;
constexpr float kLog2e = 1.4426950408889634f;

template <int HDP, int HDV>
__host__ __device__ constexpr int64_t attn_part_floats() {
  // per row block per split: 4 waves * (HDV/16 frags * 64 lanes * 4) + m,l
  return (int64_t)4 * (HDV / 16) * 64 * 4 + 2 * 64;
}

template <int ND>
__device__ __forceinline__ void store_rows(const fvx_attn_desc& p, bf16_t* O,
                                           int64_t row0, int64_t R,
                                           int64_t heads, int HD, int fr,
                                           int g, const f32x4_t* o,
                                           float l_run);

// Zero the elements e >= valid of an 8-key vector (keys past the range).
__device__ __forceinline__ bf16x8 mask_keys(bf16x8 v, int64_t valid) {
  if (valid >= 8) return v;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    if (2 * w >= valid) v.w[w] = 0u;
    else if (2 * w + 1 >= valid) v.w[w] &= 0xffffu;
  }
  return v;
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
  const int tile_chunks = kKeyTile * kchunks;
  // Register prefetch of the next K/V tile: CH 16-byte chunks per thread.
  constexpr int CH = (kKeyTile * (HDP / 8) + 255) / 256;
  bf16x8 rk[CH], rv[CH];
  auto prefetch = [&](int64_t t0) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int i = tid + 256 * c;
      rk[c] = zero8();
      rv[c] = zero8();
      if (i < tile_chunks) {
        const int64_t jk = t0 + i / kchunks;  // K: key-major chunks
        if (jk < kend) rk[c] = ld8(K + jk * p.k_tok_stride + (i % kchunks) * 8);
        if (p.v_d_stride > 0) {
          // V^T: chunk = 8 consecutive keys of one dim
          const int64_t j8 = t0 + (i % 4) * 8;
          if (j8 < kend) rv[c] = mask_keys(ld8(V + (i / 4) * p.v_d_stride + j8), kend - j8);
        } else {
          const int64_t jv = t0 + i % kKeyTile;  // V: key-minor chunks
          if (jv < kend) rv[c] = ld8(V + jv * p.v_tok_stride + (i / kKeyTile) * 8);
        }
      }
    }
  };
  if (kbeg < kend) prefetch(kbeg);

  for (int64_t t0 = kbeg; t0 < kend; t0 += kKeyTile) {
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int i = tid + 256 * c;
      if (i < tile_chunks) {
        st8(&sK[(i / kchunks) * LDK + (i % kchunks) * 8], rk[c]);
        if (p.v_d_stride > 0) {
          st8(&sVt[(i / 4) * LDV + (i % 4) * 8], rv[c]);
        } else {
          const bf16_t* ve = (const bf16_t*)&rv[c];
          const int key = i % kKeyTile, c8 = i / kKeyTile;
#pragma unroll
          for (int e = 0; e < 8; ++e) sVt[(c8 * 8 + e) * LDV + key] = ve[e];
        }
      }
    }
    __syncthreads();
    if (t0 + kKeyTile < kend) prefetch(t0 + kKeyTile);

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
  if (splits > 1) {
    // Partial (unnormalized O, running max m, sum l) of this key range; the
    // merge kernel that follows on the stream combines the splits.
    constexpr int64_t PF = attn_part_floats<HDP, HDV>();
    const int64_t blk = (int64_t)z * n_row_blocks + rb;
    float* part = (float*)p.workspace + (blk * splits + split) * PF;
#pragma unroll
    for (int df = 0; df < ND; ++df)
      *(f32x4_t*)(part + ((wave * ND + df) * 64 + lane) * 4) = o[df];
    if (g == 0) {
      part[4 * ND * 64 * 4 + wave * 16 + fr] = m_run;
      part[4 * ND * 64 * 4 + 64 + wave * 16 + fr] = l_run;
    }
    return;
  }
  store_rows<ND>(p, O, (int64_t)rb * 64 + wave * 16 + 4 * g, R, heads, HD,
                 fr, g, o, l_run);
}

// Normalize and store: lane holds d = df*16 + fr for rows row0 + j.
template <int ND>
__device__ __forceinline__ void store_rows(const fvx_attn_desc& p, bf16_t* O,
                                           int64_t row0, int64_t R,
                                           int64_t heads, int HD, int fr,
                                           int g, const f32x4_t* o,
                                           float l_run) {
  float inv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float l = __shfl(l_run, 4 * g + j, 64);
    inv[j] = l > 0.f ? 1.f / l : 0.f;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t r = row0 + j;
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

// Combine the split partials of one row block (same lane layout as the
// attention kernel): global max, rescale, sum, in split order.
template <int HDP, int HDV>
__global__ __launch_bounds__(256) void attn_merge_kernel(fvx_attn_desc p,
                                                         int n_row_blocks,
                                                         int splits) {
  constexpr int ND = HDV / 16;
  constexpr int64_t PF = attn_part_floats<HDP, HDV>();
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;
  const int rb = blockIdx.x, z = blockIdx.z;
  const int64_t R = p.sq * p.heads;
  const int64_t zb = z / p.zdiv, zh = z % p.zdiv;
  bf16_t* O = (bf16_t*)p.o + zb * p.o_zs1 + zh * p.o_zs2;
  const int64_t blk = (int64_t)z * n_row_blocks + rb;
  const float* ws = (const float*)p.workspace + blk * splits * PF;
  const float* mrow = ws + 4 * ND * 64 * 4 + wave * 16 + fr;
  float mx = -INFINITY;
  for (int s2 = 0; s2 < splits; ++s2) mx = fmaxf(mx, mrow[s2 * PF]);
  const float mref = (mx == -INFINITY) ? 0.f : mx;
  f32x4_t o[ND];
#pragma unroll
  for (int df = 0; df < ND; ++df) o[df] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float l_run = 0.f;
#pragma unroll 2
  for (int s2 = 0; s2 < splits; ++s2) {
    const float* q = ws + s2 * PF;
    f32x4_t t[ND];
#pragma unroll
    for (int df = 0; df < ND; ++df)
      t[df] = *(const f32x4_t*)(q + ((wave * ND + df) * 64 + lane) * 4);
    const float ms = q[4 * ND * 64 * 4 + wave * 16 + fr];
    const float ls = q[4 * ND * 64 * 4 + 64 + wave * 16 + fr];
    const float w = exp2f(ms - mref);
    l_run += ls * w;
    float wj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) wj[j] = __shfl(w, 4 * g + j, 64);
#pragma unroll
    for (int df = 0; df < ND; ++df)
#pragma unroll
      for (int j = 0; j < 4; ++j) o[df][j] += t[df][j] * wj[j];
  }
  store_rows<ND>(p, O, (int64_t)rb * 64 + wave * 16 + 4 * g, R, p.heads,
                 (int)p.head_dim, fr, g, o, l_run);
}

// ---------------------------------------------------------------------------
// Decode-shaped attention: no LDS, no barriers.  Work item = one wave =
// (problem z, 16 query rows, key range).  K comes straight from the cache as
// the A operand of S^T = K Q^T, with the rows of each 16-key fragment mapped
// to keys 8 * (i / 4) + 4 * kf + i % 4: lane group g then holds the 8
// consecutive keys 8g .. 8g + 7 of the 32-key tile, so its probabilities are
// a ready A operand of P V and the transposed value cache gives the B
// operand in one 16-byte load per 16 output dims.  The next tile's K loads
// are issued before the softmax and its V loads before the next QK^T.
// ---------------------------------------------------------------------------
constexpr int64_t kDecPF = 16 * 64 * 4 + 2 * 16;  // partial floats per item

__global__ __launch_bounds__(256) void attn_decode_kernel(fvx_attn_desc p,
                                                          int n_rb, int splits,
                                                          int64_t kps,
                                                          int n_items) {
  constexpr int HD = 256, NS = HD / 32, ND = HD / 16;
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= n_items) return;  // whole wave
  const int fr = lane & 15, g = lane >> 4;
  const int rb = item % n_rb, split = (item / n_rb) % splits;
  const int z = item / (n_rb * splits);
  const int64_t heads = p.heads, R = p.sq * heads;
  const int64_t zb = z / p.zdiv, zh = z % p.zdiv;
  const bf16_t* Q = (const bf16_t*)p.q + zb * p.q_zs1 + zh * p.q_zs2;
  const bf16_t* K = (const bf16_t*)p.k + zb * p.k_zs1 + zh * p.k_zs2;
  const bf16_t* Vt = (const bf16_t*)p.v + zb * p.v_zs1 + zh * p.v_zs2;
  const int32_t* kgrp = p.kgrp ? p.kgrp + zb * p.kgrp_zs1 : nullptr;
  const int32_t* qgrp = p.qgrp ? p.qgrp + zb * p.qgrp_zs1 : nullptr;

  const int64_t qrow = (int64_t)rb * 16 + fr;
  const bool qval = qrow < R;
  const int64_t qtok = qval ? qrow / heads : 0, qhead = qval ? qrow % heads : 0;
  const int32_t qg = (qgrp && qval) ? qgrp[qtok] : 0;
  bf16x8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    qf[s] = qval ? ld8(Q + qtok * p.q_tok_stride + qhead * p.q_head_stride +
                       32 * s + 8 * g)
                 : zero8();

  const int64_t kbeg = (int64_t)split * kps;
  const int64_t kend = (kbeg + kps < p.sk) ? kbeg + kps : p.sk;
  const int krow = 8 * (fr >> 2) + (fr & 3);  // tile row of this lane (kf=0)
  bf16x8 kr[2][NS], vr[ND];
  auto load_k = [&](int64_t t0) {
#pragma unroll
    for (int kf = 0; kf < 2; ++kf) {
      const int64_t j = t0 + krow + 4 * kf;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        kr[kf][s] = j < kend ? ld8(K + j * p.k_tok_stride + 32 * s + 8 * g) : zero8();
    }
  };
  auto load_v = [&](int64_t t0) {
    const int64_t j8 = t0 + 8 * g;
#pragma unroll
    for (int df = 0; df < ND; ++df)
      vr[df] = j8 < kend ? mask_keys(ld8(Vt + (df * 16 + fr) * p.v_d_stride + j8),
                                     kend - j8)
                         : zero8();
  };

  const float sc = p.scale * kLog2e;
  float m_run = -INFINITY, l_run = 0.f;
  f32x4_t o[ND];
#pragma unroll
  for (int i = 0; i < ND; ++i) o[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (kbeg < kend) {
    load_k(kbeg);
    load_v(kbeg);
  }
  for (int64_t t0 = kbeg; t0 < kend; t0 += kKeyTile) {
    float s[8];
#pragma unroll
    for (int kf = 0; kf < 2; ++kf) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ss = 0; ss < NS; ++ss) acc = mfma16x16x32(kr[kf][ss], qf[ss], acc);
#pragma unroll
      for (int e = 0; e < 4; ++e) s[4 * kf + e] = acc[e];
    }
    const bool more = t0 + kKeyTile < kend;
    if (more) load_k(t0 + kKeyTile);
    // lane group g holds keys t0 + 8g + e
    float tmax = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t j = t0 + 8 * g + e;
      bool vis = j < kend;
      if (vis && kgrp) vis = kgrp[j] <= qg;
      s[e] = vis ? s[e] * sc : -INFINITY;
      tmax = fmaxf(tmax, s[e]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float m_ref = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_ref);
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s[e] = exp2f(s[e] - m_ref);
      psum += s[e];
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
    const bf16x8 pa = pack8(s);
    float al[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) al[j] = __shfl(alpha, 4 * g + j, 64);
#pragma unroll
    for (int df = 0; df < ND; ++df) {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[df][j] *= al[j];
      o[df] = mfma16x16x32(pa, vr[df], o[df]);
    }
    if (more) load_v(t0 + kKeyTile);
  }

  if (splits > 1) {
    float* part = (float*)p.workspace + (int64_t)item * kDecPF;
#pragma unroll
    for (int df = 0; df < ND; ++df) *(f32x4_t*)(part + (df * 64 + lane) * 4) = o[df];
    if (g == 0) {
      part[ND * 64 * 4 + fr] = m_run;
      part[ND * 64 * 4 + 16 + fr] = l_run;
    }
    return;
  }
  bf16_t* O = (bf16_t*)p.o + zb * p.o_zs1 + zh * p.o_zs2;
  store_rows<ND>(p, O, (int64_t)rb * 16 + 4 * g, R, heads, HD, fr, g, o, l_run);
}

// Merge of the decode partials: one thread per (problem, 16-row block,
// output fragment float4) = 4 rows x 1 dim; every split's loads of a batch
// of 8 are issued before the running-max merge, applied in split order.
__global__ __launch_bounds__(256) void attn_decode_merge_kernel(
    fvx_attn_desc p, int n_rb, int splits) {
  constexpr int ND = 16;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n_blk = (int64_t)p.n_problems * n_rb;
  if (gid >= n_blk * ND * 64) return;
  const int64_t blk = gid / (ND * 64);
  const int fi = (int)(gid % (ND * 64));
  const int df = fi / 64, lane = fi % 64, fr = lane & 15, g = lane >> 4;
  const int z = (int)(blk / n_rb), rb = (int)(blk % n_rb);
  // item index of split s: rb + n_rb * (s + splits * z)
  float M[4], L[4];
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    M[j] = -INFINITY;
    L[j] = 0.f;
  }
  for (int s0 = 0; s0 < splits; s0 += 8) {
    f32x4_t ov[8], mv[8], lv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (s0 + i < splits) {
        const float* part =
            (const float*)p.workspace +
            ((int64_t)rb + (int64_t)n_rb * (s0 + i + (int64_t)splits * z)) * kDecPF;
        ov[i] = *(const f32x4_t*)(part + (df * 64 + lane) * 4);
        mv[i] = *(const f32x4_t*)(part + ND * 64 * 4 + 4 * g);
        lv[i] = *(const f32x4_t*)(part + ND * 64 * 4 + 16 + 4 * g);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (s0 + i < splits) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float mn = fmaxf(M[j], mv[i][j]);
          const float mr = (mn == -INFINITY) ? 0.f : mn;
          const float a = exp2f(M[j] - mr), b = exp2f(mv[i][j] - mr);
          acc[j] = acc[j] * a + ov[i][j] * b;
          L[j] = L[j] * a + lv[i][j] * b;
          M[j] = mn;
        }
      }
    }
  }
  const int64_t zb = z / p.zdiv, zh = z % p.zdiv;
  bf16_t* O = (bf16_t*)p.o + zb * p.o_zs1 + zh * p.o_zs2;
  const int64_t R = p.sq * p.heads;
  const int d = df * 16 + fr;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t r = (int64_t)rb * 16 + 4 * g + j;
    if (r >= R) break;
    const int64_t tok = r / p.heads, h = r % p.heads;
    O[tok * p.o_tok_stride + h * p.o_head_stride + d] =
        f2bf(L[j] > 0.f ? acc[j] / L[j] : 0.f);
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
    splits = (int)((160 + blocks - 1) / blocks);
    const int64_t max_split = (d.sk + 127) / 128;  // >= 4 key tiles per split
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
  a.ws_bytes = splits > 1 ? blocks * splits * pf * 4 : 0;
  return a;
}

}  // namespace fvx

using namespace fvx;

struct DecodePlan {
  int n_rb, splits, n_items;
  int64_t kps, ws_bytes;
};

static bool use_decode(const fvx_attn_desc& d) {
  return d.v_d_stride > 0 && d.head_dim == 256 && d.sq * d.heads <= 512;
}

static DecodePlan plan_decode(const fvx_attn_desc& d) {
  DecodePlan a;
  a.n_rb = (int)((d.sq * d.heads + 15) / 16);
  int splits = d.kv_splits;
  if (splits <= 0) splits = (int)((d.sk + 95) / 96);  // ~3 key tiles per wave
  if (splits < 1) splits = 1;
  int64_t kps = (d.sk + splits - 1) / splits;
  kps = (kps + kKeyTile - 1) / kKeyTile * kKeyTile;
  a.splits = (int)((d.sk + kps - 1) / kps);
  a.kps = kps;
  a.n_items = (int)(a.n_rb * a.splits * d.n_problems);
  a.ws_bytes = a.splits > 1 ? (int64_t)a.n_items * kDecPF * 4 : 0;
  return a;
}

extern "C" int64_t fvx_attention_workspace_bytes(const fvx_attn_desc* d) {
  if (!d || d->sq <= 0 || d->sk <= 0 || d->heads <= 0 || d->n_problems <= 0)
    return 0;
  if (use_decode(*d)) return plan_decode(*d).ws_bytes;
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
  FVX_REQUIRE(d.v_d_stride == 0 ||
                  (d.head_dim == 256 && d.v_d_stride % 8 == 0 &&
                   d.sk <= d.v_d_stride),
              FVX_ERR_SHAPE,
              "attention: a transposed V needs head_dim 256, v_d_stride %% 8 "
              "== 0 and sk <= v_d_stride");
  if (d.sq == 0 || d.n_problems == 0) return FVX_OK;
  FVX_REQUIRE(d.sk > 0, FVX_ERR_SHAPE, "attention: sk must be > 0");
  hipStream_t s = (hipStream_t)stream;
  if (use_decode(d)) {
    DecodePlan a = plan_decode(d);
    if (a.splits > 1 && (!d.workspace || d.workspace_bytes < a.ws_bytes))
      return set_error(FVX_ERR_WORKSPACE,
                       "attention: %d key splits need %lld workspace bytes, "
                       "got %lld", a.splits, (long long)a.ws_bytes,
                       (long long)d.workspace_bytes);
    FVX_REQUIRE(aligned16(d.workspace), FVX_ERR_ALIGN,
                "attention: workspace must be 16B aligned");
    hipLaunchKernelGGL(attn_decode_kernel, dim3((unsigned)((a.n_items + 3) / 4)),
                       dim3(256), 0, s, d, a.n_rb, a.splits, a.kps, a.n_items);
    int st = launch_status("attention(decode)");
    if (st || a.splits == 1) return st;
    const int64_t threads = (int64_t)d.n_problems * a.n_rb * 16 * 64;
    hipLaunchKernelGGL(attn_decode_merge_kernel,
                       dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       d, a.n_rb, a.splits);
    return launch_status("attention(decode merge)");
  }
  AttnPlan a = plan_attn(d);
  if (a.splits > 1 && (!d.workspace || d.workspace_bytes < a.ws_bytes)) {
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
  if (a.hdp == 256)
    hipLaunchKernelGGL((attn_kernel<256, 256>), grid, dim3(256), 0, s, d,
                       a.n_row_blocks, a.splits, a.kps);
  else
    hipLaunchKernelGGL((attn_kernel<96, 80>), grid, dim3(256), 0, s, d,
                       a.n_row_blocks, a.splits, a.kps);
  int st = launch_status("attention");
  if (st || a.splits == 1) return st;
  dim3 mgrid((unsigned)a.n_row_blocks, 1u, (unsigned)d.n_problems);
  if (a.hdp == 256)
    hipLaunchKernelGGL((attn_merge_kernel<256, 256>), mgrid, dim3(256), 0, s,
                       d, a.n_row_blocks, a.splits);
  else
    hipLaunchKernelGGL((attn_merge_kernel<96, 80>), mgrid, dim3(256), 0, s, d,
                       a.n_row_blocks, a.splits);
  return launch_status("attention");
}
