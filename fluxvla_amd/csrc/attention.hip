// Fused multi-query attention (gfx950): softmax(Q K^T * scale + mask) V.
//
// One workgroup = 4 waves x 16 query rows.  For MQA every query head of a
// token shares the single K/V head, so query rows are (token, head) pairs
// and one K/V tile in LDS feeds all of them (8 heads x 8 tokens per block for
// Gemma).  Keys stream in tiles of 64 (two barriers per tile, so the
// tile is as wide as the registers allow):
//
//   S^T(16 keys x 16 rows) = K_tile(16 x d) . Q^T(d x 16)     (MFMA, Q in VGPRs)
//
// computing S transposed leaves each lane with 16 scores of ONE query row, so
// the online-softmax statistics need only in-lane math plus two cross-lane
// shuffles, and the probabilities are already in the A-operand layout of
//
//   O(16 rows x 16 d) += P(16 x 32 keys) . V(32 keys x 16 d)   (per 32 keys)
//
// for which V is stored transposed in LDS (keys contiguous) as it is copied
// in.  K/V rows past the key range are zero-filled; masked scores are -inf
// and never produce NaN (a row that has seen no visible key yet keeps a zero
// reference).  With kv_splits > 1 each split writes (O, m, l) partials to a
// workspace and a merge kernel, the next kernel on the stream, combines them
// in split order (deterministic).  This kernel serves SigLIP (head dim 72)
// and any head dim other than 256 or a non-transposed V.  Head dim 256 with
// the transposed value cache runs attn_decode_kernel (the action expert: 408
// query rows against the 867-key prefix+suffix cache, one 64-key tile per
// workgroup) or attn_decode_t_kernel (the prefix prefill, key ranges of >= 4
// tiles), both further below.
#include <math.h>

#include "capi_util.h"
#include "common.h"

namespace fvx {

constexpr int kKeyTile = 64;
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
  if (valid <= 0) return zero8();
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
  __shared__ int32_t sG[kKeyTile];
  warm_kernargs<sizeof(fvx_attn_desc) + 32>();

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;
  const int rb = blockIdx.x, split = blockIdx.y, z = blockIdx.z;
  const int HD = (int)p.head_dim;
  const int64_t heads = p.heads;
  const int64_t R = p.sq * heads;

  const int64_t zb = (uint32_t)z / (uint32_t)p.zdiv, zh = (uint32_t)z % (uint32_t)p.zdiv;
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
  const int64_t qtok = qval ? (uint32_t)qrow / (uint32_t)heads : 0;
  const int64_t qhead = qval ? (uint32_t)qrow % (uint32_t)heads : 0;
  const int32_t qg = (qgrp && qval) ? qgrp[qtok] : 0;
  // Branch-free loads through buffer views (an out-of-range offset reads
  // zero), so that every load of a batch is in flight at once.
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(
      Q, (uint32_t)(((p.sq - 1) * p.q_tok_stride + (heads - 1) * p.q_head_stride + HD) * 2));
  bf16x8 qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int d = 32 * s + 8 * g;
    qf[s] = bload8(rq, (qval && d < HD) ? (uint32_t)((qtok * p.q_tok_stride +
                                                      qhead * p.q_head_stride + d) * 2)
                                        : kOOB);
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
  // Keys >= kend read as zero (K, row-major V: outside the buffer view; V^T:
  // masked when the tile is written to LDS).
  constexpr int CH = (kKeyTile * (HDP / 8) + 255) / 256;
  const __amdgpu_buffer_rsrc_t rkc = make_rsrc(K, (uint32_t)(kend * p.k_tok_stride * 2));
  const __amdgpu_buffer_rsrc_t rvc = make_rsrc(
      V, (uint32_t)(p.v_d_stride > 0 ? HD * p.v_d_stride * 2 : kend * p.v_tok_stride * 2));
  const __amdgpu_buffer_rsrc_t rgc =
      make_rsrc(kgrp ? (const void*)kgrp : (const void*)K, kgrp ? (uint32_t)(kend * 4) : 0u);
  bf16x8 rk[CH], rv[CH];
  int32_t rgp = 0;
  // Each thread's chunks, fixed over the tiles (computed once, 32-bit: the
  // views are below 2 GiB): global byte offsets relative to the tile's first
  // key and LDS element offsets.  K chunks are key-major (key i / kchunks,
  // dims 8 (i % kchunks)); V^T chunks 8 consecutive keys of dim i / (tile
  // / 8); row-major V chunks key i % tile, dims 8 (i / tile).
  const bool vt = p.v_d_stride > 0;
  const uint32_t kts2 = (uint32_t)p.k_tok_stride * 2u;
  const uint32_t vstep2 = vt ? 2u : (uint32_t)p.v_tok_stride * 2u;  // per key
  uint32_t koff[CH], voff[CH];
  int kl[CH], vl[CH], vkey[CH];
  bool cin[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int i = tid + 256 * c;
    cin[c] = i < tile_chunks;
    const int kr = i / kchunks, kc = i - kr * kchunks;
    koff[c] = (uint32_t)kr * kts2 + (uint32_t)kc * 16u;
    kl[c] = kr * LDK + kc * 8;
    if (vt) {
      constexpr int KG = kKeyTile / 8;  // 8-key chunks per dim
      vkey[c] = (i % KG) * 8;
      voff[c] = ((uint32_t)(i / KG) * (uint32_t)p.v_d_stride + (uint32_t)vkey[c]) * 2u;
      vl[c] = (i / KG) * LDV + vkey[c];
    } else {
      vkey[c] = i % kKeyTile;
      voff[c] = (uint32_t)vkey[c] * vstep2 + (uint32_t)(i / kKeyTile) * 16u;
      vl[c] = (i / kKeyTile) * 8 * LDV + vkey[c];
    }
  }
  auto prefetch = [&](int64_t t0) {
    const uint32_t kb = (uint32_t)t0 * kts2, vb = (uint32_t)t0 * vstep2;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      rk[c] = bload8(rkc, cin[c] ? kb + koff[c] : kOOB);
      rv[c] = bload8(rvc, cin[c] ? vb + voff[c] : kOOB);
    }
    if (kgrp && tid < kKeyTile)
      rgp = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rgc, (uint32_t)((t0 + tid) * 4), 0, 0);
  };
  if (kbeg < kend) prefetch(kbeg);

  for (int64_t t0 = kbeg; t0 < kend; t0 += kKeyTile) {
    __syncthreads();  // previous tile fully consumed
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if (cin[c]) {
        st8(&sK[kl[c]], rk[c]);
        if (vt) {
          st8(&sVt[vl[c]], mask_keys(rv[c], (int)(kend - t0) - vkey[c]));
        } else {
          const bf16_t* ve = (const bf16_t*)&rv[c];
#pragma unroll
          for (int e = 0; e < 8; ++e) sVt[vl[c] + e * LDV] = ve[e];
        }
      }
    }
    if (kgrp && tid < kKeyTile) sG[tid] = rgp;
    __syncthreads();
    if (t0 + kKeyTile < kend) prefetch(t0 + kKeyTile);

    // Scores: lane holds keys t0 + kf*16 + 4g + e for its query row.
    constexpr int KB = kKeyTile / 16, PC = kKeyTile / 32;
    float s[KB][4];
#pragma unroll
    for (int kf = 0; kf < KB; ++kf) {
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ss = 0; ss < NS; ++ss)
        acc = mfma16x16x32(ld8(&sK[(kf * 16 + fr) * LDK + ss * 32 + 8 * g]),
                           qf[ss], acc);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int64_t j = t0 + kf * 16 + 4 * g + e;
        bool vis = j < kend;
        if (vis && kgrp) vis = sG[kf * 16 + 4 * g + e] <= qg;
        s[kf][e] = vis ? acc[e] * sc : -INFINITY;
      }
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int kf = 0; kf < KB; ++kf)
#pragma unroll
      for (int e = 0; e < 4; ++e) tmax = fmaxf(tmax, s[kf][e]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m_run, tmax);
    const float m_ref = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_ref);
    float psum = 0.f;
    float pr[KB][4];
#pragma unroll
    for (int kf = 0; kf < KB; ++kf)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pr[kf][e] = __builtin_amdgcn_exp2f(s[kf][e] - m_ref);
        psum += pr[kf][e];
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;

    // P as A operand of key block c (32 keys): keys 32c + {4g+e} (e<4) and
    // 32c + {16+4g+e} (e>=4).
    bf16x8 pa[PC];
#pragma unroll
    for (int c = 0; c < PC; ++c) {
      float pf[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pf[e] = pr[2 * c][e];
        pf[4 + e] = pr[2 * c + 1][e];
      }
      pa[c] = pack8(pf);
    }
    // Rescale O rows 4g+j by alpha of that row (held by lane 4g+j).
    float al[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) al[j] = __shfl(alpha, 4 * g + j, 64);
#pragma unroll
    for (int df = 0; df < ND; ++df) {
#pragma unroll
      for (int j = 0; j < 4; ++j) o[df][j] *= al[j];
#pragma unroll
      for (int c = 0; c < PC; ++c) {
        const bf16_t* vt = &sVt[(df * 16 + fr) * LDV + 32 * c];
        bf16x8 vb;
        const uint2 lo = *(const uint2*)(vt + 4 * g);
        const uint2 hi = *(const uint2*)(vt + 16 + 4 * g);
        vb.w[0] = lo.x;
        vb.w[1] = lo.y;
        vb.w[2] = hi.x;
        vb.w[3] = hi.y;
        o[df] = mfma16x16x32(pa[c], vb, o[df]);
      }
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
    const int64_t tok = (uint32_t)r / (uint32_t)heads, h = (uint32_t)r % (uint32_t)heads;
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
  const int64_t zb = (uint32_t)z / (uint32_t)p.zdiv, zh = (uint32_t)z % (uint32_t)p.zdiv;
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
    const float w = __builtin_amdgcn_exp2f(ms - mref);
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
// Head-dim-256 attention with a transposed value cache: the action expert's
// 408 query rows (51 tokens x 8 heads) against the ~870-key prefix + suffix
// cache, and the prefix prefill (6528 rows x 816 keys).
//
// A workgroup of 4 waves owns 64 query rows and one key range, walked in
// 64-key tiles.  The waves split each tile two ways:
//   S^T = K Q^T   wave w takes keys 16 w .. 16 w + 15 of the tile for all 64
//                 rows (the 64 rows' Q fragments stay in VGPRs for the whole
//                 range);
//   O += P V      wave w takes dims 64 w .. 64 w + 63 for all 64 rows.
// Every byte moves from memory into LDS by the buffer unit (buffer_load ...
// lds), 1 KiB of contiguous rows per wave instruction: a wave load that
// gathers 16 rows x 64 B (the shape of an MFMA fragment) runs at a third of
// that rate per CU.  Each wave loads exactly the K and V^T slices it reads
// itself, so their arrival needs only the wave's own vmcnt, no barrier; a
// two-stage ring keeps the next tile in flight.  LDS rows carry an XOR
// swizzle of their 16-byte chunks (the load picks which global chunk lands
// in each slot), so the fragment reads are conflict-free.
//
// Only the probabilities cross waves: each wave writes its 64 x 16 block of
// P (bf16) and its per-row maxima to LDS and reads the whole 64 x 64 tile
// back as the A operand of P V.  Every wave derives the same running
// maximum from the exchanged maxima, so the per-wave row sums add up to the
// softmax denominator at the end.  Two barriers per tile; the exchange
// buffers alternate between tiles.  Online-softmax statistics are fp32.
//
// With several key ranges each workgroup writes its partial (O, m, l) and
// attn_decode_merge_kernel, the next kernel on the stream, combines them in
// split order (deterministic).  (Merging inside this kernel -- partials
// written through to the device-coherent level, a per-row-group arrival
// counter -- measured slower: the write-through stores of ~6 MB of partials
// alone took ~9 us.)
// ---------------------------------------------------------------------------
constexpr int kDecKT = 64;                      // keys per tile
constexpr int kDecPP = kDecKT + 8;              // LDS pitch (elements), P rows
constexpr int kDecOP = 256 + 4;                 // LDS pitch (floats), O rows
// partial per workgroup: O rows [64][256] bf16 (un-normalized), then the 64
// row references and the 64 row sums (fp32); sizes in floats
constexpr int64_t kDecPO = 64 * 256 / 2;
constexpr int64_t kDecPF = kDecPO + 2 * 64;
// An attention workspace opens with the 64-row groups' arrival counters of
// the in-launch merge (one 256-byte line each); the last line holds the
// merge status word (the number of merging workgroups that stopped waiting
// for their key ranges; fvx_attention_check reads and clears it); the split
// partials follow.
constexpr int64_t kAttnCounterBytes = 64 * 1024;
constexpr int kAttnMaxGroups = (int)(kAttnCounterBytes / 256) - 1;
constexpr int64_t kAttnStatusWord = (kAttnCounterBytes - 256) / 4;
constexpr int kDecMergeSpin = 1 << 16;  // polls before a merge stops waiting

// The value of a 32-bit word as the L2 holds it: a returning atomic add of 0
// (written out here: the compiler turns an idempotent atomic into a load,
// which may be served by the CU's L1 and never see another CU's update).
__device__ __forceinline__ uint32_t l2_atomic_read(uint32_t* p) {
  uint32_t v;
  asm volatile("global_atomic_add %0, %1, %2, off sc0\n\ts_waitcnt vmcnt(0)"
               : "=v"(v)
               : "v"(p), "v"(0u)
               : "memory");
  return v;
}
// LDS map (bytes): two stages of [K tile 64 x 512 B | V^T tile 256 x 128 B]
// (stage 1 first holds the Q rows), then P [2][64][kDecPP] bf16, the row
// maxima [2][64][4] f32, the key groups [2][4 waves][64] and the query
// groups [64]; at the end the O rows [64][kDecOP] f32 over the stages.
constexpr int kDecStage = 64 * 512 + 256 * 128;
constexpr int kDecOffP = 2 * kDecStage;
constexpr int kDecOffM = kDecOffP + 2 * 64 * kDecPP * 2;
constexpr int kDecOffG = kDecOffM + 2 * 64 * 4 * 4;
constexpr int kDecOffQG = kDecOffG + 2 * 4 * 64 * 4;
constexpr int kDecLDS = kDecOffQG + 64 * 4;
static_assert(64 * kDecOP * 4 <= 2 * kDecStage, "O rows fit the stages");
constexpr int kDecLoads = 17;  // DMA instructions per wave per tile

// Division by the small divisors of the decode kernels (heads, the problem
// divisor zdiv, the row-group and split counts): x / d = umulhi(x, m) with
// m = ceil(2^32 / d) (0 for d = 1), exact for x < 2^32 / d -- the host
// checks every dividend's bound (dec_div_exact).  One multiply in
// place of a ~20-instruction integer division: the decode prologues run
// dozens of them before their first load is issued.
struct FastDiv {
  uint32_t m;
  __device__ __forceinline__ int div(int x) const {
    return m ? (int)__umulhi((uint32_t)x, m) : x;
  }
};
struct DecDiv {
  FastDiv heads, zdiv, rg, splits, rgw;  // rgw: the 128-row groups (NW = 4)
};

// Query row r of a problem is (token r / heads, head r % heads).
__device__ __forceinline__ int row_tok(int r, const DecDiv& dv) { return dv.heads.div(r); }

// One output chunk: `n` (4 or 8) dims d0.. of query row r of problem z,
// row-major and, if requested, fragment-major for the o-projection.
template <int NE>
__device__ __forceinline__ void dec_store(const fvx_attn_desc& p, int z, int r,
                                          int d0, const DecDiv& dv, const float* v) {
  const int heads = (int)p.heads;
  const int tok = row_tok(r, dv), h = r - tok * heads;
  const int64_t zb = dv.zdiv.div(z), zh = z - zb * p.zdiv;
  // o may be NULL on this path when o_frag is given (the row-major copy
  // has no reader then)
  bf16_t* dst = p.o ? (bf16_t*)p.o + zb * p.o_zs1 + zh * p.o_zs2 + (int64_t)tok * p.o_tok_stride +
                          (int64_t)h * p.o_head_stride + d0
                    : nullptr;
  bf16_t* fdst = p.o_frag ? (bf16_t*)p.o_frag + frag_offset((int64_t)z * p.sq + tok,
                                                            h * 256 + d0)
                          : nullptr;
  if (NE == 8) {
    const bf16x8 b = pack8(v);
    if (dst) st8(dst, b);
    if (fdst) st8(fdst, b);
  } else {
    const uint2 b = {f2bf2(v[0], v[1]), f2bf2(v[2], v[3])};
    if (dst) *(uint2*)dst = b;
    if (fdst) *(uint2*)fdst = b;
  }
}

// Prefetch role of the workgroups past the attention items (prefetch
// index pw of npw, on XCD blockIdx % 8).  Each range moves in whole 1 KiB
// wave blocks by LDS DMA into one 1 KiB slot per wave, overwritten and
// never read: the point is the cache fill.  A range without tiles is split
// evenly over all prefetch workgroups; a tiled range's tile j goes to the
// prefetch workgroups on XCD j % 8 (split evenly among them), so that it
// lands in the L2 of the XCD whose workgroup will read it.  Every load
// completes before the wave ends.
__device__ void dec_prefetch(const fvx_attn_desc& p, int pw, int npw, int first,
                             unsigned char* smem) {
  prefetch_ranges<4>(p.prefetch, p.prefetch_bytes, p.prefetch_tile_bytes, pw, npw,
                     first, lds_addr(smem));
}

// Row r (problem z), dims d0 .. d0 + 7 of the merged output from the split
// partials of its 64-row group: the loads of up to NS splits in flight, then
// per pass of 16 the pass maximum first and the weighted sums after it, in
// split order (the weights exp2(m_s - max) are independent of each other, so
// no rescaling chain runs through the splits).  AUX: the loads' cache policy
// (0 for partials of an earlier launch; 1, missing in the vector L1, for
// partials other CUs of the XCD wrote in this launch).
// NS: splits per pass (4, 8 or 16; the smallest that holds `splits`, so
// no load is spent on splits that do not exist).
template <int AUX, int NS>
__device__ __forceinline__ void dec_merge8_ns(const fvx_attn_desc& p, int n_rg, int splits,
                                              const DecDiv& dv, int z, int r, int d0) {
  const int rg = r >> 6, i = r & 63;
  const float* base = (const float*)p.workspace + (((int64_t)z * n_rg + rg) * splits) * kDecPF;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(base, (uint32_t)(splits * kDecPF * 4));
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, M = -INFINITY, L = 0.f;
  for (int s0 = 0; s0 < splits; s0 += NS) {
    bf16x8 a[NS];
    float mv[NS], lv[NS];
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      // splits past the end read as zero (out of the buffer view)
      const uint32_t off = (uint32_t)((s0 + u) * kDecPF * 4);
      a[u] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                            rw, off + (uint32_t)(i * 256 + d0) * 2, 0, AUX));
      mv[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          rw, off + (uint32_t)(kDecPO + i) * 4, 0, AUX));
      lv[u] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
          rw, off + (uint32_t)(kDecPO + 64 + i) * 4, 0, AUX));
    }
    float mn = M;
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      mv[u] = s0 + u < splits ? mv[u] : -INFINITY;
      mn = fmaxf(mn, mv[u]);
    }
    // a row no split has seen keys of keeps a zero reference
    const float mr = (mn == -INFINITY) ? 0.f : mn;
    const float wa = __builtin_amdgcn_exp2f(M - mr);  // earlier passes (0 on the first)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] *= wa;
    L *= wa;
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const float wb = __builtin_amdgcn_exp2f(mv[u] - mr);
      float av[8];
      unpack8(a[u], av);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(av[e], wb, acc[e]);
      L = fmaf(lv[u], wb, L);
    }
    M = mn;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] *= inv;
  dec_store<8>(p, z, r, d0, dv, acc);
}

// dec_merge8_ns for the in-launch merge (splits <= 16, partials of this
// launch in this XCD's L2): the O rows' loads as above, the splits' row
// references and sums from sML[split][8 rows] (staged in LDS by the merging
// workgroup, one load per thread instead of two per split and thread).
__device__ __forceinline__ void dec_merge8_staged(const fvx_attn_desc& p, int n_rg, int splits,
                                                  const DecDiv& dv, int z, int r, int d0,
                                                  const float2* sML) {
  constexpr int NS = 16;
  const int rg = r >> 6, i = r & 63, rl = r & 7;
  const float* base = (const float*)p.workspace + (((int64_t)z * n_rg + rg) * splits) * kDecPF;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(base, (uint32_t)(splits * kDecPF * 4));
  bf16x8 a[NS];
#pragma unroll
  for (int u = 0; u < NS; ++u)
    a[u] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(
                                          rw, (uint32_t)(u * kDecPF * 4 + (i * 256 + d0) * 2), 0,
                                          1));
  float mv[NS], lv[NS], mn = -INFINITY;
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const float2 ml = sML[u * 8 + rl];
    mv[u] = u < splits ? ml.x : -INFINITY;
    lv[u] = u < splits ? ml.y : 0.f;
    mn = fmaxf(mn, mv[u]);
  }
  const float mr = (mn == -INFINITY) ? 0.f : mn;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, L = 0.f;
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    const float wb = __builtin_amdgcn_exp2f(mv[u] - mr);
    float av[8];
    unpack8(a[u], av);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = fmaf(av[e], wb, acc[e]);
    L = fmaf(lv[u], wb, L);
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] *= inv;
  dec_store<8>(p, z, r, d0, dv, acc);
}

template <int AUX>
__device__ __forceinline__ void dec_merge8(const fvx_attn_desc& p, int n_rg, int splits,
                                           const DecDiv& dv, int z, int r, int d0) {
  if (splits <= 4)
    dec_merge8_ns<AUX, 4>(p, n_rg, splits, dv, z, r, d0);
  else if (splits <= 8)
    dec_merge8_ns<AUX, 8>(p, n_rg, splits, dv, z, r, d0);
  else
    dec_merge8_ns<AUX, 16>(p, n_rg, splits, dv, z, r, d0);
}

// One merging workgroup of the in-launch merge: 8 rows (chunk) of 64-row
// group G = z n_rg + rg, 256 threads of (row, 8 dims), on the group's XCD.
// Thread 0 polls the group's arrival counter (an L2 atomic) until it reaches
// `splits` -- every range's workgroup has a lower block index on the same
// XCD, so it was dispatched first, and it waits on nothing; the wait is
// bounded regardless (`polls`; 0 only from the descriptor's test hook) --
// then the partials are read from that XCD's L2.  A workgroup whose polls
// run out counts itself in the status word and merges what has arrived:
// that call's output is wrong, and a range arriving after the counters'
// reset leaves a count behind, so fvx_attention_check reports the status
// and clears every counter before the next call relies on them.  The
// group's last merging workgroup resets both of its counters.
__device__ void dec_merge_wg(const fvx_attn_desc& p, int n_rg, int splits, const DecDiv& dv,
                             uint32_t* counters, int grp, int chunk, int polls,
                             unsigned char* smem) {
  const int tid = threadIdx.x;
  const int R = (int)(p.sq * p.heads);
  const int z = dv.rg.div(grp), rg = grp - z * n_rg;
  const int r = rg * 64 + 8 * chunk + (tid >> 5), d0 = (tid & 31) * 8;
  uint32_t* ctr = counters + (int64_t)grp * 64;
  if (tid == 0) {
    bool arrived = false;
#pragma unroll 1
    for (int it = 0; it < polls; ++it) {
      if (l2_atomic_read(ctr) >= (uint32_t)splits) {
        arrived = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    if (!arrived)
      __hip_atomic_fetch_add(counters + kAttnStatusWord, 1u, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  // the splits' row references and sums of this workgroup's 8 rows: thread
  // t < 16 splits loads value t & 1 (reference, sum) of row (t >> 1) & 7 of
  // split t >> 4 into sML
  float2* sML = (float2*)smem;
  if (tid < 16 * splits) {
    const int s = tid >> 4, rl = (tid >> 1) & 7, which = tid & 1;
    const float* part = (const float*)p.workspace +
                        (((int64_t)z * n_rg + rg) * splits + s) * kDecPF;
    const float v = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        make_rsrc(part, (uint32_t)(kDecPF * 4)),
        (uint32_t)(kDecPO + 64 * which + 8 * chunk + rl) * 4, 0, 1));
    ((float*)sML)[2 * (s * 8 + rl) + which] = v;
  }
  __syncthreads();
  dec_merge8_staged(p, n_rg, splits, dv, z, r, d0, sML);
  if (tid == 0) {
    const int rows = R - rg * 64 < 64 ? R - rg * 64 : 64;
    const uint32_t old =
        __hip_atomic_fetch_add(ctr + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (old == (uint32_t)(rows / 8 - 1)) {
      __hip_atomic_exchange(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_exchange(ctr + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  }
}

// counters != NULL: the key ranges of each 64-row group G = z n_rg + rg
// merge inside the launch, all on XCD G % 8 (block b runs on XCD b & 7).
// Blocks [0, n_items) compute: slot b >> 3 of XCD b & 7 is range slot %
// splits of the XCD's group slot / splits.  Blocks [n_items, merge_first)
// merge: slot j of XCD x takes rows 8 (j % 8) .. + 7 of the XCD's group
// j / 8.  The rest prefetch.  A range's partial goes to the XCD's L2 and is
// then counted in counters[64 G] (a 256-byte line per group; [64 G + 1]
// counts the group's merging workgroups).  Slots past the groups (or past
// R) do nothing.  n_items and merge_first are multiples of 8.
__global__ __launch_bounds__(256) void attn_decode_kernel(fvx_attn_desc p,
                                                          int n_rg, int splits,
                                                          int kps, DecDiv dv,
                                                          int n_items,
                                                          uint32_t* counters,
                                                          int merge_first) {
  constexpr int HD = 256, KT = kDecKT;
  __shared__ __align__(16) unsigned char smem[kDecLDS];
  __shared__ float sL[4][64], sM[64];
  warm_kernargs<sizeof(fvx_attn_desc) + 32>();
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int n_groups = (int)p.n_problems * n_rg;
  if (counters && (int)blockIdx.x >= n_items && (int)blockIdx.x < merge_first) {
    const int j = slot - n_items / 8, grp = xcd + 8 * (j / 8);
    if (grp < n_groups && (grp - dv.rg.div(grp) * n_rg) * 64 + 8 * (j % 8) < (int)(p.sq * p.heads))
      dec_merge_wg(p, n_rg, splits, dv, counters, grp, j % 8,
                   p.merge_no_wait ? 0 : kDecMergeSpin, smem);
    return;
  }
  const int pf0 = counters ? merge_first : n_items;
  if ((int)blockIdx.x >= pf0) {
    dec_prefetch(p, (int)blockIdx.x - pf0, (int)gridDim.x - pf0, pf0, smem);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, g = lane >> 4;
  int item;
  if (counters) {
    const int sq = dv.splits.div(slot);
    const int grp = xcd + 8 * sq;
    if (grp >= n_groups) return;  // an empty slot
    const int gz = dv.rg.div(grp);
    item = (gz * splits + (slot - sq * splits)) * n_rg + (grp - gz * n_rg);
  } else {
    // XCD-aware order: consecutive items (the row groups of one key range)
    // land on one XCD and share its L2 copy of the range's K / V tiles.
    const int nb = n_items, q8 = nb >> 3, r8 = nb & 7;
    item = xcd * q8 + (xcd < r8 ? xcd : r8) + slot;
  }
  const int ir = dv.rg.div(item), rg = item - ir * n_rg;
  const int z = dv.splits.div(ir), split = ir - z * splits;
  const int heads = (int)p.heads, R = (int)p.sq * heads;
  const int64_t zb = dv.zdiv.div(z), zh = z - zb * p.zdiv;
  const bf16_t* Q = (const bf16_t*)p.q + zb * p.q_zs1 + zh * p.q_zs2;
  const bf16_t* K = (const bf16_t*)p.k + zb * p.k_zs1 + zh * p.k_zs2;
  const bf16_t* Vt = (const bf16_t*)p.v + zb * p.v_zs1 + zh * p.v_zs2;
  const int32_t* kgrp = p.kgrp ? p.kgrp + zb * p.kgrp_zs1 : nullptr;
  const int32_t* qgrp = p.qgrp ? p.qgrp + zb * p.qgrp_zs1 : nullptr;
  const int kbeg = split * kps;
  const int kend = kbeg + kps < (int)p.sk ? kbeg + kps : (int)p.sk;
  const int qts = (int)p.q_tok_stride, qhs = (int)p.q_head_stride;
  const int kts = (int)p.k_tok_stride, vds = (int)p.v_d_stride;

  // Buffer views: loads past them write zeros (K: keys >= kend; V^T: past
  // its last row; Q: rows >= R get an out-of-range offset).  V^T keys past
  // kend inside the view are zeroed after they are read.
  const i32x4_t rq =
      make_rsrc4(Q, (uint32_t)(((int)p.sq - 1) * qts + (heads - 1) * qhs + HD) * 2);
  const i32x4_t rkc = make_rsrc4(K, (uint32_t)kend * kts * 2);
  const i32x4_t rvc = make_rsrc4(Vt, (uint32_t)HD * vds * 2);
  const i32x4_t rgc = make_rsrc4(kgrp ? (const void*)kgrp : (const void*)Q,
                                 kgrp ? (uint32_t)kend * 4 : 0u);
  const i32x4_t rqg = make_rsrc4(qgrp ? (const void*)qgrp : (const void*)Q,
                                 qgrp ? (uint32_t)p.sq * 4 : 0u);
  const uint32_t lbase = lds_addr(smem);
  bf16_t* sP = (bf16_t*)(smem + kDecOffP);
  float* sMx = (float*)(smem + kDecOffM);
  const int32_t* sG = (const int32_t*)(smem + kDecOffG);
  const int32_t* sQG = (const int32_t*)(smem + kDecOffQG);

  // Tile t0 into stage st, this wave's slices: K keys t0 + 16 w + 2 i +
  // (lane >> 5) (LDS slot lane & 31 of the key's 512-byte row holds global
  // chunk slot ^ (key & 15)); V^T dims 64 w + 8 i + (lane >> 3) (slot lane
  // & 7 of the dim's 128-byte row holds key chunk slot ^ ((dim >> 1) & 7));
  // the groups of keys t0 + 16 w + lane, lane < 16.
  auto issue = [&](int t0, int st) {
    const uint32_t sb = lbase + st * kDecStage;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kl = 16 * w + 2 * i + (lane >> 5);
      const int ch = (lane & 31) ^ (kl & 15);
      load_lds16(rkc, sb + (16 * w + 2 * i) * 512,
                 (uint32_t)((t0 + kl) * kts + 8 * ch) * 2);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int d = 64 * w + 8 * i + (lane >> 3);
      const int ch = (lane & 7) ^ ((d >> 1) & 7);
      load_lds16(rvc, sb + 64 * 512 + (64 * w + 8 * i) * 128,
                 (uint32_t)(d * vds + t0 + 8 * ch) * 2);
    }
    load_lds4(rgc, lbase + kDecOffG + (st * 4 + w) * 256,
              lane < 16 ? (uint32_t)(t0 + 16 * w + lane) * 4 : kOOB);
  };

  // Q rows 64 rg + 16 w + 2 i + (lane >> 5) into stage 1 (same swizzle as
  // K), their tokens' query groups, then tile 0.
  {
    const uint32_t qb = lbase + kDecStage;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int rl = 16 * w + 2 * i + (lane >> 5);
      const int r = rg * 64 + rl;
      const int tok = row_tok(r, dv);
      const int ch = (lane & 31) ^ (rl & 15);
      load_lds16(rq, qb + (16 * w + 2 * i) * 512,
                 r < R ? (uint32_t)(tok * qts + (r - tok * heads) * qhs + 8 * ch) * 2
                       : kOOB);
    }
    if (w == 0) {
      const int r = rg * 64 + lane;
      load_lds4(rqg, lbase + kDecOffQG, r < R ? (uint32_t)row_tok(r, dv) * 4 : kOOB);
    }
  }
  issue(kbeg, 0);
  wait_vmcnt<kDecLoads>();  // this wave's Q rows (and query groups) landed
  __syncthreads();

  // Q fragments (B operand of S^T): lane (fr, g) holds dims 32 ds + 8 g ..
  // + 7 of row 16 rb + fr.
  bf16x8 qf[4][8];
  int32_t qg[4];
  {
    const bf16_t* sQ = (const bf16_t*)(smem + kDecStage);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
      for (int ds = 0; ds < 8; ++ds)
        qf[rb][ds] = ld8(&sQ[(16 * rb + fr) * 256 + 8 * ((4 * ds + g) ^ fr)]);
      qg[rb] = qgrp ? sQG[16 * rb + fr] : 0;
    }
  }
  __syncthreads();  // stage 1 is free for tile 1
  if (kbeg + KT < kend) issue(kbeg + KT, 1);

  const float sc = p.scale * kLog2e;
  float m_run[4], l_w[4];
  f32x4_t o[4][4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    m_run[rb] = -INFINITY;
    l_w[rb] = 0.f;
#pragma unroll
    for (int b = 0; b < 4; ++b) o[rb][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  for (int t0 = kbeg, cs = 0; t0 < kend; t0 += KT, cs ^= 1) {
    // this wave's slices of tile t0 have landed (the next tile's may not)
    if (t0 + KT < kend)
      wait_vmcnt<kDecLoads>();
    else
      wait_vmcnt<0>();
    const unsigned char* stg = smem + cs * kDecStage;
    const bf16_t* sK = (const bf16_t*)stg;
    const bf16_t* sV = (const bf16_t*)(stg + 64 * 512);

    // S^T: lane (fr, g) ends with keys t0 + 16 w + 4 g + j of row 16 rb + fr
    bf16x8 kf[8];
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
      kf[ds] = ld8(&sK[(16 * w + fr) * 256 + 8 * ((4 * ds + g) ^ fr)]);
    const int4 kgv = *(const int4*)&sG[(cs * 4 + w) * 64 + 4 * g];
    const int32_t kgc[4] = {kgv.x, kgv.y, kgv.z, kgv.w};
    f32x4_t s[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) s[rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ds = 0; ds < 8; ++ds)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) s[rb] = mfma16x16x32(kf[ds], qf[rb][ds], s[rb]);

    float sv[4][4], mx[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      mx[rb] = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bool vis = t0 + 16 * w + 4 * g + j < kend;
        if (kgrp) vis = vis && kgc[j] <= qg[rb];
        sv[rb][j] = vis ? s[rb][j] * sc : -INFINITY;
        mx[rb] = fmaxf(mx[rb], sv[rb][j]);
      }
      mx[rb] = fmaxf(mx[rb], __shfl_xor(mx[rb], 16, 64));
      mx[rb] = fmaxf(mx[rb], __shfl_xor(mx[rb], 32, 64));
    }
    float* mxb = sMx + cs * 256;
    if (g == 0)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) mxb[(16 * rb + fr) * 4 + w] = mx[rb];
    __syncthreads();

    bf16_t* pb = sP + cs * 64 * kDecPP;
    float alpha[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const f32x4_t t = *(const f32x4_t*)&mxb[(16 * rb + fr) * 4];
      const float m_new = fmaxf(m_run[rb], fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3])));
      const float m_ref = (m_new == -INFINITY) ? 0.f : m_new;
      // the hardware exp2 (v_exp_f32; results below 2^-126 may flush to
      // zero, far under a probability's bf16 resolution)
      alpha[rb] = __builtin_amdgcn_exp2f(m_run[rb] - m_ref);
      m_run[rb] = m_new;
      float pv[4], ps = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pv[j] = __builtin_amdgcn_exp2f(sv[rb][j] - m_ref);
        ps += pv[j];
      }
      ps += __shfl_xor(ps, 16, 64);
      ps += __shfl_xor(ps, 32, 64);
      l_w[rb] = l_w[rb] * alpha[rb] + ps;
      *(uint2*)&pb[(16 * rb + fr) * kDecPP + 16 * w + 4 * g] =
          uint2{f2bf2(pv[0], pv[1]), f2bf2(pv[2], pv[3])};
    }
    if (t0 != kbeg) {  // O is still zero on the first tile
#pragma unroll
      for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float al = __shfl(alpha[rb], 4 * g + j, 64);
#pragma unroll
          for (int b = 0; b < 4; ++b) o[rb][b][j] *= al;
        }
    }
    // V fragments (B operand of P V): dim 64 w + 16 b + fr, keys t0 + 32 c +
    // 8 g .. + 7
    bf16x8 vf[8];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int d = 64 * w + 16 * b + fr;
        vf[4 * c + b] = mask_keys(ld8(&sV[d * 64 + 8 * ((4 * c + g) ^ ((d >> 1) & 7))]),
                                  kend - (t0 + 32 * c + 8 * g));
      }
    __syncthreads();

#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const bf16x8 pa = ld8(&pb[(16 * rb + fr) * kDecPP + 32 * c + 8 * g]);
#pragma unroll
        for (int b = 0; b < 4; ++b) o[rb][b] = mfma16x16x32(pa, vf[4 * c + b], o[rb][b]);
      }
    if (t0 + 2 * KT < kend) {
      // this wave's reads of stage cs are done before the stage is refilled
      __builtin_amdgcn_s_waitcnt((15 << 0) | (7 << 4) | (0 << 8) | (3 << 14));
      issue(t0 + 2 * KT, cs);
    }
  }

  // per-wave row sums; O rows -> LDS (over the stages, once every wave is
  // done with them), then row segments out
  __syncthreads();
  if (g == 0) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      sL[w][16 * rb + fr] = l_w[rb];
      if (w == 0) sM[16 * rb + fr] = m_run[rb];
    }
  }
  float* sO = (float*)smem;
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sO[(16 * rb + 4 * g + j) * kDecOP + 64 * w + 16 * b + fr] = o[rb][b][j];
  __syncthreads();
  // thread item c: row c >> 5, dims 8 (c & 31) .. + 7 (a wave writes two
  // whole rows)
  if (splits == 1) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = tid + 256 * u, i = c >> 5, d0 = (c & 31) * 8;
      const int r = rg * 64 + i;
      if (r >= R) continue;
      const float l = ((sL[0][i] + sL[1][i]) + sL[2][i]) + sL[3][i];
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const f32x4_t a = *(const f32x4_t*)&sO[i * kDecOP + d0];
      const f32x4_t b = *(const f32x4_t*)&sO[i * kDecOP + d0 + 4];
      float v[8] = {a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv,
                    b[0] * inv, b[1] * inv, b[2] * inv, b[3] * inv};
      dec_store<8>(p, z, r, d0, dv, v);
    }
    return;
  }

  float* part = (float*)p.workspace + (((int64_t)z * n_rg + rg) * splits + split) * kDecPF;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int c = tid + 256 * u, i = c >> 5, d0 = (c & 31) * 8;
    st8((bf16_t*)part + i * 256 + d0, pack8(&sO[i * kDecOP + d0]));
  }
  if (tid < 64) {
    part[kDecPO + tid] = sM[tid];
    part[kDecPO + 64 + tid] = ((sL[0][tid] + sL[1][tid]) + sL[2][tid]) + sL[3][tid];
  }
  if (!counters) return;
  // the partial is in this XCD's L2 before it is counted
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0)
    __hip_atomic_fetch_add(counters + ((int64_t)z * n_rg + rg) * 64, 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
}


// ---------------------------------------------------------------------------
// attn_decode_t_kernel: the same problems as attn_decode_kernel (head_dim 256,
// transposed value cache, 64-row groups x key ranges, the same partials for
// attn_decode_merge_kernel), computed transposed so that nothing crosses
// waves but the K / V^T tiles.  A workgroup of NW waves owns 32 NW query
// rows; wave w owns rows 32 w .. + 31 and all 256 dims, and per 64-key tile
//   S^T (64 keys x 32 rows)  = K . Q^T     v_mfma_f32_32x32x16_bf16, K from
//                                          LDS (A), Q^T in VGPRs (B);
//   O^T (256 dims x 32 rows) += V^T . P^T  V^T from LDS (A), P^T (B) straight
//                                          from the S^T accumulators.
// Lane (q, h) = (lane % 32, lane / 32) ends S^T holding 32 keys of ONE query
// row q: the A operand rows of K are read in the key order pi(i) = 16 (j >>
// 1) + 8 h' + 4 (j & 1) + (i & 3) (j = i >> 3, h' = (i >> 2) & 1), so that
// the accumulator elements 0..7 / 8..15 are keys 8 h .. + 7 / 16 + 8 h .. + 7
// of the 32-key block, i.e. exactly the B operand of P^T for the 16-key
// steps of O^T.  The softmax statistics of a row live in lanes q and q + 32
// (one shuffle), and O^T's accumulators of lane (q, h) all belong to row q,
// so nothing needs a cross-lane exchange.  There is no online rescale of
// the 128 O accumulators (which would pull them out of the AGPRs every
// tile): a row's exp2 reference is its maximum over the first 32-key block
// in which it sees a key, so P = 2^(s - ref) <= 2^32 as long as no later score
// exceeds the reference by more than 32 (in the exp2 domain) -- fp32 and
// bf16 hold that with room to spare.  Should any row of the workgroup go
// further, the workgroup runs its key range a second time with each row's
// exact maximum (tracked on the first pass) as the reference.  The K / V^T
// tiles (the same LDS images as attn_decode_kernel's) move by LDS DMA in a
// two-stage ring with one barrier per tile; tile t + 1's loads are spread
// between tile t's S^T MFMAs.  The softmax of the second 32-key block runs
// under the first P V steps, and tiles that need no masking (neither the
// range's last, partial tile nor key groups that hide a key from a row of
// the wave) skip it.
// ---------------------------------------------------------------------------
constexpr int kDtKB = 64 * 512, kDtVB = 256 * 128;
constexpr int kDtStage = kDtKB + kDtVB + 256;    // + the tile's key groups
constexpr int kDtOffQG = 2 * kDtStage;           // query groups [32 NW]
// NW waves own 32 NW query rows; the epilogue's O rows ([32 NW][kDecOP] fp32)
// reuse the LDS from its start
template <int NW>
constexpr int dt_lds() {
  return kDtOffQG + 128 * NW > 128 * NW * kDecOP ? kDtOffQG + 128 * NW
                                                 : 128 * NW * kDecOP;
}
static_assert(dt_lds<4>() <= 160 * 1024, "4-wave LDS fits the CU");
constexpr float kDtRefSlack = 32.f;              // log2 of the largest P
constexpr int kDecTKps = 4 * kDecKT;             // keys per range that select it
// waves per workgroup of attn_decode_t_kernel (2: 64 query rows, 4: 128;
// 4 measured 15-20 % faster on the prefix)
constexpr int kDtNW = 4;
// workgroups the default key-range count aims at (the CUs of an MI355X)
constexpr int64_t kDtTargetWgs = 256;
// LDS fragment ring of the tile loop: kDtRing register sets, read kDtAhead
// MFMA steps ahead of their use (deeper rings measured no faster)
constexpr int kDtAhead = 6, kDtRing = kDtAhead + 2;

// The values of lanes l and l ^ 32 combined in both (v_permlane32_swap: a
// VALU exchange of the wave's halves, where a shuffle is an LDS round trip).
// Both lanes compute the same expression of the same two values, so they
// agree bit for bit.
__device__ __forceinline__ void half_pair(float v, float& a, float& b) {
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  a = __uint_as_float(s[0]);  // lane l & 31's value
  b = __uint_as_float(s[1]);  // lane (l & 31) + 32's value
}
__device__ __forceinline__ float half_pair_max(float v) {
  float a, b;
  half_pair(v, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float half_pair_sum(float v) {
  float a, b;
  half_pair(v, a, b);
  return a + b;
}

// NW = 2 or 4 waves: with 4, every K / V^T tile brought into the LDS serves
// 128 query rows and all four SIMDs of the CU.  n_rg counts 64-row groups
// (the unit of the partials and of the merge); a 4-wave workgroup covers two
// of them.
template <int NW>
__global__ __launch_bounds__(64 * NW) void attn_decode_t_kernel(fvx_attn_desc p,
                                                                int n_rg, int splits,
                                                                int kps, DecDiv dv) {
  constexpr int HD = 256, KT = 64, RPW = 32 * NW, LPW = 32 / NW;
  static_assert(NW == 2 || NW == 4, "2 or 4 waves");
  __shared__ __align__(16) unsigned char smem[dt_lds<NW>()];
  __shared__ float sLq[RPW], sMq[RPW];
  warm_kernargs<sizeof(fvx_attn_desc) + 32>();
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane & 31, h = lane >> 5;
  const int nb = (int)gridDim.x, q8 = nb >> 3, r8 = nb & 7;
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const int item = xcd * q8 + (xcd < r8 ? xcd : r8) + slot;
  const int n_rgw = (n_rg * 64 + RPW - 1) / RPW;  // RPW-row groups
  const int ir = dv.rgw.div(item), rg = item - ir * n_rgw;
  const int z = dv.splits.div(ir), split = ir - z * splits;
  const int heads = (int)p.heads, R = (int)p.sq * heads;
  const int64_t zb = dv.zdiv.div(z), zh = z - zb * p.zdiv;
  const bf16_t* Q = (const bf16_t*)p.q + zb * p.q_zs1 + zh * p.q_zs2;
  const bf16_t* K = (const bf16_t*)p.k + zb * p.k_zs1 + zh * p.k_zs2;
  const bf16_t* Vt = (const bf16_t*)p.v + zb * p.v_zs1 + zh * p.v_zs2;
  const int32_t* kgrp = p.kgrp ? p.kgrp + zb * p.kgrp_zs1 : nullptr;
  const int32_t* qgrp = p.qgrp ? p.qgrp + zb * p.qgrp_zs1 : nullptr;
  const int kbeg = split * kps;
  const int kend = kbeg + kps < (int)p.sk ? kbeg + kps : (int)p.sk;
  const int ntile = (kend - kbeg + KT - 1) / KT;
  const int qts = (int)p.q_tok_stride, qhs = (int)p.q_head_stride;
  const int kts = (int)p.k_tok_stride, vds = (int)p.v_d_stride;

  // buffer views: K keys >= kend and Q rows >= R read zero; V^T keys past
  // kend are zeroed after they are read
  const i32x4_t rq =
      make_rsrc4(Q, (uint32_t)(((int)p.sq - 1) * qts + (heads - 1) * qhs + HD) * 2);
  const i32x4_t rkc = make_rsrc4(K, (uint32_t)kend * kts * 2);
  const i32x4_t rvc = make_rsrc4(Vt, (uint32_t)HD * vds * 2);
  const i32x4_t rgc = make_rsrc4(kgrp ? (const void*)kgrp : (const void*)Q,
                                 kgrp ? (uint32_t)kend * 4 : 0u);
  const i32x4_t rqg = make_rsrc4(qgrp ? (const void*)qgrp : (const void*)Q,
                                 qgrp ? (uint32_t)p.sq * 4 : 0u);
  const uint32_t lbase = lds_addr(smem);

  // load L (0..31) of a tile: K keys 2 L + (lane >> 5) (LDS slot lane & 31 of
  // the key's 512-byte row holds global chunk slot ^ (key & 15)); V^T dims
  // 8 L + (lane >> 3) (slot lane & 7 of the dim's 128-byte row holds key
  // chunk slot ^ ((dim >> 1) & 7)).  Wave w issues K and V loads LPW w ..
  // LPW w + LPW - 1.
  auto load_k = [&](int t0, int st, int L) {
    const int kl = 2 * L + (lane >> 5);
    const int ch = (lane & 31) ^ (kl & 15);
    load_lds16(rkc, lbase + st * kDtStage + 2 * L * 512, (uint32_t)((t0 + kl) * kts + 8 * ch) * 2);
  };
  auto load_v = [&](int t0, int st, int L) {
    const int d = 8 * L + (lane >> 3);
    const int ch = (lane & 7) ^ ((d >> 1) & 7);
    load_lds16(rvc, lbase + st * kDtStage + kDtKB + 8 * L * 128,
               (uint32_t)(d * vds + t0 + 8 * ch) * 2);
  };
  auto load_g = [&](int t0, int st) {  // the tile's 64 key groups (wave 0)
    load_lds4(rgc, lbase + st * kDtStage + kDtKB + kDtVB, (uint32_t)(t0 + lane) * 4);
  };

  // Q rows RPW rg + 2 L + (lane >> 5) into stage 1 from its start (K's
  // swizzle; 128 rows fill its K and V^T areas, 64 KB), the query groups,
  // then tile 0 into stage 0
  static_assert(RPW * 512 <= kDtKB + kDtVB, "Q rows fit stage 1");
  {
    const uint32_t qb = lbase + kDtStage;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int L = 16 * w + i, rl = 2 * L + (lane >> 5), r = rg * RPW + rl;
      const int tok = row_tok(r, dv);
      const int ch = (lane & 31) ^ (rl & 15);
      load_lds16(rq, qb + 2 * L * 512,
                 r < R ? (uint32_t)(tok * qts + (r - tok * heads) * qhs + 8 * ch) * 2 : kOOB);
    }
    if (w < NW / 2) {  // 64 rows' groups per wave
      const int r = rg * RPW + 64 * w + lane;
      load_lds4(rqg, lbase + kDtOffQG + 256 * w,
                r < R ? (uint32_t)row_tok(r, dv) * 4 : kOOB);
    }
  }
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    load_k(kbeg, 0, LPW * w + i);
    load_v(kbeg, 0, LPW * w + i);
  }
  if (kgrp && w == 0) load_g(kbeg, 0);
  wait_vmcnt<0>();
  __syncthreads();

  // Q^T fragments (B operand): lane (q, h) holds dims 16 s + 8 h .. + 7 of
  // row 32 w + q
  bf16x8 qT[16];
  int32_t qg;
  {
    const int rl = 32 * w + q;
    const bf16_t* sQ = (const bf16_t*)(smem + kDtStage);
#pragma unroll
    for (int s2 = 0; s2 < 16; ++s2) qT[s2] = ld8(&sQ[rl * 256 + 8 * ((2 * s2 + h) ^ (rl & 15))]);
    qg = qgrp ? ((const int32_t*)(smem + kDtOffQG))[rl] : 0;
  }
  // the wave's smallest query group (rows past R: their token's group or 0)
  int qg_min = qg;
#pragma unroll
  for (int x = 1; x < 64; x <<= 1) qg_min = min(qg_min, __shfl_xor(qg_min, x, 64));
  qg_min = __builtin_amdgcn_readfirstlane(qg_min);
  __syncthreads();  // stage 1 is free for tile 1

  // K A-operand row of this lane: key pi(q) of each 32-key block
  const int piq = 16 * ((q >> 3) >> 1) + 8 * ((q >> 2) & 1) + 4 * ((q >> 3) & 1) + (q & 3);
  const float sc = p.scale * kLog2e;
  // m_ref: the row's exp2 reference, fixed at its first visible key (O and
  // l are still zero then) or, on the second pass, the exact row maximum
  float m_ref = -INFINITY, l_run = 0.f, m_max = -INFINITY;
  f32x16_t o[8];
  for (int pass = 0;; ++pass) {
  bool over = false;
#pragma unroll
  for (int db = 0; db < 8; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;

  for (int t = 0; t < ntile; ++t) {
    const int t0 = kbeg + t * KT, st = t & 1;
    const bool edge = t0 + KT > kend;  // the range's last, partial tile
    const bf16_t* sK = (const bf16_t*)(smem + st * kDtStage);
    const bf16_t* sV = (const bf16_t*)(smem + st * kDtStage + kDtKB);
    const int32_t* sG = (const int32_t*)(smem + st * kDtStage + kDtKB + kDtVB);
    // this wave's loads of tile t landed
    wait_vmcnt<0>();
    if (edge) {
      // keys >= kend of this wave's V^T rows (dims 8 LPW w ..) read as zero
      // (the cache past the range may hold anything; P is 0 there)
      bf16_t* sVw = (bf16_t*)sV + 8 * LPW * w * 64;
      const int valid = kend - t0;
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int c = lane + 64 * i, row = c >> 3, slot = c & 7;
        const int kc = slot ^ (((8 * LPW * w + row) >> 1) & 7);  // key chunk in this slot
        bf16x8* ptr = (bf16x8*)&sVw[row * 64 + 8 * slot];
        if (8 * kc + 8 > valid) {
          bf16x8 v = *ptr;
#pragma unroll
          for (int x = 0; x < 4; ++x)
            v.w[x] &= 8 * kc + 2 * x + 1 < valid ? 0xffffffffu
                                                  : (8 * kc + 2 * x < valid ? 0xffffu : 0u);
          *ptr = v;
        }
      }
    }
    // the barrier publishes everyone's loads of tile t, and every wave is
    // done with tile t - 1 (stage st ^ 1)
    __syncthreads();

    // key groups mask some key of this tile for some row of this wave?
    // (uniform: any key group of the tile above the wave's smallest; one
    // ballot, no cross-lane chain)
    const bool gmask = kgrp && __ballot(sG[lane] > qg_min) != 0;
    const bool more = t + 1 < ntile;  // tile t + 1 is loaded during this one
    auto rdk = [&](int j) {  // S^T step j: key block j & 1, dims 16 (j >> 1) ..
      const int key = 32 * (j & 1) + piq;
      return ld8(&sK[key * 256 + 8 * ((2 * (j >> 1) + h) ^ (key & 15))]);
    };
    auto rdv = [&](int j) {
      const int d = 32 * (j & 7) + q;
      return ld8(&sV[d * 64 + 8 * ((2 * (j >> 3) + h) ^ ((d >> 1) & 7))]);
    };
    // the tile (masking only on the edge tile or with key groups in play)
    {
      // S^T: step j = 2 s + kb (key block kb, dims 16 s ..; the two blocks'
      // accumulations alternate, so that no MFMA waits for the previous
      // one's result), the K fragments through a ring of kDtRing register
      // sets read kDtAhead steps ahead
      f32x16_t sacc[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
      bf16x8 ring[kDtRing], pT[4];
      // softmax of key block kb (its S^T complete) -> pT[2 kb], pT[2 kb + 1]:
      // element r is key 32 kb + 16 (r >> 3) + 8 h + (r & 7).  The maximum
      // is taken on the raw scores (the scale is positive) and the scale
      // folded into the exponent's FMA.
      auto softmax = [&](auto kbc) {
        constexpr int kb = decltype(kbc)::value;
        f32x16_t& sv = sacc[kb];
        if (edge || gmask) {  // uniform
#pragma unroll
          for (int hf = 0; hf < 2; ++hf) {
            const int kl0 = 32 * kb + 16 * hf + 8 * h;
            int32_t kgv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (kgrp) {
              const int4 ga = *(const int4*)&sG[kl0];
              const int4 gb = *(const int4*)&sG[kl0 + 4];
              kgv[0] = ga.x; kgv[1] = ga.y; kgv[2] = ga.z; kgv[3] = ga.w;
              kgv[4] = gb.x; kgv[5] = gb.y; kgv[6] = gb.z; kgv[7] = gb.w;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (kgv[e] > qg || t0 + kl0 + e >= kend) sv[8 * hf + e] = -INFINITY;
          }
        }
        float mb = sv[0];
#pragma unroll
        for (int e = 1; e < 16; ++e) mb = fmaxf(mb, sv[e]);
        mb = half_pair_max(mb) * sc;
        m_max = fmaxf(m_max, mb);
        if (m_ref == -INFINITY)
          m_ref = mb;
        else
          over = over || mb > m_ref + kDtRefSlack;
        const float nm = m_ref == -INFINITY ? 0.f : -m_ref;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
          float pv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            pv[e] = __builtin_amdgcn_exp2f(fmaf(sv[8 * hf + e], sc, nm));
            l_run += pv[e];
          }
          pT[2 * kb + hf] = pack8(pv);
        }
      };
#pragma unroll
      for (int j = 0; j < kDtAhead; ++j) ring[j] = rdk(j);
      // (compile-time steps: the loops hold too much code for the unroller)
      static_for<0, 32>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if (j + kDtAhead < 32) ring[(j + kDtAhead) % kDtRing] = rdk(j + kDtAhead);
        sacc[j & 1] = mfma32x32x16(ring[j % kDtRing], qT[j >> 1], sacc[j & 1]);
        // the wave's 2 LPW loads of tile t + 1, one every 16 / LPW steps
        constexpr int EV = 16 / LPW, LL = j / EV;
        if (more && j % EV == 0) {
          if (j == 0 && kgrp && w == 0) load_g(t0 + KT, st ^ 1);
          if (LL < LPW)
            load_k(t0 + KT, st ^ 1, LPW * w + LL);
          else
            load_v(t0 + KT, st ^ 1, LPW * w + LL - LPW);
        }
      });
      softmax(IntC<0>{});
      // O^T += V^T P^T, step j = 8 u + db: V^T A operand lane (i, h) = dim
      // 32 db + i, keys 16 u + 8 h .. + 7
#pragma unroll
      for (int j = 0; j < kDtAhead; ++j) ring[j] = rdv(j);
      static_for<0, 32>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        if (j + kDtAhead < 32) ring[(j + kDtAhead) % kDtRing] = rdv(j + kDtAhead);
        o[j & 7] = mfma32x32x16(ring[j % kDtRing], pT[j >> 3], o[j & 7]);
        if (j == 3) softmax(IntC<1>{});
      });
    }
  }
  wait_vmcnt<0>();
  // every wave is done with the ring; a row whose scores rose more than
  // 2^kDtRefSlack above its reference sends the workgroup through a second
  // pass with the exact row maxima as references (P <= 1)
  if (!__syncthreads_or(over) || pass) break;
  m_ref = m_max;
  l_run = 0.f;
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    load_k(kbeg, 0, LPW * w + i);
    load_v(kbeg, 0, LPW * w + i);
  }
  if (kgrp && w == 0) load_g(kbeg, 0);
  }
  l_run = half_pair_sum(l_run);

  // O rows -> LDS: lane (q, h) holds dims 32 db + 8 (r >> 2) + 4 h + (r & 3)
  // of row 32 w + q
  float* sO = (float*)smem;
  {
    const int rl = 32 * w + q;
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j)  // elements 4 j .. 4 j + 3: 4 consecutive dims
        *(f32x4_t*)&sO[rl * kDecOP + 32 * db + 8 * j + 4 * h] =
            f32x4_t{o[db][4 * j], o[db][4 * j + 1], o[db][4 * j + 2], o[db][4 * j + 3]};
    if (h == 0) {
      sLq[rl] = l_run;
      sMq[rl] = m_ref;
    }
  }
  __syncthreads();
  // thread item c: row c >> 5, dims 8 (c & 31) .. + 7
  if (splits == 1) {
#pragma unroll 4
    for (int u = 0; u < 16; ++u) {
      const int c = tid + 64 * NW * u, i = c >> 5, d0 = (c & 31) * 8;
      const int r = rg * RPW + i;
      if (r >= R) continue;
      const float l = sLq[i];
      const float inv = l > 0.f ? 1.f / l : 0.f;
      const f32x4_t a = *(const f32x4_t*)&sO[i * kDecOP + d0];
      const f32x4_t b = *(const f32x4_t*)&sO[i * kDecOP + d0 + 4];
      float v[8] = {a[0] * inv, a[1] * inv, a[2] * inv, a[3] * inv,
                    b[0] * inv, b[1] * inv, b[2] * inv, b[3] * inv};
      dec_store<8>(p, z, r, d0, dv, v);
    }
    return;
  }
  // one partial per 64-row group (the merge's unit); a 4-wave workgroup's
  // second group does not exist when n_rg is odd and this is the last one
  for (int g = 0; g < NW / 2; ++g) {
    const int rg64 = rg * (NW / 2) + g;
    if (rg64 >= n_rg) break;
    float* part = (float*)p.workspace + (((int64_t)z * n_rg + rg64) * splits + split) * kDecPF;
#pragma unroll 4
    for (int u = 0; u < 16 / (NW / 2); ++u) {
      const int c = tid + 64 * NW * u, i = c >> 5, d0 = (c & 31) * 8;
      st8((bf16_t*)part + i * 256 + d0, pack8(&sO[(64 * g + i) * kDecOP + d0]));
    }
    if (tid < 64) {
      part[kDecPO + tid] = sMq[64 * g + tid];
      part[kDecPO + 64 + tid] = sLq[64 * g + tid];
    }
  }
}

// Merge of the decode partials (bf16 O rows: half the bytes of fp32, within
// the output's own bf16 rounding): one thread per (problem, query row, 8
// dims); the loads of up to 4, 8 or 16 splits (as many as there are) are
// issued before the merge, which is applied in split order.
__global__ __launch_bounds__(256) void attn_decode_merge_kernel(
    fvx_attn_desc p, int n_rg, int splits, DecDiv dv) {
  warm_kernargs<sizeof(fvx_attn_desc) + 32>();
  const int R = (int)(p.sq * p.heads);
  const int gid = blockIdx.x * 256 + threadIdx.x;
  if (gid >= (int)p.n_problems * R * 32) return;
  const int d0 = (gid & 31) * 8;
  const int zr = gid >> 5;
  const int z = zr / R, r = zr % R;
  dec_merge8<0>(p, n_rg, splits, dv, z, r, d0);
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
  a.ws_bytes = splits > 1 ? kAttnCounterBytes + blocks * splits * pf * 4 : 0;
  return a;
}

}  // namespace fvx

using namespace fvx;

static bool has_prefetch(const fvx_attn_desc& d) {
  for (int r = 0; r < 8; ++r)
    if (d.prefetch[r] && d.prefetch_bytes[r] > 0) return true;
  return false;
}


struct DecodePlan {
  int n_rb, splits, n_items;
  int64_t kps, ws_bytes;
};

static bool use_decode(const fvx_attn_desc& d) {
  // (its operand offsets are 32-bit)
  const int64_t lim = (int64_t)1 << 30;
  return d.v_d_stride > 0 && d.head_dim == 256 &&
         d.sq * d.q_tok_stride + d.heads * d.q_head_stride < lim &&
         d.sk * d.k_tok_stride < lim && 256 * d.v_d_stride < lim;
}

// 64-row groups x key ranges of whole 64-key tiles; by default about 128
// workgroups (one tile each for the action expert: measured faster than two
// tiles per workgroup with half the partials to merge).
static DecodePlan plan_decode(const fvx_attn_desc& d) {
  DecodePlan a;
  a.n_rb = (int)((d.sq * d.heads + 63) / 64);
  const int64_t tiles = (d.sk + kDecKT - 1) / kDecKT;
  const int64_t groups = (int64_t)a.n_rb * d.n_problems;
  int64_t splits = d.kv_splits;
  if (splits <= 0) splits = (128 + groups - 1) / groups;
  if (splits > tiles) splits = tiles;
  if (splits < 1) splits = 1;
  if (d.kv_splits <= 0 && (tiles + splits - 1) / splits * kDecKT >= kDecTKps) {
    // the prefix kernel (ranges of >= 4 tiles): as many ranges as keep its
    // 32 kDtNW-row workgroups within one per CU, each range >= 4 tiles
    const int64_t wg_groups =
        ((int64_t)a.n_rb * 64 + 32 * kDtNW - 1) / (32 * kDtNW) * d.n_problems;
    splits = kDtTargetWgs / wg_groups;
    while (splits > 1 && (tiles + splits - 1) / splits * kDecKT < kDecTKps) --splits;
    if (splits < 1) splits = 1;
  }
  const int64_t kps = (tiles + splits - 1) / splits * kDecKT;
  a.splits = (int)((d.sk + kps - 1) / kps);
  a.kps = kps;
  a.n_items = (int)(groups * a.splits);
  a.ws_bytes = a.splits > 1 ? kAttnCounterBytes + (int64_t)a.n_items * kDecPF * 4 : 0;
  return a;
}

// FastDiv of d: m = ceil(2^32 / d), 0 for d = 1 (d < 2^31).
static FastDiv fast_div(int64_t d) {
  return FastDiv{d <= 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + (uint64_t)d - 1) / (uint64_t)d)};
}
static int64_t dt_groups(int n_rb) { return ((int64_t)n_rb * 64 + 32 * kDtNW - 1) / (32 * kDtNW); }
static DecDiv dec_div(const fvx_attn_desc& d, const DecodePlan& a) {
  return DecDiv{fast_div(d.heads), fast_div(d.zdiv), fast_div(a.n_rb), fast_div(a.splits),
                fast_div(dt_groups(a.n_rb))};
}
// every dividend of a FastDiv stays below 2^32 / divisor
static bool dec_div_exact(const fvx_attn_desc& d, const DecodePlan& a) {
  const uint64_t lim = (uint64_t)1 << 32;
  const uint64_t R = (uint64_t)(d.sq * d.heads), items = (uint64_t)a.n_items + 8 * 256;
  const uint64_t wide = (uint64_t)d.n_problems * a.splits * dt_groups(a.n_rb) + 8 * 256;
  return R * (uint64_t)d.heads < lim && (uint64_t)d.n_problems * (uint64_t)d.zdiv < lim &&
         items * (uint64_t)a.n_rb < lim && items * (uint64_t)a.splits < lim &&
         wide * (uint64_t)dt_groups(a.n_rb) < lim && wide * (uint64_t)a.splits < lim;
}
// the decode kernels serve d: head_dim 256 with the transposed value cache,
// 32-bit operand offsets, exact fast divisions
static bool decode_ok(const fvx_attn_desc& d) {
  return use_decode(d) && dec_div_exact(d, plan_decode(d));
}

extern "C" int64_t fvx_attention_workspace_bytes(const fvx_attn_desc* d) {
  if (!d || d->sq <= 0 || d->sk <= 0 || d->heads <= 0 || d->n_problems <= 0)
    return 0;
  if (decode_ok(*d)) return plan_decode(*d).ws_bytes;
  return plan_attn(*d).ws_bytes;
}

// The descriptor the kernels see: the split partials start past the arrival
// counters that open every attention workspace.
static fvx_attn_desc past_counters(const fvx_attn_desc& d) {
  fvx_attn_desc k = d;
  if (d.workspace && d.workspace_bytes >= kAttnCounterBytes) {
    k.workspace = (char*)d.workspace + kAttnCounterBytes;
    k.workspace_bytes = d.workspace_bytes - kAttnCounterBytes;
  } else {
    k.workspace = nullptr;
    k.workspace_bytes = 0;
  }
  return k;
}

static int run_generic(const fvx_attn_desc& d, hipStream_t s) {
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
  const fvx_attn_desc dk = past_counters(d);
  dim3 grid((unsigned)a.n_row_blocks, (unsigned)a.splits,
            (unsigned)d.n_problems);
  if (a.hdp == 256)
    hipLaunchKernelGGL((attn_kernel<256, 256>), grid, dim3(256), 0, s, dk,
                       a.n_row_blocks, a.splits, a.kps);
  else
    hipLaunchKernelGGL((attn_kernel<96, 80>), grid, dim3(256), 0, s, dk,
                       a.n_row_blocks, a.splits, a.kps);
  int st = launch_status("attention");
  if (st || a.splits == 1) return st;
  dim3 mgrid((unsigned)a.n_row_blocks, 1u, (unsigned)d.n_problems);
  if (a.hdp == 256)
    hipLaunchKernelGGL((attn_merge_kernel<256, 256>), mgrid, dim3(256), 0, s,
                       dk, a.n_row_blocks, a.splits);
  else
    hipLaunchKernelGGL((attn_merge_kernel<96, 80>), mgrid, dim3(256), 0, s, dk,
                       a.n_row_blocks, a.splits);
  return launch_status("attention");
}

extern "C" int fvx_attention(const fvx_attn_desc* dp, void* stream) {
  clear_error();
  FVX_REQUIRE(dp, FVX_ERR_NULL, "attention: descriptor is NULL");
  const fvx_attn_desc& d = *dp;
  FVX_REQUIRE(d.q && d.k && d.v && (d.o || d.o_frag), FVX_ERR_NULL,
              "attention: q, k, v and o (or o_frag) required");
  FVX_REQUIRE(d.sq >= 0 && d.sk >= 0 && d.heads > 0 && d.n_problems >= 0 &&
                  d.zdiv > 0,
              FVX_ERR_SHAPE, "attention: bad sizes");
  // problem and query-row indices divide in 32 bits
  FVX_REQUIRE(d.zdiv < ((int64_t)1 << 31) && d.sq * d.heads < ((int64_t)1 << 31) &&
                  d.n_problems < ((int64_t)1 << 31),
              FVX_ERR_SHAPE, "attention: sq * heads, n_problems and zdiv must be < 2^31");
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
  FVX_REQUIRE(!d.o_frag || (decode_ok(d) && d.n_problems * d.sq <= 64 &&
                             d.o_head_stride % 8 == 0 && d.o_tok_stride % 8 == 0 &&
                             aligned16(d.o) && aligned16(d.o_frag)),
              FVX_ERR_ARG,
              "attention: o_frag needs the decode path (transposed V, head_dim "
              "256), n_problems * sq <= 64 and 16B-aligned outputs");
  for (int r = 0; r < 8; ++r)
    FVX_REQUIRE(!d.prefetch[r] ||
                    (aligned16(d.prefetch[r]) && d.prefetch_bytes[r] >= 0 &&
                     d.prefetch_bytes[r] % 1024 == 0 && d.prefetch_tile_bytes[r] >= 0 &&
                     d.prefetch_tile_bytes[r] % 1024 == 0),
                FVX_ERR_ARG,
                "attention: prefetch ranges need 16B-aligned pointers and byte "
                "and tile-byte counts that are multiples of 1024");
  FVX_REQUIRE(d.prefetch_wgs >= 0 && d.prefetch_wgs <= 4096, FVX_ERR_ARG,
              "attention: prefetch_wgs must be in [0, 4096]");
  if (d.sq == 0 || d.n_problems == 0) return FVX_OK;
  FVX_REQUIRE(d.sk > 0, FVX_ERR_SHAPE, "attention: sk must be > 0");
  hipStream_t s = (hipStream_t)stream;
  if (decode_ok(d)) {
    DecodePlan a = plan_decode(d);
    if (a.splits > 1 && (!d.workspace || d.workspace_bytes < a.ws_bytes))
      return set_error(FVX_ERR_WORKSPACE,
                       "attention: %d key splits need %lld workspace bytes, "
                       "got %lld", a.splits, (long long)a.ws_bytes,
                       (long long)d.workspace_bytes);
    FVX_REQUIRE(aligned16(d.workspace), FVX_ERR_ALIGN,
                "attention: workspace must be 16B aligned");
    const DecDiv dv = dec_div(d, a);
    const fvx_attn_desc dk = past_counters(d);
    // the 4-wave kernel's in-launch merge: each 64-row group's ranges and
    // its 8 merging workgroups on one XCD, all of them resident at once
    // (R % 8 == 0: a merging workgroup's 8 rows lie in one group)
    const int64_t R = d.sq * d.heads;
    const int groups = (int)(d.n_problems * a.n_rb);
    const int gpx = (groups + 7) / 8;  // groups per XCD
    const bool fused = a.kps < kDecTKps && a.splits > 1 && a.splits <= 16 && R % 8 == 0 &&
                       groups <= kAttnMaxGroups && gpx * (a.splits + 8) <= device_cus() / 8;
    const int item_blocks = fused ? 8 * gpx * a.splits : a.n_items;
    const int merge_blocks = fused ? 64 * gpx : 0;
    int pf_wgs = 0;  // prefetch workgroups (the 4-wave kernel only)
    if (a.kps < kDecTKps && has_prefetch(d)) {
      pf_wgs = d.prefetch_wgs;
      if (pf_wgs <= 0) {
        const int cus = device_cus(), used = item_blocks + merge_blocks;
        pf_wgs = cus > used ? cus - used : 0;
      }
    }
    // key ranges of >= 4 tiles (the prefix): attn_decode_t_kernel, ~8 %
    // faster there; one or two tiles per workgroup (the action expert): the
    // 4-wave kernel, whose fixed costs are lower
    if (a.kps >= kDecTKps) {
      const int64_t groups = (a.n_rb * 64 + 32 * kDtNW - 1) / (32 * kDtNW);
      const int64_t wgs = d.n_problems * a.splits * groups;
      hipLaunchKernelGGL(attn_decode_t_kernel<kDtNW>, dim3((unsigned)wgs),
                         dim3(64 * kDtNW), 0, s, dk, a.n_rb, a.splits, (int)a.kps, dv);
    } else
      hipLaunchKernelGGL(attn_decode_kernel,
                         dim3((unsigned)(item_blocks + merge_blocks + pf_wgs)), dim3(256), 0,
                         s, dk, a.n_rb, a.splits, (int)a.kps, dv, item_blocks,
                         fused ? (uint32_t*)d.workspace : nullptr,
                         item_blocks + merge_blocks);
    int st = launch_status("attention(decode)");
    if (st || a.splits == 1 || fused) return st;
    const int64_t threads = (int64_t)d.n_problems * d.sq * d.heads * 32;
    hipLaunchKernelGGL(attn_decode_merge_kernel,
                       dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       dk, a.n_rb, a.splits, dv);
    return launch_status("attention(decode merge)");
  }
  return run_generic(d, s);
}
// Zeroes the attention workspace's counter region (a fill kernel, not a
// memset node: callers may run it next to captured work).
__global__ void attn_counters_clear_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

extern "C" int fvx_attention_check(void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  clear_error();
  FVX_REQUIRE(workspace, FVX_ERR_NULL, "attention_check: workspace is NULL");
  FVX_REQUIRE(workspace_bytes >= kAttnCounterBytes, FVX_ERR_WORKSPACE,
              "attention_check: the workspace must hold the %lld-byte counter "
              "region, got %lld bytes", (long long)kAttnCounterBytes,
              (long long)workspace_bytes);
  FVX_REQUIRE(aligned16(workspace), FVX_ERR_ALIGN,
              "attention_check: workspace must be 16B aligned");
  hipStream_t s = (hipStream_t)stream;
  uint32_t* counters = (uint32_t*)workspace;
  uint32_t status = 0;
  hipError_t e = hipMemcpyAsync(&status, counters + kAttnStatusWord, 4,
                                hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess)
    return set_error(FVX_ERR_LAUNCH, "attention_check: reading the status "
                     "failed: %s", hipGetErrorString(e));
  if (status == 0) return FVX_OK;
  const int n = (int)(kAttnCounterBytes / 4);
  hipLaunchKernelGGL(attn_counters_clear_kernel, dim3((n + 255) / 256), dim3(256), 0, s,
                     counters, n);
  e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess)
    return set_error(FVX_ERR_LAUNCH, "attention_check: clearing the counters "
                     "failed: %s", hipGetErrorString(e));
  return set_error(FVX_ERR_MERGE,
                   "attention: %u merging workgroup(s) stopped waiting for "
                   "their key ranges, so an earlier call's output is wrong; "
                   "the merge counters are cleared", status);
}
