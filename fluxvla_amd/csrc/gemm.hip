// bf16 / fp8 MFMA GEMM family with fused epilogues (gfx950).
//
//   acc[m][n] = sum_k A[m][k] * B[n][k]      A: activations, B: nn.Linear weight
//
// Kernels (all share the 8-column epilogue epi_load / epi_store):
//
//  * gemm_tile_kernel<BM, BN, WGM, WGN, STAGES, MODE, FP8>: M > 64 (SigLIP
//    M=768, Gemma prefix M=816, batched expert).  64 x 128 tiles of 2 x 2
//    waves on v_mfma_f32_32x32x16_bf16 (fp8: the block-scaled 32x32x64), K in
//    64-wide slabs through a 3- or 4-stage LDS ring filled by LDS DMA
//    (buffer_load ... lds), the slab loads spread between MFMA groups.
//  * gemm_wide_kernel<MODE, SUM_A, NWV> / gemm_wide_f8_kernel: 256 x 256
//    tiles of 8 waves (64 x 128 each; fp8: 4 waves of 128 x 128, the
//    accumulators in AGPRs) for the prefix gate/up
//    at every batch, batched prefixes, and -- over up to 8 K ranges, one
//    per XCD -- long-K GEMMs with few tiles (the prefix down projection).
//  * gemm_skinny_kernel<MODE, FP8>: M <= 64 (the bs=1 action expert,
//    M=50/51).  A weight stream: a workgroup owns 16 output columns and
//    reads its weight rows straight from memory as MFMA B fragments
//    (fragment-major weights: 1 KiB per operand); K splits over workgroups
//    meet through write-through partials and an arrival counter.
//  * gemm_partial_reduce_kernel: the split-K sum (in split order,
//    deterministic) and epilogue behind the tile and wide kernels.
//
// Tiles are ordered m-fastest within a weight panel and block ids remapped
// (xcd_remap) so that one XCD owns consecutive tiles: the m-tiles of a
// panel run on one XCD and reuse the panel from its L2.
//
// Per-row RMSNorm ("rownorm") is fused: the kernel that streams A also
// accumulates sum(A[m][:]^2) (or takes the sums handed over by the GEMM that
// produced A, ss_in / ss_out) and scales the accumulator by rsqrt(mean +
// eps) in the epilogue, so (x * r) @ W' == r * (x @ W') needs no separate
// normalization pass (the (1 + w) Gemma scale is folded into W').
#include <mutex>

#include "capi_util.h"
#include "common.h"

namespace fvx {

typedef fvx_gemm_desc GemmArgs;

// The first kCounterBytes of a GEMM workspace hold the per-column-tile
// arrival counters of the split-K skinny kernel; fp32 partials follow.
constexpr int kCounterBytes = 4096;
constexpr int kMaxSkinnyTiles = kCounterBytes / 4;


// Row indices and the epilogue's periods (row_group, gate_group,
// pos_period, rtc_period) are below 2^31 (the host checks), so quotients and
// remainders take the 32-bit unsigned divide: the 64-bit one is a long
// software sequence per lane.
__device__ __forceinline__ uint32_t udiv32(int64_t a, int64_t b) {
  return (uint32_t)a / (uint32_t)b;
}
__device__ __forceinline__ uint32_t umod32(int64_t a, int64_t b) {
  return (uint32_t)a % (uint32_t)b;
}

__device__ __forceinline__ int64_t out_row(const GemmArgs& p, int64_t m) {
  if (p.row_group <= 0) return m;
  const uint32_t q = udiv32(m, p.row_group);
  return (int64_t)q * p.row_group_stride + ((uint32_t)m - q * (uint32_t)p.row_group);
}

// sum of squares of 8 bf16 values: four v_dot2c_f32_bf16 (fp32 accumulate)
__device__ __forceinline__ float sumsq8(const bf16x8& v) {
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const bf16x2v h = __builtin_bit_cast(bf16x2v, v.w[i]);
    s = __builtin_amdgcn_fdot2_f32_bf16(h, h, s, false);
  }
  return s;
}

// sum of 8 bf16 values: four dot products with (1, 1) (exact products)
__device__ __forceinline__ float sum8(const bf16x8& v) {
  typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
  const bf16x2v one = {(__bf16)1.0f, (__bf16)1.0f};
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, v.w[i]), one, s, false);
  return s;
}

// ---------------------------------------------------------------------------
// Row-chunk epilogue: output columns n .. n + 7 of one row m.
//
// epi_load_col and epi_load_row issue every global read the epilogue needs
// (the column operands: bias, fp32 biases, the RTC lock; the row operands:
// residual, gate, position table, Euler state, RoPE table) and epi_store
// computes and writes.  Callers issue the reads for all of their chunks
// before the first epi_store: an in-place operand (residual == c, xt) may
// alias the output, so a read issued after a store would wait for a full
// memory round trip per element.  A lane of the tile and wide kernels keeps
// one column chunk in every item, so those kernels read the column operands
// once per lane.  `vec`: the chunk holds 8 columns and every operand is
// 16-byte aligned, so each operand moves as one 16-byte (fp32: two) access;
// otherwise `cnt` columns are handled one by one.
// ---------------------------------------------------------------------------
struct EpiIn {
  bf16x8 res, gate, pos, bias;
  float f0[8];    // bias_f32 (PLAIN, EULER) or RoPE (cos, sin) x 4 (QKV_ROPE)
  float xt[8];    // EULER state
  float prev[8];  // EULER with RTC: the previous chunk's actions
  float cw;       // EULER with RTC guidance: the row's correction weight
  float cs[8];    // PLAIN with a folded LayerNorm: the weight's column sums
  bool locked;    // PLAIN, EULER: the row is in the RTC locked prefix
};

__device__ __forceinline__ void st_b8(bf16_t* dst, const float* x, bool vec,
                                      int cnt) {
  if (vec) {
    st8(dst, pack8(x));
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < cnt) dst[e] = f2bf(x[e]);
  }
}

__device__ __forceinline__ void st_f8(float* dst, const float* x, bool vec,
                                      int cnt) {
  if (vec) {
    *(f32x4_t*)dst = f32x4_t{x[0], x[1], x[2], x[3]};
    *(f32x4_t*)(dst + 4) = f32x4_t{x[4], x[5], x[6], x[7]};
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < cnt) dst[e] = x[e];
  }
}

// Buffer-view reads for the epilogue: a NULL operand gets an empty view (all
// reads return zero) and no load sits behind a branch, so the compiler can
// keep every load of a batch in flight (a branch around a load makes it
// wait for that load at the join).
__device__ __forceinline__ uint32_t rec_bytes(int64_t b) {
  return b > 0x7fffffff ? 0x7fffffffu : (uint32_t)b;
}

__device__ __forceinline__ bf16x8 bl_b8(__amdgpu_buffer_rsrc_t r, uint32_t off,
                                        bool vec) {
  if (vec) return bload8(r, off);
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    v.w[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off + 4 * i, 0, 0) |
             ((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off + 4 * i + 2, 0, 0) << 16);
  return v;
}

__device__ __forceinline__ void bl_f8(__amdgpu_buffer_rsrc_t r, uint32_t off,
                                      bool vec, float* d) {
  if (vec) {
    const f32x4_t a = bload4f(r, off), b = bload4f(r, off + 16);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      d[e] = a[e];
      d[4 + e] = b[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) d[e] = bload1f(r, off + 4 * e);
  }
}

// Buffer views of the epilogue's operands: uniform, built once per wave
// outside the item loops (an absent operand gets an empty view, whose reads
// return zeros).
struct EpiViews {
  __amdgpu_buffer_rsrc_t bias, bf32, gate, res, pos, xt, prev, cw, rope, positions, csum;
};

// (SP: the plain-epilogue build -- PLAIN with bias, fp32 bias, activation,
// a per-row gate, residual and the fragment-major copy only; the host
// checks that the call uses nothing else)
template <int MODE, bool SP = false>
__device__ __forceinline__ EpiViews epi_views(const GemmArgs& p) {
  EpiViews V;
  const int64_t N = p.n;
  V.bias = V.bf32 = V.gate = V.res = V.pos = V.xt = V.prev = V.cw = V.rope = V.positions =
      V.csum = make_rsrc(nullptr, 0u);
  if constexpr (SP) {
    V.bias = make_rsrc(p.bias, p.bias ? rec_bytes(N * 2) : 0u);
    V.bf32 = make_rsrc(p.bias_f32, p.bias_f32 ? rec_bytes(N * 4) : 0u);
    V.res = make_rsrc(p.residual, p.residual ? rec_bytes(p.m * p.ldr * 2) : 0u);
    V.gate = make_rsrc(p.gate, p.gate ? rec_bytes(p.m * p.ldg * 2) : 0u);
    return V;
  }
  if (MODE == FVX_GEMM_QKV_ROPE) {
    V.positions = make_rsrc(p.positions, rec_bytes(p.m * 4));
    V.rope = make_rsrc(p.rope, 0x7fffffffu);
  }
  if (MODE == FVX_GEMM_PLAIN || MODE == FVX_GEMM_EULER) {
    V.bias = make_rsrc(p.bias, p.bias ? rec_bytes(N * 2) : 0u);
    V.bf32 = make_rsrc(p.bias_f32, p.bias_f32 ? rec_bytes(N * 4) : 0u);
  }
  if (MODE == FVX_GEMM_EULER) {
    V.xt = make_rsrc(p.xt, rec_bytes(p.m * p.ldx * 4));
    V.prev = make_rsrc(p.rtc_prev, p.rtc_prev ? rec_bytes(p.m * p.ld_prev * 4) : 0u);
    V.cw = make_rsrc(p.rtc_cw, p.rtc_cw ? rec_bytes(p.rtc_period * 4) : 0u);
  }
  if (MODE == FVX_GEMM_PLAIN) {
    V.csum = make_rsrc(p.ln_csum, p.ln_csum ? rec_bytes(N * 4) : 0u);
    const bool gdiv = p.gate_group > 1;
    const int64_t grows = gdiv ? udiv32(p.m + p.gate_group - 1, p.gate_group) : p.m;
    V.gate = make_rsrc(p.gate, p.gate ? rec_bytes(grows * p.ldg * 2) : 0u);
    V.res = make_rsrc(p.residual,
                      p.residual ? rec_bytes((out_row(p, p.m - 1) + 1) * p.ldr * 2) : 0u);
    const int64_t pp = p.pos_period > 0 ? p.pos_period : 1;
    V.pos = make_rsrc(p.pos, p.pos ? rec_bytes(pp * p.ldp * 2) : 0u);
  }
  return V;
}

__device__ __align__(16) const float kZeros8[8] = {};

// the column operands of columns n .. n + 7 (bias_f32: the unlocked rows')
// (LN: the kernel build with the folded LayerNorm, which reads ln_csum)
template <int MODE, bool LN = false>
__device__ __forceinline__ void epi_load_col(const EpiViews& V, int64_t n, bool vec,
                                             EpiIn& in) {
  if (MODE != FVX_GEMM_PLAIN && MODE != FVX_GEMM_EULER) return;
  in.bias = bl_b8(V.bias, (uint32_t)(n * 2), vec);
  bl_f8(V.bf32, (uint32_t)(n * 4), vec, in.f0);
  if (MODE == FVX_GEMM_PLAIN && LN) bl_f8(V.csum, (uint32_t)(n * 4), vec, in.cs);
}

// the row operands of row m, columns n .. n + 7
template <int MODE, bool SP = false>
__device__ __forceinline__ void epi_load_row(const GemmArgs& p, const EpiViews& V, int64_t m,
                                             int64_t n, bool vec, int cnt, EpiIn& in) {
  if (MODE == FVX_GEMM_GEGLU) return;
  if constexpr (SP) {
    // 32-bit offsets: the host keeps m * ldr and m * ldg below 2^31
    in.res = bl_b8(V.res, ((uint32_t)m * (uint32_t)p.ldr + (uint32_t)n) * 2u, vec);
    in.gate = bl_b8(V.gate, ((uint32_t)m * (uint32_t)p.ldg + (uint32_t)n) * 2u, vec);
    return;
  }
  if (MODE == FVX_GEMM_QKV_ROPE) {
    const int hd = p.head_dim;
    const bool rot = n < (int64_t)(p.n_q_heads + 1) * hd;
    const int64_t pos =
        (int32_t)__builtin_amdgcn_raw_buffer_load_b32(V.positions, (uint32_t)(m * 4), 0, 0);
    bl_f8(V.rope, rot ? (uint32_t)((pos * (hd >> 1) + (umod32(n, hd) >> 1)) * 8) : kOOB, vec,
          in.f0);
    return;
  }
  // real-time chunking: the row's position within its chunk and the locked
  // prefix (*rtc_lock: one scalar load, which waits for no vector load)
  const int rr = p.rtc_period > 0 ? (int)umod32(m, p.rtc_period) : 0;
  in.locked = false;
  if (p.rtc_lock) in.locked = rr < *(const __attribute__((address_space(4))) int32_t*)p.rtc_lock;
  if (p.bias_f32_locked) {
    // the row picks its fp32 bias array: a per-lane address, so global loads
    // (a per-lane buffer view would loop over the lanes' views); an absent
    // array or a column past cnt reads kZeros8
    const float* b = in.locked ? p.bias_f32_locked : p.bias_f32;
    if (vec) {
      const f32x4_t* q = (const f32x4_t*)(b ? b + n : kZeros8);
      const f32x4_t x0 = q[0], x1 = q[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        in.f0[e] = x0[e];
        in.f0[4 + e] = x1[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) in.f0[e] = *(b && e < cnt ? b + n + e : kZeros8 + e);
    }
  }
  if (MODE == FVX_GEMM_EULER) {
    bl_f8(V.xt, (uint32_t)((m * p.ldx + n) * 4), vec, in.xt);
    bl_f8(V.prev, (uint32_t)((m * p.ld_prev + n) * 4), vec, in.prev);
    in.cw = bload1f(V.cw, (uint32_t)(rr * 4));
    return;
  }
  in.gate = bl_b8(V.gate, (uint32_t)(((p.gate_group > 1 ? udiv32(m, p.gate_group) : m) * p.ldg + n) * 2),
                  vec);
  in.res = bl_b8(V.res, (uint32_t)((out_row(p, m) * p.ldr + n) * 2), vec);
  in.pos = bl_b8(V.pos,
                 (uint32_t)(((p.pos_period > 1 ? umod32(m, p.pos_period) : 0) * p.ldp + n) * 2),
                 vec);
}

template <int MODE>
__device__ __forceinline__ void epi_load(const GemmArgs& p, const EpiViews& V, int64_t m,
                                         int64_t n, bool vec, int cnt, EpiIn& in) {
  epi_load_col<MODE>(V, n, vec, in);
  epi_load_row<MODE>(p, V, m, n, vec, cnt, in);
}

// v: main accumulators, u: GEGLU up accumulators, r: RMS factor of row m
// (LN build with a folded LayerNorm: its rsqrt(var + eps), with mr =
// mean * r).  want_xo (PLAIN, GEGLU): xo receives the 8 values as stored
// (bf16-rounded unless out_f32), for the hand-over outputs (epi_handoff).
template <int MODE, bool LN = false, bool SP = false>
__device__ __forceinline__ void epi_store(const GemmArgs& p, int64_t m,
                                          int64_t n, bool vec, int cnt,
                                          const float* v, const float* u,
                                          float r, const EpiIn& in,
                                          bool want_xo, float* xo, float mr = 0.f) {
  float x[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = v[e] * r;
  if constexpr (SP && MODE == FVX_GEMM_PLAIN) {
    // the same operations in the same order as below, with 32-bit row
    // offsets (the host keeps m * ldc below 2^31)
    float t[8];
    unpack8(in.bias, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] += t[e] + in.f0[e];
    if (p.act == FVX_ACT_SILU) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = silu(x[e]);
    } else if (p.act == FVX_ACT_GELU_TANH) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = gelu_tanh(x[e]);
    }
    if (p.gate) {
      unpack8(in.gate, t);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= t[e];
    }
    if (p.residual) {
      unpack8(in.res, t);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] += t[e];
    }
    st_b8((bf16_t*)p.c + ((uint32_t)m * (uint32_t)p.ldc + (uint32_t)n), x, vec, cnt);
    if (p.c_frag) st8((bf16_t*)p.c_frag + frag_offset(m, n), pack8(x));
    if (want_xo) unpack8(pack8(x), xo);
    return;
  }
  if (MODE == FVX_GEMM_PLAIN && LN && p.ln_csum)
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = fmaf(-mr, in.cs[e], x[e]);
  if (MODE == FVX_GEMM_GEGLU) {
    if (p.gu_out) {
      // the pre-activations the product is taken from (gate | up)
      float uu[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) uu[e] = u[e] * r;
      bf16_t* g = (bf16_t*)p.gu_out + out_row(p, m) * p.ld_gu + n;
      st_b8(g, x, vec, cnt);
      st_b8(g + p.n, uu, vec, cnt);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = gelu_tanh(x[e]) * (u[e] * r);
    st_b8((bf16_t*)p.c + out_row(p, m) * p.ldc + n, x, vec, cnt);
    if (p.c_frag) st8((bf16_t*)p.c_frag + frag_offset(m, n), pack8(x));
    if (want_xo) unpack8(pack8(x), xo);
    return;
  }
  if (MODE == FVX_GEMM_QKV_ROPE) {
    const int hd = p.head_dim;
    const int64_t qcols = (int64_t)p.n_q_heads * hd;
    if (n < qcols + hd) {
      // pair (2i, 2i+1) = (x_i, x_{i+hd/2}) rotated by (cos, sin)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = x[2 * i], b = x[2 * i + 1];
        const float c = in.f0[2 * i], s = in.f0[2 * i + 1];
        x[2 * i] = a * c - b * s;
        x[2 * i + 1] = b * c + a * s;
      }
      if (n < qcols) {
        st_b8((bf16_t*)p.q_out + m * p.ldq + n, x, vec, cnt);
      } else {
        st_b8((bf16_t*)p.k_out + out_row(p, m) * p.ldk + (n - qcols), x, vec,
              cnt);
        if (p.k_t_out) {
          // the keys transposed as well ([group][head_dim][ld_kt])
          const int64_t b = p.row_group > 0 ? udiv32(m, p.row_group) : 0;
          const int64_t t = p.row_group > 0 ? umod32(m, p.row_group) : m;
          bf16_t* dst = (bf16_t*)p.k_t_out + (b * hd + (n - qcols)) * p.ld_kt + t;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (e < cnt) dst[e * p.ld_kt] = f2bf(x[e]);
        }
      }
    } else if (p.v_transposed) {
      // V^T cache: [group][head_dim][ldv], tokens contiguous
      const int64_t b = p.row_group > 0 ? udiv32(m, p.row_group) : 0;
      const int64_t t = p.row_group > 0 ? umod32(m, p.row_group) : m;
      bf16_t* dst = (bf16_t*)p.v_out + (b * hd + (n - qcols - hd)) * p.ldv + t;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (e < cnt) dst[e * p.ldv] = f2bf(x[e]);
      if (p.v_rows_out)  // the values row-major as well
        st_b8((bf16_t*)p.v_rows_out + out_row(p, m) * p.ld_vr + (n - qcols - hd), x, vec,
              cnt);
    } else {
      st_b8((bf16_t*)p.v_out + out_row(p, m) * p.ldv + (n - qcols - hd), x,
            vec, cnt);
    }
    return;
  }
  float t[8];
  unpack8(in.bias, t);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] += t[e] + in.f0[e];
  if (MODE == FVX_GEMM_EULER) {
    float nx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) nx[e] = in.xt[e] + p.dt * x[e];
    if (p.rtc_cw) {
      // guidance: x_1 = xt - omt * v is the predicted clean chunk; the
      // velocity is corrected by gw * w_r * (prev - x_1)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        nx[e] += in.cw * (in.prev[e] - in.xt[e] + p.rtc_omt * x[e]);
    }
    if (in.locked && p.rtc_prev) {
#pragma unroll
      for (int e = 0; e < 8; ++e) nx[e] = in.prev[e];
    }
    st_f8(p.xt + m * p.ldx + n, nx, vec, cnt);
    if (p.xt_bf16) st_b8((bf16_t*)p.xt_bf16 + m * p.ldxb + n, nx, vec, cnt);
    return;
  }
  if (p.act == FVX_ACT_SILU) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = silu(x[e]);
  } else if (p.act == FVX_ACT_GELU_TANH) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = gelu_tanh(x[e]);
  }
  if (p.gate) {
    unpack8(in.gate, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= t[e];
  }
  if (p.residual) {
    unpack8(in.res, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] += t[e];
  }
  if (p.pos) {
    unpack8(in.pos, t);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] += t[e];
  }
  const int64_t orow = out_row(p, m);
  if (p.out_f32)
    st_f8((float*)p.c + orow * p.ldc + n, x, vec, cnt);
  else
    st_b8((bf16_t*)p.c + orow * p.ldc + n, x, vec, cnt);
  if (p.c_frag) st8((bf16_t*)p.c_frag + frag_offset(m, n), pack8(x));
  if (want_xo) {
    if (p.out_f32) {
#pragma unroll
      for (int e = 0; e < 8; ++e) xo[e] = x[e];
    } else {
      unpack8(pack8(x), xo);
    }
  }
}

// Hand-over outputs of one row's 64-column block, held as 8-column chunks
// n .. n + 7 by 8 consecutive lanes (every lane runs the shuffles; `valid`:
// this lane's chunk exists; the block's first lane stores): the row's sum of
// squares of the stored values (ss_out) and the e4m3 copy with the block's
// E8M0 exponent (a8_out), quantized exactly as quant_fp8x32 quantizes an A
// block.
__device__ __forceinline__ void epi_handoff(const GemmArgs& p, bool valid, int64_t m,
                                            int64_t n, int cnt, const float* xo) {
  const bool lead = ((n >> 3) & 7) == 0;
  if (p.ss_out) {
    float q = 0.f;
    if (valid)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (e < cnt) q += xo[e] * xo[e];
    q += __shfl_xor(q, 1, 64);
    q += __shfl_xor(q, 2, 64);
    q += __shfl_xor(q, 4, 64);
    if (lead && valid) p.ss_out[(n / 64) * p.ss_ld + m] = q;
  }
  if (p.a8_out) {
    const bf16x8 b = pack8(xo);
    uint32_t mx = 0;
    if (valid)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t w = b.w[j] & 0x7fff7fffu;
        const uint32_t lo = 2 * j < cnt ? (w & 0xffffu) : 0u;
        const uint32_t hi = 2 * j + 1 < cnt ? (w >> 16) : 0u;
        mx = lo > mx ? lo : mx;
        mx = hi > mx ? hi : mx;
      }
#pragma unroll
    for (int sh = 1; sh <= 4; sh <<= 1) {
      const uint32_t o = (uint32_t)__shfl_xor((int)mx, sh, 64);
      mx = o > mx ? o : mx;
    }
    const int e = e8m0_for_amax(mx);
    if (valid) {
      const float scale = __uint_as_float((uint32_t)e << 23);
      uint32_t q[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        i16x2_t r = {0, 0};
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(
            r, __builtin_bit_cast(bf16x2_t, b.w[2 * j]), scale, false);
        r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(
            r, __builtin_bit_cast(bf16x2_t, b.w[2 * j + 1]), scale, true);
        q[j] = __builtin_bit_cast(uint32_t, r);
      }
      unsigned char* dst = (unsigned char*)p.a8_out + m * p.a8_out_ld + n;
      if (cnt == 8) {
        *(uint2*)dst = uint2{q[0], q[1]};
      } else {
#pragma unroll
        for (int x = 0; x < 8; ++x)
          if (x < cnt) dst[x] = (unsigned char)(q[x >> 2] >> (8 * (x & 3)));
      }
      if (lead) ((unsigned char*)p.a8_out_scale)[(n / 64) * p.a8_out_sld + m] = (unsigned char)e;
    }
  }
}

// The handed-over sums of squares (`parts`: ss_in) of rows m0 .. m0 + R - 1,
// with every thread of an NT-thread workgroup: thread t loads parts
// t / R, t / R + NT / R, ... of row t % R, all loads in flight (up to 64
// parts per row; more take a loop), and thread t < R receives its row's
// total, added in a fixed order.  A loop over the parts in one thread per row
// waited for a memory round trip per 8 parts before its wave could start
// the K loop.  Every thread must call it (two barriers); sTmp: NT floats
// of LDS.
template <int R, int NT>
__device__ float rows_parts_sum(const GemmArgs& p, const float* parts, int64_t m0, int64_t M,
                                float* sTmp) {
  static_assert(NT % R == 0, "whole rows per thread group");
  constexpr int STEP = NT / R, MAXL = (64 + STEP - 1) / STEP;
  const int tid = threadIdx.x, row = tid % R, j0 = tid / R;
  const int64_t m = m0 + row;
  const bool mv = m < M;
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(parts, rec_bytes((int64_t)p.ss_parts * p.ss_ld * 4));
  float acc = 0.f;
  if (p.ss_parts <= STEP * MAXL) {
    float t[MAXL];
#pragma unroll
    for (int u = 0; u < MAXL; ++u) {
      const int q = j0 + STEP * u;
      t[u] = bload1f(rs, (mv && q < p.ss_parts) ? (uint32_t)(((int64_t)q * p.ss_ld + m) * 4)
                                                : kOOB);
    }
#pragma unroll
    for (int u = 0; u < MAXL; ++u) acc += t[u];
  } else {
    for (int q = j0; q < p.ss_parts; q += STEP)
      acc += bload1f(rs, mv ? (uint32_t)(((int64_t)q * p.ss_ld + m) * 4) : kOOB);
  }
  sTmp[tid] = acc;
  __syncthreads();
  float tot = 0.f;
  if (tid < R)
#pragma unroll
    for (int j = 0; j < STEP; ++j) tot += sTmp[j * R + tid];
  __syncthreads();  // sTmp may be reused
  return tot;
}

// The tile kernel's handed-over row sums of squares (ss_in) of rows m0 ..
// m0 + R - 1, split in two so that no wait sits in front of the K loop:
// issue() puts every load in flight ahead of the first slabs (thread t takes
// parts t / R, t / R + NT / R, ... of row t % R, up to STEP * L parts per row
// in registers), finish() adds them after the K loop, when they have long
// landed; rows with more parts are loaded by finish() itself.  Thread t < R
// receives its row's total, added in a fixed order.  Every thread calls
// finish() (one barrier); sTmp: NT floats of LDS, not to be rewritten before
// the caller's next barrier.
template <int R, int NT>
struct RowParts {
  static_assert(NT % R == 0, "whole rows per thread group");
  static constexpr int STEP = NT / R, L = STEP >= 4 ? (48 + STEP - 1) / STEP : 12;
  float q[L];

  __device__ __forceinline__ bool in_regs(const GemmArgs& p) const {
    return p.ss_parts <= STEP * L;
  }
  // byte offset of part qi of row m (the host keeps the array below 2^31
  // bytes); kOOB (a zero) past the parts or the rows
  __device__ __forceinline__ static uint32_t off(uint32_t row4, uint32_t ld4, int qi, int parts,
                                                 bool mv) {
    const uint32_t o = row4 + (uint32_t)qi * ld4;
    return (mv && qi < parts) ? o : kOOB;
  }
  __device__ __forceinline__ void issue(const GemmArgs& p, int64_t m0, int64_t M) {
    const int tid = threadIdx.x, j0 = tid / R, parts = p.ss_parts;
    const int64_t m = m0 + tid % R;
    const bool mv = m < M && in_regs(p);
    const uint32_t row4 = (uint32_t)m * 4u, ld4 = (uint32_t)p.ss_ld * 4u;
    const __amdgpu_buffer_rsrc_t rq =
        make_rsrc(p.ss_in, rec_bytes((int64_t)parts * p.ss_ld * 4));
#pragma unroll
    for (int u = 0; u < L; ++u) q[u] = bload1f(rq, off(row4, ld4, j0 + STEP * u, parts, mv));
  }
  __device__ __forceinline__ float finish(const GemmArgs& p, int64_t m0, int64_t M,
                                          float* sTmp) {
    const int tid = threadIdx.x, j0 = tid / R, parts = p.ss_parts;
    const int64_t m = m0 + tid % R;
    float aq = 0.f;
    if (in_regs(p)) {
      // the sum starts here, after the K loop, not where the loads were
      // issued (an add hoisted there would wait for them)
#pragma unroll
      for (int u = 0; u < L; ++u) {
        asm volatile("" : "+v"(q[u]));
        aq += q[u];
      }
    } else {
      const uint32_t row4 = (uint32_t)m * 4u, ld4 = (uint32_t)p.ss_ld * 4u;
      const __amdgpu_buffer_rsrc_t rq =
          make_rsrc(p.ss_in, rec_bytes((int64_t)parts * p.ss_ld * 4));
      for (int qi = j0; qi < parts; qi += STEP) aq += bload1f(rq, off(row4, ld4, qi, parts, m < M));
    }
    sTmp[tid] = aq;
    __syncthreads();
    float tq = 0.f;
    if (tid < R)
#pragma unroll
      for (int j = 0; j < STEP; ++j) tq += sTmp[j * R + tid];
    return tq;
  }
};

// Host check: may the chunk epilogue use 16-byte accesses for full chunks?
static bool epi_vec_ok(const GemmArgs& d) {
  auto al = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
  switch (d.mode) {
    case FVX_GEMM_GEGLU:
      return al(d.c) && d.ldc % 8 == 0;
    case FVX_GEMM_QKV_ROPE:
      return d.head_dim % 8 == 0 && al(d.rope) && al(d.q_out) &&
             d.ldq % 8 == 0 && al(d.k_out) && d.ldk % 8 == 0 &&
             (d.v_transposed || (al(d.v_out) && d.ldv % 8 == 0));
    case FVX_GEMM_EULER:
      return al(d.bias) && al(d.bias_f32) && al(d.bias_f32_locked) && al(d.xt) &&
             d.ldx % 4 == 0 && (!d.xt_bf16 || (al(d.xt_bf16) && d.ldxb % 8 == 0)) &&
             (!d.rtc_prev || (al(d.rtc_prev) && d.ld_prev % 4 == 0));
    default:
      return al(d.c) && d.ldc % (d.out_f32 ? 4 : 8) == 0 && al(d.bias) &&
             al(d.bias_f32) && al(d.bias_f32_locked) &&
             (!d.gate || (al(d.gate) && d.ldg % 8 == 0)) &&
             (!d.residual || (al(d.residual) && d.ldr % 8 == 0)) &&
             (!d.pos || (al(d.pos) && d.ldp % 8 == 0));
  }
}

// ---------------------------------------------------------------------------
// Tiled kernel (M > 64)
// ---------------------------------------------------------------------------
// WGM x WGN waves own a BM x BN output tile.  GEGLU tiles hold BN / 2
// columns of each weight, and wave wn holds the gate and the up accumulators
// of the same output columns, so the GeGLU product needs no exchange.  Each
// wave computes a (BM / WGM) x (BN / WGN) sub-tile with
// v_mfma_f32_32x32x16_bf16 (on MI355X it sustains ~1.4x the rate of the
// 16x16x32 form).
//
// K moves through a STAGES-deep LDS ring in 64-wide slabs fetched with
// buffer_load_dwordx4 ... lds: the data goes from L2 straight into LDS (no
// staging registers, no ds_write).  One wave instruction moves 8 rows of 128
// bytes; lane l fetches row l / 8, 16-byte chunk (l % 8) ^ ((row >> 1) & 7),
// so the LDS image is XOR-swizzled and both the fetch and the fragment reads
// (16 consecutive rows of one chunk per 16 lanes) are free of bank
// conflicts.  One barrier per slab: at slab t each wave waits for its own
// loads of slab t, the barrier publishes everyone's and frees the stage of
// slab t - 1, which then receives slab t + STAGES - 1.  Those loads are
// spread evenly between slab t's MFMA groups rather than issued in one burst
// (a burst fills the texture-address queue and holds the MFMAs back).  Loads
// of slabs past the K range use out-of-view offsets (zeros), so the loop has
// no branch around a load.
//
// Per-row sums of squares for the fused RMSNorm are taken from the A
// fragments as they feed the MFMAs.  The epilogue moves each wave's 32-row
// blocks through LDS so that every lane finishes 8 consecutive columns of a
// row with 16-byte accesses.  With splits > 1 the K range is split over
// blockIdx.y and fp32 partials go to the workspace for
// gemm_partial_reduce_kernel.
template <int BM, int BN, int WGM, int WGN, int STAGES, int MODE, bool F8>
struct TileCfg {
  static constexpr int NW = WGM * WGN, NT = 64 * NW;
  static constexpr int NB = MODE == FVX_GEMM_GEGLU ? 2 : 1;
  static constexpr int WM = BM / WGM, WN = BN / WGN;  // WN counts both weights
  static constexpr int FM = WM / 32, FN = WN / 32;
  // bf16: slabs of 64 k, one 128-byte LDS row per A and B row.  F8 (e4m3
  // weights): slabs of 128 k, A rows split into two 128-byte half rows (k
  // 0..63 then 64..127), B rows of 128 fp8 bytes.
  static constexpr int BK = F8 ? 128 : 64;
  static constexpr int AROWS = F8 ? 2 * BM : BM;
  static constexpr int ROWS = AROWS + BN;             // LDS rows per stage
  static constexpr int STAGE_BYTES = ROWS * 128;
  static constexpr int LPW = ROWS / (8 * NW);         // loads per wave per slab
  static constexpr int WNO = WN / NB;                 // output columns per wave
  static constexpr int ELD = WN + 4;                  // epilogue scratch stride
  static constexpr int EPI_BYTES = NW * 32 * ELD * 4;
  static constexpr int LDS_BYTES =
      STAGES * STAGE_BYTES > EPI_BYTES ? STAGES * STAGE_BYTES : EPI_BYTES;
  static_assert(BM % (32 * WGM) == 0 && BN % (32 * NB * WGN) == 0, "tile");
  static_assert(ROWS % (8 * NW) == 0 && STAGES >= 2, "loader");
  static_assert(NT >= BM, "row sums");
};

// F8 && A16 (W8A16): the F8 LDS layout (128-k slabs, e4m3 weight rows), but
// A stays bf16 and each 8 weight bytes become one bf16 MFMA fragment.
// XF: the optional paths compiled in (bit 0: handed-over row sums of
// squares read, ss_in; bit 1: hand-over outputs, ss_out / a8_out; bit 2,
// PLAIN, not with bit 0: the folded LayerNorm, ln_csum, on sums of A's
// values and squares taken in the K loop; bit 3, PLAIN: the plain epilogue,
// see plain_epilogue_ok).  GEMMs without a path run a build without its
// code: compiled in but not taken, the row-sum paths cost such 20 us
// launches ~0.7 us.  bf16 bit-0 builds have no K-loop sum of squares: the
// host picks them only for rownorm GEMMs with ss_in (fp8-weight tiles keep
// one build, XF = 3, with both row-sum paths).
template <int BM, int BN, int WGM, int WGN, int STAGES, int MODE, bool F8, bool A16,
          int XF = 3>
__global__ __launch_bounds__(64 * WGM * WGN, 1) void gemm_tile_kernel(
    GemmArgs p, int m_tiles, int n_tiles, int splits, int64_t kchunk,
    int vec_ok) {
  static_assert(!A16 || F8, "W8A16 is an fp8-weight variant");
  constexpr bool RPX = (XF & 1) != 0, HOX = (XF & 2) != 0;
  constexpr bool SUMX = !RPX || F8;  // builds with the K-loop sum of squares
  // ... and of values, for the folded LayerNorm
  constexpr bool LN = (XF & 4) != 0 && MODE == FVX_GEMM_PLAIN && !F8 && !RPX;
  // the plain epilogue (32-bit row offsets, no unused features)
  constexpr bool SP = (XF & 8) != 0 && MODE == FVX_GEMM_PLAIN && !F8;
  typedef TileCfg<BM, BN, WGM, WGN, STAGES, MODE, F8> C;
  constexpr int NB = C::NB, WM = C::WM, WN = C::WN, FM = C::FM, FN = C::FN;
  constexpr int LPW = C::LPW, WNO = C::WNO, ELD = C::ELD, BK = C::BK;
  constexpr int AROWS = C::AROWS;
  __shared__ __align__(16) char smem[C::LDS_BYTES];
  __shared__ float sRow[BM], sSum[BM], sTmp[64 * WGM * WGN];
  // per-wave partial row sums (bf16, K-loop sums: squares, values)
  __shared__ float sPart[LN ? 2 : 1][F8 || !SUMX ? 1 : WGN][F8 || !SUMX ? 1 : BM];
  warm_kernargs<sizeof(GemmArgs) + 24>();

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave % WGN;

  // XCD-aware order over (split, tile): consecutive ids (the M tiles of one
  // weight panel, m fastest, then the panels of one K range) land on one
  // XCD and share its L2 -- with splits, an XCD works on one K range and
  // reads only that slice of A and B.
  const int nblk = m_tiles * n_tiles;
  const int lid = xcd_remap(blockIdx.x + nblk * blockIdx.y, nblk * splits);
  const int bid = lid % nblk, split = lid / nblk;
  const int m_tile = bid % m_tiles, n_tile = bid / m_tiles;
  const int64_t M = p.m, N = p.n, K = p.k;
  const int64_t m0 = (int64_t)m_tile * BM, n0 = (int64_t)n_tile * (BN / NB);
  const int64_t kb = (int64_t)split * kchunk;
  const int64_t ke = (kb + kchunk < K) ? kb + kchunk : K;
  const int nk = (int)((ke - kb + BK - 1) / BK);

  // Buffer views of the tile's A rows and B rows: rows past M / N read zero.
  // Grouped A rows (a_row_group > 0): a view of the whole of A, each row's
  // offset from its group, rows past M kept out by kmax.
  const int64_t a_rows = (M - m0 < BM) ? M - m0 : BM;
  const int64_t b_rows = (N - n0 < BN / NB) ? N - n0 : BN / NB;
  const uint32_t lda2 = (uint32_t)p.lda * 2, ldb2 = (uint32_t)p.ldb * (F8 ? 1 : 2);
  const bool agrp = p.a_row_group > 0;
  auto a_phys = [&](int64_t m) -> int64_t {  // physical row of product row m
    const uint32_t q = udiv32(m, p.a_row_group);
    return (int64_t)q * p.a_row_group_stride + ((uint32_t)m - q * (uint32_t)p.a_row_group);
  };
  const i32x4_t rA =
      agrp ? make_rsrc4((const bf16_t*)p.a, (uint32_t)((a_phys(M - 1) + 1) * lda2))
           : make_rsrc4((const bf16_t*)p.a + m0 * p.lda, (uint32_t)(a_rows * lda2));
  const i32x4_t rB0 =
      make_rsrc4((const char*)p.b + n0 * ldb2, (uint32_t)(b_rows * ldb2));
  const i32x4_t rB1 =
      make_rsrc4((const char*)(NB == 2 ? p.b2 : p.b) + n0 * ldb2,
                 (uint32_t)(b_rows * ldb2));

  // Load i of this wave fills LDS rows R0 = (wave LPW + i) 8 .. + 7 of a
  // stage: A rows (F8: half rows) first, then BN / NB rows of each weight.
  // Either way a slab advances 128 bytes along a B row and 2 BK along an A
  // row; a 16-byte chunk spans 8 k of A and 8 (F8: 16) k of B.
  const int lr = lane >> 3, lc = lane & 7;
  uint32_t voff[LPW];
  int kmax[LPW];  // slab t of load i is in range iff BK t < kmax[i]
  bool isa[LPW];
  i32x4_t rsel[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int R0 = (wave * LPW + i) * 8, R = R0 + lr;
    const int gc = lc ^ ((R >> 1) & 7);
    isa[i] = R0 < AROWS;
    if (R0 < AROWS) {
      const int hk = R0 / BM;  // F8: which 64-k half of the slab
      const int ar = R0 % BM + lr;
      rsel[i] = rA;
      voff[i] = (uint32_t)(agrp ? a_phys(m0 + ar) : ar) * lda2 +
                (uint32_t)(kb + hk * 64 + gc * 8) * 2;
      kmax[i] = (agrp && m0 + ar >= M) ? 0 : (int)(ke - kb) - hk * 64 - gc * 8;
    } else {
      // 8-row groups never straddle the two weights' regions (BN / NB % 8 == 0)
      const int br0 = R0 - AROWS;
      const int kc = F8 ? 16 : 8;
      rsel[i] = br0 < BN / NB ? rB0 : rB1;
      voff[i] = (uint32_t)(br0 % (BN / NB) + lr) * ldb2 +
                (uint32_t)(kb + gc * kc) * (F8 ? 1 : 2);
      kmax[i] = (int)(ke - kb) - gc * kc;
    }
  }
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem) + wave * LPW * 1024);
  auto issue1 = [&](int t, int stage, int i) {
    load_lds16(rsel[i], lds0 + stage * C::STAGE_BYTES + i * 1024,
               BK * t < kmax[i] ? voff[i] + (uint32_t)t * (isa[i] ? 2 * BK : 128) : kOOB);
  };
  auto issue = [&](int t, int stage) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) issue1(t, stage, i);
  };
  // slab tn's loads spread over the G MFMA groups of a slab: load i goes
  // after group i G / LPW
  auto issue_group = [&](int g, int G, int tn, int tst) {
#pragma unroll
    for (int i = 0; i < LPW; ++i)
      if ((i * G) / LPW == g) issue1(tn, tst, i);
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  float ss[FM], sv[FM];
#pragma unroll
  for (int i = 0; i < FM; ++i) ss[i] = sv[i] = 0.f;
  // the fused RMSNorm sums A's squares in the K loop unless they are handed
  // over (ss_in)
  const bool sum_a = SUMX && p.rownorm && !p.ss_in;
  const int wn_u = __builtin_amdgcn_readfirstlane(wn);

  // LDS row of B fragment j of this wave (GEGLU: gate blocks, then up)
  auto brow = [&](int j) {
    if (NB == 2)
      return j < FN / 2 ? AROWS + wn * (WN / 2) + 32 * j
                        : AROWS + BN / 2 + wn * (WN / 2) + 32 * (j - FN / 2);
    return AROWS + wn * WN + 32 * j;
  };
  // rows of a fragment are (multiple of 32) + lane % 32: swizzle (lane >> 1) & 7
  const int sw = (lane >> 1) & 7, fr = lane & 31, hk = lane >> 5;
  auto compute = [&](int stage, auto with_ss, int tn, int tst) {
    constexpr bool SS = decltype(with_ss)::value;
    const char* s = smem + stage * C::STAGE_BYTES;
    if (F8) {
      // two 64-k steps; lane (fr, hk) takes k = 64 ks + 32 hk .. + 31: A as
      // four bf16 chunks of half row ks (quantized here with one scale per
      // row and step), B as two fp8 chunks
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        i32x8_t aq[FM], bq[FN];
        int ae[FM];
        bf16x8 av[FM][4], bw[FN][4];
#pragma unroll
        for (int i = 0; i < FM; ++i) {
          const char* row = s + (ks * BM + wm * WM + 32 * i + fr) * 128;
#pragma unroll
          for (int c = 0; c < 4; ++c)
            av[i][c] = *(const bf16x8*)(row + (((4 * hk + c) ^ sw) * 16));
          if (SS)
#pragma unroll
            for (int c = 0; c < 4; ++c) ss[i] += sumsq8(av[i][c]);
          if (!A16) aq[i] = quant_fp8x32<32, 0>(av[i], &ae[i]);  // (row, 64-k step) scale
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const char* row = s + (brow(j) + fr) * 128;
          const bf16x8 b0 = *(const bf16x8*)(row + (((4 * ks + 2 * hk) ^ sw) * 16));
          const bf16x8 b1 = *(const bf16x8*)(row + (((4 * ks + 2 * hk + 1) ^ sw) * 16));
          if (A16) {
            // k = 64 ks + 32 hk + 8 c + j: bytes 8c .. of b0 (c < 2), b1
            bw[j][0] = e4m3x8_to_bf16(b0.w[0], b0.w[1]);
            bw[j][1] = e4m3x8_to_bf16(b0.w[2], b0.w[3]);
            bw[j][2] = e4m3x8_to_bf16(b1.w[0], b1.w[1]);
            bw[j][3] = e4m3x8_to_bf16(b1.w[2], b1.w[3]);
          } else {
#pragma unroll
            for (int x = 0; x < 4; ++x) {
              bq[j][x] = (int)b0.w[x];
              bq[j][4 + x] = (int)b1.w[x];
            }
          }
        }
        if (A16) {
          // lane (fr, hk) holds A row / B column fr at k = 64 ks + 32 hk +
          // 8 c + j: MFMA c sums those 16 k (hk = 0, 1) of the 64
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
              for (int j = 0; j < FN; ++j)
                acc[i][j] = mfma32x32x16(av[i][c], bw[j][c], acc[i][j]);
        } else {
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
              acc[i][j] = mfma32x32x64_f8(aq[i], ae[i], bq[j], 127, acc[i][j]);
        }
        issue_group(ks, 2, tn, tst);
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    }
    // k step ks + 1's fragments are read before step ks's MFMAs are issued
    // (two register sets), so each step's LDS latency hides under the
    // previous step's MFMAs
    bf16x8 af[2][FM], bfr[2][FN];
    auto rd = [&](int ks, int b) {
      const int cpos = ((2 * ks + hk) ^ sw) * 16;
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[b][i] = *(const bf16x8*)(s + (wm * WM + 32 * i + fr) * 128 + cpos);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[b][j] = *(const bf16x8*)(s + (brow(j) + fr) * 128 + cpos);
    };
    rd(0, 0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int b = ks & 1;
      if (ks < 3) rd(ks + 1, b ^ 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        // the waves of a row band share the sums: wave wn takes the steps
        // ks = wn (mod WGN)
        if (SS && (ks % WGN) == wn_u) {
          ss[i] += sumsq8(af[b][i]);
          if (LN) sv[i] += sum8(af[b][i]);
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma32x32x16(af[b][i], bfr[b][j], acc[i][j]);
        issue_group(ks * FM + i, 4 * FM, tn, tst);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  // handed-over row sums of squares: in flight ahead of the first slabs,
  // added after the K loop
  RowParts<BM, 64 * WGM * WGN> rparts;
  const bool rp_on = RPX && p.rownorm && p.ss_in;
  if constexpr (RPX)
    if (rp_on) rparts.issue(p, m0, M);
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue(s, s);
  auto k_loop = [&](auto with_ss) {
    for (int t0 = 0; t0 < nk; t0 += STAGES) {
#pragma unroll
      for (int s = 0; s < STAGES; ++s) {
        const int t = t0 + s;
        if (t >= nk) break;
        wait_vmcnt<LPW * (STAGES - 2)>();  // this wave's loads of slab t landed
        __syncthreads();                   // everyone's, and slab t-1 is consumed
        compute(s, with_ss, t + STAGES - 1, (s + STAGES - 1) % STAGES);
      }
    }
  };
  if constexpr (SUMX) {
    if (sum_a)
      k_loop(BoolC<true>{});
    else
      k_loop(BoolC<false>{});
  } else {
    k_loop(BoolC<false>{});
  }
  // Loads past the end may still be in flight into the ring: drain them
  // before the ring becomes epilogue scratch.
  wait_vmcnt<0>();
  float ss_pre = 0.f;
  if constexpr (RPX)
    if (rp_on) ss_pre = rparts.finish(p, m0, M, sTmp);

  // Row sums of squares (and of values): lanes l and l ^ 32 hold the two
  // k halves of row l % 32 of block i; bf16: wave wn summed the k steps
  // ks = wn (mod WGN), added across the waves in wn order (fp8: waves with
  // wn > 0 computed the same sums).
  if (!sum_a) {
    if (tid < BM) sRow[tid] = ss_pre;
  } else if constexpr (F8) {
    if (wn == 0)
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const float s2 = ss[i] + __shfl_xor(ss[i], 32, 64);
        if (lane < 32) sRow[wm * WM + 32 * i + lane] = s2;
      }
  } else if constexpr (SUMX) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const float s2 = ss[i] + __shfl_xor(ss[i], 32, 64);
      const float v2 = sv[i] + __shfl_xor(sv[i], 32, 64);
      if (lane < 32) {
        sPart[0][wn][wm * WM + 32 * i + lane] = s2;
        if constexpr (LN) sPart[1][wn][wm * WM + 32 * i + lane] = v2;
      }
    }
    __syncthreads();
    if (tid < BM) {
      float a = 0.f, c = 0.f;
#pragma unroll
      for (int w = 0; w < WGN; ++w) {
        a += sPart[0][w][tid];
        if constexpr (LN) c += sPart[1][w][tid];
      }
      sRow[tid] = a;
      if constexpr (LN) sSum[tid] = c;
    }
  }
  __syncthreads();

  float* ws = (float*)((char*)p.workspace + kCounterBytes);
  const int64_t plane = (int64_t)splits * M * N;
  // (handed-over sums are complete: split 0 carries them)
  if (splits > 1 && n_tile == 0 && tid < BM && m0 + tid < M)
    ws[NB * plane + (int64_t)split * M + m0 + tid] = (p.ss_in && split) ? 0.f : sRow[tid];

  // Epilogue: each 32-row block of the wave's sub-tile goes through the
  // wave's own LDS scratch [32][ELD] fp32 (GEGLU: gate columns, then up).
  // Lane item q = lane + 64 e covers row q / CH, columns 8 (q % CH) ..: the
  // same column chunk in every item (64 % CH == 0), so the column operands
  // and the fp8 weight scales are read once per lane.
  float* scr = (float*)smem + wave * 32 * ELD;
  constexpr int CH = WNO / 8;               // 8-column chunks per row
  constexpr int ITEMS = 32 * CH / 64;       // chunks per lane per block
  constexpr int EB = ITEMS < 4 ? ITEMS : 4; // chunks whose loads fly together
  constexpr int RS = 64 / CH;               // row step between a lane's items
  static_assert(64 % CH == 0, "one column chunk per lane");
  const int ch = lane % CH, row0 = lane / CH;
  const int64_t nn = n0 + wn * WNO + 8 * ch;
  const int cnt = (int)(N - nn < 8 ? N - nn : 8);
  // hand-over outputs: the 8 lanes of a row (CH == 8: one 64-column block
  // per wave); the shuffles run in every lane
  constexpr bool HO = MODE == FVX_GEMM_PLAIN && WNO == 64;
  const bool ho = HOX && HO && (p.ss_out || p.a8_out) && splits == 1;
  const EpiViews V = epi_views<MODE, SP>(p);
  // VA: every operand is 16B-aligned and N % 8 == 0 (uniform), so every
  // chunk with columns left holds 8 and moves as whole vectors
  auto epilogue = [&](auto va) {
    const bool vec = decltype(va)::value || (vec_ok && cnt == 8);
    EpiIn col;
    if (splits == 1) epi_load_col<MODE, LN>(V, nn, vec, col);
    float w0[8], w1[8];  // fp8: per-output-channel weight scales
    if (F8) {
      bl_f8(make_rsrc(p.b_scale, rec_bytes(N * 4)), (uint32_t)(nn * 4), vec, w0);
      bl_f8(make_rsrc(NB == 2 ? p.b2_scale : p.b_scale, rec_bytes(N * 4)), (uint32_t)(nn * 4),
            vec, w1);
    }
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          scr[(8 * (r >> 2) + 4 * hk + (r & 3)) * ELD + 32 * j + fr] = acc[i][j][r];
      const int64_t rb = m0 + wm * WM + 32 * i + row0;
#pragma unroll
      for (int e0 = 0; e0 < ITEMS; e0 += EB) {
        EpiIn in[EB];
        if (splits == 1) {
#pragma unroll
          for (int e = 0; e < EB; ++e) {
            in[e] = col;
            epi_load_row<MODE, SP>(p, V, rb + RS * (e0 + e), nn, vec, cnt, in[e]);
          }
        }
#pragma unroll
        for (int e = 0; e < EB; ++e) {
          const int row = row0 + RS * (e0 + e);
          const int64_t m = rb + RS * (e0 + e);
          float xo[8];
          if (m < M && cnt > 0) {
            float v[8], u[8];
            const float* sv = scr + row * ELD + 8 * ch;
#pragma unroll
            for (int x = 0; x < 8; ++x) {
              v[x] = sv[x];
              u[x] = NB == 2 ? sv[WNO + x] : 0.f;
            }
            if (F8) {
#pragma unroll
              for (int x = 0; x < 8; ++x) {
                v[x] *= w0[x];
                u[x] *= w1[x];
              }
            }
            if (splits > 1) {
#pragma unroll
              for (int b = 0; b < NB; ++b) {
                float* dst = ws + b * plane + ((int64_t)split * M + m) * N + nn;
#pragma unroll
                for (int x = 0; x < 8; ++x)
                  if (x < cnt) dst[x] = b ? u[x] : v[x];
              }
            } else {
              float r = 1.f, mr = 0.f;
              if (p.rownorm) {
                if (LN && p.ln_csum) {
                  // LayerNorm: mean and variance from the handed-over sums
                  const float mean = sSum[m - m0] / (float)K;
                  const float var = fmaxf(sRow[m - m0] / (float)K - mean * mean, 0.f);
                  r = rsqrtf(var + p.rownorm_eps);
                  mr = mean * r;
                } else {
                  r = rsqrtf(sRow[m - m0] / (float)K + p.rownorm_eps);
                }
              }
              epi_store<MODE, LN, SP>(p, m, nn, vec, cnt, v, u, r, in[e], ho, xo, mr);
            }
          }
          if (ho) epi_handoff(p, m < M && cnt > 0, m, nn, cnt, xo);
        }
      }
    }
  };
  if (vec_ok && (N & 7) == 0)
    epilogue(BoolC<true>{});
  else
    epilogue(BoolC<false>{});
}

// ---------------------------------------------------------------------------
// gemm_wide_kernel: large-M GEMMs (the prefix gate/up projection at every
// batch; the other prefix and SigLIP GEMMs once a batch gives them >= 128
// such tiles).  A 256 x 256 tile (GEGLU: 256 rows x 128 columns of each
// weight) for NWV waves.  With 4, wave (wm, wn) owns rows 128 wm .. + 127
// and columns 128 wn .. + 127 (GEGLU: 64 wn .. + 63 of both weights), 16
// 32x32 accumulators, so 8 fragment reads from LDS feed 16 MFMAs; with 8
// (two waves per SIMD, the build's choice) rows 64 wm .. + 63 of the same
// columns, 8 accumulators, 6 reads for 8 MFMAs -- more LDS bytes per MFMA,
// but the second wave on a SIMD issues its LDS reads while the first waits.
// Each wave loads one 512 / NWV-row band of every slab by LDS DMA (the first
// half of the waves the A rows, the others the B rows: GEGLU the gate, then
// the up rows): per load one
// VGPR offset, the slab advance in the scalar offset, rows past the operand
// out of the buffer view (zeros).  K moves in 64-wide slabs through a
// 2-stage ring; K % 64 == 0, one pass (no split).  The slab's 16 (8 waves:
// 8) loads per wave are spread between MFMA groups, two after each group
// (issued in one burst they fill the texture-address queue and hold the
// MFMAs back): the first half of slab t + 2's during the last k step of
// slab t, the second half during the first k step of slab t + 1.  The one barrier per slab sits before the
// last k step: it publishes slab t + 1 and frees slab t's stage, and the
// first fragments of slab t + 1 are read while that step's MFMAs run.
// LDS rows are 128 bytes with the 16-byte chunk index XOR (row >> 1) & 7,
// as in gemm_tile_kernel.  The epilogue is gemm_tile_kernel's (epi_load /
// epi_store per 8-column chunk), including ss_out for PLAIN.
// ---------------------------------------------------------------------------
constexpr int kGwBM = 256, kGwBN = 256;  // rows, columns (GEGLU: 2 x 128)
#ifndef FVX_WIDE_EB
#define FVX_WIDE_EB 4
#endif
constexpr int kGwStage = 512 * 128;
constexpr int kGwELD = 128 + 4;          // epilogue scratch stride (floats)
constexpr int kGhP = 64 + 8;             // GeGLU product scratch stride (bf16)
// waves of the bf16 wide kernel: 8 (prefix GeGLU 119 -> 110 us, chunk
// 16.8 -> 16.4 ms against 4)
template <int MODE>
constexpr int wide_waves() { return 8; }

// NWV waves: 4 (one per SIMD; wave (wm, wn) of 2 x 2 owns 128 rows) or 8
// (two per SIMD, 4 x 2 waves of 64 rows: half the accumulators per wave, so
// that a second wave on each SIMD hides the LDS reads of the first -- one
// wave per SIMD gets ~1 KB per 40-50 cycles out of the LDS, two ~1 KB per
// 25).
template <int NWV>
constexpr int wide_lds_bytes() {
  return 2 * kGwStage > NWV * 32 * kGwELD * 4 ? 2 * kGwStage : NWV * 32 * kGwELD * 4;
}

template <int MODE, bool SUM_A, int NWV>  // SUM_A: the fused RMSNorm sums A's squares here
__global__ __launch_bounds__(64 * NWV, 1) void gemm_wide_kernel(GemmArgs p, int m_tiles,
                                                                int n_tiles, int vec_ok,
                                                                int splits, int kchunk) {
  constexpr bool GG = MODE == FVX_GEMM_GEGLU;
  constexpr int WNO = GG ? 64 : 128;  // output columns per wave
  constexpr int WM = NWV == 8 ? 64 : 128, RB = WM / 32;  // rows, row blocks per wave
  constexpr int BAND = 512 / NWV, LW = BAND / 8;          // DMA band rows, loads per slab
  static_assert(NWV == 4 || NWV == 8, "4 or 8 waves");
  __shared__ __align__(16) char smem[wide_lds_bytes<NWV>()];
  __shared__ float sRow[kGwBM], sTmp[64 * NWV];
  warm_kernargs<sizeof(GemmArgs) + 24>();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-aware order over (split, tile): consecutive ids (the M tiles of one
  // weight panel, then the panels of one K range) share an XCD's L2
  const int nblk = m_tiles * n_tiles;
  const int lid = xcd_remap(blockIdx.x, nblk * splits);
  const int bid = lid % nblk, split = lid / nblk;
  const int m_tile = bid % m_tiles, n_tile = bid / m_tiles;
  const int64_t M = p.m, N = p.n, K = p.k;
  const int64_t m0 = (int64_t)m_tile * kGwBM, n0 = (int64_t)n_tile * (GG ? 128 : 256);
  // K range [kb, kb + 64 nk) (splits > 1: PLAIN without rownorm, fp32
  // partials for gemm_partial_reduce_kernel)
  const int64_t kb = (int64_t)split * kchunk;
  const int nk = (int)(((kb + kchunk < K ? kb + kchunk : K) - kb) / 64);

  // this wave's band: BAND rows of A (the first NWV / 2 waves) or of B (the
  // others; GEGLU: the gate rows, then the up rows)
  const int bw = wave - NWV / 2;
  const bool isa = bw < 0;
  const int64_t r0 = isa ? m0 + BAND * wave
                         : n0 + BAND * (GG ? bw % (NWV / 4) : bw);
  const int64_t rlim = (isa ? M : N) - r0;
  const int64_t nrows = rlim <= 0 ? 0 : (rlim < BAND ? rlim : BAND);
  const uint32_t ld2 = (uint32_t)(isa ? p.lda : p.ldb) * 2;
  const bf16_t* band = isa ? (const bf16_t*)p.a + r0 * p.lda + kb
                           : (const bf16_t*)((GG && bw >= NWV / 4) ? p.b2 : p.b) + r0 * p.ldb + kb;
  const i32x4_t rs = make_rsrc4(band, (uint32_t)(nrows * ld2));
  // load i: LDS rows BAND wave + 8 i + (lane >> 3), slot lane & 7 holds
  // global chunk slot ^ (((8 i + (lane >> 3)) >> 1) & 7)
  const int lr = lane >> 3, lc = lane & 7;
  const uint32_t vo0 = (uint32_t)lr * ld2 + 16u * (uint32_t)(lc ^ (lr >> 1));
  const uint32_t vo1 = (uint32_t)lr * ld2 + 16u * (uint32_t)(lc ^ (lr >> 1) ^ 4);
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem) + wave * BAND * 128);
  // load i (8 rows of the band) of slab t into ring stage `stage`
  auto issue1 = [&](int t, int stage, int i) {
    load_lds16_so(rs, lds0 + stage * kGwStage + i * 1024,
                  ((i & 1) ? vo1 : vo0) + (uint32_t)(8 * i) * ld2, (uint32_t)t * 128u);
  };
  auto issue = [&](int t, int stage) {
#pragma unroll
    for (int i = 0; i < LW; ++i) issue1(t, stage, i);
  };

  f32x16_t acc[RB][4];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  float ss[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) ss[i] = 0.f;
  const int sw = (lane >> 1) & 7, fr = lane & 31, hk = lane >> 5;
  // LDS row of B fragment j of this wave (GEGLU: gate blocks, then up)
  auto brow = [&](int j) {
    return GG ? 256 + (j >> 1) * 128 + wn * 64 + 32 * (j & 1) : 256 + wn * 128 + 32 * j;
  };
  issue(0, 0);
  // handed-over row sums: thread t < 256 takes row m0 + t (waits with slab 0)
  float ss_pre = 0.f;
  if (!SUM_A && p.rownorm) ss_pre = rows_parts_sum<kGwBM, 64 * NWV>(p, p.ss_in, m0, M, sTmp);
  bf16x8 af[2][RB], bfr[2][4];
  auto rd = [&](int stage, int ks, int b) {
    const char* s = smem + stage * kGwStage;
    const int cpos = ((2 * ks + hk) ^ sw) * 16;
#pragma unroll
    for (int i = 0; i < RB; ++i)
      af[b][i] = *(const bf16x8*)(s + (wm * WM + 32 * i + fr) * 128 + cpos);
#pragma unroll
    for (int j = 0; j < 4; ++j) bfr[b][j] = *(const bf16x8*)(s + (brow(j) + fr) * 128 + cpos);
  };
  // 32-row blocks of this wave that hold rows < M (the last M tile of the
  // prefix, 816 = 3 x 256 + 48 rows, has 2 of 8): the others skip their
  // MFMAs, so that tile finishes early and its CU takes the next one
  bool blk_ok[RB];
#pragma unroll
  for (int i = 0; i < RB; ++i) blk_ok[i] = m0 + wm * WM + 32 * i < M;
  for (int x = 0; x < LW / 2; ++x) issue1(nk > 1 ? 1 : 0, 1, x);
  wait_vmcnt<LW / 2>();
  __syncthreads();
  rd(0, 0, 0);
  for (int t = 0; t < nk; ++t) {
    const int st = t & 1;
    const int t1 = t + 1 < nk ? t + 1 : nk - 1, t2 = t + 2 < nk ? t + 2 : nk - 1;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int b = ks & 1;
      if (ks < 3) {
        rd(st, ks + 1, b ^ 1);
      } else {
        wait_vmcnt<0>();   // slab t + 1 landed (this wave's loads)
        __syncthreads();   // everyone's, and every read of slab t is done
        rd(st ^ 1, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      // the wave's LW loads of a slab: the second half of slab t + 1's in
      // k step 0, the first half of slab t + 2's in k step 3 (after the
      // barrier that frees its stage), LW / (2 RB) after each MFMA group
      constexpr int PG = LW / (2 * RB);
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        if (SUM_A) ss[i] += sumsq8(af[b][i]);
        if (blk_ok[i])
#pragma unroll
          for (int j = 0; j < 4; ++j) acc[i][j] = mfma32x32x16(af[b][i], bfr[b][j], acc[i][j]);
#pragma unroll
        for (int g = 0; g < PG; ++g) {
          if (ks == 0)
            issue1(t1, st ^ 1, LW / 2 + PG * i + g);
          else if (ks == 3)
            issue1(t2, st, PG * i + g);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  wait_vmcnt<0>();

  // row sums of squares: lanes l and l ^ 32 hold the two k halves of row
  // l % 32 of block i
  if (!SUM_A) {
    if (tid < kGwBM) sRow[tid] = ss_pre;
  } else if (wn == 0) {
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const float s2 = ss[i] + __shfl_xor(ss[i], 32, 64);
      if (lane < 32) sRow[wm * WM + 32 * i + lane] = s2;
    }
  }
  __syncthreads();  // also: every wave is done with the ring
  // each row's RMS factor, once (the epilogue reads it per row)
  if (p.rownorm) {
    if (tid < kGwBM) sRow[tid] = rsqrtf(sRow[tid] / (float)K + p.rownorm_eps);
    __syncthreads();
  }

  // each 32-row block through the wave's LDS scratch [32][kGwELD] (GEGLU:
  // gate columns 0..63, up 64..127); lane item q = lane + 64 e: row q / CH,
  // 8 columns 8 (q % CH) with CH = WNO / 8 chunks per row, the lane's own
  // column chunk in every item (EB items' epilogue inputs in flight;
  // PLAIN's, with 8 waves, one at a time and column operands included:
  // more do not fit the 256 registers of two waves per SIMD)
  constexpr int EB0 = NWV == 8 && MODE == FVX_GEMM_PLAIN ? 1 : FVX_WIDE_EB;
  constexpr int CH = WNO / 8, ITEMS = 32 * CH / 64, EB = EB0 < ITEMS ? EB0 : ITEMS;
  constexpr int RS = 64 / CH;  // row step between a lane's items
  static_assert(64 % CH == 0, "one column chunk per lane");
  float* scr = (float*)smem + wave * 32 * kGwELD;
  const int ch = lane % CH, row0 = lane / CH;
  const int64_t nn = n0 + wn * WNO + 8 * ch;
  const int cnt = (int)(N - nn < 8 ? N - nn : 8);
  const bool ho = (MODE == FVX_GEMM_PLAIN || GG) && (p.ss_out || p.a8_out);
  const EpiViews V = epi_views<MODE>(p);
  // block i of the accumulators -> scratch (compile-time indices, so the
  // accumulators stay in registers); the item loops below are real loops,
  // which keeps the epilogue code small enough for the kernel arguments to
  // stay in SGPRs
  auto to_scr = [&](auto ic) {
    constexpr int i = decltype(ic)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        scr[(8 * (r >> 2) + 4 * hk + (r & 3)) * kGwELD + 32 * j + fr] = acc[i][j][r];
  };
  // with N % 8 == 0 every chunk with columns left holds 8: vec is uniform
  const bool vec = vec_ok && (cnt == 8 || (N & 7) == 0);
  // GeGLU without hand-overs, whole vectors: gelu(gate) * up straight from
  // the accumulators (gate block j and up block j + 2 share the lane layout:
  // lane (fr, hk), register q holds row 8 (q >> 2) + 4 hk + (q & 3), column
  // 32 j + fr), so only the bf16 products pass through the scratch, a
  // quarter of the fp32 gate | up rows' bytes
  if (GG && !ho && vec_ok && (N & 7) == 0 && splits == 1) {
    bf16_t* sh = (bf16_t*)scr;  // [32][kGhP] bf16
    auto gg_to_scr = [&](auto ic) {
      constexpr int i = decltype(ic)::value;
      float r[16];
#pragma unroll
      for (int q = 0; q < 16; ++q)
        r[q] = p.rownorm ? sRow[wm * WM + 32 * i + 8 * (q >> 2) + 4 * hk + (q & 3)] : 1.f;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const float g = acc[i][jj][q] * r[q], u = acc[i][jj + 2][q] * r[q];
          sh[(8 * (q >> 2) + 4 * hk + (q & 3)) * kGhP + 32 * jj + fr] = f2bf(gelu_tanh(g) * u);
        }
    };
#pragma unroll 1
    for (int i = 0; i < RB; ++i) {
      switch (i) {
        case 0: gg_to_scr(IntC<0>{}); break;
        case 1: gg_to_scr(IntC<1>{}); break;
        case 2: gg_to_scr(IntC<2 % RB>{}); break;
        default: gg_to_scr(IntC<3 % RB>{}); break;
      }
      const int64_t rb = m0 + wm * WM + 32 * i + row0;
#pragma unroll
      for (int e = 0; e < ITEMS; ++e) {
        const int64_t m = rb + RS * e;
        const bf16x8 h = ld8(sh + (row0 + RS * e) * kGhP + 8 * ch);
        if (m < M && cnt > 0) {
          st8((bf16_t*)p.c + out_row(p, m) * p.ldc + nn, h);
          if (p.c_frag) st8((bf16_t*)p.c_frag + frag_offset(m, nn), h);
        }
      }
    }
    return;
  }
  {
#pragma unroll 1
    for (int i = 0; i < RB; ++i) {
      switch (i) {
        case 0: to_scr(IntC<0>{}); break;
        case 1: to_scr(IntC<1>{}); break;
        case 2: to_scr(IntC<2 % RB>{}); break;
        default: to_scr(IntC<3 % RB>{}); break;
      }
      const int64_t rb = m0 + wm * WM + 32 * i + row0;
      if (splits > 1) {
        // fp32 partials of this K range: ws[(split M + m) N + n]
        float* ws = (float*)((char*)p.workspace + kCounterBytes) + (int64_t)split * M * N;
#pragma unroll 1
        for (int e = 0; e < ITEMS; ++e) {
          const int row = row0 + RS * e;
          const int64_t m = rb + RS * e;
          if (m < M && cnt > 0) {
            const float* sv = scr + row * kGwELD + 8 * ch;
            float v[8];
#pragma unroll
            for (int x = 0; x < 8; ++x) v[x] = sv[x];
            st_f8(ws + m * N + nn, v, (N & 3) == 0 && cnt == 8, cnt);
          }
        }
        continue;
      }
#pragma unroll 1
      for (int e0 = 0; e0 < ITEMS; e0 += EB) {
        EpiIn in[EB];
#pragma unroll
        for (int e = 0; e < EB; ++e) epi_load<MODE>(p, V, rb + RS * (e0 + e), nn, vec, cnt, in[e]);
#pragma unroll
        for (int e = 0; e < EB; ++e) {
          const int row = row0 + RS * (e0 + e);
          const int64_t m = rb + RS * (e0 + e);
          float xo[8];
          if (m < M && cnt > 0) {
            float v[8], u[8];
            const float* sv = scr + row * kGwELD + 8 * ch;
#pragma unroll
            for (int x = 0; x < 8; ++x) {
              v[x] = sv[x];
              u[x] = GG ? sv[64 + x] : 0.f;
            }
            const float r = p.rownorm ? sRow[m - m0] : 1.f;
            epi_store<MODE>(p, m, nn, vec, cnt, v, u, r, in[e], ho, xo);
          }
          // the 8 lanes of a row's 64-column block
          if (ho) epi_handoff(p, m < M && cnt > 0, m, nn, cnt, xo);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// gemm_wide_f8_kernel: gemm_wide_kernel with fp8 (e4m3) weights.  Same tile
// and wave split; the MFMA is the block-scaled v_mfma_scale_f32_32x32x64
// (A and B as e4m3, one power-of-two scale per A row and 64-k slab, the
// weights' per-channel scales applied in the epilogue).  The bf16 A tile is
// quantized as it feeds the MFMAs, the same way as gemm_tile_kernel's fp8
// path: one scale per (row, 64-k slab) from the slab's largest magnitude,
// shared by the two lanes (l, l ^ 32) holding the row's two 32-k halves.
// Slabs of 64 k: A 256 rows x 128 B (bf16) and B 256 rows x 64 B (e4m3),
// 48 KiB per stage, a 3-stage ring; slab t + 2's loads go between slab t's
// four MFMA groups.  B rows carry the 16-byte chunk index XOR (row >> 2) & 3
// (4 chunks per 64-byte row).
// ---------------------------------------------------------------------------
// F8A: A arrives as an e4m3 copy with its exponents (a8 / a8_scale, see
// fvx_gemm_desc): A rows of 64 bytes per slab like the B rows, 256 exponent
// bytes per slab, no quantization here.
constexpr int kGw8Stages = 3;
template <bool F8A>
struct Gw8Layout {
  static constexpr int A = F8A ? 256 * 64 : 256 * 128;  // A tile bytes
  static constexpr int B = 256 * 64;                    // B tile bytes
  static constexpr int E = F8A ? 256 : 0;               // A exponents
  static constexpr int STAGE = A + B + E;
};

// A16 (W8A16): A stays bf16 (no quantization, F8A off) and each 8 weight
// bytes become one bf16 fragment of v_mfma_f32_32x32x16_bf16: per slab and
// wave 64 bf16 MFMAs, as in gemm_wide_kernel, on half its B bytes.
template <int MODE, bool SUM_A, bool F8A, bool A16>
__global__ __launch_bounds__(256, 1) void gemm_wide_f8_kernel(GemmArgs p, int m_tiles,
                                                              int n_tiles, int vec_ok,
                                                              int splits, int kchunk) {
  static_assert(!(A16 && F8A), "W8A16 reads a bf16 A");
  typedef Gw8Layout<F8A> LY;
  constexpr bool GG = MODE == FVX_GEMM_GEGLU;
  constexpr int WNO = GG ? 64 : 128;  // output columns per wave
  constexpr int kGw8AStage = LY::A, kGw8Stage = LY::STAGE;
  static_assert(!(F8A && SUM_A), "an e4m3 A has no bf16 squares to sum");
  __shared__ __align__(16) char smem[kGw8Stages * kGw8Stage];
  __shared__ float sRow[kGwBM], sTmp[256];
  warm_kernargs<sizeof(GemmArgs) + 24>();
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-aware order over (split, tile), as in gemm_wide_kernel
  const int nblk = m_tiles * n_tiles;
  const int lid = xcd_remap(blockIdx.x, nblk * splits);
  const int bid = lid % nblk, split = lid / nblk;
  const int m_tile = bid % m_tiles, n_tile = bid / m_tiles;
  const int64_t M = p.m, N = p.n, K = p.k;
  const int64_t m0 = (int64_t)m_tile * kGwBM, n0 = (int64_t)n_tile * (GG ? 128 : 256);
  // K range [kb, kb + 64 nk) (splits > 1: PLAIN without rownorm, partials
  // scaled by the weight scales for gemm_partial_reduce_kernel)
  const int64_t kb = (int64_t)split * kchunk;
  const int nk = (int)(((kb + kchunk < K ? kb + kchunk : K) - kb) / 64);

  // this wave's band: 128 rows of A (waves 0, 1; 16 loads of 8 rows x 128 B
  // per slab) or of B (2, 3; 8 loads of 16 rows x 64 B)
  const bool isa = wave < 2;
  const int64_t r0 = isa ? m0 + 128 * wave : (GG ? n0 : n0 + 128 * (wave - 2));
  const int64_t rlim = (isa ? M : N) - r0;
  const int64_t nrows = rlim <= 0 ? 0 : (rlim < 128 ? rlim : 128);
  const uint32_t ld = isa ? (F8A ? (uint32_t)p.a8_ld : (uint32_t)p.lda * 2)
                          : (uint32_t)p.ldb;  // bytes per row
  const char* band = isa ? (F8A ? (const char*)p.a8 + r0 * p.a8_ld + kb
                                : (const char*)p.a + r0 * p.lda * 2 + kb * 2)
                         : (const char*)((GG && wave == 3) ? p.b2 : p.b) + r0 * p.ldb + kb;
  const i32x4_t rs = make_rsrc4(band, (uint32_t)(nrows * ld));
  // F8A: the slab's 256 A exponents, one dword per lane (rows 4 l .. 4 l + 3)
  const i32x4_t rse = make_rsrc4(F8A ? p.a8_scale : p.a,
                                 F8A ? (uint32_t)((K / 64) * p.a8_sld) : 0u);
  uint32_t vo0, vo1, lds0;
  if (isa && !F8A) {
    // rows 8 i + (lane >> 3), slot lane & 7 <- chunk slot ^ ((row >> 1) & 7)
    const int lr = lane >> 3, lc = lane & 7;
    vo0 = (uint32_t)lr * ld + 16u * (uint32_t)(lc ^ (lr >> 1));
    vo1 = (uint32_t)lr * ld + 16u * (uint32_t)(lc ^ (lr >> 1) ^ 4);
    lds0 = __builtin_amdgcn_readfirstlane(lds_addr(smem) + wave * 128 * 128);
  } else {
    // rows 16 i + (lane >> 2), slot lane & 3 <- chunk slot ^ ((row >> 2) & 3)
    const int lr = lane >> 2, lc = lane & 3;
    vo0 = vo1 = (uint32_t)lr * ld + 16u * (uint32_t)(lc ^ ((lr >> 2) & 3));
    lds0 = __builtin_amdgcn_readfirstlane(
        lds_addr(smem) + (isa ? wave * 128 * 64 : kGw8AStage + (wave - 2) * 128 * 64));
  }
  // quarter q of slab t's loads into ring stage `stage` (the four quarters
  // go between the four MFMA groups of a slab)
  auto issue_q = [&](int t, int stage, int q) {
    if (F8A && wave == 0 && q == 0)
      load_lds4(rse, lds_addr(smem) + stage * kGw8Stage + LY::A + LY::B,
                (uint32_t)((kb / 64 + t) * p.a8_sld + m0 + 4 * lane));
    if (isa && !F8A) {
      const uint32_t so = (uint32_t)t * 128u;
#pragma unroll
      for (int i = 4 * q; i < 4 * q + 4; ++i)
        load_lds16_so(rs, lds0 + stage * kGw8Stage + i * 1024,
                      ((i & 1) ? vo1 : vo0) + (uint32_t)(8 * i) * ld, so);
    } else {
      const uint32_t so = (uint32_t)t * 64u;  // 64 one-byte k per row and slab
#pragma unroll
      for (int i = 2 * q; i < 2 * q + 2; ++i)
        load_lds16_so(rs, lds0 + stage * kGw8Stage + i * 1024, vo0 + (uint32_t)(16 * i) * ld, so);
    }
  };
  auto issue = [&](int t, int stage) {
#pragma unroll
    for (int q = 0; q < 4; ++q) issue_q(t, stage, q);
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  float ss[4] = {0.f, 0.f, 0.f, 0.f};
  const int sw = (lane >> 1) & 7, fr = lane & 31, hk = lane >> 5;
  const int swb = (fr >> 2) & 3;
  auto brow = [&](int j) {
    return GG ? (j >> 1) * 128 + wn * 64 + 32 * (j & 1) : wn * 128 + 32 * j;
  };
  // lane (fr, hk): k = 32 hk .. + 31 of the slab for A row / B column fr;
  // slab tn's loads go into stage tst between the MFMA groups
  auto compute = [&](int stage, int tn, int tst) {
    const char* sa = smem + stage * kGw8Stage;
    const char* sb = sa + kGw8AStage;
    const unsigned char* se = (const unsigned char*)(sb + LY::B);
    i32x8_t bq[4];
    bf16x8 bw[4][4];  // A16: [j][c], k = 32 hk + 8 c + 0..7
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const char* row = sb + (brow(j) + fr) * 64;
      const bf16x8 b0 = *(const bf16x8*)(row + (((2 * hk) ^ swb) * 16));
      const bf16x8 b1 = *(const bf16x8*)(row + (((2 * hk + 1) ^ swb) * 16));
      if (A16) {
        bw[j][0] = e4m3x8_to_bf16(b0.w[0], b0.w[1]);
        bw[j][1] = e4m3x8_to_bf16(b0.w[2], b0.w[3]);
        bw[j][2] = e4m3x8_to_bf16(b1.w[0], b1.w[1]);
        bw[j][3] = e4m3x8_to_bf16(b1.w[2], b1.w[3]);
      } else {
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          bq[j][x] = (int)b0.w[x];
          bq[j][4 + x] = (int)b1.w[x];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      int ae;
      i32x8_t aq;
      if (F8A) {
        const int ra = wm * 128 + 32 * i + fr;
        const char* row = sa + ra * 64;
        const bf16x8 a0 = *(const bf16x8*)(row + (((2 * hk) ^ swb) * 16));
        const bf16x8 a1 = *(const bf16x8*)(row + (((2 * hk + 1) ^ swb) * 16));
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          aq[x] = (int)a0.w[x];
          aq[4 + x] = (int)a1.w[x];
        }
        ae = se[ra];
      } else {
        const char* row = sa + (wm * 128 + 32 * i + fr) * 128;
        bf16x8 av[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) av[c] = *(const bf16x8*)(row + (((4 * hk + c) ^ sw) * 16));
        if (SUM_A)
#pragma unroll
          for (int c = 0; c < 4; ++c) ss[i] += sumsq8(av[c]);
        if (A16) {
          // MFMA c sums k = 32 hk + 8 c + 0..7 (hk = 0, 1) of the slab
#pragma unroll
          for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma32x32x16(av[c], bw[j][c], acc[i][j]);
        } else {
          aq = quant_fp8x32<32, 0>(av, &ae);
        }
      }
      if (!A16)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma32x32x64_f8(aq, ae, bq[j], 127, acc[i][j]);
      issue_q(tn, tst, i);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // every iteration loads a slab (past the end: slab nk - 1 again, into the
  // free stage), so one slab's loads are in flight behind slab t's
  issue(0, 0);
  issue(nk > 1 ? 1 : 0, 1);
  float ss_pre = 0.f;
  if (!SUM_A && p.rownorm) ss_pre = rows_parts_sum<kGwBM, 256>(p, p.ss_in, m0, M, sTmp);
  for (int t = 0; t < nk; ++t) {
    // this wave's loads of slab t landed (slab t + 1's may still fly)
    if (F8A && wave == 0)
      wait_vmcnt<9>();
    else if (isa && !F8A)
      wait_vmcnt<16>();
    else
      wait_vmcnt<8>();
    __syncthreads();  // everyone's, and slab t - 1 is consumed
    compute(t % kGw8Stages, t + 2 < nk ? t + 2 : nk - 1, (t + 2) % kGw8Stages);
  }
  wait_vmcnt<0>();

  if (!SUM_A) {
    sRow[tid] = ss_pre;
  } else if (wn == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s2 = ss[i] + __shfl_xor(ss[i], 32, 64);
      if (lane < 32) sRow[wm * 128 + 32 * i + lane] = s2;
    }
  }
  __syncthreads();  // also: every wave is done with the ring

  // lane item q = lane + 64 e: row q / CH, columns 8 (q % CH) .. -- the
  // lane's own column chunk in every item, so its column operands and
  // weight scales are read once
  constexpr int CH = WNO / 8, ITEMS = 32 * CH / 64, EB = 4, RS = 64 / CH;
  static_assert(64 % CH == 0, "one column chunk per lane");
  float* scr = (float*)smem + wave * 32 * kGwELD;
  const int ch = lane % CH, row0 = lane / CH;
  const int64_t nn = n0 + wn * WNO + 8 * ch;
  const int cnt = (int)(N - nn < 8 ? N - nn : 8);
  const bool ho = (MODE == FVX_GEMM_PLAIN || GG) && (p.ss_out || p.a8_out);
  const EpiViews V = epi_views<MODE>(p);
  auto to_scr = [&](auto ic) {
    constexpr int i = decltype(ic)::value;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        scr[(8 * (r >> 2) + 4 * hk + (r & 3)) * kGwELD + 32 * j + fr] = acc[i][j][r];
  };
  // with N % 8 == 0 every chunk with columns left holds 8: vec is uniform
  const bool vec = vec_ok && (cnt == 8 || (N & 7) == 0);
  {
    EpiIn col;
    if (splits == 1) epi_load_col<MODE>(V, nn, vec, col);
    float w0[8], w1[8];
    bl_f8(make_rsrc(p.b_scale, rec_bytes(N * 4)), (uint32_t)(nn * 4), vec, w0);
    if (GG) bl_f8(make_rsrc(p.b2_scale, rec_bytes(N * 4)), (uint32_t)(nn * 4), vec, w1);
#pragma unroll 1
    for (int i = 0; i < 4; ++i) {
      switch (i) {
        case 0: to_scr(IntC<0>{}); break;
        case 1: to_scr(IntC<1>{}); break;
        case 2: to_scr(IntC<2>{}); break;
        default: to_scr(IntC<3>{}); break;
      }
      const int64_t rb = m0 + wm * 128 + 32 * i + row0;
      if (splits > 1) {
        // partials of this K range, scaled by the weight scales:
        // ws[(split M + m) N + n]
        float* ws = (float*)((char*)p.workspace + kCounterBytes) + (int64_t)split * M * N;
#pragma unroll 1
        for (int e = 0; e < ITEMS; ++e) {
          const int row = row0 + RS * e;
          const int64_t m = rb + RS * e;
          if (m < M && cnt > 0) {
            float v[8];
            const float* sv = scr + row * kGwELD + 8 * ch;
#pragma unroll
            for (int x = 0; x < 8; ++x) v[x] = sv[x] * w0[x];
            st_f8(ws + m * N + nn, v, (N & 3) == 0 && cnt == 8, cnt);
          }
        }
        continue;
      }
#pragma unroll 1
      for (int e0 = 0; e0 < ITEMS; e0 += EB) {
        EpiIn in[EB];
#pragma unroll
        for (int e = 0; e < EB; ++e) {
          in[e] = col;
          epi_load_row<MODE>(p, V, rb + RS * (e0 + e), nn, vec, cnt, in[e]);
        }
#pragma unroll
        for (int e = 0; e < EB; ++e) {
          const int row = row0 + RS * (e0 + e);
          const int64_t m = rb + RS * (e0 + e);
          float xo[8];
          if (m < M && cnt > 0) {
            float v[8], u[8];
            const float* sv = scr + row * kGwELD + 8 * ch;
#pragma unroll
            for (int x = 0; x < 8; ++x) {
              v[x] = sv[x] * w0[x];
              u[x] = GG ? sv[64 + x] * w1[x] : 0.f;
            }
            const float r = p.rownorm ? rsqrtf(sRow[m - m0] / (float)K + p.rownorm_eps) : 1.f;
            epi_store<MODE>(p, m, nn, vec, cnt, v, u, r, in[e], ho, xo);
          }
          if (ho) epi_handoff(p, m < M && cnt > 0, m, nn, cnt, xo);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny (M <= 64) weight-streaming kernels
// ---------------------------------------------------------------------------
// gemm_skinny_kernel: M <= 64 (the bs=1 action expert, M = 50/51).  The op is
// a weight stream.  A workgroup of 8 waves owns 16 output columns (GEGLU: 16
// of each weight) and one K range of the split-K grid (blockIdx.y); wave w
// takes the slice [w kw, (w + 1) kw) of that range.  Both MFMA operands come
// straight from global memory: lane (fr, g) reads the 16 bytes at k = 32 t +
// 8 g of weight row n0 + fr and of activation rows 16 f + fr (the activations
// are a few hundred KB and stay L2-resident).  The slice moves through two
// register sets of 3 MFMA steps (GEGLU: 2), the loads of the next set issued
// before the MFMAs of the current one.  The waves' partial tiles and row sums of squares
// meet in LDS and are added in wave order.
//
// With one K range 128 threads run the chunk epilogue at once.  Otherwise
// every workgroup writes its fp32 partial tile (and row sums) with stores
// that write through to the device-coherent level (sc1), waits for them to
// complete, and bumps the arrival counter of its column tile; the last
// workgroup of the tile to arrive re-reads the splits' partials with sc1
// loads, adds them in split order (deterministic, whatever the arrival
// order), runs the epilogue and resets the counter to zero for the next
// call.  No device-scope fence is involved: the shared data never sits
// dirty in a non-coherent L2, which is what a release/acquire pair would
// have to write back and invalidate (tens of microseconds per GEMM here).
constexpr int kSkWaves = 8;
// W8A8 (fp8 weights, A quantized here): 4 waves, each with the full
// 512-register file (its A quantization does not fit 256 registers with two
// sets of loads in flight); bf16 and W8A16 (fp8 weights converted to bf16
// in registers, A bf16): 8
constexpr int sk_waves(bool f8, bool a16) { return f8 && !a16 ? 4 : kSkWaves; }
// steps per register set: W8A8 one 128-k fp8 block; W8A16 one 16-byte half
// of a lane's 32 weight bytes (2 steps; 4 spilled in the PLAIN kernel);
// bf16: as many 32-k steps as the registers hold with two sets in flight --
// fewer activation row blocks per workgroup (rb) leave room for more
constexpr int sk_steps(int nb, bool f8, bool a16, int rb) {
  return f8 ? (a16 ? 2 : 4)
            : (rb == 4 ? (nb == 2 ? 2 : 3) : rb == 2 ? (nb == 2 ? 3 : 4) : (nb == 2 ? 6 : 8));
}
// K granule of one wave's slice (a multiple of the register-set steps that
// the weight layout needs: W8A8 a 128-k block, W8A16 a 64-k half)
constexpr int sk_kgran(bool f8, bool a16) { return f8 ? (a16 ? 64 : 128) : 32; }
constexpr int kSkMaxSplits = 4;

__host__ __device__ constexpr int skinny_block_floats(int nb) {
  return nb * 64 * 16 + 64;  // [nb][64 rows][16 cols] + 64 row sums
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kSc1 = 16;  // buffer cache policy bit: write through / read at
                          // the device-coherent level

__device__ __forceinline__ void sc1_store8(__amdgpu_buffer_rsrc_t r, int off,
                                           const float* x) {
  __builtin_amdgcn_raw_buffer_store_b128(
      u32x4_t{__float_as_uint(x[0]), __float_as_uint(x[1]),
              __float_as_uint(x[2]), __float_as_uint(x[3])},
      r, off, 0, kSc1);
  __builtin_amdgcn_raw_buffer_store_b128(
      u32x4_t{__float_as_uint(x[4]), __float_as_uint(x[5]),
              __float_as_uint(x[6]), __float_as_uint(x[7])},
      r, off + 16, 0, kSc1);
}

__device__ __forceinline__ void sc1_load8(__amdgpu_buffer_rsrc_t r, int off,
                                          float* x) {
  const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1);
  const u32x4_t b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, kSc1);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[e] = __uint_as_float(a[e]);
    x[4 + e] = __uint_as_float(b[e]);
  }
}

template <int MODE, bool F8, bool A16, int RB, bool ASC, bool SP = false>
__global__ __launch_bounds__(64 * sk_waves(F8, A16)) void gemm_skinny_kernel(GemmArgs p,
                                                          int splits,
                                                          int64_t kc,
                                                          int vec_ok) {
  constexpr int NB = (MODE == FVX_GEMM_GEGLU) ? 2 : 1;
  // RB activation row blocks of 16 per workgroup: row group blockIdx.z
  // covers rows 16 RB z .. + 16 RB - 1 (fewer row blocks, more workgroups)
  static_assert(RB == 4 || !F8 || A16, "W8A8 skinny GEMMs take all 4 row blocks");
  // ASC: adaptive RMSNorm folded in -- A's column k scaled by (1 +
  // a_scale[k]) as it is loaded (bf16 A, i.e. bf16 or W8A16 weights)
  static_assert(!ASC || !F8 || A16, "a_scale needs bf16 activations");
  constexpr int RR = 16 * RB;
  // W8A8: one register set = one 128-k step of the fp8 MFMA (4 A blocks of
  // 32); W8A16: S 32-k steps of bf16 MFMAs whose B fragments are converted
  // from 8 e4m3 bytes each (a 16-byte load holds two steps)
  static_assert(!A16 || F8, "W8A16 is an fp8-weight variant");
  constexpr int W = sk_waves(F8, A16), S = sk_steps(NB, F8, A16, RB);
  __shared__ float sP[W][NB][RR][16 + 1];
  __shared__ float sS[W][RR];
  __shared__ int s_last;
  warm_kernargs<sizeof(GemmArgs) + 24>();

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;
  const int tile = blockIdx.x, split = blockIdx.y, rg = blockIdx.z;
  const int fb0 = rg * RB;  // first row block of the workgroup
  const int64_t M = p.m, N = p.n, K = p.k;
  const int64_t n0 = (int64_t)tile * 16;
  const int64_t n = n0 + fr;
  const bool nval = n < N;
  const int64_t kw = kc / W;  // multiple of 32
  const int64_t kb = (int64_t)split * kc + wave * kw;
  const int64_t ke0 = kb + kw, kend = (int64_t)(split + 1) * kc;
  const int64_t ke = ke0 < K ? (ke0 < kend ? ke0 : kend) : K;
  const int nst = kb < ke ? (int)((ke - kb + 31) / 32) : 0;
  // Operand byte offsets: fragment (f, step ks) of A at a0 + ks * a_ks +
  // f * a_f, of B at b0 + ks * b_ks (32-bit, through buffer resources).
  // Fragment-major operands (a_frag / b_frag) hold each MFMA step as one
  // contiguous 1 KiB block, so every wave load is fully coalesced; row-major
  // ones give 16 rows x 64 B per load.
  const uint32_t ks0 = (uint32_t)(kb >> 5);
  uint32_t a0, a_ks, a_f, b0, b_ks;
  if (p.a_frag) {
    a0 = lane * 16;
    a_ks = 4 * 64 * 16;
    a_f = 64 * 16;
  } else {
    a0 = (uint32_t)(fr * p.lda + 8 * g) * 2;
    a_ks = 64;
    a_f = (uint32_t)(16 * p.lda * 2);
  }
  if (F8) {
    // fp8 fragment-major: one 2 KiB block per (16 columns, 128 k), 32 B per
    // lane; b_ks counts 32-k steps (a block spans four)
    b0 = (uint32_t)(((int64_t)tile * (K >> 7) * 64 + lane) * 32);
    b_ks = 512;
  } else if (p.b_frag) {
    b0 = (uint32_t)(((int64_t)tile * (K >> 5) * 64 + lane) * 16);
    b_ks = 64 * 16;
  } else {
    b0 = (uint32_t)(((nval ? n : 0) * p.ldb + 8 * g) * 2);
    b_ks = 64;
  }
  const bool bval = nval || p.b_frag;
  const __amdgpu_buffer_rsrc_t ra_rs = make_rsrc(p.a, 0x7fffffffu);
  const __amdgpu_buffer_rsrc_t rb_rs[2] = {make_rsrc(p.b, 0x7fffffffu),
                                           make_rsrc(NB == 2 ? p.b2 : p.b, 0x7fffffffu)};
  auto bld = [](__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  };

  bf16x8 ra[2][S][RB], rb[2][S][NB];
  bf16x8 rsc[2][S];  // ASC: a_scale of the lane's 8 k positions per step
  const __amdgpu_buffer_rsrc_t rsc_rs = make_rsrc(p.a_scale, ASC ? rec_bytes(K * 2) : 0u);
  // unconditional loads: a masked-out fragment gets an offset past the view
  auto load = [&](int t0, int set) {
#pragma unroll
    for (int t = 0; t < S; ++t) {
      const uint32_t ks = ks0 + t0 + t;
      const bool kin = kb + 32 * (t0 + t) + 8 * g < ke;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (!F8)
          rb[set][t][b] = bld(rb_rs[b], (kin && bval) ? b0 + ks * b_ks : kOOB);
        else if (A16) {
          // steps ks, ks + 1 (ks even): half (ks / 2) % 2 of the lane's 32
          // bytes in 128-k block ks / 4
          if (t % 2 == 0)
            rb[set][t / 2][b] =
                bld(rb_rs[b], kin ? b0 + (ks >> 2) * 2048u + ((ks >> 1) & 1u) * 16u : kOOB);
        } else if (t < 2)  // the step's 32 fp8 bytes: two 16-byte halves
          rb[set][t][b] = bld(rb_rs[b], kin ? b0 + (ks0 + t0) * b_ks + 16 * t : kOOB);
      }
#pragma unroll
      for (int f = 0; f < RB; ++f) {
        const bool rin = p.a_frag || (fb0 + f) * 16 + fr < M;
        ra[set][t][f] = bld(ra_rs, (kin && rin) ? a0 + ks * a_ks + (fb0 + f) * a_f : kOOB);
      }
      if (ASC) rsc[set][t] = bld(rsc_rs, kin ? ks * 64u + 16u * (uint32_t)g : kOOB);
    }
  };
  f32x4_t acc[NB][RB];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int f = 0; f < RB; ++f) acc[b][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float ss[RB];
#pragma unroll
  for (int f = 0; f < RB; ++f) ss[f] = 0.f;
  // ASC: the A fragment as the MFMA sees it, bf16(x[k] * (1 + a_scale[k]))
  // with the factor in fp32 (as GemmaRMSNorm forms it)
  auto scaled = [&](const bf16x8& a, const bf16x8& sc) {
    if (!ASC) return a;
    float x[8], y[8];
    unpack8(a, x);
    unpack8(sc, y);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= 1.f + y[e];
    return pack8(x);
  };
  auto compute = [&](int set) {
    if (A16) {
      // lane (fr, g) holds weight bytes k = 32 t + 8 g + j of column n0 + fr
      // (the k positions of its A fragments): bf16 MFMAs on the converted
      // weights
#pragma unroll
      for (int t = 0; t < S; ++t) {
        bf16x8 bw[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const bf16x8& raw = rb[set][t / 2][b];
          bw[b] = (t % 2 == 0) ? e4m3x8_to_bf16(raw.w[0], raw.w[1])
                               : e4m3x8_to_bf16(raw.w[2], raw.w[3]);
        }
#pragma unroll
        for (int f = 0; f < RB; ++f) {
          if (p.rownorm) ss[f] += sumsq8(ra[set][t][f]);
          const bf16x8 av = scaled(ra[set][t][f], rsc[set][t]);
#pragma unroll
          for (int b = 0; b < NB; ++b) acc[b][f] = mfma16x16x32(av, bw[b], acc[b][f]);
        }
      }
      return;
    }
    if (F8) {
      // lane (fr, g) holds k = 32 t + 8 g + j of row 16 f + fr: quantize the
      // row's 128 values of the step with one power-of-two scale, one fp8
      // MFMA per row block
#pragma unroll
      for (int f = 0; f < RB; ++f) {
        const bf16x8 av[4] = {ra[set][0][f], ra[set][1][f], ra[set][2][f], ra[set][3][f]};
        if (p.rownorm)
#pragma unroll
          for (int t = 0; t < 4; ++t) ss[f] += sumsq8(av[t]);
        int e8;  // one scale per (row, 128-k step): lanes fr + 16 g, g = 0..3
        const i32x8_t aq = quant_fp8x32<16, 32>(av, &e8);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          i32x8_t bq;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            bq[i] = (int)rb[set][0][b].w[i];
            bq[4 + i] = (int)rb[set][1][b].w[i];
          }
          acc[b][f] = mfma16x16x128_f8(aq, e8, bq, 127, acc[b][f]);
        }
      }
      return;
    }
#pragma unroll
    for (int t = 0; t < S; ++t)
#pragma unroll
      for (int f = 0; f < RB; ++f) {
        if (p.rownorm) ss[f] += sumsq8(ra[set][t][f]);
        const bf16x8 av = scaled(ra[set][t][f], rsc[set][t]);
#pragma unroll
        for (int b = 0; b < NB; ++b)
          acc[b][f] = mfma16x16x32(av, rb[set][t][b], acc[b][f]);
      }
  };
  if (nst > 0) load(0, 0);
  // The epilogue's reads (residual, gate, bias, RoPE table, Euler state) do
  // not depend on the product: issue them now so that their latency hides
  // under the K loop.  Thread t < 2 RR owns local row t / 2 (global row
  // 16 fb0 + t / 2), columns n0 + 8 (t % 2).
  const int lrow = (tid >> 1) & (RR - 1), half = tid & 1;
  const int row = fb0 * 16 + lrow;
  const int64_t ncol = n0 + 8 * half;
  const int cnt = (int)(N - ncol < 8 ? N - ncol : 8);
  const bool mine = tid < 2 * RR && row < M && cnt > 0;
  const bool vec = vec_ok && cnt == 8;
  EpiIn in;
  if (mine) {
    const EpiViews V = epi_views<MODE, SP>(p);
    epi_load_col<MODE>(V, ncol, vec, in);
    epi_load_row<MODE, SP>(p, V, row, ncol, vec, cnt, in);
  }
  // ASC with QKV_ROPE / GEGLU: the folded shift's fp32 biases (gate, up)
  constexpr bool FB = ASC && (MODE == FVX_GEMM_QKV_ROPE || MODE == FVX_GEMM_GEGLU);
  float fb[8], fb2[8];
  if (FB) {
    bl_f8(make_rsrc(p.bias_f32, p.bias_f32 ? rec_bytes(N * 4) : 0u), (uint32_t)(ncol * 4), vec,
          fb);
    bl_f8(make_rsrc(p.bias2_f32, p.bias2_f32 ? rec_bytes(N * 4) : 0u), (uint32_t)(ncol * 4),
          vec, fb2);
  }
  float wsc[8], wsc2[8];  // fp8 per-channel weight scales of the 8 columns
  if (F8) {
    bl_f8(make_rsrc(p.b_scale, rec_bytes(N * 4)), (uint32_t)(ncol * 4), vec, wsc);
    bl_f8(make_rsrc(NB == 2 ? p.b2_scale : p.b_scale, rec_bytes(N * 4)), (uint32_t)(ncol * 4),
          vec, wsc2);
  }
  for (int t0 = 0; t0 < nst; t0 += 2 * S) {
    if (t0 + S < nst) load(t0 + S, 1);
    compute(0);
    if (t0 + S >= nst) break;
    if (t0 + 2 * S < nst) load(t0 + 2 * S, 0);
    compute(1);
  }

  // wave partials -> LDS; lane holds column fr, local rows 16 f + 4 g + j
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int f = 0; f < RB; ++f)
#pragma unroll
      for (int j = 0; j < 4; ++j) sP[wave][b][f * 16 + 4 * g + j][fr] = acc[b][f][j];
  if (p.rownorm) {
#pragma unroll
    for (int f = 0; f < RB; ++f) {
      float v = ss[f];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      if (g == 0) sS[wave][f * 16 + fr] = v;
    }
  }
  __syncthreads();

  // thread t < 2 RR: local row t / 2, columns n0 + 8 (t % 2) .. + 7
  float v[8], u[8], rsum = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = u[e] = 0.f;
  if (mine) {
#pragma unroll
    for (int w = 0; w < W; ++w) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] += sP[w][0][lrow][8 * half + e];
        if (NB == 2) u[e] += sP[w][NB - 1][lrow][8 * half + e];
      }
      if (p.rownorm) rsum += sS[w][lrow];
    }
  }

  if (splits > 1) {
    // partial block of (tile, split): [NB][64][16] floats, then 64 row sums
    constexpr int BLK = skinny_block_floats(NB);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (char*)p.workspace + kCounterBytes, 0, 0x7fffffff, 0x00020000);
    const int cell = tile * (int)gridDim.z + rg;  // (column tile, row group)
    const int base = (cell * splits + split) * BLK * 4;
    if (mine) {
      sc1_store8(rs, base + (row * 16 + 8 * half) * 4, v);
      if (NB == 2) sc1_store8(rs, base + ((64 + row) * 16 + 8 * half) * 4, u);
      if (p.rownorm && half == 0)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(rsum), rs,
                                              base + (NB * 1024 + row) * 4, 0, kSc1);
    }
    // every store of this workgroup completes before it is counted
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      uint32_t* ctr = (uint32_t*)p.workspace + cell;
      const uint32_t old =
          __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = old == (uint32_t)(splits - 1);
      if (last) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_last = last;
    }
    __syncthreads();
    if (!s_last || !mine) return;
    // last arrival: every split's loads in flight, added in split order
    float tv[kSkMaxSplits][8], tu[kSkMaxSplits][8], tr[kSkMaxSplits];
#pragma unroll
    for (int s = 0; s < kSkMaxSplits; ++s) {
      if (s < splits) {
        const int bs = (cell * splits + s) * BLK * 4;
        sc1_load8(rs, bs + (row * 16 + 8 * half) * 4, tv[s]);
        if (NB == 2) sc1_load8(rs, bs + ((64 + row) * 16 + 8 * half) * 4, tu[s]);
        tr[s] = p.rownorm ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                                rs, bs + (NB * 1024 + row) * 4, 0, kSc1))
                          : 0.f;
      }
    }
    rsum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = u[e] = 0.f;
#pragma unroll
    for (int s = 0; s < kSkMaxSplits; ++s) {
      if (s < splits) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v[e] += tv[s][e];
          if (NB == 2) u[e] += tu[s][e];
        }
        rsum += tr[s];
      }
    }
  }
  if (!mine) return;
  float r = p.rownorm ? rsqrtf(rsum / (float)K + p.rownorm_eps) : 1.f;
  if (F8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] *= wsc[e];
      u[e] *= wsc2[e];
    }
  }
  if (FB) {
    // RMS factor, then the shift's biases (the QKV / GeGLU epilogues have
    // no bias of their own)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = v[e] * r + fb[e];
      u[e] = u[e] * r + fb2[e];
    }
    r = 1.f;
  }
  epi_store<MODE, false, SP>(p, row, ncol, vec, cnt, v, u, r, in, false, nullptr);
}

// Sum of the split partials of the tile or wide kernel + epilogue.  Thread t
// owns 8 consecutive columns of one row (chunk c = 256 blockIdx.x + t: row
// c / CH, columns 8 (c % CH) .., CH = ceil(N / 8) chunks per row) and runs
// the tile kernel's 8-column epilogue on them; the partials are read 16
// bytes at a time (N % 4 == 0) through a buffer view (past it: zeros),
// the loads of up to 8 splits in flight before their adds, which follow
// split order (deterministic).
// (SP: the plain-epilogue build, as the tile kernel's XF bit 3)
template <int MODE, bool SP = false>
__global__ __launch_bounds__(256) void gemm_partial_reduce_kernel(GemmArgs p,
                                                                  int splits,
                                                                  int vec_ok) {
  warm_kernargs<sizeof(GemmArgs) + 24>();
  constexpr int NB = (MODE == FVX_GEMM_GEGLU) ? 2 : 1;
  constexpr int UN = 8;  // splits in flight per pass
  const int64_t N = p.n, K = p.k, M = p.m;
  const int64_t CH = (N + 7) / 8;
  // M * CH < 2^31 (the split partials fit a 2 GiB buffer view): 32-bit divide
  const uint32_t c = blockIdx.x * 256u + threadIdx.x;
  const int64_t m = udiv32(c, CH), nn = (int64_t)(c - (uint32_t)m * (uint32_t)CH) * 8;
  if (m >= M) return;
  const int cnt = (int)(N - nn < 8 ? N - nn : 8);
  const bool v4 = (N & 3) == 0;
  const float* ws = (const float*)((const char*)p.workspace + kCounterBytes);
  const int64_t plane = (int64_t)splits * M * N;
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(ws, rec_bytes((NB * plane + (int64_t)splits * M) * 4));
  EpiIn in;
  {
    const EpiViews V = epi_views<MODE, SP>(p);
    epi_load_col<MODE>(V, nn, vec_ok && cnt == 8, in);
    epi_load_row<MODE, SP>(p, V, m, nn, vec_ok && cnt == 8, cnt, in);
  }
  float v[8], u[8], ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = u[e] = 0.f;
  auto ld8f = [&](int64_t off, float* d) {  // 8 floats at element offset off
    if (v4) {
      const f32x4_t a = bload4f(rw, (uint32_t)(off * 4));
      const f32x4_t b = bload4f(rw, cnt > 4 ? (uint32_t)((off + 4) * 4) : kOOB);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        d[e] = a[e];
        d[4 + e] = b[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] = bload1f(rw, e < cnt ? (uint32_t)((off + e) * 4) : kOOB);
    }
  };
  for (int s0 = 0; s0 < splits; s0 += UN) {
    float t[UN][NB][8], q[UN];
#pragma unroll
    for (int i = 0; i < UN; ++i) {
      const int sp = s0 + i;
      const bool in_ = sp < splits;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        if (in_)
          ld8f(b * plane + ((int64_t)sp * M + m) * N + nn, t[i][b]);
        else
#pragma unroll
          for (int e = 0; e < 8; ++e) t[i][b][e] = 0.f;
      }
      q[i] = bload1f(rw, (in_ && p.rownorm) ? (uint32_t)((NB * plane + (int64_t)sp * M + m) * 4)
                                            : kOOB);
    }
#pragma unroll
    for (int i = 0; i < UN; ++i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[e] += t[i][0][e];
        u[e] += t[i][NB - 1][e];
      }
      ss += q[i];
    }
  }
  const float r = p.rownorm ? rsqrtf(ss / (float)K + p.rownorm_eps) : 1.f;
  // hand-over outputs (PLAIN, N % 64 == 0): the 8 consecutive lanes of a
  // row's 64-column block
  const bool ho = MODE == FVX_GEMM_PLAIN && (p.ss_out || p.a8_out);
  float xo[8];
  epi_store<MODE, false, SP>(p, m, nn, vec_ok && cnt == 8, cnt, v, u, r, in, ho, xo);
  if (ho) epi_handoff(p, cnt > 0, m, nn, cnt, xo);
}

// ---------------------------------------------------------------------------
// Host side: validation and kernel selection
// ---------------------------------------------------------------------------
struct SkinnyPlan {
  int n_tiles, splits;
  int rb, row_groups;  // activation row blocks per workgroup, row groups
  int64_t kc, ws_bytes;
};

// 16-column tiles over the whole K.  A split of K costs a round trip through
// the device-coherent level (~4 us measured), so K is split only when one
// workgroup would otherwise stream more than ~400 KB of operands (64
// activation rows + 16 NB weight rows per k), and never beyond 256
// workgroups.  Ranges are multiples of 8 waves x 32 k.
static SkinnyPlan plan_skinny(const GemmArgs& d) {
  SkinnyPlan s;
  const int nb = d.mode == FVX_GEMM_GEGLU ? 2 : 1;
  s.n_tiles = (int)((d.n + 15) / 16);
  const bool f8 = d.b_fp8 != 0, a16 = f8 && !d.fp8_act;
  // Fewer activation row blocks per workgroup spread a GEMM with few column
  // tiles over more CUs with no K split: per-CU operand bytes, not HBM,
  // bound these kernels (~115 GB/s per CU from L2).  The smallest row block
  // count whose grid still fits one workgroup per CU wins; past 256
  // workgroups the second round costs more than the narrower tiles save.
  s.rb = 4;
  if (!(f8 && !a16) && d.split_k <= 0) {
    for (int rb = 1; rb < 4; rb *= 2) {
      const int64_t groups = (d.m + 16 * rb - 1) / (16 * rb);
      const int64_t bytes = (16 * rb * 2 + 16 * nb * (f8 ? 1 : 2)) * d.k;
      if (s.n_tiles * groups <= 256 && bytes <= 400 * 1024) {
        s.rb = rb;
        break;
      }
    }
  }
  s.row_groups = (int)((d.m + 16 * s.rb - 1) / (16 * s.rb));
  if (s.row_groups < 1) s.row_groups = 1;
  const int64_t unit = (int64_t)sk_kgran(f8, a16) * sk_waves(f8, a16);
  const int64_t max_splits = (d.k + unit - 1) / unit;
  int64_t sp = d.split_k;
  if (sp <= 0 && s.rb < 4) sp = 1;
  if (sp <= 0) {
    const int64_t bytes = (64 * 2 + 16 * nb * (d.b_fp8 ? 1 : 2)) * d.k;
    sp = (bytes + 400 * 1024 - 1) / (400 * 1024);
    const int64_t cap = 256 / s.n_tiles;
    if (sp > cap) sp = cap;
  }
  if (sp > kSkMaxSplits) sp = kSkMaxSplits;
  if (sp > max_splits) sp = max_splits;
  if (sp < 1) sp = 1;
  int64_t kc = (d.k + sp - 1) / sp;
  kc = (kc + unit - 1) / unit * unit;
  s.splits = (int)((d.k + kc - 1) / kc);
  s.kc = kc;
  s.ws_bytes = s.splits > 1 ? kCounterBytes + (int64_t)s.n_tiles * s.row_groups * s.splits *
                                                   skinny_block_floats(nb) * 4
                             : 0;
  return s;
}

// The skinny kernel serves M <= 64 while its arrival counters fit the
// counter area and its partial offsets fit 31 bits; anything else is tiled.
// A's rows in groups with gaps between them (fvx_gemm_desc.a_row_group)
static bool a_grouped(const GemmArgs& d) { return d.a_row_group > 0 && d.m > d.a_row_group; }

static bool use_skinny(const GemmArgs& d) {
  if (d.m > 64 || a_grouped(d)) return false;
  if (d.b_fp8 && !d.b_frag) return false;  // fp8 skinny reads fragment-major B
  const SkinnyPlan s = plan_skinny(d);
  // operand byte offsets are 32-bit
  const int64_t a_bytes = d.a_frag ? (d.k / 32) * 4 * 1024 : 64 * d.lda * 2;
  const int64_t b_bytes = d.b_frag ? (int64_t)s.n_tiles * 16 * d.k * (d.b_fp8 ? 1 : 2)
                                   : (int64_t)s.n_tiles * 16 * d.ldb * 2;
  return s.n_tiles * s.row_groups <= kMaxSkinnyTiles && s.ws_bytes < ((int64_t)1 << 31) &&
         a_bytes < ((int64_t)1 << 31) && b_bytes < ((int64_t)1 << 31);
}

static int validate(const GemmArgs& d) {
  FVX_REQUIRE(d.a && d.b, FVX_ERR_NULL, "gemm: a and b are required");
  FVX_REQUIRE(d.m >= 0 && d.n > 0 && d.k > 0, FVX_ERR_SHAPE,
              "gemm: need m >= 0, n > 0, k > 0 (m=%lld n=%lld k=%lld)",
              (long long)d.m, (long long)d.n, (long long)d.k);
  FVX_REQUIRE(d.k % 8 == 0 && d.lda % 8 == 0 && d.ldb % 8 == 0 &&
                  d.lda >= d.k && d.ldb >= d.k,
              FVX_ERR_SHAPE,
              "gemm: k, lda, ldb must be multiples of 8 with lda, ldb >= k "
              "(k=%lld lda=%lld ldb=%lld)",
              (long long)d.k, (long long)d.lda, (long long)d.ldb);
  FVX_REQUIRE(aligned16(d.a) && aligned16(d.b) && aligned16(d.b2),
              FVX_ERR_ALIGN, "gemm: a, b, b2 must be 16B aligned");
  FVX_REQUIRE(d.mode >= 0 && d.mode <= 3, FVX_ERR_ARG, "gemm: bad mode %d",
              d.mode);
  FVX_REQUIRE(d.act >= 0 && d.act <= 2, FVX_ERR_ARG, "gemm: bad act %d",
              d.act);
  FVX_REQUIRE(!d.ss_out || (d.mode == FVX_GEMM_PLAIN && d.m > 64 && d.ss_ld >= d.m &&
                            aligned16(d.ss_out)),
              FVX_ERR_ARG, "gemm: ss_out needs mode PLAIN, m > 64 and ss_ld >= m");
  FVX_REQUIRE(!d.ss_in || (d.rownorm && d.ss_parts > 0 && d.ss_ld >= d.m), FVX_ERR_ARG,
              "gemm: ss_in needs rownorm, ss_parts > 0 and ss_ld >= m");
  {
    // the kernels address the row-sum arrays with 32-bit byte offsets
    const int64_t parts_in = d.ss_in ? d.ss_parts : 0;
    const int64_t parts_out = d.ss_out ? (d.n + 63) / 64 : 0;
    const int64_t parts = parts_in > parts_out ? parts_in : parts_out;
    FVX_REQUIRE(parts == 0 || parts * d.ss_ld < ((int64_t)1 << 29), FVX_ERR_ARG,
                "gemm: row-sum arrays must hold fewer than 2^29 floats (parts %lld, ss_ld %lld)",
                (long long)parts, (long long)d.ss_ld);
  }
  FVX_REQUIRE(d.a_row_group >= 0 && d.a_row_group < ((int64_t)1 << 31) &&
                  (d.a_row_group == 0 ||
                   (d.a_row_group_stride >= d.a_row_group &&
                    d.a_row_group_stride < ((int64_t)1 << 31))),
              FVX_ERR_SHAPE, "gemm: need 0 <= a_row_group <= a_row_group_stride < 2^31");
  if (a_grouped(d)) {
    const int64_t last = (d.m - 1) / d.a_row_group * d.a_row_group_stride +
                         (d.m - 1) % d.a_row_group;
    FVX_REQUIRE(!d.a_frag && !d.a8 && (last + 1) * d.lda * 2 < ((int64_t)1 << 31), FVX_ERR_ARG,
                "gemm: grouped A rows take a row-major bf16 A below 2 GiB");
  }
  FVX_REQUIRE(!d.ln_csum || (d.mode == FVX_GEMM_PLAIN && d.rownorm && !d.ss_in && d.m > 64 &&
                             d.split_k <= 1 && !d.b_fp8 && !d.a_scale && !d.ss_out &&
                             !d.a8_out),
              FVX_ERR_ARG,
              "gemm: ln_csum needs mode PLAIN, rownorm without ss_in, m > 64, one K range, "
              "bf16 weights and no hand-over outputs");
  FVX_REQUIRE(!d.a8_out || ((d.mode == FVX_GEMM_PLAIN || d.mode == FVX_GEMM_GEGLU) &&
                            !d.out_f32 && d.m > 64 && d.a8_out_scale &&
                            d.a8_out_ld >= d.n && d.a8_out_ld % 8 == 0 &&
                            d.a8_out_sld >= d.m && ((uintptr_t)d.a8_out & 7) == 0),
              FVX_ERR_ARG,
              "gemm: a8_out needs mode PLAIN or GEGLU, a bf16 output, m > 64, "
              "a8_out_scale, a8_out_ld >= n (multiple of 8), a8_out_sld >= m");
  FVX_REQUIRE(!d.a8 || (d.a8_scale && d.a8_ld >= d.k && d.a8_ld % 16 == 0 &&
                        d.a8_sld >= d.m && d.a8_sld % 4 == 0 && aligned16(d.a8) &&
                        ((uintptr_t)d.a8_scale & 3) == 0),
              FVX_ERR_ARG,
              "gemm: a8 needs a8_scale, a8_ld >= k (multiple of 16, 16B aligned) "
              "and a8_sld >= m (multiple of 4)");
  FVX_REQUIRE(!d.rownorm || d.rownorm_eps >= 0.f, FVX_ERR_ARG,
              "gemm: rownorm_eps must be >= 0");
  FVX_REQUIRE(d.row_group >= 0, FVX_ERR_ARG, "gemm: row_group must be >= 0");
  FVX_REQUIRE(d.m < ((int64_t)1 << 31) && d.row_group < ((int64_t)1 << 31) &&
                  d.gate_group < ((int64_t)1 << 31) && d.pos_period < ((int64_t)1 << 31) &&
                  d.rtc_period < ((int64_t)1 << 31),
              FVX_ERR_SHAPE,
              "gemm: m, row_group, gate_group, pos_period and rtc_period must be < 2^31");
  switch (d.mode) {
    case FVX_GEMM_PLAIN:
      FVX_REQUIRE(d.c, FVX_ERR_NULL, "gemm: c is required");
      FVX_REQUIRE(d.ldc >= d.n, FVX_ERR_SHAPE, "gemm: ldc < n");
      FVX_REQUIRE(!d.gate || d.gate_group > 0, FVX_ERR_ARG,
                  "gemm: gate_group must be > 0 when gate is given");
      FVX_REQUIRE(!d.pos || d.pos_period > 0, FVX_ERR_ARG,
                  "gemm: pos_period must be > 0 when pos is given");
      break;
    case FVX_GEMM_GEGLU:
      FVX_REQUIRE(d.c && d.b2, FVX_ERR_NULL, "gemm(geglu): c and b2 required");
      FVX_REQUIRE(d.ldc >= d.n, FVX_ERR_SHAPE, "gemm: ldc < n");
      break;
    case FVX_GEMM_QKV_ROPE:
      FVX_REQUIRE(d.rope && d.positions && d.q_out && d.k_out && d.v_out,
                  FVX_ERR_NULL,
                  "gemm(qkv_rope): rope, positions, q_out, k_out, v_out "
                  "required");
      FVX_REQUIRE(d.head_dim > 0 && d.head_dim % 2 == 0 && d.n_q_heads >= 0 &&
                      d.n == (int64_t)(d.n_q_heads + 2) * d.head_dim,
                  FVX_ERR_SHAPE,
                  "gemm(qkv_rope): n must be (n_q_heads + 2) * head_dim with "
                  "even head_dim");
      break;
    case FVX_GEMM_EULER:
      FVX_REQUIRE(d.xt, FVX_ERR_NULL, "gemm(euler): xt required");
      break;
  }
  const bool rtc = d.rtc_lock || d.bias_f32_locked || d.rtc_prev || d.rtc_cw;
  FVX_REQUIRE(!rtc || ((d.mode == FVX_GEMM_PLAIN || d.mode == FVX_GEMM_EULER) &&
                       d.rtc_period > 0),
              FVX_ERR_ARG, "gemm: RTC fields need mode PLAIN or EULER and rtc_period > 0");
  FVX_REQUIRE(!d.bias_f32_locked || (d.rtc_lock && d.bias_f32), FVX_ERR_ARG,
              "gemm: bias_f32_locked needs rtc_lock and bias_f32");
  FVX_REQUIRE(!(d.rtc_prev || d.rtc_cw) || d.mode == FVX_GEMM_EULER, FVX_ERR_ARG,
              "gemm: rtc_prev / rtc_cw need mode EULER");
  FVX_REQUIRE(!d.rtc_cw || d.rtc_prev, FVX_ERR_ARG, "gemm: rtc_cw needs rtc_prev");
  FVX_REQUIRE(!d.a_scale || ((d.mode == FVX_GEMM_QKV_ROPE || d.mode == FVX_GEMM_GEGLU ||
                              d.mode == FVX_GEMM_EULER) &&
                             !(d.b_fp8 && d.fp8_act) && aligned16(d.a_scale) && use_skinny(d)),
              FVX_ERR_ARG,
              "gemm: a_scale needs mode QKV_ROPE, GEGLU or EULER, bf16 activations, "
              "M <= 64 (skinny) and a 16B-aligned bf16 [K] vector");
  FVX_REQUIRE(!((d.mode == FVX_GEMM_QKV_ROPE || d.mode == FVX_GEMM_GEGLU) &&
                (d.bias || ((d.bias_f32 || d.bias2_f32) && !d.a_scale))),
              FVX_ERR_ARG,
              "gemm: QKV_ROPE / GEGLU take fp32 biases only with a_scale, no bf16 bias");
  FVX_REQUIRE(!d.bias2_f32 || d.mode == FVX_GEMM_GEGLU, FVX_ERR_ARG,
              "gemm: bias2_f32 is the GEGLU up half's bias");
  FVX_REQUIRE((!d.k_t_out && !d.v_rows_out) ||
                  (d.mode == FVX_GEMM_QKV_ROPE && d.v_transposed &&
                   (!d.k_t_out || d.ld_kt > 0) &&
                   (!d.v_rows_out || (d.ld_vr >= d.head_dim && d.ld_vr % 8 == 0 &&
                                      aligned16(d.v_rows_out)))),
              FVX_ERR_ARG, "gemm: k_t_out / v_rows_out need QKV_ROPE with a transposed "
                           "v_out (and ld_vr >= head_dim, a multiple of 8)");
  FVX_REQUIRE(!d.gu_out || (d.mode == FVX_GEMM_GEGLU && d.ld_gu >= 2 * d.n &&
                            d.ld_gu % 8 == 0 && aligned16(d.gu_out)),
              FVX_ERR_ARG, "gemm: gu_out needs GEGLU mode, ld_gu >= 2 n (a multiple of 8) "
                           "and a 16-byte aligned buffer");
  FVX_REQUIRE(((uintptr_t)d.bias2_f32 & 15) == 0, FVX_ERR_ALIGN,
              "gemm: bias2_f32 must be 16B aligned");
  FVX_REQUIRE(!d.rtc_prev || (d.ld_prev >= d.n && (d.rtc_lock || d.rtc_cw)), FVX_ERR_ARG,
              "gemm: rtc_prev needs ld_prev >= n and rtc_lock or rtc_cw");
  FVX_REQUIRE(((uintptr_t)d.rtc_lock & 3) == 0 && ((uintptr_t)d.rtc_prev & 3) == 0 &&
                  ((uintptr_t)d.rtc_cw & 3) == 0 && ((uintptr_t)d.bias_f32_locked & 3) == 0,
              FVX_ERR_ALIGN, "gemm: RTC pointers must be 4B aligned");
  FVX_REQUIRE(d.fp8_act == 0 || (d.fp8_act == 1 && d.b_fp8), FVX_ERR_ARG,
              "gemm: fp8_act must be 0, or 1 with b_fp8 (got %d)", d.fp8_act);
  if (d.b_fp8) {
    FVX_REQUIRE(d.b_scale && (d.mode != FVX_GEMM_GEGLU || d.b2_scale), FVX_ERR_NULL,
                "gemm(fp8): b_scale (and b2_scale for GEGLU) required");
    FVX_REQUIRE(aligned16(d.b_scale) && aligned16(d.b2_scale), FVX_ERR_ALIGN,
                "gemm(fp8): weight scales must be 16B aligned");
    FVX_REQUIRE(d.k % 128 == 0 && d.ldb % 16 == 0, FVX_ERR_SHAPE,
                "gemm(fp8): needs k %% 128 == 0 and ldb %% 16 == 0 (k=%lld ldb=%lld)",
                (long long)d.k, (long long)d.ldb);
  }
  if (d.a_frag || d.b_frag || d.c_frag) {
    FVX_REQUIRE(d.m <= 64 && use_skinny(d), FVX_ERR_ARG,
                "gemm: fragment-major operands need m <= 64 (m=%lld)",
                (long long)d.m);
    FVX_REQUIRE(!(d.a_frag || d.b_frag) || d.k % 32 == 0, FVX_ERR_SHAPE,
                "gemm: fragment-major A/B need k %% 32 == 0 (k=%lld)",
                (long long)d.k);
    FVX_REQUIRE(!d.b_frag || d.n % 16 == 0, FVX_ERR_SHAPE,
                "gemm: fragment-major B needs n %% 16 == 0 (n=%lld)",
                (long long)d.n);
    FVX_REQUIRE(!d.c_frag || ((d.mode == FVX_GEMM_PLAIN || d.mode == FVX_GEMM_GEGLU) &&
                              !d.out_f32 && d.n % 32 == 0 && aligned16(d.c_frag)),
                FVX_ERR_ARG,
                "gemm: c_frag needs PLAIN/GEGLU bf16 output, n %% 32 == 0 and a "
                "16B-aligned buffer");
  }
  return FVX_OK;
}

#define FVX_MODE_DISPATCH_NG(MODE_RT, LAUNCH)                 \
  switch (MODE_RT) {                                          \
    case FVX_GEMM_QKV_ROPE: LAUNCH(FVX_GEMM_QKV_ROPE); break; \
    case FVX_GEMM_EULER: LAUNCH(FVX_GEMM_EULER); break;       \
    default: LAUNCH(FVX_GEMM_PLAIN); break;                   \
  }

#define FVX_MODE_DISPATCH(MODE_RT, LAUNCH)         \
  switch (MODE_RT) {                               \
    case FVX_GEMM_PLAIN: LAUNCH(FVX_GEMM_PLAIN); break;       \
    case FVX_GEMM_GEGLU: LAUNCH(FVX_GEMM_GEGLU); break;       \
    case FVX_GEMM_QKV_ROPE: LAUNCH(FVX_GEMM_QKV_ROPE); break; \
    default: LAUNCH(FVX_GEMM_EULER); break;                   \
  }

// Tile configurations: {BM, BN (all weights' columns), waves M x N, stages}.
//   0:  64 x 128, 2 x 2 waves of 32 x 64,  2 stages (48 KiB of LDS: two
//       workgroups per CU)
//   1: 256 x 256, 2 x 4 waves of 128 x 64, 2 stages (128 KiB: one workgroup
//      of 8 waves per CU; half the L2 traffic per flop of a 128 x 128 tile)
//   2:  64 x 128 with 4 stages (96 KiB, one workgroup per CU: three slabs in
//       flight instead of one, for grids that leave CUs free anyway)
// Measured on MI355X (us; bs=1 chunk shapes):
//   prefix GeGLU 816 x 16384 x2 x 2048   128x128: 158, 1: 151 (0: 154)
//   prefix QKV   816 x 2560 x 2048   (260 tiles)   0: 26.2   2: 37.4
//   prefix O     816 x 2048 x 2048   (208 tiles)   0: 23.7   2: 19.9
//   SigLIP fc1   768 x 4304 x 1152   (408 tiles)   0: 23.4   2: 30.4
//   SigLIP fc2   768 x 1152 x 4304   (108 tiles)   0 split 4: 37.6, 2 split 2: 33.6
//   bs=8 QKV     408 x 2560 x 1024   (140 tiles)   0: 16.5   2: 14.1
// Small tiles win on these shapes: the extra workgroups hide more latency
// than they cost in LDS traffic per flop; deeper rings win only when the
// grid leaves CUs idle.
static const int kTileBM[] = {64, 256, 64, 256, 64};
static const int kTileBN[] = {128, 256, 128, 256, 64};
constexpr int kTileCfgs = 5;
constexpr int kWideCfg = 3;  // gemm_wide_kernel
// 4: 64 x 64, 2 x 2 waves of 32 x 32, 4 stages -- bf16 PLAIN / QKV / EULER
// GEMMs with fewer than 128 tiles of 64 x 128 (SigLIP o-proj, fc2: M = 768,
// N = 1152): twice the workgroups instead of idle CUs or a split-K pass
constexpr int kSmallCfg = 4;
#ifndef FVX_WIDE_MIN_TILES
#define FVX_WIDE_MIN_TILES 128
#endif
#ifndef FVX_WIDE_MIN_K
#define FVX_WIDE_MIN_K 2048
#endif
#ifndef FVX_WIDE_F8
#define FVX_WIDE_F8 1
#endif
#ifndef FVX_WIDE_SPLIT_MIN_K
#define FVX_WIDE_SPLIT_MIN_K 8192
#endif
#ifndef FVX_SMALL_TILES
#define FVX_SMALL_TILES 1
#endif
#ifndef FVX_SMALL_STAGES
#define FVX_SMALL_STAGES 4
#endif
#ifndef FVX_SMALL_SPLIT
#define FVX_SMALL_SPLIT 1
#endif
#ifndef FVX_SMALL_SPLIT_MIN_K
#define FVX_SMALL_SPLIT_MIN_K 4096
#endif
#ifndef FVX_SMALL_MAX_TILES
#define FVX_SMALL_MAX_TILES 128
#endif

static int tile_bm(int cfg, int fp8) {
  if (fp8) return cfg == 1 ? 128 : (cfg == 3 ? 256 : 64);
  return kTileBM[cfg];
}

struct TilePlan {
  int cfg, splits;
};

// The wide kernel (bf16, K % 64 == 0, PLAIN / GEGLU / QKV_ROPE) once its
// 256 x 256 tiles number >= 256 (GEGLU) or, for PLAIN / QKV_ROPE, fill the
// CUs (below) with K >= FVX_WIDE_MIN_K; config 1
// for other GeGLU projections with >= 256 such tiles (fp8); else 64 x 128
// tiles: the 4-stage ring (config 2, 96 KiB of LDS, one workgroup per CU)
// when they number <= 256, else the 3-stage ring (config 0, 72 KiB: two
// workgroups per CU share the second round; with cold weights 2 stages lose
// up to 25 % and 4 stages more).  A long
// K (>= 4096) with fewer than 128 tiles is split in two (SigLIP fc2); with
// more tiles the partials cost more than the idle CUs.
// The wide kernels split K for PLAIN GEMMs without a fused RMSNorm;
// the reduce kernel's hand-over outputs need whole 64-column blocks.
static bool wide_split_ok(const GemmArgs& d) {
  return d.mode == FVX_GEMM_PLAIN && (!d.b_fp8 || FVX_WIDE_F8) && !d.rownorm && d.n % 64 == 0;
}

static TilePlan plan_tile(const GemmArgs& d) {
  TilePlan t;
  const bool gg = d.mode == FVX_GEMM_GEGLU;
  const int64_t bn = 128 / (gg ? 2 : 1);
  const int64_t tiles = ((d.m + 63) / 64) * ((d.n + bn - 1) / bn);
  const int64_t wtiles = ((d.m + 255) / 256) * ((d.n + 2 * bn - 1) / (2 * bn));
  const bool wide_ok = (!d.b_fp8 || FVX_WIDE_F8) && d.k % 64 == 0 && d.split_k <= 1 &&
                       !d.ln_csum && !a_grouped(d) && !d.gu_out &&
                       (d.mode == FVX_GEMM_PLAIN || gg || d.mode == FVX_GEMM_QKV_ROPE);
  t.splits = 1;
  // PLAIN / QKV: one workgroup of 256 x 256 per CU at a time, so the tiles
  // must fill the last round (>= 3/4 of 256 CUs) and K must amortize the
  // epilogue's 256 x 256 operand stream (measured: K = 2048 gains a little,
  // K = 1152 loses; 260 tiles lose to the 64 x 128 kernel)
  const int64_t rounds = (wtiles + 255) / 256;
  const bool fill = wtiles >= FVX_WIDE_MIN_TILES && 4 * wtiles >= 3 * 256 * rounds;
  if (wide_ok && (gg ? wtiles >= 256 : (fill && d.k >= FVX_WIDE_MIN_K))) {
    t.cfg = kWideCfg;
    return t;
  }
  // A long K with few wide tiles (the prefix down projection at bs=1: 32
  // tiles, K = 16384): the wide kernel over up to 8 K ranges, one per XCD,
  // so that every byte of A and B passes one L2 (the 64 x 128 grid makes
  // each XCD stream all of A); fp32 partials, then
  // gemm_partial_reduce_kernel runs the epilogue and the hand-overs
  if (wide_ok && wide_split_ok(d) && d.split_k == 0 && d.m > 256 && wtiles <= 64 &&
      d.k >= FVX_WIDE_SPLIT_MIN_K) {
    t.cfg = kWideCfg;
    t.splits = (int)(256 / wtiles < 8 ? 256 / wtiles : 8);
    return t;
  }
  if (gg && wtiles >= 256) t.cfg = 1;
  else t.cfg = tiles <= 256 ? 2 : 0;
  // hand-overs are written by the one-pass epilogue of 64-column waves
  if (d.ss_out || d.a8_out) return t;
  if (FVX_SMALL_TILES && !gg && !d.b_fp8 && d.split_k == 0 && tiles < FVX_SMALL_MAX_TILES) {
    t.cfg = kSmallCfg;
    if (FVX_SMALL_SPLIT > 1 && d.k >= FVX_SMALL_SPLIT_MIN_K && !d.ln_csum)
      t.splits = FVX_SMALL_SPLIT;
    return t;
  }
  if (d.ln_csum) return t;  // one K range
  if (d.split_k > 0) t.splits = d.split_k;
  else if (t.cfg != 1 && tiles < 128 && d.k >= 4096) t.splits = 2;
  return t;
}

// May a PLAIN GEMM's epilogue take the plain-epilogue build (the tile
// kernel's XF bit 3, the skinny kernel's and the split-K reduce's SP)?
// Bias, fp32 bias, activation, a per-row gate, residual, the fragment-major
// copy, the fused RMSNorm and the hand-overs only, bf16 output rows below
// 2^31 elements from the start of c, of the residual and of the gate.
static bool plain_epilogue_ok(const GemmArgs& d) {
  return d.mode == FVX_GEMM_PLAIN && !d.pos && !d.out_f32 && d.row_group == 0 && !d.rtc_lock &&
         !d.bias_f32_locked && !d.ln_csum && d.m * d.ldc < ((int64_t)1 << 31) &&
         (!d.residual || d.m * d.ldr < ((int64_t)1 << 31)) &&
         (!d.gate || (d.gate_group <= 1 && d.m * d.ldg < ((int64_t)1 << 31)));
}

// The tile kernel build for a launch: xf = the row-sum paths it needs
// (gemm_tile_kernel's XF; bits 1 and 2 only matter for PLAIN, and a folded
// LayerNorm hands nothing over) and bit 3 for the plain epilogue.  fp8-weight
// tiles keep one build with the row-sum paths but the LayerNorm.
template <int BM, int BN, int WGM, int WGN, int ST, int MODE, bool F8, bool A16>
static void launch_tile(dim3 grid, hipStream_t s, const GemmArgs& d, int xf, int m_tiles,
                        int n_tiles, int splits, int64_t kchunk, int vec_ok) {
  auto go = [&](auto xc) {
    constexpr int X = decltype(xc)::value;
    hipLaunchKernelGGL((gemm_tile_kernel<BM, BN, WGM, WGN, ST, MODE, F8, A16, X>), grid,
                       dim3(64 * WGM * WGN), 0, s, d, m_tiles, n_tiles, splits, kchunk,
                       vec_ok);
  };
  if constexpr (F8) {
    go(IntC<3>{});
  } else if constexpr (MODE != FVX_GEMM_PLAIN) {
    if (xf & 1) go(IntC<1>{});
    else go(IntC<0>{});
  } else {
    switch (xf) {
      case 0: go(IntC<0>{}); break;
      case 1: go(IntC<1>{}); break;
      case 2: go(IntC<2>{}); break;
      case 3: go(IntC<3>{}); break;
      case 4: go(IntC<4>{}); break;  // folded LayerNorm, alone
      case 8: go(IntC<8>{}); break;
      case 10: go(IntC<10>{}); break;
      default: go(IntC<3>{}); break;
    }
  }
}

// bf16 256 x 256 tiles (config 1): GEGLU only (the planner's choice for
// GeGLU projections with >= 256 wide tiles)
template <int MODE>
static void launch_big_tile(dim3 grid, hipStream_t s, const GemmArgs& d, int xf, int m_tiles,
                            int n_tiles, int splits, int64_t kchunk, int vec_ok) {
  if constexpr (MODE == FVX_GEMM_GEGLU)
    launch_tile<256, 256, 2, 4, 2, MODE, false, false>(grid, s, d, xf, m_tiles, n_tiles, splits,
                                                       kchunk, vec_ok);
}

// 64 x 64 tiles (kSmallCfg): not instantiated for GEGLU, whose tiles hold
// two weights' columns
template <int MODE>
static void launch_small_tile(dim3 grid, hipStream_t s, const GemmArgs& d, int xf, int m_tiles,
                              int n_tiles, int splits, int64_t kchunk, int vec_ok) {
  if constexpr (MODE != FVX_GEMM_GEGLU)
    launch_tile<64, 64, 2, 2, FVX_SMALL_STAGES, MODE, false, false>(
        grid, s, d, xf, m_tiles, n_tiles, splits, kchunk, vec_ok);
}

static int run_tile(GemmArgs d, int cfg, int splits, hipStream_t s) {
  FVX_REQUIRE(cfg >= 0 && cfg < kTileCfgs, FVX_ERR_ARG, "gemm: bad tile config %d", cfg);
  FVX_REQUIRE(cfg != 1 || d.mode == FVX_GEMM_GEGLU || d.b_fp8, FVX_ERR_ARG,
              "gemm: the bf16 256 x 256 tile configuration is built for GEGLU only");
  FVX_REQUIRE(cfg != kSmallCfg || (d.mode != FVX_GEMM_GEGLU && !d.b_fp8), FVX_ERR_ARG,
              "gemm: the 64 x 64 tile configuration takes no GEGLU / fp8 weights");
  FVX_REQUIRE(cfg != kSmallCfg || (!d.a8_out && !d.ss_out), FVX_ERR_ARG,
              "gemm: the 64 x 64 tile configuration hands nothing over");
  const bool gg = d.mode == FVX_GEMM_GEGLU;
  const int bm = tile_bm(cfg, d.b_fp8), bn = kTileBN[cfg] / (gg ? 2 : 1);
  const int m_tiles = (int)((d.m + bm - 1) / bm);
  const int n_tiles = (int)((d.n + bn - 1) / bn);
  // hand-overs come from a one-pass epilogue, except through the reduce
  // kernel behind a split wide kernel
  if (splits < 1 ||
      (cfg == kWideCfg ? !wide_split_ok(d) : (d.ss_out || d.a8_out || d.ln_csum)))
    splits = 1;
  const int64_t bk = d.b_fp8 ? 128 : 64;
  int64_t kchunk = (d.k + splits - 1) / splits;
  kchunk = (kchunk + bk - 1) / bk * bk;
  splits = (int)((d.k + kchunk - 1) / kchunk);
  const int nbm = gg ? 2 : 1;
  const int64_t need = splits > 1 ? kCounterBytes + ((int64_t)nbm * splits * d.m * d.n +
                                                     (int64_t)splits * d.m) * 4
                                   : 0;
  // the partials are read through one buffer view (< 2 GiB)
  if (splits > 1 && (!d.workspace || d.workspace_bytes < need || need >= ((int64_t)1 << 31))) {
    if (d.split_k > 1)
      return set_error(FVX_ERR_WORKSPACE,
                       "gemm: split_k=%d needs %lld workspace bytes (below 2 GiB), got %lld",
                       d.split_k, (long long)need, (long long)d.workspace_bytes);
    splits = 1;
    kchunk = d.k;
  }
  FVX_REQUIRE(splits == 1 || aligned16(d.workspace), FVX_ERR_ALIGN,
              "gemm: workspace must be 16B aligned");
  const int vec_ok = epi_vec_ok(d) ? 1 : 0;
  FVX_REQUIRE(!(gg && d.a8_out) || cfg == kWideCfg, FVX_ERR_ARG,
              "gemm: a8_out on a GeGLU GEMM needs the wide kernel (>= 256 of its tiles)");
  if (cfg == kWideCfg) {
    FVX_REQUIRE(d.k % 64 == 0 && d.mode != FVX_GEMM_EULER, FVX_ERR_ARG,
                "gemm: the wide kernel needs K %% 64 == 0, no EULER");
    // 256 x 256 tiles (GEGLU: 256 x 2 x 128), 4 waves of 128 x 128; with
    // splits, (split, tile) workgroups
    const unsigned nb = (unsigned)(m_tiles * n_tiles);
    const unsigned nbs = nb * (unsigned)splits;
#define LW(MODE)                                                                       \
  if (d.rownorm && !d.ss_in)                                                           \
    hipLaunchKernelGGL((gemm_wide_kernel<MODE, true, wide_waves<MODE>()>), dim3(nbs),    \
                       dim3(64 * wide_waves<MODE>()), 0, s, d, m_tiles, n_tiles, vec_ok, \
                       splits,                                                         \
                       (int)kchunk);                                                   \
  else                                                                                 \
    hipLaunchKernelGGL((gemm_wide_kernel<MODE, false, wide_waves<MODE>()>), dim3(nbs),   \
                       dim3(64 * wide_waves<MODE>()), 0, s, d, m_tiles, n_tiles, vec_ok, \
                       splits,                                                         \
                       (int)kchunk)
    // the e4m3 copy of A is used when given (a rownorm then needs ss_in)
    const bool f8a = d.a8 && d.a8_scale && (!d.rownorm || d.ss_in);
#define LW8(MODE)                                                                           \
  if (!d.fp8_act && d.rownorm && !d.ss_in)                                                  \
    hipLaunchKernelGGL((gemm_wide_f8_kernel<MODE, true, false, true>), dim3(nbs), dim3(256), \
                       0, s, d, m_tiles, n_tiles, vec_ok, splits, (int)kchunk);             \
  else if (!d.fp8_act)                                                                      \
    hipLaunchKernelGGL((gemm_wide_f8_kernel<MODE, false, false, true>), dim3(nbs), dim3(256),\
                       0, s, d, m_tiles, n_tiles, vec_ok, splits, (int)kchunk);             \
  else if (d.rownorm && !d.ss_in)                                                           \
    hipLaunchKernelGGL((gemm_wide_f8_kernel<MODE, true, false, false>), dim3(nbs), dim3(256),\
                       0, s, d, m_tiles, n_tiles, vec_ok, splits, (int)kchunk);             \
  else if (f8a)                                                                             \
    hipLaunchKernelGGL((gemm_wide_f8_kernel<MODE, false, true, false>), dim3(nbs), dim3(256),\
                       0, s, d, m_tiles, n_tiles, vec_ok, splits, (int)kchunk);             \
  else                                                                                      \
    hipLaunchKernelGGL((gemm_wide_f8_kernel<MODE, false, false, false>), dim3(nbs),         \
                       dim3(256), 0, s, d, m_tiles, n_tiles, vec_ok, splits, (int)kchunk)
    if (d.b_fp8) {
      switch (d.mode) {
        case FVX_GEMM_GEGLU: LW8(FVX_GEMM_GEGLU); break;
        case FVX_GEMM_QKV_ROPE: LW8(FVX_GEMM_QKV_ROPE); break;
        default: LW8(FVX_GEMM_PLAIN); break;
      }
    } else {
      switch (d.mode) {
        case FVX_GEMM_GEGLU: LW(FVX_GEMM_GEGLU); break;
        case FVX_GEMM_QKV_ROPE: LW(FVX_GEMM_QKV_ROPE); break;
        default: LW(FVX_GEMM_PLAIN); break;
      }
    }
#undef LW8
#undef LW
    const int stw = launch_status("gemm(wide)");
    if (stw || splits == 1) return stw;
  } else {
    dim3 grid((unsigned)(m_tiles * n_tiles), (unsigned)splits);
    // row-sum paths: handed-over sums read (the tile kernel's bit-0 build
    // has no K-loop sum of squares), hand-over outputs (one-pass epilogue)
    int xf = ((d.rownorm && d.ss_in) ? 1 : 0) |
             ((splits == 1 && (d.ss_out || d.a8_out)) ? 2 : 0) | (d.ln_csum ? 4 : 0);
    if ((xf == 0 || xf == 2) && !d.b_fp8 && splits == 1 && plain_epilogue_ok(d)) xf |= 8;
#define LT(BM_, BN_, WGM_, WGN_, ST_, MODE, F8_, A16_)                                 \
    launch_tile<BM_, BN_, WGM_, WGN_, ST_, MODE, F8_, A16_>(grid, s, d, xf, m_tiles,    \
                                                           n_tiles, splits, kchunk, vec_ok)
    // fp8 tiles hold 128-k slabs (bf16 A rows of 256 bytes): config 1 becomes
    // 128 x 256 to stay within the LDS
#define LCFG8(MODE, A16_)                                                             \
      if (cfg == 1) LT(128, 256, 2, 4, 2, MODE, true, A16_);                          \
      else if (cfg == 2) LT(64, 128, 2, 2, 4, MODE, true, A16_);                      \
      else LT(64, 128, 2, 2, 2, MODE, true, A16_);
#define LCFG(MODE)                                                                    \
    if (d.b_fp8 && d.fp8_act) {                                                       \
      LCFG8(MODE, false)                                                              \
    } else if (d.b_fp8) {                                                             \
      LCFG8(MODE, true)                                                               \
    } else {                                                                          \
      if (cfg == 1)                                                                   \
        launch_big_tile<MODE>(grid, s, d, xf, m_tiles, n_tiles, splits, kchunk, vec_ok); \
      else if (cfg == 2) LT(64, 128, 2, 2, 4, MODE, false, false);                    \
      else if (cfg == kSmallCfg)                                                      \
        launch_small_tile<MODE>(grid, s, d, xf, m_tiles, n_tiles, splits, kchunk, vec_ok); \
      else LT(64, 128, 2, 2, 3, MODE, false, false);                                  \
    }
    FVX_MODE_DISPATCH(d.mode, LCFG)
#undef LCFG
#undef LCFG8
#undef LT
    int st3 = launch_status("gemm(tile)");
    if (st3 || splits == 1) return st3;
  }
  const int64_t chunks = d.m * ((d.n + 7) / 8);
  const dim3 rgrid((unsigned)((chunks + 255) / 256));
  if (plain_epilogue_ok(d)) {
    hipLaunchKernelGGL((gemm_partial_reduce_kernel<FVX_GEMM_PLAIN, true>), rgrid, dim3(256), 0,
                       s, d, splits, vec_ok);
    return launch_status("gemm(reduce)");
  }
#define L(MODE)                                                                           \
  hipLaunchKernelGGL(gemm_partial_reduce_kernel<MODE>, rgrid, dim3(256), 0, s, d, splits, \
                     vec_ok)
  FVX_MODE_DISPATCH(d.mode, L)
#undef L
  return launch_status("gemm(reduce)");
}

}  // namespace fvx

using namespace fvx;

extern "C" int64_t fvx_gemm_workspace_bytes(const fvx_gemm_desc* d) {
  if (!d || d->m <= 0) return 0;
  if (use_skinny(*d)) return plan_skinny(*d).ws_bytes;
  // tiled path: fp32 partials (+ row sums) of every K split
  const int64_t sp = plan_tile(*d).splits;
  if (sp <= 1) return 0;
  const int nb = d->mode == FVX_GEMM_GEGLU ? 2 : 1;
  const int64_t need = kCounterBytes + ((int64_t)nb * sp * d->m * d->n + sp * d->m) * 4;
  return need < ((int64_t)1 << 31) ? need : 0;  // larger: the launch runs unsplit
}

// Skinny GEMMs with the adaptive RMSNorm folded in (a_scale): QKV_ROPE,
// GEGLU and EULER, bf16 or W8A16 weights.
template <int MODE>
static void launch_skinny_asc(const GemmArgs& d, const SkinnyPlan& sp, dim3 grid,
                              hipStream_t s, int vec_ok) {
  if constexpr (MODE == FVX_GEMM_PLAIN) {
    return;  // refused by validate()
  } else {
#define LA(F8, RBV)                                                                   \
  hipLaunchKernelGGL((gemm_skinny_kernel<MODE, F8, F8, RBV, true>), grid,             \
                     dim3(64 * sk_waves(F8, F8)), 0, s, d, sp.splits, sp.kc, vec_ok)
    if (d.b_fp8) {
      if (sp.rb == 1) LA(true, 1); else if (sp.rb == 2) LA(true, 2); else LA(true, 4);
    } else {
      if (sp.rb == 1) LA(false, 1); else if (sp.rb == 2) LA(false, 2); else LA(false, 4);
    }
#undef LA
  }
}

extern "C" int fvx_gemm(const fvx_gemm_desc* dp, void* stream) {
  clear_error();
  FVX_REQUIRE(dp, FVX_ERR_NULL, "gemm: descriptor is NULL");
  GemmArgs d = *dp;
  int st = validate(d);
  if (st) return st;
  if (d.m == 0) return FVX_OK;
  hipStream_t s = (hipStream_t)stream;
  if (use_skinny(d)) {
    SkinnyPlan sp = plan_skinny(d);
    if (sp.splits > 1 && (!d.workspace || d.workspace_bytes < sp.ws_bytes))
      return set_error(FVX_ERR_WORKSPACE,
                       "gemm: m=%lld n=%lld k=%lld needs %lld workspace bytes "
                       "for %d K ranges, got %lld",
                       (long long)d.m, (long long)d.n, (long long)d.k,
                       (long long)sp.ws_bytes, sp.splits,
                       (long long)d.workspace_bytes);
    FVX_REQUIRE(aligned16(d.workspace), FVX_ERR_ALIGN,
                "gemm: workspace must be 16B aligned");
    dim3 grid((unsigned)sp.n_tiles, (unsigned)sp.splits, (unsigned)sp.row_groups);
    const int vec_ok = epi_vec_ok(d) ? 1 : 0;
    // bf16 PLAIN calls that the plain epilogue covers take its build
    if (d.mode == FVX_GEMM_PLAIN && !d.b_fp8 && !d.a_scale && plain_epilogue_ok(d)) {
#define LS(RB_)                                                                          \
  hipLaunchKernelGGL((gemm_skinny_kernel<FVX_GEMM_PLAIN, false, false, RB_, false, true>), \
                     grid, dim3(64 * kSkWaves), 0, s, d, sp.splits, sp.kc, vec_ok)
      if (sp.rb == 1) LS(1);
      else if (sp.rb == 2) LS(2);
      else LS(4);
#undef LS
      return launch_status("gemm(skinny)");
    }
#define L(MODE)                                                                 \
  if (d.b_fp8 && d.fp8_act)                                                      \
    hipLaunchKernelGGL((gemm_skinny_kernel<MODE, true, false, 4, false>), grid,  \
                       dim3(64 * sk_waves(true, false)), 0, s, d, sp.splits, sp.kc, vec_ok); \
  else if (d.a_scale)                                                           \
    launch_skinny_asc<MODE>(d, sp, grid, s, vec_ok);                             \
  else if (d.b_fp8 && sp.rb == 1)                                                \
    hipLaunchKernelGGL((gemm_skinny_kernel<MODE, true, true, 1, false>), grid,   \
                       dim3(64 * sk_waves(true, true)), 0, s, d, sp.splits, sp.kc, vec_ok); \
  else if (d.b_fp8 && sp.rb == 2)                                                \
    hipLaunchKernelGGL((gemm_skinny_kernel<MODE, true, true, 2, false>), grid,   \
                       dim3(64 * sk_waves(true, true)), 0, s, d, sp.splits, sp.kc, vec_ok); \
  else if (d.b_fp8)                                                              \
    hipLaunchKernelGGL((gemm_skinny_kernel<MODE, true, true, 4, false>), grid,   \
                       dim3(64 * sk_waves(true, true)), 0, s, d, sp.splits, sp.kc, vec_ok); \
  else if (sp.rb == 1)                                                           \
    hipLaunchKernelGGL((gemm_skinny_kernel<MODE, false, false, 1, false>), grid, \
                       dim3(64 * kSkWaves), 0, s, d, sp.splits, sp.kc, vec_ok);  \
  else if (sp.rb == 2)                                                           \
    hipLaunchKernelGGL((gemm_skinny_kernel<MODE, false, false, 2, false>), grid, \
                       dim3(64 * kSkWaves), 0, s, d, sp.splits, sp.kc, vec_ok);  \
  else                                                                           \
    hipLaunchKernelGGL((gemm_skinny_kernel<MODE, false, false, 4, false>), grid, \
                       dim3(64 * kSkWaves), 0, s, d, sp.splits, sp.kc, vec_ok)
    FVX_MODE_DISPATCH(d.mode, L)
#undef L
    return launch_status("gemm(skinny)");
  }
  TilePlan tp = plan_tile(d);
  return run_tile(d, tp.cfg, tp.splits, s);
}

// ---------------------------------------------------------------------------
// fvx_gemm_noalloc: fvx_gemm with its split-K scratch in a file-scope device
// array instead of a caller-passed workspace, for callers that cannot
// allocate.  The array's name is only a host-side stand-in: its device
// address (one copy per GPU) comes from hipGetSymbolAddress, taken once per
// device with that device current, and only that address is handed to
// kernels.  The first kCounterBytes hold the split-K arrival counters, which
// must start at zero: a fill kernel clears them at set-up and every call
// leaves them zero again.  Calls that overlap on one GPU share the array and
// race.
// ---------------------------------------------------------------------------
namespace fvx {

constexpr int64_t kScratchBytes = FVX_GEMM_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

__global__ void scratch_clear_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

constexpr int kScratchMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kScratchMaxDevices];  // device address per GPU

// Device address of `scratch` on the stream's device (set up on first use).
static int scratch_for_stream(hipStream_t s, void** out) {
  int dev = -1, cur = -1;
  hipError_t e = hipStreamGetDevice(s, &dev);
  if (e == hipSuccess) e = hipGetDevice(&cur);
  if (e != hipSuccess)
    return set_error(FVX_ERR_LAUNCH, "gemm_noalloc: device query failed: %s",
                     hipGetErrorString(e));
  FVX_REQUIRE(dev >= 0 && dev < kScratchMaxDevices, FVX_ERR_ARG,
              "gemm_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess)
      return set_error(FVX_ERR_LAUNCH, "gemm_noalloc: hipSetDevice(%d) failed: %s", dev,
                       hipGetErrorString(e));
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) hipSetDevice(cur);
    if (e != hipSuccess || !p)
      return set_error(FVX_ERR_LAUNCH, "gemm_noalloc: hipGetSymbolAddress failed: %s",
                       hipGetErrorString(e));
    const int words = kCounterBytes / 4;
    hipLaunchKernelGGL(scratch_clear_kernel, dim3((words + 255) / 256), dim3(256), 0, s,
                       (uint32_t*)p, words);
    const int st = launch_status("gemm_noalloc(clear)");
    if (st) return st;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FVX_OK;
}

}  // namespace fvx

extern "C" int fvx_gemm_noalloc(const fvx_gemm_desc* dp, void* stream) {
  clear_error();
  FVX_REQUIRE(dp, FVX_ERR_NULL, "gemm_noalloc: descriptor is NULL");
  fvx_gemm_desc d = *dp;
  d.workspace = nullptr;
  d.workspace_bytes = 0;
  const int64_t need = fvx_gemm_workspace_bytes(&d);
  if (need > kScratchBytes)
    return set_error(FVX_ERR_WORKSPACE,
                     "gemm_noalloc: m=%lld n=%lld k=%lld needs %lld bytes of split-K "
                     "scratch; the static scratch holds %lld",
                     (long long)d.m, (long long)d.n, (long long)d.k, (long long)need,
                     (long long)kScratchBytes);
  void* ws = nullptr;
  const int st = scratch_for_stream((hipStream_t)stream, &ws);
  if (st) return st;
  d.workspace = ws;
  d.workspace_bytes = kScratchBytes;
  return fvx_gemm(&d, stream);
}
