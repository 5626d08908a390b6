// bf16 MFMA GEMM family with fused epilogues (gfx950).
//
//   acc[m][n] = sum_k A[m][k] * B[n][k]      A: activations, B: nn.Linear weight
//
// Two kernels share one epilogue:
//
//  * gemm_tile_kernel<BM, BN, MODE>: 256 threads, 2x2 waves, BMxBN output tile,
//    K staged through LDS 64 at a time (register prefetch of the next K slab
//    while the current one feeds v_mfma_f32_16x16x32_bf16).  Used when M > 64
//    (SigLIP M=768, Gemma prefix M=816, batched expert).  Tiles are ordered
//    m-fastest within an n-panel and block ids are remapped so that one XCD
//    owns consecutive tiles: the m-tiles of one weight panel run on the same
//    XCD back to back and reuse that panel from its L2.
//
//  * gemm_skinny_kernel<MODE>: M <= 64 (the bs=1 action expert, M=50/51).
//    The op is a weight stream: each wave owns 16 output columns and pulls
//    its weight rows straight from HBM as MFMA B fragments (16 contiguous
//    bytes per lane); the activation slab is staged once per workgroup in
//    LDS.  K is split over blockIdx.y in ranges of <= 256 so that ~256+
//    workgroups stream weights; fp32 partials go to a workspace and
//    gemm_partial_reduce_kernel, the next kernel on the stream, sums them in
//    split order (deterministic) and runs the epilogue.  (A single-kernel
//    variant in which the last workgroup to arrive reduced the partials
//    behind device-scope fences cost 30-40 us per GEMM on MI355X: the
//    agent-scope release/acquire writes back and invalidates the per-XCD
//    L2.)
//
// Per-row RMSNorm ("rownorm") is fused: the kernel that streams A also
// accumulates sum(A[m][:]^2) and scales the accumulator by
// rsqrt(mean + eps) in the epilogue, so (x * r) @ W' == r * (x @ W') needs no
// separate normalization pass (the (1 + w) Gemma scale is folded into W').
#include "capi_util.h"
#include "common.h"

namespace fvx {

typedef fvx_gemm_desc GemmArgs;


__device__ __forceinline__ int64_t out_row(const GemmArgs& p, int64_t m) {
  return p.row_group > 0
             ? (m / p.row_group) * p.row_group_stride + (m % p.row_group)
             : m;
}

// Epilogue for one MFMA output fragment: rows row0 + j (j < 4) of column n.
// v: main accumulator, u: GEGLU up accumulator, pv: value of column n ^ 1
// (QKV_ROPE partner), rs: per-row RMS factors (used when p.rownorm).
template <int MODE, int NR = 4>
__device__ __forceinline__ void epilogue4(const GemmArgs& p, int64_t row0,
                                          int64_t n, const float* v,
                                          const float* u, const float* pv,
                                          const float* rs) {
  if (n >= p.n) return;
#pragma unroll
  for (int j = 0; j < NR; ++j) {
    const int64_t m = row0 + j;
    if (m >= p.m) break;
    const float r = p.rownorm ? rs[j] : 1.f;
    float x = v[j] * r;
    if (MODE == FVX_GEMM_GEGLU) {
      x = gelu_tanh(x) * (u[j] * r);
      ((bf16_t*)p.c)[out_row(p, m) * p.ldc + n] = f2bf(x);
      continue;
    }
    if (MODE == FVX_GEMM_QKV_ROPE) {
      const int hd = p.head_dim;
      const int64_t qcols = (int64_t)p.n_q_heads * hd;
      if (n < qcols + hd) {
        const int i = (int)(n % hd) >> 1;
        const float2 cs =
            *(const float2*)(p.rope + ((int64_t)p.positions[m] * (hd >> 1) + i) * 2);
        const float px = pv[j] * r;
        x = (n & 1) ? (x * cs.x + px * cs.y) : (x * cs.x - px * cs.y);
        if (n < qcols)
          ((bf16_t*)p.q_out)[m * p.ldq + n] = f2bf(x);
        else
          ((bf16_t*)p.k_out)[out_row(p, m) * p.ldk + (n - qcols)] = f2bf(x);
      } else if (p.v_transposed) {
        // V^T cache: [group][head_dim][ldv], tokens contiguous
        const int64_t b = p.row_group > 0 ? m / p.row_group : 0;
        const int64_t t = p.row_group > 0 ? m % p.row_group : m;
        ((bf16_t*)p.v_out)[(b * hd + (n - qcols - hd)) * p.ldv + t] = f2bf(x);
      } else {
        ((bf16_t*)p.v_out)[out_row(p, m) * p.ldv + (n - qcols - hd)] = f2bf(x);
      }
      continue;
    }
    if (p.bias) x += bf2f(((const bf16_t*)p.bias)[n]);
    if (p.bias_f32) x += p.bias_f32[n];
    if (MODE == FVX_GEMM_EULER) {
      float* xt = p.xt + m * p.ldx + n;
      const float nx = *xt + p.dt * x;
      *xt = nx;
      if (p.xt_bf16) ((bf16_t*)p.xt_bf16)[m * p.ldxb + n] = f2bf(nx);
      continue;
    }
    if (p.act == FVX_ACT_SILU)
      x = silu(x);
    else if (p.act == FVX_ACT_GELU_TANH)
      x = gelu_tanh(x);
    if (p.gate)
      x *= bf2f(((const bf16_t*)p.gate)[(m / p.gate_group) * p.ldg + n]);
    const int64_t orow = out_row(p, m);
    if (p.residual) x += bf2f(((const bf16_t*)p.residual)[orow * p.ldr + n]);
    if (p.pos) x += bf2f(((const bf16_t*)p.pos)[(m % p.pos_period) * p.ldp + n]);
    if (p.out_f32)
      ((float*)p.c)[orow * p.ldc + n] = x;
    else
      ((bf16_t*)p.c)[orow * p.ldc + n] = f2bf(x);
  }
}

__device__ __forceinline__ float sumsq8(const bf16x8& v) {
  float f[8];
  unpack8(v, f);
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += f[e] * f[e];
  return s;
}

// ---------------------------------------------------------------------------
// Tiled kernel (M > 64)
// ---------------------------------------------------------------------------
// 256 threads = 2 x 2 waves; block tile BM x BN (GEGLU: BN columns of each
// of the two weights).  K moves through a 2-stage LDS ring in 64-wide slabs
// with ONE barrier per slab: while slab t feeds the MFMAs, slab t+1 (already
// in registers) is written to the other LDS stage and slab t+2's global
// loads are issued.  LDS rows are XOR-swizzled (see the loader) so neither
// the staging writes nor the fragment reads conflict.  <= 256 registers and
// <= 64 KiB of LDS keep two workgroups per CU.  With
// splits > 1 the K range is split over blockIdx.y and fp32 partials go to
// the workspace for gemm_partial_reduce_kernel.
template <int BM, int BN, int MODE>
constexpr int tile_min_blocks() {
  // two workgroups per CU when the 2-stage ring fits twice in 160 KiB
  return (2 * (BM + (MODE == FVX_GEMM_GEGLU ? 2 : 1) * BN) * 64 * 2 <= 80 * 1024 &&
          MODE != FVX_GEMM_QKV_ROPE) ? 2 : 1;
}

template <int BM, int BN, int MODE>
__global__ __launch_bounds__(256, (tile_min_blocks<BM, BN, MODE>())) void gemm_tile_kernel(GemmArgs p,
                                                           int m_tiles,
                                                           int n_tiles,
                                                           int splits,
                                                           int64_t kchunk) {
  constexpr int BK = 64;
  constexpr int LD = BK;  // 128-byte rows, XOR-swizzled chunks (see loader)
  constexpr int NB = (MODE == FVX_GEMM_GEGLU) ? 2 : 1;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int AI = BM / 32, BI = BN / 32;
  constexpr int STAGE = BM * LD + NB * BN * LD;  // bf16 elements per stage
  __shared__ __align__(16) bf16_t smem[2 * STAGE];
  __shared__ float sRow[BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-aware tile order: consecutive tile ids (the M tiles of one weight
  // panel, m fastest) land on one XCD and share its L2.
  const int nblk = m_tiles * n_tiles;
  int bid = blockIdx.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int m_tile = bid % m_tiles, n_tile = bid / m_tiles;
  const int split = blockIdx.y;
  const int64_t m0 = (int64_t)m_tile * BM, n0 = (int64_t)n_tile * BN;
  const int64_t M = p.m, N = p.n, K = p.k;
  const int64_t kb = (int64_t)split * kchunk;
  const int64_t ke = (kb + kchunk < K) ? kb + kchunk : K;
  const int nk = (int)((ke - kb + BK - 1) / BK);

  const bf16_t* A = (const bf16_t*)p.a;
  const bf16_t* Bm[2] = {(const bf16_t*)p.b, (const bf16_t*)p.b2};

  // Loader: 8 consecutive lanes move one 128-byte row slab (coalesced).
  // LDS rows have no padding; chunk c of row r lives at chunk position
  // c ^ ((r >> 1) & 7).  With 64 banks and 16 lanes per LDS cycle, the
  // loader's 16 lanes (rows 2j, 2j+1, all chunks) and a fragment read's 16
  // lanes (16 consecutive rows, one chunk) both land on 16 distinct 4-bank
  // groups: no bank conflicts on either side.
  const int lrow = tid >> 3, lchk = tid & 7;
  // Two register sets: slab t is loaded into set t & 1 two slabs before it
  // is written to LDS, so its global latency overlaps two slabs of MFMAs.
  bf16x8 ra[2][AI], rb[2][NB][BI];
  float ss[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) ss[i] = 0.f;

  auto gload = [&](int t, int set) {
    const int64_t kk = kb + (int64_t)t * BK + lchk * 8;
    const bool kin = t < nk && kk < ke;
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const int64_t r = m0 + lrow + 32 * i;
      ra[set][i] = (kin && r < M) ? ld8(A + r * p.lda + kk) : zero8();
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < BI; ++i) {
        const int64_t c = n0 + lrow + 32 * i;
        rb[set][b][i] = (kin && c < N) ? ld8(Bm[b] + c * p.ldb + kk) : zero8();
      }
  };
  const int wpos = (lchk ^ ((lrow >> 1) & 7)) * 8;  // same for rows lrow + 32 i
  auto swrite = [&](int buf, int set) {
    bf16_t* sa = smem + buf * STAGE;
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      st8(&sa[(lrow + 32 * i) * LD + wpos], ra[set][i]);
      if (p.rownorm) ss[i] += sumsq8(ra[set][i]);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < BI; ++i)
        st8(&sa[BM * LD + (b * BN + lrow + 32 * i) * LD + wpos], rb[set][b][i]);
  };

  f32x4_t acc[NB][FM][FN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[b][i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, fk = (lane >> 4) * 8;
  auto compute = [&](int buf) {
    const bf16_t* sa = smem + buf * STAGE;
    const bf16_t* sb = sa + BM * LD;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 af[FM], bfr[NB][FN];
      // rows here are (multiple of 16) + fr, so (row >> 1) & 7 == fr >> 1
      const int rpos = ((4 * ks + (lane >> 4)) ^ ((fr >> 1) & 7)) * 8;
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = ld8(&sa[(wm * WM + i * 16 + fr) * LD + rpos]);
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[b][j] = ld8(&sb[(b * BN + wn * WN + j * 16 + fr) * LD + rpos]);
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[b][i][j] = mfma16x16x32(af[i], bfr[b][j], acc[b][i][j]);
    }
  };

  // slab t: loaded into register set t&1, written to LDS stage t&1.
  gload(0, 0);
  gload(1, 1);
  if (nk > 0) swrite(0, 0);
  gload(2, 0);
  __syncthreads();
  for (int t = 0; t < nk; t += 2) {
    compute(0);                          // slab t
    if (t + 1 < nk) {
      swrite(1, 1);                      // slab t+1
      gload(t + 3, 1);
    }
    __syncthreads();
    if (t + 1 >= nk) break;
    compute(1);                          // slab t+1
    if (t + 2 < nk) {
      swrite(0, 0);                      // slab t+2
      gload(t + 4, 0);
    }
    __syncthreads();
  }

  // Row sums of squares of this K range: 8 consecutive lanes share a row.
  if (p.rownorm) {
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      float s2 = ss[i];
      s2 += __shfl_xor(s2, 1, 64);
      s2 += __shfl_xor(s2, 2, 64);
      s2 += __shfl_xor(s2, 4, 64);
      if (lchk == 0) sRow[lrow + 32 * i] = s2;
    }
    __syncthreads();
  }

  if (splits > 1) {
    float* ws = (float*)p.workspace;
    const int64_t plane = (int64_t)splits * M * N;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const int64_t n = n0 + wn * WN + j * 16 + fr;
          const int64_t r0 = m0 + wm * WM + i * 16 + 4 * (lane >> 4);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n < N && r0 + e < M)
              ws[b * plane + ((int64_t)split * M + r0 + e) * N + n] = acc[b][i][j][e];
        }
    if (n_tile == 0 && p.rownorm && tid < BM && m0 + tid < M)
      ws[NB * plane + (int64_t)split * M + m0 + tid] = sRow[tid];
    return;
  }

#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int lr0 = wm * WM + i * 16 + 4 * (lane >> 4);
    float rs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      rs[j] = p.rownorm ? rsqrtf(sRow[lr0 + j] / (float)K + p.rownorm_eps) : 1.f;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int64_t n = n0 + wn * WN + j * 16 + fr;
      float v[4], u[4], pv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = acc[0][i][j][e];
        u[e] = acc[NB - 1][i][j][e];
        pv[e] = (MODE == FVX_GEMM_QKV_ROPE) ? __shfl_xor(v[e], 1, 64) : 0.f;
      }
      epilogue4<MODE>(p, m0 + lr0, n, v, u, pv, rs);
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny (M <= 64) weight-streaming kernels
// ---------------------------------------------------------------------------
// gemm_skinny_kernel: a workgroup owns 64 output columns (4 waves x 16) and a
// K range of at most kSkinnyKc.  Each wave first issues every weight
// fragment load of its range (up to 8 x 16 B per lane per weight matrix, so
// ~32-64 KiB per CU are in flight -- what HBM latency needs), then the whole
// workgroup stages the 64 x Kc activation slab once in LDS, where all four
// waves read their A fragments (activation traffic = weight traffic / 1.25
// instead of 4x when every wave fetched its own copy).
//
// With one K range (splits == 1) the epilogue runs in place.  Otherwise the
// fp32 partial tile and the partial row sums of squares go to the workspace
// with plain stores, and gemm_partial_reduce_kernel -- the next kernel on the
// stream, so the partials are visible without any fence -- adds the splits
// in order and runs the epilogue (deterministic).
constexpr int kSkinnyKc = 256;
constexpr int kSkinnyLDA = kSkinnyKc + 8;  // LDS pitch: conflict-free frag reads

template <int MODE>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(GemmArgs p,
                                                          int splits,
                                                          int64_t kchunk) {
  constexpr int NB = (MODE == FVX_GEMM_GEGLU) ? 2 : 1;
  constexpr int KS = kSkinnyKc / 32;  // k-steps per workgroup (max)
  __shared__ __align__(16) bf16_t sA[64 * kSkinnyLDA];
  __shared__ float s_ss[64];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, g = lane >> 4;
  const int ntile = blockIdx.x, split = blockIdx.y;
  const int64_t M = p.m, N = p.n, K = p.k;
  const int64_t n = (int64_t)ntile * 64 + wave * 16 + fr;
  const bool nval = n < N;
  const int64_t kb = (int64_t)split * kchunk;
  const int64_t ke = (kb + kchunk < K) ? kb + kchunk : K;
  const int nks = (int)((ke - kb + 31) / 32);

  // 1. weight fragments for the whole K range, all loads in flight
  const bf16_t* Bp[2] = {(const bf16_t*)p.b + (nval ? n : 0) * p.ldb,
                         (const bf16_t*)(NB == 2 ? p.b2 : p.b) +
                             (nval ? n : 0) * p.ldb};
  bf16x8 bw[KS][NB];
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    const int64_t kk = kb + 32 * t + 8 * g;
#pragma unroll
    for (int b = 0; b < NB; ++b)
      bw[t][b] = (t < nks && kk < ke && nval) ? ld8(Bp[b] + kk) : zero8();
  }
  // 2. activation slab [64 x Kc] -> LDS (zero rows >= M / columns >= ke)
  const bf16_t* A = (const bf16_t*)p.a;
  constexpr int ACH = 64 * (kSkinnyKc / 8) / 256;  // 16 B chunks per thread
  float ssp[ACH];
#pragma unroll
  for (int c = 0; c < ACH; ++c) {
    const int i = tid + 256 * c;
    const int r = i / (kSkinnyKc / 8), ck = i % (kSkinnyKc / 8);
    const int64_t kk = kb + ck * 8;
    const bf16x8 v = (r < M && kk < ke) ? ld8(A + r * p.lda + kk) : zero8();
    st8(&sA[r * kSkinnyLDA + ck * 8], v);
    ssp[c] = p.rownorm ? sumsq8(v) : 0.f;
  }
  // row sums: the 32 chunks of a row sit in 32 consecutive threads
  if (p.rownorm) {
#pragma unroll
    for (int c = 0; c < ACH; ++c) {
      float v = ssp[c];
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) v += __shfl_xor(v, o, 64);
      ssp[c] = v;
    }
  }
  if (p.rownorm && (tid & 31) == 0) {
#pragma unroll
    for (int c = 0; c < ACH; ++c) s_ss[(tid + 256 * c) / 32] = ssp[c];
  }
  __syncthreads();

  // 3. MFMA over the K range
  f32x4_t acc[NB][4];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b][f] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    if (t < nks) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const bf16x8 a = ld8(&sA[(f * 16 + fr) * kSkinnyLDA + 32 * t + 8 * g]);
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b][f] = mfma16x16x32(a, bw[t][b], acc[b][f]);
      }
    }
  }

  if (splits > 1) {
    // partials: [NB][split][M rows][N] fp32, then [split][M] row sums
    float* ws = (float*)p.workspace;
    const int64_t plane = (int64_t)splits * M * N;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (nval && f * 16 + 4 * g + j < M)
            ws[b * plane + ((int64_t)split * M + f * 16 + 4 * g + j) * N + n] =
                acc[b][f][j];
    if (ntile == 0 && p.rownorm && tid < M) ws[NB * plane + split * M + tid] = s_ss[tid];
    return;
  }

  // Epilogue: lane holds column n, rows f*16 + 4g + j.
#pragma unroll
  for (int f = 0; f < 4; ++f) {
    float rs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      rs[j] = p.rownorm ? rsqrtf(s_ss[f * 16 + 4 * g + j] / (float)K + p.rownorm_eps)
                        : 1.f;
    float v[4], u[4], pv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = acc[0][f][e];
      u[e] = acc[NB - 1][f][e];
      pv[e] = (MODE == FVX_GEMM_QKV_ROPE) ? __shfl_xor(v[e], 1, 64) : 0.f;
    }
    epilogue4<MODE>(p, (int64_t)f * 16 + 4 * g, n, v, u, pv, rs);
  }
}

// Sum of the split partials of either GEMM kernel + epilogue.  Thread t of
// block (x, y): column 64 x + t % 64, row 4 y + t / 64; the loads of 16
// splits are issued before their adds (one memory latency per 16), added in
// split order (deterministic).
template <int MODE>
__global__ __launch_bounds__(256) void gemm_partial_reduce_kernel(GemmArgs p,
                                                                  int splits) {
  constexpr int NB = (MODE == FVX_GEMM_GEGLU) ? 2 : 1;
  constexpr int UN = 16;  // loads in flight per pass
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t N = p.n, K = p.k;
  const int64_t n = (int64_t)blockIdx.x * 64 + lane;
  const int64_t row = (int64_t)blockIdx.y * 4 + (tid >> 6);
  const bool ok = n < N && row < p.m;
  const float* ws = (const float*)p.workspace;
  const int64_t M = p.m;
  const int64_t plane = (int64_t)splits * M * N;
  float v = 0.f, u = 0.f, ss = 0.f;
  for (int s0 = 0; s0 < splits; s0 += UN) {
    float t[NB][UN], q[UN];
#pragma unroll
    for (int i = 0; i < UN; ++i) {
      const int s = s0 + i;
      const bool in = ok && s < splits;
#pragma unroll
      for (int b = 0; b < NB; ++b)
        t[b][i] = in ? ws[b * plane + ((int64_t)s * M + row) * N + n] : 0.f;
      q[i] = (in && p.rownorm) ? ws[NB * plane + (int64_t)s * M + row] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < UN; ++i) {
      v += t[0][i];
      u += t[NB - 1][i];
      ss += q[i];
    }
  }
  float rs[1] = {p.rownorm ? rsqrtf(ss / (float)K + p.rownorm_eps) : 1.f};
  float vv[1] = {v}, uu[1] = {u};
  float pv[1] = {(MODE == FVX_GEMM_QKV_ROPE) ? __shfl_xor(v, 1, 64) : 0.f};
  if (ok) epilogue4<MODE, 1>(p, row, n, vv, uu, pv, rs);
}

// ---------------------------------------------------------------------------
// Host side: validation and kernel selection
// ---------------------------------------------------------------------------
struct SkinnyPlan {
  int n_tiles, splits;
  int64_t kchunk, ws_bytes;
};

static SkinnyPlan plan_skinny(const GemmArgs& d) {
  SkinnyPlan s;
  const int nb = d.mode == FVX_GEMM_GEGLU ? 2 : 1;
  s.n_tiles = (int)((d.n + 63) / 64);
  int64_t kchunk;
  if (d.split_k > 0) {
    kchunk = (d.k + d.split_k - 1) / d.split_k;
    kchunk = (kchunk + 31) / 32 * 32;
  } else {
    // 256-wide K ranges when that already gives ~200+ workgroups, else 128
    kchunk = s.n_tiles * ((d.k + kSkinnyKc - 1) / kSkinnyKc) >= 200 ? 256 : 128;
  }
  if (kchunk > kSkinnyKc) kchunk = kSkinnyKc;
  if (kchunk < 32) kchunk = 32;
  s.splits = (int)((d.k + kchunk - 1) / kchunk);
  s.kchunk = kchunk;
  s.ws_bytes = s.splits > 1
                   ? ((int64_t)nb * s.splits * d.m * d.n + (int64_t)s.splits * d.m) * 4
                   : 0;
  return s;
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
  FVX_REQUIRE(!d.rownorm || d.rownorm_eps >= 0.f, FVX_ERR_ARG,
              "gemm: rownorm_eps must be >= 0");
  FVX_REQUIRE(d.row_group >= 0, FVX_ERR_ARG, "gemm: row_group must be >= 0");
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
  return FVX_OK;
}

}  // namespace fvx

using namespace fvx;

extern "C" int64_t fvx_gemm_workspace_bytes(const fvx_gemm_desc* d) {
  if (!d || d->m <= 0) return 0;
  if (d->m <= 64) return plan_skinny(*d).ws_bytes;
  // tiled path: at most 4 K splits of fp32 partials (+ row sums)
  const int nb = d->mode == FVX_GEMM_GEGLU ? 2 : 1;
  return ((int64_t)nb * 4 * d->m * d->n + 4 * d->m) * 4;
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

extern "C" int fvx_gemm(const fvx_gemm_desc* dp, void* stream) {
  clear_error();
  FVX_REQUIRE(dp, FVX_ERR_NULL, "gemm: descriptor is NULL");
  GemmArgs d = *dp;
  int st = validate(d);
  if (st) return st;
  if (d.m == 0) return FVX_OK;
  hipStream_t s = (hipStream_t)stream;
  if (d.m <= 64) {
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
    dim3 grid((unsigned)sp.n_tiles, (unsigned)sp.splits);
#define L(MODE)                                                          \
  hipLaunchKernelGGL(gemm_skinny_kernel<MODE>, grid, dim3(256), 0, s, d, \
                     sp.splits, sp.kchunk)
    FVX_MODE_DISPATCH(d.mode, L)
#undef L
    int st2 = launch_status("gemm(skinny)");
    if (st2 || sp.splits == 1) return st2;
#define L(MODE)                                                            \
  hipLaunchKernelGGL(gemm_partial_reduce_kernel<MODE>,                      \
                     dim3(sp.n_tiles, (unsigned)((d.m + 3) / 4)), dim3(256), \
                     0, s, d, sp.splits)
    FVX_MODE_DISPATCH(d.mode, L)
#undef L
    return launch_status("gemm(skinny reduce)");
  }
  // Tiled path: 128 x 128 tiles (GEGLU: 128 x 64 of each weight) when that
  // gives >= 512 workgroups (two per CU), else 64 x 128.  Projections with a long K and
  // too few tiles to fill 256 CUs split K.
  const bool gg = d.mode == FVX_GEMM_GEGLU;
  const int64_t mt128 = (d.m + 127) / 128, mt64 = (d.m + 63) / 64;
  const int64_t ncols = gg ? 2 * d.n : d.n;  // output columns incl. both weights
  int cfg;  // 1: 128x128, 2: 64x128  (128x256 needs >110 KiB of LDS: one
            // workgroup per CU, measured 3-4x slower than two of 128x128)
  if (mt128 * ((ncols + 127) / 128) >= 512) cfg = 1;
  else cfg = 2;
  const int bm = cfg == 2 ? 64 : 128;
  const int bn = 128 / (gg ? 2 : 1);
  const int m_tiles = (int)(cfg == 2 ? mt64 : mt128);
  const int n_tiles = (int)((d.n + bn - 1) / bn);
  const int tiles = m_tiles * n_tiles;
  int splits = d.split_k > 0 ? d.split_k : 1;
  if (d.split_k <= 0 && tiles < 160 && d.k >= 4096) {
    splits = (int)((256 + tiles - 1) / tiles);
    if (splits > 4) splits = 4;
  }
  int64_t kchunk = (d.k + splits - 1) / splits;
  kchunk = (kchunk + 63) / 64 * 64;
  splits = (int)((d.k + kchunk - 1) / kchunk);
  const int nbm = gg ? 2 : 1;
  const int64_t need = splits > 1 ? ((int64_t)nbm * splits * d.m * d.n + (int64_t)splits * d.m) * 4 : 0;
  if (splits > 1 && (!d.workspace || d.workspace_bytes < need)) {
    if (d.split_k > 1)
      return set_error(FVX_ERR_WORKSPACE,
                       "gemm: split_k=%d needs %lld workspace bytes, got %lld",
                       d.split_k, (long long)need, (long long)d.workspace_bytes);
    splits = 1;
    kchunk = d.k;
  }
  dim3 grid((unsigned)tiles, (unsigned)splits);
#define LT(BM_, BN_, MODE)                                                  \
  hipLaunchKernelGGL((gemm_tile_kernel<BM_, BN_, MODE>), grid, dim3(256), 0, \
                     s, d, m_tiles, n_tiles, splits, kchunk)
  if (gg) {
    if (cfg == 1) LT(128, 64, FVX_GEMM_GEGLU);
    else LT(64, 64, FVX_GEMM_GEGLU);
  } else if (cfg == 1) {
#define L(MODE) LT(128, 128, MODE)
    FVX_MODE_DISPATCH_NG(d.mode, L)
#undef L
  } else {
#define L(MODE) LT(64, 128, MODE)
    FVX_MODE_DISPATCH_NG(d.mode, L)
#undef L
  }
#undef LT
  int st3 = launch_status("gemm(tile)");
  if (st3 || splits == 1) return st3;
#define L(MODE)                                                            \
  hipLaunchKernelGGL(gemm_partial_reduce_kernel<MODE>,                     \
                     dim3((unsigned)((d.n + 63) / 64), (unsigned)((d.m + 3) / 4)), \
                     dim3(256), 0, s, d, splits)
  FVX_MODE_DISPATCH(d.mode, L)
#undef L
  return launch_status("gemm(reduce)");
}
