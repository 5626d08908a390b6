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
//    gemm_skinny_reduce_kernel, the next kernel on the stream, sums them in
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
// Big-tile kernel
// ---------------------------------------------------------------------------
template <int BM, int BN, int MODE>
__global__ __launch_bounds__(256) void gemm_tile_kernel(GemmArgs p, int m_tiles,
                                                        int n_tiles) {
  constexpr int BK = 64;
  constexpr int LD = BK + 8;  // LDS row pitch (bf16): 144 B, conflict-free reads
  constexpr int NB = (MODE == FVX_GEMM_GEGLU) ? 2 : 1;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int FM = WM / 16, FN = WN / 16;
  constexpr int AI = BM / 32, BI = BN / 32;
  __shared__ __align__(16) bf16_t sA[BM * LD];
  __shared__ __align__(16) bf16_t sB[NB][BN * LD];
  __shared__ float sRow[BM];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // XCD-aware tile order (see file comment).
  const int nblk = m_tiles * n_tiles;
  int bid = blockIdx.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int m_tile = bid % m_tiles, n_tile = bid / m_tiles;
  const int64_t m0 = (int64_t)m_tile * BM, n0 = (int64_t)n_tile * BN;

  const bf16_t* A = (const bf16_t*)p.a;
  const bf16_t* Bm[2] = {(const bf16_t*)p.b, (const bf16_t*)p.b2};
  const int64_t M = p.m, N = p.n, K = p.k;

  const int lrow = tid >> 3, lchk = tid & 7;
  bf16x8 ra[AI], rb[NB][BI];
  float ss[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) ss[i] = 0.f;

  auto gload = [&](int64_t k0) {
    const int64_t kk = k0 + lchk * 8;
    const bool kin = kk < K;
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const int64_t r = m0 + lrow + 32 * i;
      ra[i] = (kin && r < M) ? ld8(A + r * p.lda + kk) : zero8();
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < BI; ++i) {
        const int64_t c = n0 + lrow + 32 * i;
        rb[b][i] = (kin && c < N) ? ld8(Bm[b] + c * p.ldb + kk) : zero8();
      }
  };
  auto swrite = [&]() {
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      st8(&sA[(lrow + 32 * i) * LD + lchk * 8], ra[i]);
      if (p.rownorm) ss[i] += sumsq8(ra[i]);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int i = 0; i < BI; ++i)
        st8(&sB[b][(lrow + 32 * i) * LD + lchk * 8], rb[b][i]);
  };

  f32x4_t acc[NB][FM][FN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc[b][i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)((K + BK - 1) / BK);
  gload(0);
  swrite();
  __syncthreads();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    if (kt + 1 < nk) gload((int64_t)(kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 af[FM], bfr[NB][FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = ld8(&sA[(wm * WM + i * 16 + fr) * LD + ks * 32 + fk]);
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          bfr[b][j] = ld8(&sB[b][(wn * WN + j * 16 + fr) * LD + ks * 32 + fk]);
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
            acc[b][i][j] = mfma16x16x32(af[i], bfr[b][j], acc[b][i][j]);
    }
    __syncthreads();
    if (kt + 1 < nk) {
      swrite();
      __syncthreads();
    }
  }

  if (p.rownorm) {
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      float s = ss[i];
      s += __shfl_xor(s, 1, 64);
      s += __shfl_xor(s, 2, 64);
      s += __shfl_xor(s, 4, 64);
      if (lchk == 0) sRow[lrow + 32 * i] = rsqrtf(s / (float)K + p.rownorm_eps);
    }
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int lr0 = wm * WM + i * 16 + 4 * (lane >> 4);
    float rs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) rs[j] = p.rownorm ? sRow[lr0 + j] : 1.f;
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
// with plain stores, and gemm_skinny_reduce_kernel -- the next kernel on the
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
    // partials: [NB][split][64 rows][N] fp32, then [split][64] row sums
    float* ws = (float*)p.workspace;
    const int64_t plane = (int64_t)splits * 64 * N;
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int f = 0; f < 4; ++f)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (nval && f * 16 + 4 * g + j < M)
            ws[b * plane + ((int64_t)split * 64 + f * 16 + 4 * g + j) * N + n] =
                acc[b][f][j];
    if (ntile == 0 && tid < 64) ws[NB * plane + split * 64 + tid] = s_ss[tid];
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

// Sum of the split partials + epilogue.  Thread t of block (x, y): column
// 64 x + t % 64, row 4 y + t / 64; the loads of all splits are issued before
// the adds (one memory latency) and added in split order (deterministic).

template <int MODE>
__global__ __launch_bounds__(256) void gemm_skinny_reduce_kernel(GemmArgs p,
                                                                 int splits) {
  constexpr int NB = (MODE == FVX_GEMM_GEGLU) ? 2 : 1;
  constexpr int UN = 16;  // loads in flight per pass
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t N = p.n, K = p.k;
  const int64_t n = (int64_t)blockIdx.x * 64 + lane;
  const int64_t row = (int64_t)blockIdx.y * 4 + (tid >> 6);
  const bool ok = n < N && row < p.m;
  const float* ws = (const float*)p.workspace;
  const int64_t plane = (int64_t)splits * 64 * N;
  float v = 0.f, u = 0.f, ss = 0.f;
  for (int s0 = 0; s0 < splits; s0 += UN) {
    float t[NB][UN], q[UN];
#pragma unroll
    for (int i = 0; i < UN; ++i) {
      const int s = s0 + i;
      const bool in = ok && s < splits;
#pragma unroll
      for (int b = 0; b < NB; ++b)
        t[b][i] = in ? ws[b * plane + ((int64_t)s * 64 + row) * N + n] : 0.f;
      q[i] = (in && p.rownorm) ? ws[NB * plane + s * 64 + row] : 0.f;
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
                   ? ((int64_t)nb * s.splits * 64 * d.n + (int64_t)s.splits * 64) * 4
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
  if (!d || d->m > 64 || d->m <= 0) return 0;
  return plan_skinny(*d).ws_bytes;
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
  hipLaunchKernelGGL(gemm_skinny_reduce_kernel<MODE>,                      \
                     dim3(sp.n_tiles, (unsigned)((d.m + 3) / 4)), dim3(256), \
                     0, s, d, sp.splits)
    FVX_MODE_DISPATCH(d.mode, L)
#undef L
    return launch_status("gemm(skinny reduce)");
  }
  // Big tiles: 128x128 when that fills the GPU, else 64-row tiles.
  const int64_t mt128 = (d.m + 127) / 128, nt128 = (d.n + 127) / 128;
  const bool big = mt128 * nt128 >= 256;
  const int m_tiles = (int)(big ? mt128 : (d.m + 63) / 64);
  const int n_tiles = (int)nt128;
  dim3 grid((unsigned)(m_tiles * n_tiles));
  if (big) {
#define L(MODE)                                                              \
  hipLaunchKernelGGL((gemm_tile_kernel<128, 128, MODE>), grid, dim3(256), 0, \
                     s, d, m_tiles, n_tiles)
    FVX_MODE_DISPATCH(d.mode, L)
#undef L
  } else {
#define L(MODE)                                                             \
  hipLaunchKernelGGL((gemm_tile_kernel<64, 128, MODE>), grid, dim3(256), 0, \
                     s, d, m_tiles, n_tiles)
    FVX_MODE_DISPATCH(d.mode, L)
#undef L
  }
  return launch_status("gemm(tile)");
}
