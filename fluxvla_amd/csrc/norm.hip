// Row normalizations: fused residual + RMSNorm, LayerNorm, adaptive RMSNorm.
//
// Layout: WPR 64-lane wavefronts per row (RMSNorm and LayerNorm: 4 from
// 2048 columns, else 1; adaRMS: 1), 256-thread workgroups of 4 / WPR rows.
// Each lane moves 16-byte vectors (8 bf16); vector v of a row belongs to
// lane v % 64 of the row's wave (v / 64) % WPR, so a wavefront reads 1 KiB
// contiguous per instruction; the row is held in fp32 registers between
// the reduction and the write, so HBM sees each input byte once and each
// output byte once.  Reductions are wavefront shuffles, then (WPR > 1) the
// row's wave sums through LDS.  Several waves per row keep more waves per
// SIMD in flight for the same bytes.
#include "capi_util.h"
#include "common.h"

namespace fvx {

constexpr int kRowsPerBlock = 4;
constexpr int kMaxVec = 8;  // up to 64 lanes * 8 vectors * 8 = 4096 columns

// All of a row's loads (and the per-column weights) are issued before any
// is used, through buffer views: a vector past the row end or of an absent
// operand reads zero without a branch (a load behind a branch makes the
// compiler wait for it at the join, serializing the loads).
__device__ __forceinline__ uint32_t vec_off(int v, int nvec, int64_t base) {
  return v < nvec ? (uint32_t)((base + (int64_t)v * 8) * 2) : kOOB;
}

// Sum of v over the WPR waves of a row: shuffles within each wave, then the
// waves' sums through `slot` (this row's WPR floats of LDS) in wave order.
// Every thread of the workgroup must call it (it holds a barrier when
// WPR > 1); a slot array serves one reduction.
template <int WPR>
__device__ __forceinline__ float row_sum(float v, float* slot, int lane, int wr) {
  v = wave_sum(v);
  if (WPR == 1) return v;
  if (lane == 0) slot[wr] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < WPR; ++j) s += slot[j];
  return s;
}

// Row of this wave (rl: row within the workgroup, wr: wave within the row)
// and the vector index of its i-th vector.
template <int WPR>
struct RowLanes {
  int lane, rl, wr;
  int64_t row;
  __device__ RowLanes() {
    lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    rl = wave / WPR;
    wr = wave % WPR;
    row = (int64_t)blockIdx.x * (kRowsPerBlock / WPR) + rl;
  }
  __device__ int vec(int i) const { return lane + 64 * (wr + WPR * i); }
};

template <int NV, int WPR>
__global__ __launch_bounds__(256) void rms_norm_residual_kernel(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ res,
    const bf16_t* __restrict__ w, bf16_t* __restrict__ out,
    bf16_t* __restrict__ res_out, int64_t rows, int cols, float eps) {
  __shared__ float sred[kRowsPerBlock / WPR][WPR];
  const RowLanes<WPR> L;
  // a row past the end reads zeros and writes nothing (its waves still
  // reach the barrier of the row sum)
  const bool live = L.row < rows;
  const int64_t row = live ? L.row : 0;
  const int nvec = cols >> 3;
  const uint32_t rb = live ? (uint32_t)cols * 2 : 0u;  // views of this row only
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + row * cols, rb);
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(res ? res + row * cols : x, res ? rb : 0u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w ? w : x, w ? (uint32_t)cols * 2 : 0u);
  bf16x8 xv[NV], rv[NV], wv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    xv[i] = bload8(rx, vec_off(L.vec(i), nvec, 0));
    rv[i] = bload8(rr, vec_off(L.vec(i), nvec, 0));
    wv[i] = bload8(rw, vec_off(L.vec(i), nvec, 0));
  }
  float h[NV][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    float r[8];
    unpack8(xv[i], h[i]);
    unpack8(rv[i], r);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h[i][e] += r[e];
      ss += h[i][e] * h[i][e];
    }
  }
  ss = row_sum<WPR>(ss, sred[L.rl], L.lane, L.wr);
  if (!live) return;
  const float f = rsqrtf(ss / (float)cols + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = L.vec(i);
    if (v < nvec) {
      if (res_out) st8(res_out + row * cols + v * 8, pack8(h[i]));
      float y[8], wf[8];
      unpack8(wv[i], wf);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = h[i][e] * f * (w ? wf[e] : 1.f);
      st8(out + row * cols + v * 8, pack8(y));
    }
  }
}

template <int NV, int WPR>
__global__ __launch_bounds__(256) void layer_norm_kernel(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
    const bf16_t* __restrict__ b, bf16_t* __restrict__ out, int64_t rows,
    int cols, float eps) {
  __shared__ float sred[2][kRowsPerBlock / WPR][WPR];
  const RowLanes<WPR> L;
  const bool live = L.row < rows;
  const int64_t row = live ? L.row : 0;
  const int nvec = cols >> 3;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + row * cols, live ? (uint32_t)cols * 2 : 0u);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, (uint32_t)cols * 2);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(b, (uint32_t)cols * 2);
  bf16x8 xv[NV], wv[NV], bv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    xv[i] = bload8(rx, vec_off(L.vec(i), nvec, 0));
    wv[i] = bload8(rw, vec_off(L.vec(i), nvec, 0));
    bv[i] = bload8(rb, vec_off(L.vec(i), nvec, 0));
  }
  float h[NV][8];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    unpack8(xv[i], h[i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) s += h[i][e];
  }
  const float mean = row_sum<WPR>(s, sred[0][L.rl], L.lane, L.wr) / (float)cols;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const bool in = L.vec(i) < nvec;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      h[i][e] -= mean;
      if (in) ss += h[i][e] * h[i][e];
    }
  }
  const float inv = rsqrtf(row_sum<WPR>(ss, sred[1][L.rl], L.lane, L.wr) / (float)cols + eps);
  if (!live) return;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = L.vec(i);
    if (v < nvec) {
      float wf[8], bf[8], y[8];
      unpack8(wv[i], wf);
      unpack8(bv[i], bf);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = h[i][e] * inv * wf[e] + bf[e];
      st8(out + row * cols + v * 8, pack8(y));
    }
  }
}

template <int NV>
__global__ __launch_bounds__(256) void adarms_norm_kernel(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ style,
    bf16_t* __restrict__ out, bf16_t* __restrict__ gate_out, int64_t rows,
    int cols, int64_t rows_per_style, int64_t style_stride, float eps,
    const bf16_t* __restrict__ style_locked, const int32_t* __restrict__ lock,
    int64_t lock_period) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int nvec = cols >> 3;
  // rows of the locked prefix (real-time chunking) use the time-0 style row
  const bool locked = lock && (row % lock_period) < (int64_t)*lock;
  const bf16_t* srow = locked ? style_locked : style + (row / rows_per_style) * style_stride;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + row * cols, (uint32_t)cols * 2);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(srow, (uint32_t)cols * 6);
  bf16x8 xv[NV], scv[NV], shv[NV], gv[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    xv[i] = bload8(rx, vec_off(v, nvec, 0));
    scv[i] = bload8(rs, vec_off(v, nvec, 0));
    shv[i] = bload8(rs, vec_off(v, nvec, cols));
    gv[i] = bload8(rs, vec_off(v, nvec, 2 * cols));
  }
  float h[NV][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    unpack8(xv[i], h[i]);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += h[i][e] * h[i][e];
  }
  const float f = rsqrtf(wave_sum(ss) / (float)cols + eps);
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int v = lane + 64 * i;
    if (v < nvec) {
      float sc[8], sh[8], y[8];
      unpack8(scv[i], sc);
      unpack8(shv[i], sh);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = h[i][e] * f * (1.f + sc[e]) + sh[e];
      st8(out + row * cols + v * 8, pack8(y));
      if (gate_out) st8(gate_out + row * cols + v * 8, gv[i]);
    }
  }
}

#define FVX_NV_DISPATCH(NV_RUNTIME, LAUNCH) \
  switch (NV_RUNTIME) {                     \
    case 1: LAUNCH(1); break;               \
    case 2: LAUNCH(2); break;               \
    case 3: LAUNCH(3); break;               \
    case 4: LAUNCH(4); break;               \
    case 5: LAUNCH(5); break;               \
    case 6: LAUNCH(6); break;               \
    case 7: LAUNCH(7); break;               \
    default: LAUNCH(8); break;              \
  }

// RMSNorm / LayerNorm: 4 waves per row from 256 vectors (2048 columns: C1
// 6.33 -> 5.70 us), else one (two waves on SigLIP's 1152-column LayerNorm
// measured 3.65 -> 3.75 us); vectors per lane: up to 4096 columns, 2 with
// 4 waves, 8 with one
static int waves_per_row(int64_t nvec) { return nvec >= 256 ? 4 : 1; }

#define FVX_ROW_DISPATCH(WPR, NV, LAUNCH) \
  if (WPR == 4) {                          \
    if (NV == 1) LAUNCH(1, 4);             \
    else LAUNCH(2, 4);                     \
  } else {                                 \
    switch (NV) {                          \
      case 1: LAUNCH(1, 1); break;         \
      case 2: LAUNCH(2, 1); break;         \
      case 3: LAUNCH(3, 1); break;         \
      default: LAUNCH(4, 1); break;        \
    }                                      \
  }

static int check_rows(const char* what, int64_t rows, int64_t cols) {
  FVX_REQUIRE(rows >= 0, FVX_ERR_SHAPE, "%s: rows=%lld < 0", what,
              (long long)rows);
  FVX_REQUIRE(cols > 0 && cols % 8 == 0 && cols <= 64 * 8 * kMaxVec,
              FVX_ERR_SHAPE,
              "%s: cols=%lld must be a positive multiple of 8 and <= 4096",
              what, (long long)cols);
  return FVX_OK;
}

}  // namespace fvx

using namespace fvx;

extern "C" int fvx_rms_norm_residual(const void* x, const void* residual,
                                     const void* weight, void* out,
                                     void* residual_out, int64_t rows,
                                     int64_t cols, float eps, void* stream) {
  clear_error();
  FVX_REQUIRE(x && out, FVX_ERR_NULL, "rms_norm_residual: x and out required");
  int st = check_rows("rms_norm_residual", rows, cols);
  if (st) return st;
  FVX_REQUIRE(aligned16(x) && aligned16(out) && aligned16(residual) &&
                  aligned16(weight) && aligned16(residual_out),
              FVX_ERR_ALIGN, "rms_norm_residual: pointers must be 16B aligned");
  if (rows == 0) return FVX_OK;
  const int wpr = waves_per_row(cols / 8);
  const int nv = (int)((cols / 8 + 64 * wpr - 1) / (64 * wpr));
  const int rpb = kRowsPerBlock / wpr;
  dim3 grid((unsigned)((rows + rpb - 1) / rpb));
  hipStream_t s = (hipStream_t)stream;
#define L(NV, WPR)                                                                 \
  hipLaunchKernelGGL((rms_norm_residual_kernel<NV, WPR>), grid, dim3(256), 0, s,   \
                     (const bf16_t*)x, (const bf16_t*)residual,                    \
                     (const bf16_t*)weight, (bf16_t*)out,                          \
                     (bf16_t*)residual_out, rows, (int)cols, eps)
  FVX_ROW_DISPATCH(wpr, nv, L)
#undef L
  return launch_status("rms_norm_residual");
}

extern "C" int fvx_layer_norm(const void* x, const void* weight,
                              const void* bias, void* out, int64_t rows,
                              int64_t cols, float eps, void* stream) {
  clear_error();
  FVX_REQUIRE(x && weight && bias && out, FVX_ERR_NULL,
              "layer_norm: x, weight, bias, out required");
  int st = check_rows("layer_norm", rows, cols);
  if (st) return st;
  FVX_REQUIRE(aligned16(x) && aligned16(out) && aligned16(weight) &&
                  aligned16(bias),
              FVX_ERR_ALIGN, "layer_norm: pointers must be 16B aligned");
  if (rows == 0) return FVX_OK;
  const int wpr = waves_per_row(cols / 8);
  const int nv = (int)((cols / 8 + 64 * wpr - 1) / (64 * wpr));
  const int rpb = kRowsPerBlock / wpr;
  dim3 grid((unsigned)((rows + rpb - 1) / rpb));
  hipStream_t s = (hipStream_t)stream;
#define L(NV, WPR)                                                                  \
  hipLaunchKernelGGL((layer_norm_kernel<NV, WPR>), grid, dim3(256), 0, s,           \
                     (const bf16_t*)x, (const bf16_t*)weight,                       \
                     (const bf16_t*)bias, (bf16_t*)out, rows, (int)cols, eps)
  FVX_ROW_DISPATCH(wpr, nv, L)
#undef L
  return launch_status("layer_norm");
}

static int adarms_launch(const void* x, const void* style,
                         const void* style_locked, const int32_t* lock,
                         int64_t lock_period, void* out, void* gate_out,
                         int64_t rows, int64_t cols, int64_t rows_per_style,
                         int64_t style_stride, float eps, void* stream) {
  FVX_REQUIRE(x && style && out, FVX_ERR_NULL,
              "adarms_norm: x, style, out required");
  int st = check_rows("adarms_norm", rows, cols);
  if (st) return st;
  FVX_REQUIRE(rows_per_style > 0 && style_stride >= 3 * cols &&
                  style_stride % 8 == 0,
              FVX_ERR_SHAPE,
              "adarms_norm: rows_per_style > 0 and style_stride >= 3*cols "
              "(multiple of 8) required");
  FVX_REQUIRE(aligned16(x) && aligned16(out) && aligned16(style) &&
                  aligned16(gate_out),
              FVX_ERR_ALIGN, "adarms_norm: pointers must be 16B aligned");
  if (rows == 0) return FVX_OK;
  const int nv = (int)((cols / 8 + 63) / 64);
  dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
  hipStream_t s = (hipStream_t)stream;
#define L(NV)                                                               \
  hipLaunchKernelGGL(adarms_norm_kernel<NV>, grid, dim3(256), 0, s,         \
                     (const bf16_t*)x, (const bf16_t*)style, (bf16_t*)out,  \
                     (bf16_t*)gate_out, rows, (int)cols, rows_per_style,    \
                     style_stride, eps, (const bf16_t*)style_locked, lock,  \
                     lock_period)
  FVX_NV_DISPATCH(nv, L)
#undef L
  return launch_status("adarms_norm");
}

extern "C" int fvx_adarms_norm(const void* x, const void* style, void* out,
                               void* gate_out, int64_t rows, int64_t cols,
                               int64_t rows_per_style, int64_t style_stride,
                               float eps, void* stream) {
  clear_error();
  return adarms_launch(x, style, nullptr, nullptr, 1, out, gate_out, rows,
                       cols, rows_per_style, style_stride, eps, stream);
}

extern "C" int fvx_adarms_norm_locked(const void* x, const void* style,
                                      const void* style_locked,
                                      const int32_t* lock, int64_t lock_period,
                                      void* out, void* gate_out, int64_t rows,
                                      int64_t cols, int64_t rows_per_style,
                                      int64_t style_stride, float eps,
                                      void* stream) {
  clear_error();
  FVX_REQUIRE(style_locked && lock, FVX_ERR_NULL,
              "adarms_norm_locked: style_locked and lock required");
  FVX_REQUIRE(lock_period > 0, FVX_ERR_SHAPE,
              "adarms_norm_locked: lock_period must be > 0");
  FVX_REQUIRE(aligned16(style_locked) && ((uintptr_t)lock & 3) == 0,
              FVX_ERR_ALIGN,
              "adarms_norm_locked: style_locked 16B, lock 4B aligned");
  return adarms_launch(x, style, style_locked, lock, lock_period, out,
                       gate_out, rows, cols, rows_per_style, style_stride, eps,
                       stream);
}
