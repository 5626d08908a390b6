// Small data-movement kernels around the GEMMs, and the library's error
// plumbing.  All of them are HBM/latency bound byte movers: 16-byte vector
// accesses where the layout allows, one thread per output vector.
#include <string.h>

#include "capi_util.h"
#include "common.h"

namespace fvx {

static thread_local char g_err[512];

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = 0; }

// images [n, 3, H, W] -> patches [n * (H/P) * (W/P), k_pad], column
// (c * P + ky) * P + kx; one thread per output element pair is too fine, so
// each thread builds 8 consecutive columns of one patch row.
__global__ void im2col_kernel(const void* __restrict__ img, int in_f32,
                              int chlast, bf16_t* __restrict__ out,
                              int64_t n_img, int H,
                              int W, int P, int k_pad, float scale,
                              float shift) {
  const int gw = W / P, gh = H / P;
  const int64_t vecs_per_row = k_pad / 8;
  const int64_t total = n_img * gh * gw * vecs_per_row;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t row = idx / vecs_per_row;
  const int col0 = (int)(idx % vecs_per_row) * 8;
  const int64_t im = row / (gh * gw);
  const int pr = (int)(row % (gh * gw));
  const int py = pr / gw, px = pr % gw;
  const int kreal = 3 * P * P;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int col = col0 + e;
    if (col < kreal) {
      const int c = col / (P * P), rem = col % (P * P);
      const int ky = rem / P, kx = rem % P;
      const int64_t y = py * P + ky, xx = px * P + kx;
      const int64_t off = chlast ? ((im * H + y) * W + xx) * 3 + c
                                 : ((im * 3 + c) * H + y) * W + xx;
      const float x = in_f32 ? ((const float*)img)[off]
                             : bf2f(((const bf16_t*)img)[off]);
      v[e] = x * scale + shift;
    } else {
      v[e] = 0.f;
    }
  }
  st8(out + row * k_pad + col0, pack8(v));
}

__global__ void embed_kernel(const bf16_t* __restrict__ table,
                             const int64_t* __restrict__ ids,
                             bf16_t* __restrict__ out, int64_t n, int dim,
                             int64_t vocab, float scale, int64_t rg,
                             int64_t rgs) {
  const int64_t vpr = dim / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n * vpr) return;
  const int64_t t = idx / vpr;
  const int c = (int)(idx % vpr) * 8;
  int64_t id = ids[t];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  float f[8];
  unpack8(ld8(table + id * dim + c), f);
#pragma unroll
  for (int e = 0; e < 8; ++e) f[e] *= scale;
  const int64_t orow = rg > 0 ? (t / rg) * rgs + t % rg : t;
  st8(out + orow * dim + c, pack8(f));
}

__global__ void copy_rows_kernel(const bf16_t* __restrict__ src,
                                 int64_t src_ld, bf16_t* __restrict__ dst,
                                 int64_t dst_ld, int64_t rows, int cols,
                                 int64_t rg, int64_t rgs) {
  const int64_t vpr = cols / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * vpr) return;
  const int64_t r = idx / vpr;
  const int c = (int)(idx % vpr) * 8;
  const int64_t orow = rg > 0 ? (r / rg) * rgs + r % rg : r;
  st8(dst + orow * dst_ld + c, ld8(src + r * src_ld + c));
}

// Row-major [m <= 64, k] -> fragment-major (frag_offset); one thread per
// 8-column chunk.
__global__ void pack_frag_kernel(const bf16_t* __restrict__ src, int64_t src_ld,
                                 bf16_t* __restrict__ dst, int64_t rows,
                                 int64_t cols) {
  const int64_t vpr = cols / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * vpr) return;
  const int64_t r = idx / vpr, c = (idx % vpr) * 8;
  st8(dst + frag_offset(r, c), ld8(src + r * src_ld + c));
}

}  // namespace fvx

using namespace fvx;

extern "C" int fvx_version(void) { return 1; }

extern "C" const char* fvx_last_error(void) { return g_err; }

extern "C" int fvx_im2col_patches(const void* images, int in_f32,
                                  int channels_last, void* patches,
                                  int64_t n_img, int64_t height,
                                  int64_t width, int64_t patch, int64_t k_pad,
                                  float in_scale, float in_shift,
                                  void* stream) {
  clear_error();
  FVX_REQUIRE(images && patches, FVX_ERR_NULL,
              "im2col_patches: images and patches required");
  FVX_REQUIRE(n_img >= 0 && patch > 0 && height % patch == 0 &&
                  width % patch == 0 && k_pad % 8 == 0 &&
                  k_pad >= 3 * patch * patch,
              FVX_ERR_SHAPE,
              "im2col_patches: H, W must be multiples of patch and k_pad a "
              "multiple of 8 >= 3*patch^2");
  FVX_REQUIRE(aligned16(patches), FVX_ERR_ALIGN,
              "im2col_patches: patches must be 16B aligned");
  const int64_t total = n_img * (height / patch) * (width / patch) * (k_pad / 8);
  if (total == 0) return FVX_OK;
  hipLaunchKernelGGL(im2col_kernel, dim3((unsigned)((total + 255) / 256)),
                     dim3(256), 0, (hipStream_t)stream, images, in_f32,
                     channels_last ? 1 : 0, (bf16_t*)patches, n_img,
                     (int)height, (int)width,
                     (int)patch, (int)k_pad, in_scale, in_shift);
  return launch_status("im2col_patches");
}

extern "C" int fvx_embed_tokens(const void* table, const int64_t* ids,
                                void* out, int64_t n_tokens, int64_t dim,
                                int64_t vocab, float scale, int64_t row_group,
                                int64_t row_group_stride, void* stream) {
  clear_error();
  FVX_REQUIRE(table && ids && out, FVX_ERR_NULL,
              "embed_tokens: table, ids, out required");
  FVX_REQUIRE(n_tokens >= 0 && dim > 0 && dim % 8 == 0 && vocab > 0 &&
                  row_group >= 0,
              FVX_ERR_SHAPE, "embed_tokens: bad sizes");
  FVX_REQUIRE(aligned16(table) && aligned16(out), FVX_ERR_ALIGN,
              "embed_tokens: table and out must be 16B aligned");
  const int64_t total = n_tokens * (dim / 8);
  if (total == 0) return FVX_OK;
  hipLaunchKernelGGL(embed_kernel, dim3((unsigned)((total + 255) / 256)),
                     dim3(256), 0, (hipStream_t)stream, (const bf16_t*)table,
                     ids, (bf16_t*)out, n_tokens, (int)dim, vocab, scale,
                     row_group, row_group_stride);
  return launch_status("embed_tokens");
}

extern "C" int fvx_copy_rows(const void* src, int64_t src_ld, void* dst,
                             int64_t dst_ld, int64_t rows, int64_t cols,
                             int64_t row_group, int64_t dst_group_stride,
                             void* stream) {
  clear_error();
  FVX_REQUIRE(src && dst, FVX_ERR_NULL, "copy_rows: src and dst required");
  FVX_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && src_ld % 8 == 0 &&
                  dst_ld % 8 == 0 && row_group >= 0,
              FVX_ERR_SHAPE, "copy_rows: bad sizes");
  FVX_REQUIRE(aligned16(src) && aligned16(dst), FVX_ERR_ALIGN,
              "copy_rows: pointers must be 16B aligned");
  const int64_t total = rows * (cols / 8);
  if (total == 0) return FVX_OK;
  hipLaunchKernelGGL(copy_rows_kernel, dim3((unsigned)((total + 255) / 256)),
                     dim3(256), 0, (hipStream_t)stream, (const bf16_t*)src,
                     src_ld, (bf16_t*)dst, dst_ld, rows, (int)cols, row_group,
                     dst_group_stride);
  return launch_status("copy_rows");
}

extern "C" int fvx_pack_frag(const void* src, int64_t src_ld, void* dst,
                             int64_t rows, int64_t cols, void* stream) {
  clear_error();
  FVX_REQUIRE(src && dst, FVX_ERR_NULL, "pack_frag: src and dst required");
  FVX_REQUIRE(rows >= 0 && rows <= 64 && cols > 0 && cols % 32 == 0 &&
                  src_ld % 8 == 0 && src_ld >= cols,
              FVX_ERR_SHAPE,
              "pack_frag: need rows <= 64, cols %% 32 == 0, src_ld %% 8 == 0");
  FVX_REQUIRE(aligned16(src) && aligned16(dst), FVX_ERR_ALIGN,
              "pack_frag: pointers must be 16B aligned");
  const int64_t total = rows * (cols / 8);
  if (total == 0) return FVX_OK;
  hipLaunchKernelGGL(pack_frag_kernel, dim3((unsigned)((total + 255) / 256)),
                     dim3(256), 0, (hipStream_t)stream, (const bf16_t*)src,
                     src_ld, (bf16_t*)dst, rows, cols);
  return launch_status("pack_frag");
}
