// Camera-frame preprocessing on the device: resize (optionally into a padded
// region), per-channel normalization and the HWC -> CHW / BGR -> RGB
// reordering, written straight into the fp32 image planes the patch
// embedding reads.  Replaces the host transforms ResizeImages /
// ResizeImagesWithPad / NormalizeImages / TransformImage
// (fluxvla/transforms/transform_images.py:80-200, 313-390, 414-560) and
// resize_with_pad (fluxvla/engines/utils/model_utils.py:98-120).
//
// One thread per output pixel (all three channels).  Two filters:
//  * LINEAR: two-tap bilinear with half-pixel centres and edge clamping, in
//    fp32 -- the arithmetic of torch's bilinear interpolate
//    (align_corners=False, no antialiasing), which is also what OpenCV's
//    INTER_LINEAR computes (there with 11-bit fixed-point weights); the
//    result may be rounded to uint8 as a uint8 resize returns it.
//  * PIL_BILINEAR: Pillow's BILINEAR resample -- a triangle filter widened by
//    the downscale factor (antialiasing), weights normalized per output pixel
//    and quantized to 22 fractional bits, a horizontal pass rounded to uint8
//    followed by a vertical pass rounded to uint8.  Coefficients are computed
//    per thread in double precision with contraction off, so they equal the
//    host computation bit for bit.
// The kernels are tiny and memory bound (a 224 x 224 view is 150 KB of
// input, 600 KB of fp32 output).
#include "capi_util.h"
#include "common.h"

namespace fvx {

constexpr int kPilPrec = 22;      // fractional bits of the fixed-point weights
constexpr int kPilMaxTaps = 32;   // taps per direction (downscale <= 15x)

struct PilTaps {
  int lo, cnt;
  int k[kPilMaxTaps];
};

// Taps of output index `o` for a resize of `in` samples to `out` samples.
__device__ __noinline__ void pil_taps(int o, int in, int out, PilTaps& t) {
#pragma clang fp contract(off)
  const double scale = (double)in / (double)out;
  const double fs = scale < 1.0 ? 1.0 : scale;
  const double support = fs;  // bilinear support 1, widened by the scale
  const double center = ((double)o + 0.5) * scale;
  const double ss = 1.0 / fs;
  int lo = (int)(center - support + 0.5);
  if (lo < 0) lo = 0;
  int hi = (int)(center + support + 0.5);
  if (hi > in) hi = in;
  int cnt = hi - lo;
  if (cnt > kPilMaxTaps) cnt = kPilMaxTaps;  // excluded by the host check
  double w[kPilMaxTaps];
  double ww = 0.0;
  for (int x = 0; x < cnt; ++x) {
    double a = ((double)(x + lo) - center + 0.5) * ss;
    if (a < 0.0) a = -a;
    w[x] = a < 1.0 ? 1.0 - a : 0.0;
    ww += w[x];
  }
  for (int x = 0; x < cnt; ++x) {
    const double v = ww != 0.0 ? w[x] / ww : w[x];
    const double f = v * (double)(1 << kPilPrec);
    t.k[x] = v < 0.0 ? (int)(-0.5 + f) : (int)(0.5 + f);
  }
  t.lo = lo;
  t.cnt = cnt;
}

__device__ __forceinline__ int pil_clip8(int v) {
  if (v >= (1 << kPilPrec << 8)) return 255;
  if (v <= 0) return 0;
  return v >> kPilPrec;
}

__device__ __forceinline__ float src_px(const void* src, int u8, int hwc,
                                        int64_t base, int64_t h, int64_t w,
                                        int c, int64_t y, int64_t x) {
  const int64_t off = hwc ? base + (y * w + x) * 3 + c : base + (c * h + y) * w + x;
  return u8 ? (float)((const uint8_t*)src)[off] : ((const float*)src)[off];
}

__global__ void resize_normalize_kernel(fvx_image_desc d) {
  const int64_t total = d.n * d.dst_h * d.dst_w;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int64_t img = idx / (d.dst_h * d.dst_w);
  const int64_t y = (idx / d.dst_w) % d.dst_h;
  const int64_t x = idx % d.dst_w;
  const int64_t sbase = img * d.src_img_stride;
  float v[3];
  const int64_t ry = y - d.off_y, rx = x - d.off_x;
  if (ry < 0 || ry >= d.rh || rx < 0 || rx >= d.rw) {
#pragma unroll
    for (int c = 0; c < 3; ++c) v[c] = d.pad_per_channel ? d.pad_rgb[c] : d.pad_value;
  } else if (d.filter == FVX_RESIZE_PIL_BILINEAR) {
    PilTaps tx, ty;
    pil_taps((int)rx, (int)d.src_w, (int)d.rw, tx);
    pil_taps((int)ry, (int)d.src_h, (int)d.rh, ty);
    int acc[3] = {1 << (kPilPrec - 1), 1 << (kPilPrec - 1), 1 << (kPilPrec - 1)};
    for (int j = 0; j < ty.cnt; ++j) {
      const int64_t sy = ty.lo + j;
      int hs[3] = {1 << (kPilPrec - 1), 1 << (kPilPrec - 1), 1 << (kPilPrec - 1)};
      for (int i = 0; i < tx.cnt; ++i) {
        const int64_t sx = tx.lo + i;
#pragma unroll
        for (int c = 0; c < 3; ++c)
          hs[c] += (int)src_px(d.src, 1, d.src_hwc, sbase, d.src_h, d.src_w,
                               d.swap_rb ? 2 - c : c, sy, sx) * tx.k[i];
      }
#pragma unroll
      for (int c = 0; c < 3; ++c) acc[c] += pil_clip8(hs[c]) * ty.k[j];
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) v[c] = (float)pil_clip8(acc[c]);
  } else {
    // source coordinate of a half-pixel-centred sample, clamped at 0
    const float scy = (float)d.src_h / (float)d.rh;
    const float scx = (float)d.src_w / (float)d.rw;
    float fy = scy * ((float)ry + 0.5f) - 0.5f;
    float fx = scx * ((float)rx + 0.5f) - 0.5f;
    fy = fy < 0.f ? 0.f : fy;
    fx = fx < 0.f ? 0.f : fx;
    const int64_t y0 = (int64_t)fy, x0 = (int64_t)fx;
    const int64_t y1 = y0 + (y0 < d.src_h - 1 ? 1 : 0);
    const int64_t x1 = x0 + (x0 < d.src_w - 1 ? 1 : 0);
    const float ly1 = fy - (float)y0, lx1 = fx - (float)x0;
    const float ly0 = 1.f - ly1, lx0 = 1.f - lx1;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const int cs = d.swap_rb ? 2 - c : c;
      const float p00 = src_px(d.src, d.src_u8, d.src_hwc, sbase, d.src_h, d.src_w, cs, y0, x0);
      const float p01 = src_px(d.src, d.src_u8, d.src_hwc, sbase, d.src_h, d.src_w, cs, y0, x1);
      const float p10 = src_px(d.src, d.src_u8, d.src_hwc, sbase, d.src_h, d.src_w, cs, y1, x0);
      const float p11 = src_px(d.src, d.src_u8, d.src_hwc, sbase, d.src_h, d.src_w, cs, y1, x1);
      float r = ly0 * (lx0 * p00 + lx1 * p01) + ly1 * (lx0 * p10 + lx1 * p11);
      if (d.round_u8) {
        r = floorf(r + 0.5f);
        r = r < 0.f ? 0.f : (r > 255.f ? 255.f : r);
      }
      v[c] = r;
    }
  }
  float* out = d.dst + img * d.dst_img_stride + y * d.dst_w + x;
  const int64_t plane = d.dst_h * d.dst_w;
#pragma unroll
  for (int c = 0; c < 3; ++c) out[c * plane] = (v[c] / d.pre_div - d.mean[c]) / d.den[c];
}

}  // namespace fvx

using namespace fvx;

extern "C" int fvx_resize_normalize(const fvx_image_desc* desc, void* stream) {
  clear_error();
  FVX_REQUIRE(desc, FVX_ERR_NULL, "resize_normalize: desc required");
  const fvx_image_desc& d = *desc;
  FVX_REQUIRE(d.src && d.dst, FVX_ERR_NULL, "resize_normalize: src and dst required");
  FVX_REQUIRE(d.n >= 0 && d.src_h > 0 && d.src_w > 0 && d.dst_h > 0 && d.dst_w > 0 &&
                  d.rh > 0 && d.rw > 0 && d.off_y >= 0 && d.off_x >= 0 &&
                  d.off_y + d.rh <= d.dst_h && d.off_x + d.rw <= d.dst_w,
              FVX_ERR_SHAPE,
              "resize_normalize: sizes must be positive and the resized region "
              "[off_y, off_y + rh) x [off_x, off_x + rw) inside dst");
  FVX_REQUIRE(d.src_h < (1 << 24) && d.src_w < (1 << 24) && d.rh < (1 << 24) &&
                  d.rw < (1 << 24),
              FVX_ERR_SHAPE, "resize_normalize: image sides must be < 2^24");
  FVX_REQUIRE(d.src_img_stride >= 3 * d.src_h * d.src_w &&
                  d.dst_img_stride >= 3 * d.dst_h * d.dst_w,
              FVX_ERR_SHAPE, "resize_normalize: image strides too small");
  FVX_REQUIRE(d.filter == FVX_RESIZE_LINEAR || d.filter == FVX_RESIZE_PIL_BILINEAR,
              FVX_ERR_ARG, "resize_normalize: bad filter %d", d.filter);
  FVX_REQUIRE(d.src_u8 || (d.filter == FVX_RESIZE_LINEAR && !d.round_u8), FVX_ERR_ARG,
              "resize_normalize: fp32 sources take the LINEAR filter without "
              "uint8 rounding");
  if (d.filter == FVX_RESIZE_PIL_BILINEAR) {
    const double sy = (double)d.src_h / (double)d.rh, sx = (double)d.src_w / (double)d.rw;
    const double s = sy > sx ? sy : sx;
    const int taps = 2 * (int)ceil(s < 1.0 ? 1.0 : s) + 1;
    FVX_REQUIRE(taps <= kPilMaxTaps, FVX_ERR_SHAPE,
                "resize_normalize: PIL filter downscale of %.2fx exceeds %d taps", s,
                kPilMaxTaps);
  }
  for (int c = 0; c < 3; ++c)
    FVX_REQUIRE(d.den[c] != 0.f, FVX_ERR_ARG, "resize_normalize: den[%d] is 0", c);
  FVX_REQUIRE(d.pre_div != 0.f, FVX_ERR_ARG, "resize_normalize: pre_div is 0");
  const int64_t total = d.n * d.dst_h * d.dst_w;
  if (total == 0) return FVX_OK;
  const int threads = 256;
  hipLaunchKernelGGL(resize_normalize_kernel, dim3((unsigned)((total + threads - 1) / threads)),
                     dim3(threads), 0, (hipStream_t)stream, d);
  return launch_status("resize_normalize");
}
