// Shared device helpers for the gfx950 kernels of libfluxvla_amd.
//
// Storage type for bf16 is a raw uint16_t; arithmetic is always fp32.
// Conversions use round-to-nearest-even (the same rounding torch uses when it
// casts fp32 -> bf16), so a kernel that rounds at the same point as the
// reference's PyTorch path produces the same bits there.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fvx {

typedef uint16_t bf16_t;
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(bf16_t v) {
  return __uint_as_float(((uint32_t)v) << 16);
}

// fp32 -> bf16 with round-to-nearest-even (NaN stays a quiet NaN): gfx950's
// v_cvt_pk_bf16_f32, two values per instruction.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

__device__ __forceinline__ bf16_t f2bf(float f) {
  return __builtin_bit_cast(bf16_t, (__bf16)f);
}

// 8 packed bf16 values (one 16-byte vector).
struct __align__(16) bf16x8 {
  uint32_t w[4];
};

__device__ __forceinline__ void unpack8(const bf16x8& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(v.w[i] << 16);
    f[2 * i + 1] = __uint_as_float(v.w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ bf16x8 pack8(const float* f) {
  bf16x8 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v.w[i] = f2bf2(f[2 * i], f[2 * i + 1]);
  return v;
}

__device__ __forceinline__ bf16x8 ld8(const bf16_t* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}

__device__ __forceinline__ void st8(bf16_t* p, const bf16x8& v) {
  *reinterpret_cast<bf16x8*>(p) = v;
}

__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 v;
  v.w[0] = v.w[1] = v.w[2] = v.w[3] = 0u;
  return v;
}

__device__ __forceinline__ bf16x8_t as_mfma(const bf16x8& v) {
  return __builtin_bit_cast(bf16x8_t, v);
}

// D(16x16, fp32) += A(16x32) * B(32x16), bf16 inputs.
// Lane l supplies A row (l % 16) and B column (l % 16), each with 8 k-values
// of the k-group (l / 16). D lane l holds column (l % 16), rows 4*(l/16)+j.
__device__ __forceinline__ f32x4_t mfma16x16x32(const bf16x8& a,
                                                const bf16x8& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_mfma(a), as_mfma(b), c, 0,
                                                 0, 0);
}

// D(32x32, fp32) += A(32x16) * B(16x32), bf16 inputs.
// Lane l supplies A row (l % 32) and B column (l % 32), each with the 8
// k-values 8 (l / 32) .. + 7.  D lane l holds column (l % 32), rows
// 8 (r / 4) + 4 (l / 32) + r % 4 for r = 0..15.
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mfma32x32x16(const bf16x8& a,
                                                 const bf16x8& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_mfma(a), as_mfma(b), c, 0,
                                                 0, 0);
}

// ---------------------------------------------------------------------------
// fp8 (OCP e4m3fn, max 448) with power-of-two block scales (E8M0)
// ---------------------------------------------------------------------------
typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef short i16x2_t __attribute__((ext_vector_type(2)));

// E8M0 exponent e (scale 2^(e - 127)) of a block whose largest magnitude has
// bf16 bits `amax`: the smallest power of two with amax / 2^(e-127) <= 448.
// amax = (1 + m/128) 2^(E-127) with E its exponent field; 448 = 1.75 2^8, so
// e = E - 8, one more when m > 96 (1 + m/128 > 1.75).  Clamped to [1, 254].
__device__ __forceinline__ int e8m0_for_amax(uint32_t amax) {
  const int E = (int)((amax >> 7) & 0xff), m = (int)(amax & 0x7f);
  int e = E - 8 + (m > 96 ? 1 : 0);
  return e < 1 ? 1 : (e > 254 ? 254 : e);
}

// Quantize the 32 bf16 values of four 8-vectors (one MFMA lane's share of a
// row's k step) to e4m3, q = fp8(x / 2^(e-127)), round to nearest even
// (v_cvt_scalef32_pk_fp8_bf16).  The scale is shared by all lanes holding
// the same row of the step (the lanes l ^ X1 [^ X2]): the block-scaled MFMAs
// apply a lane's scale to 16-byte halves of other lanes of its row, so one
// scale per (row, step) is what keeps the product exact whatever that
// assignment is.  No value can overflow (see e8m0_for_amax).  Returns the
// packed bytes in k order; *e8 receives the E8M0 exponent.
template <int X1, int X2>
__device__ __forceinline__ i32x8_t quant_fp8x32(const bf16x8* v, int* e8) {
  uint32_t mx = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = v[i].w[j] & 0x7fff7fffu;
      const uint32_t a = w & 0xffffu, b = w >> 16;
      mx = a > mx ? a : mx;
      mx = b > mx ? b : mx;
    }
  uint32_t o = (uint32_t)__shfl_xor((int)mx, X1, 64);
  mx = o > mx ? o : mx;
  if (X2) {
    o = (uint32_t)__shfl_xor((int)mx, X2, 64);
    mx = o > mx ? o : mx;
  }
  const int e = e8m0_for_amax(mx);
  const float scale = __uint_as_float((uint32_t)e << 23);
  i32x8_t q;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      i16x2_t r = {0, 0};
      r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(
          r, __builtin_bit_cast(bf16x2_t, v[i].w[2 * j]), scale, false);
      r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(
          r, __builtin_bit_cast(bf16x2_t, v[i].w[2 * j + 1]), scale, true);
      q[2 * i + j] = __builtin_bit_cast(int, r);
    }
  *e8 = e;
  return q;
}

// Eight e4m3 bytes (k order, `lo` holds the first four) -> eight bf16
// (v_cvt_scalef32_pk_bf16_fp8 with scale 1, two values per instruction).
// Exact: every e4m3 value, subnormals included, is a bf16 value (3 mantissa
// bits within bf16's 7, exponents 2^-9 .. 2^8 within its range).
__device__ __forceinline__ bf16x8 e4m3x8_to_bf16(uint32_t lo, uint32_t hi) {
  bf16x8 r;
  r.w[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.f, false));
  r.w[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.f, true));
  r.w[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.f, false));
  r.w[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.f, true));
  return r;
}

// D(16x16) += A(16x128) * B(128x16), e4m3 inputs with E8M0 block scales:
// lane l holds 32 k-values of A row (l % 16) and of B column (l % 16) (the
// same k positions in A and B), scaled by 2^(sa - 127) and 2^(sb - 127).
__device__ __forceinline__ f32x4_t mfma16x16x128_f8(const i32x8_t& a, int sa,
                                                   const i32x8_t& b, int sb,
                                                   f32x4_t c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, sa,
                                                          0, sb);
}

// D(32x32) += A(32x64) * B(64x32), e4m3 with E8M0 block scales; lane l holds
// 32 k-values of A row (l % 32) / B column (l % 32); D as in mfma32x32x16.
__device__ __forceinline__ f32x16_t mfma32x32x64_f8(const i32x8_t& a, int sa,
                                                    const i32x8_t& b, int sb,
                                                    f32x16_t c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa,
                                                         0, sb);
}

// Raw buffer access: loads at byte offsets >= `bytes` return zero without
// touching memory, so a guarded load needs no branch (a branch around each
// load makes the compiler wait for it at the join, serializing the loads).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base,
                                                            uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                           (int)bytes, 0x00020000);
}

constexpr uint32_t kOOB = 0x80000000u;  // an offset beyond any buffer here

// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4 ...
// lds): lane l's bytes land at LDS address lds + 16 l (wave-uniform `lds`,
// passed in M0).  An out-of-view offset writes zeros.  Issued through inline
// asm: the compiler then does not treat every later LDS read as dependent on
// the load (it would wait for all loads in flight, i.e. for the prefetch),
// so the caller must wait for the load with s_waitcnt vmcnt before reading.
typedef int i32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i32x4_t make_rsrc4(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4_t r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b of a
// 1-D grid runs on XCD b % 8), and each XCD has its own L2.  xcd_remap gives
// XCD x the contiguous logical ids [start(x), start(x) + count(x)), count(x)
// = nblk / 8 (+1 for x < nblk % 8), so that neighbouring tiles (the M tiles
// of one weight panel) share an L2.  A bijection of [0, nblk) for any nblk.
__device__ __forceinline__ int xcd_remap(int bid, int nblk) {
  const int x = bid & 7, local = bid >> 3, per = nblk >> 3, rem = nblk & 7;
  return x * per + (x < rem ? x : rem) + local;
}

typedef __attribute__((address_space(3))) char lds_char_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_char_t*)p;
}

__device__ __forceinline__ void load_lds16(i32x4_t rsrc, uint32_t lds,
                                           uint32_t off) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds), "v"(off), "s"(rsrc)
               : "memory");
}

// load_lds16 with a scalar offset added to every lane's offset.
__device__ __forceinline__ void load_lds16_so(i32x4_t rsrc, uint32_t lds,
                                              uint32_t off, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds), "v"(off), "s"(rsrc), "s"(soff)
               : "memory");
}

// 4 bytes per lane into LDS (buffer_load_dword ... lds): lane l's word lands
// at lds + 4 l.
__device__ __forceinline__ void load_lds4(i32x4_t rsrc, uint32_t lds,
                                          uint32_t off) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds), "v"(off), "s"(rsrc)
               : "memory");
}

// Wait until at most N vector memory operations of this wave are in flight
// (the LDS loads above are invisible to the compiler's own accounting).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  // s_waitcnt: vmcnt[3:0] | expcnt[6:4] = 7 | lgkmcnt[11:8] = 15 | vmcnt[5:4] at [15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ bf16x8 bload8(__amdgpu_buffer_rsrc_t r,
                                         uint32_t off) {
  return __builtin_bit_cast(bf16x8,
                            __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ f32x4_t bload4f(__amdgpu_buffer_rsrc_t r,
                                           uint32_t off) {
  return __builtin_bit_cast(f32x4_t,
                            __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

__device__ __forceinline__ float bload1f(__amdgpu_buffer_rsrc_t r,
                                         uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Element offset of (row m, column k) of an M <= 64 operand in the
// fragment-major layout [K / 32 steps][4 row blocks][64 lanes][8]: lane =
// 16 g + m % 16 with g = (k % 32) / 8, so one 16x32 MFMA A fragment is one
// contiguous 1 KiB block.
__host__ __device__ __forceinline__ int64_t frag_offset(int64_t m, int64_t k) {
  return (((k >> 5) * 4 + (m >> 4)) * 64 + ((k & 31) >> 3) * 16 + (m & 15)) * 8 +
         (k & 7);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Compile-time flag for generic lambdas (a kernel path chosen once, outside
// its loops).
template <bool B>
struct BoolC {
  static constexpr bool value = B;
};

// Compile-time loop: f(IntC<B>{}), ..., f(IntC<E - 1>{}).  Array indices
// derived from the argument are constants before any optimization, so a
// large register array indexed in the body stays in registers.
template <int V>
struct IntC {
  static constexpr int value = V;
};
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(IntC<B>{});
    static_for<B + 1, E>(f);
  }
}

// GeGLU's backward at one element: with h = gelu_tanh(g) * u and the
// incoming dh, dg = dh u gelu'(g) and du = dh gelu(g), where gelu_tanh(g) =
// g s, s = 1 / (1 + exp(-2v)), v = sqrt(2/pi) (g + 0.044715 g^3), so
// gelu' = s + g s (1 - s) 2 sqrt(2/pi) (1 + 3 * 0.044715 g^2).
__device__ __forceinline__ void geglu_grad(float dh, float g, float u, float& dg,
                                           float& du) {
  constexpr float k2 = 1.5957691216057308f;  // 2 sqrt(2 / pi)
  constexpr float k1 = 0.044715f;
  const float s = 1.f / (1.f + expf(-k2 * (g + k1 * g * g * g)));
  dg = dh * u * (s + g * s * (1.f - s) * k2 * (1.f + 3.f * k1 * g * g));
  du = dh * (g * s);
}

__device__ __forceinline__ float gelu_tanh(float x) {
  // 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), written through the
  // identity 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)) with the exponent in
  // base 2 and its constants folded: exp(-2u) = 2^(x (a + b x^2)).  The
  // hardware exp2 and reciprocal (1 ulp) replace the library exp and the
  // IEEE division; at the ends of the range the reciprocal of 1 + inf is 0
  // and of 1 + 0 is 1, the limits of the sigmoid.
  constexpr float a = -1.5957691216057308f * 1.4426950408889634f;  // -2 sqrt(2/pi) log2(e)
  constexpr float b = a * 0.044715f;
  const float t = x * fmaf(b, x * x, a);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// Warm the scalar cache with the first BYTES of the kernel's argument block:
// one scalar load per 64-byte line.  The compiler reads a large descriptor
// argument in several batches of scalar loads, each behind a branch or a use
// and each waited for; cold (the caches start empty in every launch) each
// batch is a memory round trip (~0.3-0.6 us measured) before the first
// operand load can even issue.  After this call those batches hit the
// scalar cache.  The loads are plain ones that an empty asm statement
// consumes: the compiler issues them together with its own first argument
// loads, ahead of their one wait (loads inside the asm statement came after
// that wait, a second round trip).
template <int BYTES>
__device__ __forceinline__ void warm_kernargs() {
  static_assert(BYTES > 0 && BYTES <= 640, "up to ten 64-byte lines");
  constexpr int last = (BYTES - 1) / 64 * 64;
  // line k's offset (lines past the block repeat the last one)
  constexpr int o0 = 0, o1 = 64 < BYTES ? 64 : last, o2 = 128 < BYTES ? 128 : last,
                o3 = 192 < BYTES ? 192 : last, o4 = 256 < BYTES ? 256 : last,
                o5 = 320 < BYTES ? 320 : last, o6 = 384 < BYTES ? 384 : last,
                o7 = 448 < BYTES ? 448 : last, o8 = 512 < BYTES ? 512 : last,
                o9 = 576 < BYTES ? 576 : last;
  const uint32_t* kp = (const uint32_t*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" ::"s"(kp[o0 / 4]), "s"(kp[o1 / 4]), "s"(kp[o2 / 4]), "s"(kp[o3 / 4]),
               "s"(kp[o4 / 4]), "s"(kp[o5 / 4]), "s"(kp[o6 / 4]), "s"(kp[o7 / 4]),
               "s"(kp[o8 / 4]), "s"(kp[o9 / 4]));
}

// Cache prefetch by the idle workgroups of a launch (no counterpart in the
// reference).  Workgroup pw of npw prefetching ones (linear block ids first,
// first + 1, ...; block b runs on XCD b % 8), NW waves, reads up to 8 device
// ranges [ptr[r], ptr[r] + bytes[r]) by LDS DMA into a discarded 1 KiB slot
// per wave (lds_base + 1024 w), so that the next kernels find them in the
// caches.  tile_bytes[r] > 0: the range is a sequence of tiles of that size
// (the 16-column tiles of a fragment-major weight) and tile j is read only by
// the prefetching workgroups of XCD j % 8 -- the XCD whose GEMM workgroup
// will read it -- so it lands in that XCD's L2; 0: an even split over all
// prefetching workgroups (the memory-side cache).  Bytes and tile bytes are
// multiples of 1024.
template <int NW>
__device__ void prefetch_ranges(const void* const* ptr, const int64_t* bytes_of,
                                const int64_t* tile_bytes, int pw, int npw, int first,
                                uint32_t lds_base) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_base + w * 1024);
  const int xcd = (pw + first) & 7;
  // prefetching workgroups on this XCD: indices q0, q0 + 8, ... < npw
  const int q0 = ((xcd - first) % 8 + 8) % 8;
  const int xrank = (pw - q0) / 8, xcount = (npw - q0 + 7) / 8;
#pragma unroll 1
  for (int r = 0; r < 8; ++r) {
    const int64_t bytes = bytes_of[r];
    if (!ptr[r] || bytes <= 0) continue;
    // 32-bit offsets: a range of up to 2 GiB per view
    const i32x4_t rs = make_rsrc4(ptr[r], bytes < 0x7fffffff ? (uint32_t)bytes : 0x7fffffffu);
    const int64_t tb = tile_bytes[r];
    if (tb > 0) {
      // this XCD's tiles j = xcd, xcd + 8, ...: their 1 KiB blocks in order,
      // a contiguous share per prefetching workgroup of the XCD
      const int64_t bpt = tb / 1024, ntiles = bytes / tb;
      const int64_t xt = ntiles > xcd ? (ntiles - xcd + 7) / 8 : 0;
      const int64_t nblk = xt * bpt;
      const int64_t per = (nblk + xcount - 1) / xcount;
      const int64_t b0 = (int64_t)xrank * per;
      const int64_t b1 = b0 + per < nblk ? b0 + per : nblk;
      // block b of the XCD's list is block b % bpt of tile xcd + 8 (b /
      // bpt): one division for the wave's first block, then steps of NW
      // blocks carried into the next tile
      const int nb = b1 > b0 + w ? (int)((b1 - b0 - w + NW - 1) / NW) : 0;
      if (nb > 0) {
        const uint32_t ubpt = (uint32_t)bpt, b = (uint32_t)(b0 + w);
        uint32_t bb = b % ubpt;
        uint32_t off = (uint32_t)(xcd + 8 * (b / ubpt)) * (uint32_t)tb + bb * 1024u;
        const uint32_t wrap = 8u * (uint32_t)tb - ubpt * 1024u;
#pragma unroll 1
        for (int q = 0; q < nb; ++q) {
          load_lds16(rs, lds, off + (uint32_t)lane * 16u);
          bb += NW;
          off += NW * 1024u;
          while (bb >= ubpt) {
            bb -= ubpt;
            off += wrap;
          }
        }
      }
    } else {
      const int64_t nblk = (bytes + 1023) / 1024;
      const int64_t per = (nblk + npw - 1) / npw;
      const int64_t b0 = (int64_t)pw * per;
      const int64_t b1 = b0 + per < nblk ? b0 + per : nblk;
#pragma unroll 1
      for (uint32_t off = (uint32_t)(b0 + w) * 1024u; off < (uint32_t)b1 * 1024u;
           off += NW * 1024u)
        load_lds16(rs, lds, off + (uint32_t)lane * 16u);
    }
  }
  wait_vmcnt<0>();
}

}  // namespace fvx
