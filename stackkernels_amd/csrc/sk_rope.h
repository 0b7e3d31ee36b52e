// Rotary position embedding as a load-time transform of a head vector.
//
// The rotation is the reference's apply_rope_single
// (src/stackkernels/_reference/torch/rope.py:40-58 with rotate_half :32-37):
// out = x * cos + rotate_half(x) * sin in fp32, rotate_half(x) = (-x2, x1)
// over the two halves of the head dim, cast back to the tensor's type.  The
// two products and the sum are separate fp32 roundings (never fused into a
// multiply-add), which is what the reference's
// elementwise fp32 ops do, so a rotated 16-bit vector matches it bit for bit.
#pragma once

#include "sk_common.h"
#include "sk_kernels.h"

namespace sk {

// Table entry idx (element index) as fp32.
__device__ __forceinline__ float rope_entry(const RopeParams& r, const void* tab, int64_t idx) {
  if (r.dtype == 0) return ((const float*)tab)[idx];
  const uint16_t w = ((const uint16_t*)tab)[idx];
  return r.dtype == 1 ? to_f32<F16>(w) : to_f32<BF16>(w);
}

// Table row of token t of batch row b, or -1 when the rotation is off or the
// position lies outside the table (the vector is then left as it is).
__device__ __forceinline__ int rope_row(const RopeParams& r, int b, int t) {
  if (!r.cos) return -1;
  const int64_t pos = (int64_t)(r.pos_b ? r.pos_b[b] : 0) + r.start + t;
  return (pos >= 0 && pos < r.rows) ? (int)pos : -1;
}

// x * c + (-partner or partner) * s, with the first-half sign when lo_half.
// Each product passes through an empty asm statement, so the backend cannot
// fuse it with the sum into a fused multiply-add (the library is compiled
// with -ffp-contract=fast).
__device__ __forceinline__ float rope_mix(float x, float partner, bool lo_half, float c,
                                          float s) {
  float xc = x * c;
  float ps = (lo_half ? -partner : partner) * s;
  asm volatile("" : "+v"(xc), "+v"(ps));
  return xc + ps;
}

// Table entries [d0, d0 + N) of row `row` of cos and sin as fp32 (N = 4 or
// 8, d0 % N == 0).  The tables are 16-byte aligned with row strides that are
// multiples of 16 bytes, so each is one or two vector loads.
template <int N>
__device__ __forceinline__ void rope_coeffs(const RopeParams& r, int row, int d0, float (&c)[N],
                                            float (&s)[N]) {
  static_assert(N == 4 || N == 8, "4 or 8 entries");
  const int64_t off = (int64_t)row * r.stride + d0;
  if (r.dtype == 0) {
    const f32x4* cp = reinterpret_cast<const f32x4*>((const float*)r.cos + off);
    const f32x4* sp = reinterpret_cast<const f32x4*>((const float*)r.sin + off);
#pragma unroll
    for (int q = 0; q < N / 4; ++q) {
      const f32x4 a = cp[q], b = sp[q];
#pragma unroll
      for (int e = 0; e < 4; ++e) c[4 * q + e] = a[e], s[4 * q + e] = b[e];
    }
    return;
  }
  uint32_t cw[N / 2], sw[N / 2];
  if constexpr (N == 8) {
    const u32x4 a = *reinterpret_cast<const u32x4*>((const uint16_t*)r.cos + off);
    const u32x4 b = *reinterpret_cast<const u32x4*>((const uint16_t*)r.sin + off);
#pragma unroll
    for (int e = 0; e < 4; ++e) cw[e] = a[e], sw[e] = b[e];
  } else {
    const u32x2 a = *reinterpret_cast<const u32x2*>((const uint16_t*)r.cos + off);
    const u32x2 b = *reinterpret_cast<const u32x2*>((const uint16_t*)r.sin + off);
#pragma unroll
    for (int e = 0; e < 2; ++e) cw[e] = a[e], sw[e] = b[e];
  }
  const bool f16 = r.dtype == 1;
#pragma unroll
  for (int e = 0; e < N / 2; ++e) {
    const uint16_t c0 = (uint16_t)(cw[e] & 0xffffu), c1 = (uint16_t)(cw[e] >> 16);
    const uint16_t s0 = (uint16_t)(sw[e] & 0xffffu), s1 = (uint16_t)(sw[e] >> 16);
    c[2 * e] = f16 ? to_f32<F16>(c0) : to_f32<BF16>(c0);
    c[2 * e + 1] = f16 ? to_f32<F16>(c1) : to_f32<BF16>(c1);
    s[2 * e] = f16 ? to_f32<F16>(s0) : to_f32<BF16>(s0);
    s[2 * e + 1] = f16 ? to_f32<F16>(s1) : to_f32<BF16>(s1);
  }
}

// Eight 16-bit elements d0..d0+7 of a head vector (x) and the eight at
// d0 +- D/2 (partner; the chunk lies in one half because D/2 % 8 == 0),
// rotated with the table entries c, s of those columns; lo: d0 < D/2.
template <class T>
__device__ __forceinline__ u32x4 rope8(u32x4 x, u32x4 partner, bool lo, const float (&c)[8],
                                       const float (&s)[8]) {
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t xw = x[i], pw = partner[i];
    const float a = rope_mix(to_f32<T>((uint16_t)(xw & 0xffffu)),
                             to_f32<T>((uint16_t)(pw & 0xffffu)), lo, c[2 * i], s[2 * i]);
    const float b = rope_mix(to_f32<T>((uint16_t)(xw >> 16)), to_f32<T>((uint16_t)(pw >> 16)),
                             lo, c[2 * i + 1], s[2 * i + 1]);
    out[i] = pack2<T>(a, b);
  }
  return out;
}

// rope8 with the table entries of row `row` loaded here.
template <class T>
__device__ __forceinline__ u32x4 rope8_at(u32x4 x, u32x4 partner, int d0, int half,
                                          const RopeParams& r, int row) {
  float c[8], s[8];
  rope_coeffs<8>(r, row, d0, c, s);
  return rope8<T>(x, partner, d0 < half, c, s);
}

// One fp32 element d of the head vector at xrow (D elements), rotated.
__device__ __forceinline__ float rope1(const float* xrow, int d, int half, const RopeParams& r,
                                       int row) {
  const bool lo = d < half;
  const float partner = xrow[lo ? d + half : d - half];
  const int64_t e = (int64_t)row * r.stride + d;
  return rope_mix(xrow[d], partner, lo, rope_entry(r, r.cos, e), rope_entry(r, r.sin, e));
}

}  // namespace sk
