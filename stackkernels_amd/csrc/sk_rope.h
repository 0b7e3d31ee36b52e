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

// Eight 16-bit elements d0..d0+7 of a head vector (x) and the eight at
// d0 +- D/2 (partner; the chunk lies in one half because D/2 % 8 == 0),
// rotated for table row `row`.
template <class T>
__device__ __forceinline__ u32x4 rope8(u32x4 x, u32x4 partner, int d0, int half,
                                       const RopeParams& r, int row) {
  const bool lo = d0 < half;
  const int64_t base = (int64_t)row * r.stride + d0;
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t e = base + 2 * i;
    const float a = rope_mix(to_f32<T>((uint16_t)(x[i] & 0xffffu)),
                             to_f32<T>((uint16_t)(partner[i] & 0xffffu)), lo,
                             rope_entry(r, r.cos, e), rope_entry(r, r.sin, e));
    const float b = rope_mix(to_f32<T>((uint16_t)(x[i] >> 16)),
                             to_f32<T>((uint16_t)(partner[i] >> 16)), lo,
                             rope_entry(r, r.cos, e + 1), rope_entry(r, r.sin, e + 1));
    out[i] = pack2<T>(a, b);
  }
  return out;
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
