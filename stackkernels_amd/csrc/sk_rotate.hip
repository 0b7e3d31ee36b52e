// RoPE rotation of a whole (B, H, S, D) tensor, forward or adjoint.
//
// The fused prefill forward rotates q as it loads it and never writes the
// rotated q out; its backward needs that q (for dK and to recompute P) and
// owes dq = R^T dq_rot.  This kernel provides both passes, with the same
// rotation the fused kernels apply (sk_rope.h), so the rotated q is bit for
// bit the one the forward used.  It is also the reference's unfused RoPE:
// rope_fwd / _rope_fwd_kernel and rope_bwd / _rope_bwd_kernel
// (src/stackkernels/_core/positional/rope.py:12-222), whose backward rotates
// by -theta (dx = dy * cos - rotate_half(dy) * sin,
// src/stackkernels/torch/embedding.py:46-66).
//
// One thread rotates one pair of 16-byte chunks of a row, for up to four
// heads of the same token: chunk c of the first half and chunk c of the
// second half, which are each other's partners, so the thread reads both and
// writes both and the pass can run in place.  Consecutive threads walk a
// row's chunk pairs, so a wave reads and writes contiguous runs of each half.
#include "sk_common.h"
#include "sk_kernels.h"
#include "sk_rope.h"

namespace sk {

// Columns d < D/2 and d + D/2 form one plane each: the rotation is
//   y_lo = x_lo c_lo - x_hi s_lo,   y_hi = x_hi c_hi + x_lo s_hi,
// and its adjoint (the transpose, the gradient with respect to x)
//   x_lo = y_lo c_lo + y_hi s_hi,   x_hi = y_hi c_hi - y_lo s_lo,
// each product and the sum rounded to fp32, then to the element type.  With
// tables whose halves are equal (precompute_freqs) the adjoint is the
// rotation by -theta of the reference's backward, bit for bit.
// Heads per thread: the position, and so the table entries, are the same for
// every head of a token, so a thread reads them once and rotates the chunk
// pair of up to kHeads heads (the table reads were twice the bytes of the
// data they rotate).
constexpr int kRotHeads = 4;

template <class T>
__global__ void __launch_bounds__(256) rope_rotate_kernel(RotateParams p) {
  constexpr bool kF32 = __is_same(T, float);
  constexpr int EPC = kF32 ? 4 : 8;  // elements per 16-byte chunk
  using E = typename std::conditional<kF32, float, uint16_t>::type;
  const int half = p.D >> 1;
  const int pairs = half / EPC;
  const int hg_n = (p.H + kRotHeads - 1) / kRotHeads;
  // Thread i: chunk pair c of token t of batch row b, heads h0 .. h0 + 3;
  // consecutive threads walk a row's chunks, then the tokens.
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t tokens = (int64_t)p.B * hg_n * p.S;
  if (i >= tokens * pairs) return;
  const int64_t tok = i / pairs;
  const int c = (int)(i - tok * pairs);
  const int t = (int)(tok % p.S);
  const int64_t bg = tok / p.S;
  const int h0 = (int)(bg % hg_n) * kRotHeads;
  const int b = (int)(bg / hg_n);
  const int nh = min(kRotHeads, p.H - h0);
  const int d0 = c * EPC, d1 = d0 + half;
  const E* xs = (const E*)p.x + b * p.x_sb + h0 * p.x_sh + t * p.x_ss;
  E* os = (E*)p.out + b * p.o_sb + h0 * p.o_sh + t * p.o_ss;
  u32x4 lo[kRotHeads], hi[kRotHeads];
#pragma unroll
  for (int k = 0; k < kRotHeads; ++k)
    if (k < nh) {
      lo[k] = *reinterpret_cast<const u32x4*>(xs + k * p.x_sh + d0);
      hi[k] = *reinterpret_cast<const u32x4*>(xs + k * p.x_sh + d1);
    }
  const int rrow = rope_row(p.rope, b, t);
  if (rrow >= 0) {
    float c0[EPC], s0[EPC], c1[EPC], s1[EPC];
    rope_coeffs<EPC>(p.rope, rrow, d0, c0, s0);
    rope_coeffs<EPC>(p.rope, rrow, d1, c1, s1);
    // rope_mix(x, partner, neg, c, s) = x c + (neg ? -partner : partner) s
    const bool fwd = p.inverse == 0;
    const float(&sl)[EPC] = fwd ? s0 : s1;  // sine multiplying the partner of x_lo
    const float(&sh)[EPC] = fwd ? s1 : s0;  // ... of x_hi
#pragma unroll
    for (int k = 0; k < kRotHeads; ++k) {
      if (k >= nh) continue;
      u32x4 nlo, nhi;
      if constexpr (kF32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // (Elements are copied out before the bit casts: clang's bit cast of
          // a vector element expression reads element 0 whatever the index.)
          const uint32_t lw = lo[k][e], hw = hi[k][e];
          const float xl = __builtin_bit_cast(float, lw), xh = __builtin_bit_cast(float, hw);
          nlo[e] = __builtin_bit_cast(uint32_t, rope_mix(xl, xh, fwd, c0[e], sl[e]));
          nhi[e] = __builtin_bit_cast(uint32_t, rope_mix(xh, xl, !fwd, c1[e], sh[e]));
        }
      } else {
        nlo = rope8<T>(lo[k], hi[k], fwd, c0, sl);
        nhi = rope8<T>(hi[k], lo[k], !fwd, c1, sh);
      }
      lo[k] = nlo, hi[k] = nhi;
    }
  }
#pragma unroll
  for (int k = 0; k < kRotHeads; ++k)
    if (k < nh) {
      *reinterpret_cast<u32x4*>(os + k * p.o_sh + d0) = lo[k];
      *reinterpret_cast<u32x4*>(os + k * p.o_sh + d1) = hi[k];
    }
}

hipError_t launch_rope_rotate(const RotateParams& p, hipStream_t s) {
  const int epc = p.dtype == 0 ? 4 : 8;
  if (p.D % (2 * epc) != 0) return hipErrorInvalidValue;
  const int64_t threads =
      (int64_t)p.B * ((p.H + kRotHeads - 1) / kRotHeads) * p.S * (p.D / (2 * epc));
  if (threads == 0) return hipSuccess;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)blocks);
  switch (p.dtype) {
    case 0: hipLaunchKernelGGL(rope_rotate_kernel<float>, grid, dim3(256), 0, s, p); break;
    case 1: hipLaunchKernelGGL(rope_rotate_kernel<F16>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(rope_rotate_kernel<BF16>, grid, dim3(256), 0, s, p); break;
  }
  return hipGetLastError();
}

}  // namespace sk
