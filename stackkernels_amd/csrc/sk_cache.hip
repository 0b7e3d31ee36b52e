// KV-cache append for decode: write T new key/value rows per (batch, KV head)
// into cache positions given per token.
//
// Realises the reference's planned kv_cache_update(k, v, k_cache, v_cache,
// slot_indices) (docs/user_guide/dropout_cache_sampling.md:66-72; stub
// modules src/stackkernels/torch/cache.py, src/stackkernels/_core/cache/kv_update.py).
//
// One thread moves one UNIT-byte chunk of a new token's K row and the same
// chunk of V, for up to four KV heads: consecutive threads walk a row's
// chunks, so every wave's loads and stores are contiguous runs, and the
// token's slot is read once per four heads.
// A slot outside [0, S) skips the token, which lets callers pad ragged
// batches with -1.  Plain byte copies: the cache holds exactly the input's
// bits.
//
// With RoPE tables the keys are rotated on their way into the cache (the
// reference's apply_rope on k followed by the append, in one pass over the
// new rows): one thread then moves an aligned 16-byte chunk of a token's K
// row, which it rotates with the chunk half a head away, and the same chunk of
// V, for up to four KV heads, so the token's slot, position and table entries
// are read once per four heads.
#include "sk_common.h"
#include "sk_kernels.h"
#include "sk_rope.h"

namespace sk {

template <int UNIT>
struct CopyUnit;
template <>
struct CopyUnit<16> {
  using type = u32x4;
};
template <>
struct CopyUnit<8> {
  using type = u32x2;
};
template <>
struct CopyUnit<4> {
  using type = uint32_t;
};
template <>
struct CopyUnit<2> {
  using type = uint16_t;
};

// Thread i of grid row y copies UNIT-byte chunk c of new token t of batch
// row b, (b, t, c) = split(i), for the KV heads [kHeadsPerThread * y,
// kHeadsPerThread * (y + 1)): the token's slot is read once for all of them.
constexpr int kHeadsPerThread = 4;

template <int UNIT>
__global__ void __launch_bounds__(256) kv_cache_update_kernel(CacheParams p) {
  using U = typename CopyUnit<UNIT>::type;
  const int chunks = p.row_bytes / UNIT;
  const int i = blockIdx.x * 256 + threadIdx.x;  // < B * T * chunks (checked on the host)
  if (i >= p.B * p.T * chunks) return;
  const int bt = i / chunks;
  const int c = i - bt * chunks;
  const int b = bt / p.T;
  const int t = bt - b * p.T;
  const int64_t slot = p.slots[bt];
  if (slot < 0 || slot >= p.S) return;
  // Contiguous: row slot of batch row b's cache.  Paged: in-page row of a page.
  const int64_t unit = p.page_size > 0 ? slot / p.page_size : b;
  const int64_t row = p.page_size > 0 ? slot % p.page_size : slot;
  const int64_t e = p.esize;
  const int h0 = blockIdx.y * kHeadsPerThread;
#pragma unroll
  for (int j = 0; j < kHeadsPerThread; ++j) {
    const int h = h0 + j;
    if (h >= p.Hkv) break;
    const char* ks = (const char*)p.k + (b * p.k_sb + h * p.k_sh + t * p.k_ss) * e + (int64_t)c * UNIT;
    const char* vs = (const char*)p.v + (b * p.v_sb + h * p.v_sh + t * p.v_ss) * e + (int64_t)c * UNIT;
    char* kd = (char*)p.kc + (unit * p.kc_sb + h * p.kc_sh + row * p.kc_ss) * e + (int64_t)c * UNIT;
    char* vd = (char*)p.vc + (unit * p.vc_sb + h * p.vc_sh + row * p.vc_ss) * e + (int64_t)c * UNIT;
    const U kx = *reinterpret_cast<const U*>(ks);
    const U vx = *reinterpret_cast<const U*>(vs);
    *reinterpret_cast<U*>(kd) = kx;
    *reinterpret_cast<U*>(vd) = vx;
  }
}

// Rotating append.  Thread i of grid row y handles 16-byte chunk c of new
// token t of batch row b, (b, t, c) = split(i), for the KV heads
// [kHeadsPerThread * y, kHeadsPerThread * (y + 1)): the slot, the position
// and the table entries are loaded once for all of them.  T: BF16 / F16 (8
// elements per chunk) or float (4).
template <class T>
__global__ void __launch_bounds__(256) kv_cache_update_rope_kernel(CacheParams p) {
  constexpr bool kF32 = __is_same(T, float);
  constexpr int EPC = kF32 ? 4 : 8;  // elements per 16-byte chunk
  using E = typename std::conditional<kF32, float, uint16_t>::type;
  const int chunks = p.D / EPC;
  const int i = blockIdx.x * 256 + threadIdx.x;  // < B * T * chunks (checked on the host)
  if (i >= p.B * p.T * chunks) return;
  const int bt = i / chunks;
  const int c = i - bt * chunks;
  const int b = bt / p.T;
  const int t = bt - b * p.T;
  const int64_t slot = p.slots[bt];
  if (slot < 0 || slot >= p.S) return;
  const int64_t unit = p.page_size > 0 ? slot / p.page_size : b;
  const int64_t row = p.page_size > 0 ? slot % p.page_size : slot;
  const int d0 = c * EPC;
  const int half = p.D >> 1;
  const bool lo = d0 < half;
  const int dp = lo ? d0 + half : d0 - half;  // partner chunk, half a head away
  const int rrow = rope_row(p.rope, b, t);
  float cs[EPC], sn[EPC];
  if (rrow >= 0) rope_coeffs<EPC>(p.rope, rrow, d0, cs, sn);
  const int h0 = blockIdx.y * kHeadsPerThread;
#pragma unroll
  for (int j = 0; j < kHeadsPerThread; ++j) {
    const int h = h0 + j;
    if (h >= p.Hkv) break;
    const E* ks = (const E*)p.k + b * p.k_sb + h * p.k_sh + t * p.k_ss;
    const E* vs = (const E*)p.v + b * p.v_sb + h * p.v_sh + t * p.v_ss;
    E* kd = (E*)p.kc + unit * p.kc_sb + h * p.kc_sh + row * p.kc_ss;
    E* vd = (E*)p.vc + unit * p.vc_sb + h * p.vc_sh + row * p.vc_ss;
    const u32x4 vx = *reinterpret_cast<const u32x4*>(vs + d0);
    u32x4 kx = *reinterpret_cast<const u32x4*>(ks + d0);
    if (rrow >= 0) {
      const u32x4 kp = *reinterpret_cast<const u32x4*>(ks + dp);
      if constexpr (kF32) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // (Elements are copied out before the bit casts: clang's bit cast
          // of a vector element expression reads element 0 whatever the index.)
          const uint32_t xw = kx[e], pw = kp[e];
          const float r = rope_mix(__builtin_bit_cast(float, xw), __builtin_bit_cast(float, pw),
                                   lo, cs[e], sn[e]);
          kx[e] = __builtin_bit_cast(uint32_t, r);
        }
      } else {
        kx = rope8<T>(kx, kp, lo, cs, sn);
      }
    }
    *reinterpret_cast<u32x4*>(kd + d0) = kx;
    *reinterpret_cast<u32x4*>(vd + d0) = vx;
  }
}

// Largest copy unit (16, 8, 4 or 2 bytes) that divides the row and every
// byte address and stride involved.
static int copy_unit(const CacheParams& p) {
  uint64_t bits = (uint64_t)p.row_bytes;
  const void* ptrs[4] = {p.k, p.v, p.kc, p.vc};
  for (const void* q : ptrs) bits |= (uint64_t)(uintptr_t)q;
  const int64_t strides[12] = {p.k_sb, p.k_sh, p.k_ss, p.v_sb, p.v_sh, p.v_ss,
                               p.kc_sb, p.kc_sh, p.kc_ss, p.vc_sb, p.vc_sh, p.vc_ss};
  for (int64_t st : strides) bits |= (uint64_t)(st * p.esize);
  for (int u = 16; u >= 2; u /= 2)
    if ((bits & (uint64_t)(u - 1)) == 0) return u;
  return 1;
}

hipError_t launch_kv_cache_update(const CacheParams& p, hipStream_t s) {
  const int unit = copy_unit(p);
  if (p.rope.cos) {
    // Rotating path: 16-byte chunks; D / 2 a multiple of the chunk.
    const int epc = 16 / p.esize;
    if (unit < 16 || p.D % (2 * epc) != 0) return hipErrorInvalidValue;
    const int64_t threads = (int64_t)p.B * p.T * (p.D / epc);
    if (threads == 0) return hipSuccess;
    if (threads > 0x7fffffffLL - 255) return hipErrorInvalidConfiguration;
    const int64_t head_groups = (p.Hkv + kHeadsPerThread - 1) / kHeadsPerThread;
    if (head_groups > 65535) return hipErrorInvalidConfiguration;
    const dim3 grid((unsigned)((threads + 255) / 256), (unsigned)head_groups);
    switch (p.dtype) {
      case 0: hipLaunchKernelGGL(kv_cache_update_rope_kernel<float>, grid, dim3(256), 0, s, p); break;
      case 1: hipLaunchKernelGGL(kv_cache_update_rope_kernel<F16>, grid, dim3(256), 0, s, p); break;
      default: hipLaunchKernelGGL(kv_cache_update_rope_kernel<BF16>, grid, dim3(256), 0, s, p); break;
    }
    return hipGetLastError();
  }
  if (unit < 2) return hipErrorInvalidValue;
  const int64_t threads = (int64_t)p.B * p.T * (p.row_bytes / unit);
  if (threads == 0) return hipSuccess;
  if (threads > 0x7fffffffLL - 255) return hipErrorInvalidConfiguration;
  const int64_t head_groups = (p.Hkv + kHeadsPerThread - 1) / kHeadsPerThread;
  if (head_groups > 65535) return hipErrorInvalidConfiguration;
  const dim3 grid((unsigned)((threads + 255) / 256), (unsigned)head_groups);
  switch (unit) {
    case 16: hipLaunchKernelGGL(kv_cache_update_kernel<16>, grid, dim3(256), 0, s, p); break;
    case 8: hipLaunchKernelGGL(kv_cache_update_kernel<8>, grid, dim3(256), 0, s, p); break;
    case 4: hipLaunchKernelGGL(kv_cache_update_kernel<4>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(kv_cache_update_kernel<2>, grid, dim3(256), 0, s, p); break;
  }
  return hipGetLastError();
}

}  // namespace sk
