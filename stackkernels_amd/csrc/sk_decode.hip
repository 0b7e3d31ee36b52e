// Split-KV single-token decode for bf16 / fp16 on gfx950, plus the
// LSE-weighted combine.
//
// Replaces _flash_decode_split_kernel and _flash_decode_reduce_kernel
// (reference: src/stackkernels/_core/attention/decode.py:15-121, 124-189).
// Differences by design, none of them visible in the result:
//
// * One workgroup per (batch, KV head, key split) serves every query head of
//   that KV head's group, so each K/V byte is read from HBM once per call
//   (the reference reads it once per query head).  The group's heads are the
//   16-wide column dimension of v_mfma_f32_16x16x32: S^T = K Q^T for 32 keys
//   at a time, then O^T += V^T P^T with V^T read transposed from LDS by
//   ds_read_b64_tr_b16.  Up to 16 heads per wave; a group of 32 or 64 heads
//   (MQA) runs 2 or 4 waves that share each K/V tile.
// * K/V tiles arrive through fully coalesced 16-byte loads (a 64-lane load
//   instruction covers four whole 256-byte rows), are staged in registers one
//   tile ahead of use, and pass through a single padded LDS buffer.
// * Splits write a normalised partial output and its LSE (fp32).  The
//   combine kernel merges them with weights exp(LSE_s - max LSE), which is
//   the reference's (acc, l, m) merge (decode.py:166-186) rewritten on
//   normalised partials.  With one split the kernel writes O directly.
#include "sk_common.h"
#include "sk_kernels.h"

namespace sk {

template <int DP>
struct DecTile {
  static constexpr int kBN = 32;                      // keys per tile
  static constexpr int kStride = DP + 16;             // 16-bit words per LDS row
  static constexpr int kWords = kBN * kStride;
  static constexpr int kChunksPerRow = DP / 8;
  static constexpr int kChunks = kBN * kChunksPerRow;
};

template <class T, int DP, int NWH>
__global__ void __launch_bounds__(NWH * 64) decode_split_kernel(DecParams p) {
  using Tile = DecTile<DP>;
  constexpr int BN = Tile::kBN;
  constexpr int NT = NWH * 64;
  constexpr int LOADS = (Tile::kChunks + NT - 1) / NT;
  constexpr bool kRagged = Tile::kChunks % NT != 0;  // last round covers part of the tile
  constexpr int KD = DP / 32;  // k-steps over the head dim (32 wide)
  constexpr int DB = DP / 16;  // 16-wide head-dim blocks of O^T

  __shared__ __attribute__((aligned(16))) uint16_t ks[Tile::kWords];
  __shared__ __attribute__((aligned(16))) uint16_t vs[Tile::kWords];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int c16 = lane & 15;
  const int g = lane >> 4;

  const int split = blockIdx.x;
  const int bk = blockIdx.y;
  const int b = bk / p.Hkv;
  const int hkv = bk % p.Hkv;
  const int k_lo = split * p.keys_per_split;
  const int k_hi = min(p.Sk, k_lo + p.keys_per_split);
  const int n_tiles = k_hi > k_lo ? (k_hi - k_lo + BN - 1) / BN : 0;

  const int hd = 16 * wave + c16;  // head within the group for this lane's column
  const bool head_ok = hd < p.group;
  const int hq = hkv * p.group + (head_ok ? hd : 0);

  const uint16_t* kbase = (const uint16_t*)p.k + b * p.k_sb + hkv * p.k_sh;
  const uint16_t* vbase = (const uint16_t*)p.v + b * p.v_sb + hkv * p.v_sh;

  // Q^T operand: lane holds q[hq][32*s + 8*g .. +7].
  u32x4 qreg[KD];
  {
    const uint16_t* qp = (const uint16_t*)p.q + b * p.q_sb + hq * p.q_sh;
#pragma unroll
    for (int s = 0; s < KD; ++s) {
      const int d0 = 32 * s + 8 * g;
      u32x4 x = {0u, 0u, 0u, 0u};
      if (head_ok && d0 < p.D) x = ldg_b128_cached(qp + d0);
      qreg[s] = x ^ p.q_sign;
    }
  }

  u32x4 kreg[LOADS], vreg[LOADS];
  auto load_tile = [&](int t) {
    const int n0 = k_lo + t * BN;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * NT;
      const int r = c / Tile::kChunksPerRow;
      const int d = (c % Tile::kChunksPerRow) * 8;
      const int n = n0 + r;
      u32x4 kx = {0u, 0u, 0u, 0u}, vx = {0u, 0u, 0u, 0u};
      if (n < k_hi && d < p.D && (!kRagged || c < Tile::kChunks)) {
        kx = ldg_b128(kbase + (int64_t)n * p.k_ss + d);
        vx = ldg_b128(vbase + (int64_t)n * p.v_ss + d);
      }
      kreg[i] = kx;
      vreg[i] = vx;
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * NT;
      const int r = c / Tile::kChunksPerRow;
      const int d = (c % Tile::kChunksPerRow) * 8;
      if (kRagged && c >= Tile::kChunks) continue;
      *reinterpret_cast<u32x4*>(ks + r * Tile::kStride + d) = kreg[i];
      *reinterpret_cast<u32x4*>(vs + r * Tile::kStride + d) = vreg[i];
    }
  };

  f32x4 oacc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) oacc[c] = f32x4{};
  float m_run = kNegInf;
  float l_run = 0.f;

  const int k_off = c16 * Tile::kStride + 8 * g;
  const int v_off = (4 * g + c16 / 4) * Tile::kStride + 4 * (c16 & 3);

  if (n_tiles > 0) load_tile(0);
  for (int t = 0; t < n_tiles; ++t) {
    store_tile();
    __syncthreads();
    if (t + 1 < n_tiles) load_tile(t + 1);
    const int n0 = k_lo + t * BN;

    f32x4 sacc[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sacc[kb] = f32x4{};
#pragma unroll
      for (int s = 0; s < KD; ++s) {
        const u32x4 a = lds_read_b128(ks + k_off + 16 * kb * Tile::kStride + 32 * s);
        sacc[kb] = mfma16<T>(a, qreg[s], sacc[kb]);
      }
    }
    if (n0 + BN > k_hi) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n0 + 16 * kb + 4 * g + r >= k_hi) sacc[kb][r] = kNegInf;
    }
    float mt = fmaxf(fmaxf(fmaxf(sacc[0][0], sacc[0][1]), fmaxf(sacc[0][2], sacc[0][3])),
                     fmaxf(fmaxf(sacc[1][0], sacc[1][1]), fmaxf(sacc[1][2], sacc[1][3])));
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = xhalf_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const float m_sub = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = fast_exp2((m_run - m_sub) * p.scale_log2);
    const float neg_m = -m_sub * p.scale_log2;
    m_run = m_new;
    float e[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      e[j] = fast_exp2(fmaf(sacc[0][j], p.scale_log2, neg_m));
      e[4 + j] = fast_exp2(fmaf(sacc[1][j], p.scale_log2, neg_m));
    }
    l_run = l_run * alpha + ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
    const u32x4 pk = {pack2<T>(e[0], e[1]), pack2<T>(e[2], e[3]), pack2<T>(e[4], e[5]),
                      pack2<T>(e[6], e[7])};
#pragma unroll
    for (int c = 0; c < DB; ++c) {
      const uint16_t* vp = vs + v_off + 16 * c;
      const u32x2 lo = lds_read_tr(vp);
      const u32x2 hi = lds_read_tr(vp + 16 * Tile::kStride);
      const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
      oacc[c] = mfma16<T>(a, pk, oacc[c] * alpha);
    }
    __syncthreads();
  }

  float l_tot = l_run + __shfl_xor(l_run, 16);
  l_tot = xhalf_sum(l_tot);
  if (!head_ok) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (p.num_splits == 1) {
    uint16_t* op = (uint16_t*)p.o + b * p.o_sb + hq * p.o_sh;
#pragma unroll
    for (int c = 0; c < DB; ++c) {
      const int d = 16 * c + 4 * g;
      if (d < p.D) {
        const u32x2 w = {pack2<T>(oacc[c][0] * inv, oacc[c][1] * inv),
                         pack2<T>(oacc[c][2] * inv, oacc[c][3] * inv)};
        *reinterpret_cast<u32x2*>(op + d) = w;
      }
    }
  } else {
    const int64_t row = ((int64_t)b * p.Hq + hq) * p.num_splits + split;
    float* po = p.part_o + row * p.dpad;
#pragma unroll
    for (int c = 0; c < DB; ++c) {
      const int d = 16 * c + 4 * g;
      *reinterpret_cast<f32x4*>(po + d) = oacc[c] * inv;
    }
    if (g == 0) p.part_lse[row] = l_tot > 0.f ? m_run * p.scale + __logf(l_tot) : kNegInf;
  }
}

// Merge split partials: one 64-lane workgroup per (batch, query head).
template <class T>
__global__ void __launch_bounds__(64) decode_combine_kernel(DecParams p) {
  __shared__ float w[1024];
  const int lane = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / p.Hq;
  const int hq = bh % p.Hq;
  const int ns = p.num_splits;
  const float* lse = p.part_lse + (int64_t)bh * ns;

  float mx = kNegInf;
  for (int s = lane; s < ns; s += 64) mx = fmaxf(mx, lse[s]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  float den = 0.f;
  for (int s = lane; s < ns; s += 64) {
    const float x = mx == kNegInf ? 0.f : __expf(lse[s] - mx);
    w[s] = x;
    den += x;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o);
  __syncthreads();
  const float inv = den > 0.f ? 1.f / den : 0.f;
  const float* po = p.part_o + (int64_t)bh * ns * p.dpad;
  uint16_t* op = (uint16_t*)p.o + b * p.o_sb + hq * p.o_sh;
  for (int d = 2 * lane; d < p.D; d += 128) {
    float a0 = 0.f, a1 = 0.f;
    for (int s = 0; s < ns; ++s) {
      const float ws = w[s];
      const f32x2 x = *reinterpret_cast<const f32x2*>(po + (int64_t)s * p.dpad + d);
      a0 = fmaf(ws, x[0], a0);
      a1 = fmaf(ws, x[1], a1);
    }
    *reinterpret_cast<uint32_t*>(op + d) = pack2<T>(a0 * inv, a1 * inv);
  }
}

template <class T, int DP>
static hipError_t launch_decode_dp(const DecParams& p, hipStream_t s) {
  const dim3 grid((unsigned)p.num_splits, (unsigned)(p.B * p.Hkv));
  if (p.group <= 16)
    hipLaunchKernelGGL((decode_split_kernel<T, DP, 1>), grid, dim3(64), 0, s, p);
  else if (p.group <= 32)
    hipLaunchKernelGGL((decode_split_kernel<T, DP, 2>), grid, dim3(128), 0, s, p);
  else if (p.group <= 64)
    hipLaunchKernelGGL((decode_split_kernel<T, DP, 4>), grid, dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <class T>
static hipError_t launch_decode_t(const DecParams& p, hipStream_t s) {
  switch (padded_head_dim(p.D)) {
    case 64:
      return launch_decode_dp<T, 64>(p, s);
    case 96:
      return launch_decode_dp<T, 96>(p, s);
    case 128:
      return launch_decode_dp<T, 128>(p, s);
    case 256:
      return launch_decode_dp<T, 256>(p, s);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_decode_mfma(int dtype, const DecParams& p, hipStream_t s) {
  if (dtype == BF16::code) return launch_decode_t<BF16>(p, s);
  if (dtype == F16::code) return launch_decode_t<F16>(p, s);
  return hipErrorInvalidValue;
}

hipError_t launch_decode_combine(int dtype, const DecParams& p, hipStream_t s) {
  const dim3 grid((unsigned)(p.B * p.Hq));
  if (dtype == BF16::code)
    hipLaunchKernelGGL((decode_combine_kernel<BF16>), grid, dim3(64), 0, s, p);
  else if (dtype == F16::code)
    hipLaunchKernelGGL((decode_combine_kernel<F16>), grid, dim3(64), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace sk
