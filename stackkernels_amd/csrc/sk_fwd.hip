// FlashAttention-2 forward for bf16 / fp16 on gfx950 MFMA.
//
// Replaces the reference's _flash_fwd_kernel
// (src/stackkernels/_core/attention/flash_fwd.py:15-179); same math, a
// gfx950-first organisation:
//
// * A workgroup owns BM = 32*NW query rows of one (batch, query head); each
//   wave owns 32 of them.  Key/value tiles of BN rows stream through LDS,
//   double-buffered, loaded by coalesced 16-byte global reads.
// * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16:
//   every lane then holds one query column (its l%32) and 16 keys per 32-key
//   block, so the softmax row max needs one cross-half swap
//   (v_permlane32_swap) per tile and the row sum none until the end.
// * The output is accumulated transposed as well, O^T += V^T P^T.  The P^T
//   operand comes straight from the score registers (the contraction order
//   over keys is permuted consistently on both sides), and V^T is read from
//   the row-major V tile with ds_read_b64_tr_b16.
// * Online softmax in base 2 with |sm_scale|*log2(e) folded into one FMA per
//   score; a negative sm_scale is applied by negating q's sign bits.
// * Bottom-right causal masking (key j visible to query i iff
//   j <= i + Sk - Sq, reference flash_fwd.py:122-128) is applied only on the
//   tiles that straddle the diagonal or the end of the keys; tiles a wave
//   cannot see are skipped.  Rows that see no key end with O = 0 and
//   LSE = -inf, as the reference path does (_reference/torch/attention.py:70-73).
// * Online-softmax rescaling is lazy: the exponent offset moves only when a
//   tile's maximum exceeds it by more than 2^8, so the O rescale (DP/2
//   multiplies per lane) runs on a handful of tiles per row block.
// * XCD-aware order: each of the 8 XCDs walks a contiguous range of
//   (head, query block) items, head-major, heaviest query block first, so
//   the heads an XCD has in flight share its L2 and the causal triangle's
//   long rows do not trail at the end of the grid.
#include "sk_common.h"
#include "sk_kernels.h"

namespace sk {

// LDS tile geometry.  K rows are padded by 8 words (an odd multiple of 4
// banks), so the 16-byte row reads of 8 consecutive lanes hit 8 disjoint bank
// quads; V rows by 16 words (8 banks), so the four 32-byte row segments a
// 16-lane ds_read_b64_tr_b16 group touches are disjoint.
template <int DP, int BN>
struct FwdTile {
  static constexpr int kKStride = DP + 8;              // 16-bit words per K row
  static constexpr int kVStride = DP + 16;             // 16-bit words per V row
  static constexpr int kKWords = BN * kKStride;
  static constexpr int kVWords = BN * kVStride;
  static constexpr int kBufWords = kKWords + kVWords;  // one K + V stage
  static constexpr int kChunksPerRow = DP / 8;         // 16-byte chunks per row
  static constexpr int kChunks = BN * kChunksPerRow;   // chunks per tile
};

template <class T, int DP, int BN, int NW, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64, DP <= 128 ? 2 : 1) fwd_mfma_kernel(FwdParams p) {
  using Tile = FwdTile<DP, BN>;
  constexpr int BM = 32 * NW;
  constexpr int NT = NW * 64;
  constexpr int LOADS = Tile::kChunks / NT;
  static_assert(Tile::kChunks % NT == 0, "tile chunks must divide over the workgroup");
  constexpr int KD = DP / 16;  // k-steps over the head dim for S^T
  constexpr int KB = BN / 32;  // 32-key blocks per tile
  constexpr int DB = DP / 32;  // 32-wide head-dim blocks of O^T
  constexpr int KN = BN / 16;  // k-steps over keys for O^T

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * Tile::kBufWords];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  // Work order.  The dispatcher hands workgroup i to XCD i % 8; remap so each
  // XCD walks a contiguous run of (head, query block) items, head-major and
  // heaviest query block first, which keeps the one or two heads it has in
  // flight resident in that XCD's L2.
  const int w = xcd_work_index(blockIdx.x, gridDim.x);
  const int bh = w / p.n_mblocks;
  const int mblk = p.n_mblocks - 1 - (w - bh * p.n_mblocks);
  const int b = bh / p.Hq;
  const int hq = bh % p.Hq;
  const int hkv = hq / p.group;
  const int m0 = mblk * BM;
  const int mw = m0 + wave * 32;
  const int row = mw + l32;
  const int diag = p.Sk - p.Sq;  // causal offset

  const uint16_t* qb = (const uint16_t*)p.q + b * p.q_sb + hq * p.q_sh;
  const uint16_t* kbase = (const uint16_t*)p.k + b * p.k_sb + hkv * p.k_sh;
  const uint16_t* vbase = (const uint16_t*)p.v + b * p.v_sb + hkv * p.v_sh;

  int n_end = p.Sk;
  if (CAUSAL) n_end = min(p.Sk, m0 + BM + diag);
  const int n_tiles = n_end > 0 ? (n_end + BN - 1) / BN : 0;

  // Q^T operand: lane holds q[row][16*s + 8*hl .. +7].
  u32x4 qreg[KD];
#pragma unroll
  for (int s = 0; s < KD; ++s) {
    const int d0 = 16 * s + 8 * hl;
    u32x4 x = {0u, 0u, 0u, 0u};
    if (row < p.Sq && d0 < p.D) x = ldg_b128_cached(qb + (int64_t)row * p.q_ss + d0);
    x ^= p.q_sign;
    qreg[s] = x;
  }

  // K/V tiles arrive by buffer loads: a per-tile resource covers the tile's
  // valid rows, so rows past S_k (and head-dim padding, via an out-of-range
  // offset) read as zero in hardware, with no branches or 64-bit address math.
  u32x4 kreg[LOADS], vreg[LOADS];
  uint32_t koff[LOADS], voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int c = tid + i * NT;
    const int r = c / Tile::kChunksPerRow;
    const int d = (c % Tile::kChunksPerRow) * 8;
    koff[i] = d < p.D ? (uint32_t)((r * p.k_ss + d) * 2) : kBufferOob;
    voff[i] = d < p.D ? (uint32_t)((r * p.v_ss + d) * 2) : kBufferOob;
  }
  auto load_tile = [&](int t) {
    const int n0 = t * BN;
    const int rows = min(BN, p.Sk - n0);
    const buf_rsrc kr = make_rsrc(kbase + (int64_t)n0 * p.k_ss, tile_bytes(rows, p.k_ss, p.D));
    const buf_rsrc vr = make_rsrc(vbase + (int64_t)n0 * p.v_ss, tile_bytes(rows, p.v_ss, p.D));
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      kreg[i] = buffer_load_b128(kr, koff[i]);
      vreg[i] = buffer_load_b128(vr, voff[i]);
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* ks = smem + buf * Tile::kBufWords;
    uint16_t* vs = ks + Tile::kKWords;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * NT;
      const int r = c / Tile::kChunksPerRow;
      const int d = (c % Tile::kChunksPerRow) * 8;
      *reinterpret_cast<u32x4*>(ks + r * Tile::kKStride + d) = kreg[i];
      *reinterpret_cast<u32x4*>(vs + r * Tile::kVStride + d) = vreg[i];
    }
  };

  f32x16 oacc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) oacc[c] = f32x16{};
  float m_run = kNegInf;
  float l_run = 0.f;

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  // Lane-constant parts of the LDS addresses.
  const int k_off = l32 * Tile::kKStride + 8 * hl;  // K row l32, column 8*hl
  const int j16 = lane & 15;
  const int v_off = (4 * hl + j16 / 4) * Tile::kVStride + 16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
  const bool wave_has_rows = mw < p.Sq;

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_tiles) load_tile(t + 1);
    const uint16_t* ks = smem + buf * Tile::kBufWords;
    const uint16_t* vs = ks + Tile::kKWords;
    const int n0 = t * BN;

    bool active = wave_has_rows;
    if (CAUSAL) active = active && (n0 <= mw + 31 + diag);
    if (active) {
      f32x16 sacc[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        sacc[kb] = f32x16{};
#pragma unroll
        for (int s = 0; s < KD; ++s) {
          const u32x4 a = lds_read_b128(ks + k_off + kb * 32 * Tile::kKStride + 16 * s);
          sacc[kb] = mfma32<T>(a, qreg[s], sacc[kb]);
        }
      }

      const bool tail = n0 + BN > p.Sk;
      const bool straddle = CAUSAL && (n0 + BN - 1 > mw + diag);
      if (tail || straddle) {
        int lim = p.Sk - 1;
        if (CAUSAL) lim = min(lim, row + diag);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = n0 + 32 * kb + 8 * (r >> 2) + 4 * hl + (r & 3);
            if (key > lim) sacc[kb][r] = kNegInf;
          }
      }

      float mt = kNegInf;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[kb][r]);
      mt = xhalf_max(mt);
      // Lazy rescaling: the exponent offset m_run only moves when a score
      // exceeds it by more than kRescaleLog2 (in log2 units), so P <= 2^8
      // and the O / l rescale runs on a few tiles instead of every tile.
      const bool grow = (mt - m_run) * p.scale_log2 > kRescaleLog2;
      if (__any(grow)) {
        // Lanes that do not grow keep alpha = 1 (their offset may still be
        // -inf on a row that has seen no key yet).
        const float alpha = grow ? fast_exp2((m_run - mt) * p.scale_log2) : 1.f;
        m_run = grow ? mt : m_run;
        l_run *= alpha;
#pragma unroll
        for (int c = 0; c < DB; ++c) oacc[c] *= alpha;
      }
      const float neg_m = (m_run == kNegInf) ? 0.f : -m_run * p.scale_log2;

      float psum = 0.f;
      u32x4 pk[KN];
#pragma unroll
      for (int s2 = 0; s2 < KN; ++s2) {
        const int kb = s2 >> 1;
        const int base = 8 * (s2 & 1);
        float e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          e[j] = fast_exp2(fmaf(sacc[kb][base + j], p.scale_log2, neg_m));
          psum += e[j];
        }
        pk[s2] = u32x4{pack2<T>(e[0], e[1]), pack2<T>(e[2], e[3]), pack2<T>(e[4], e[5]),
                       pack2<T>(e[6], e[7])};
      }
      l_run += psum;

#pragma unroll
      for (int c = 0; c < DB; ++c) {
#pragma unroll
        for (int s2 = 0; s2 < KN; ++s2) {
          const uint16_t* vp = vs + v_off + 16 * s2 * Tile::kVStride + 32 * c;
          const u32x2 lo = lds_read_tr(vp);
          const u32x2 hi = lds_read_tr(vp + 8 * Tile::kVStride);
          const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
          oacc[c] = mfma32<T>(a, pk[s2], oacc[c]);
        }
      }
    }

    if (t + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = xhalf_sum(l_run);
  if (row < p.Sq) {
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint16_t* ob = (uint16_t*)p.o + b * p.o_sb + hq * p.o_sh + (int64_t)row * p.o_ss;
#pragma unroll
    for (int c = 0; c < DB; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * c + 8 * i + 4 * hl;
        if (d < p.D) {
          u32x2 w = {pack2<T>(oacc[c][4 * i] * inv, oacc[c][4 * i + 1] * inv),
                     pack2<T>(oacc[c][4 * i + 2] * inv, oacc[c][4 * i + 3] * inv)};
          *reinterpret_cast<u32x2*>(ob + d) = w;
        }
      }
    if (hl == 0) {
      const float lse = l_tot > 0.f ? m_run * p.scale + __logf(l_tot) : kNegInf;
      p.lse[(int64_t)bh * p.Sq + row] = lse;
    }
  }
}

// gfx950 tile table for the forward kernel: (padded head dim) -> BN, waves.
// BN = 64 keys per tile up to D = 128 (two 32x32 score blocks per wave per
// tile), 32 at D = 256 to keep the double-buffered K/V tiles and the
// accumulators inside the two-waves-per-SIMD budget (256 VGPR+AGPR).
template <class T, int DP, int BN, int NW>
static hipError_t launch_fwd_t(const FwdParams& p, bool causal, hipStream_t s) {
  const dim3 grid((unsigned)(p.n_mblocks * p.B * p.Hq));
  const dim3 block(NW * 64);
  if (causal)
    hipLaunchKernelGGL((fwd_mfma_kernel<T, DP, BN, NW, true>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((fwd_mfma_kernel<T, DP, BN, NW, false>), grid, block, 0, s, p);
  return hipGetLastError();
}

int fwd_rows_per_block(int dtype, int dpad) {
  (void)dtype;
  (void)dpad;
  return 128;  // NW = 4 waves x 32 rows
}

template <class T>
static hipError_t launch_fwd_dt(const FwdParams& p, bool causal, hipStream_t s) {
  switch (padded_head_dim(p.D)) {
    case 64:
      return launch_fwd_t<T, 64, 64, 4>(p, causal, s);
    case 96:
      return launch_fwd_t<T, 96, 64, 4>(p, causal, s);
    case 128:
      return launch_fwd_t<T, 128, 64, 4>(p, causal, s);
    case 256:
      return launch_fwd_t<T, 256, 32, 4>(p, causal, s);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_fwd_mfma(int dtype, const FwdParams& p, bool causal, hipStream_t s) {
  if (dtype == BF16::code) return launch_fwd_dt<BF16>(p, causal, s);
  if (dtype == F16::code) return launch_fwd_dt<F16>(p, causal, s);
  return hipErrorInvalidValue;
}

int padded_head_dim(int d) {
  if (d <= 0 || d % 8 != 0) return 0;
  if (d <= 64) return 64;
  if (d <= 96) return 96;
  if (d <= 128) return 128;
  if (d <= 256) return 256;
  return 0;
}

}  // namespace sk
