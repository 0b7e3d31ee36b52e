// FlashAttention-2 backward for bf16 / fp16 on gfx950 MFMA.
//
// Replaces the reference's _flash_bwd_dq_kernel and _flash_bwd_dkv_kernel
// (src/stackkernels/_core/attention/flash_bwd.py:58-198, 201-359); the row
// statistics pass (_bwd_preprocess_kernel, :15-55) is bwd_prep_kernel in
// sk_fp32.hip and writes delta = rowsum(dO * O) and lse * log2(e).
//
// Both kernels recompute P = exp2(S * scale * log2 e - lse * log2 e) from the
// saved LSE; rows with LSE = -inf (no visible key) get P = 0 and so add
// nothing.  dS = P * (dP - delta), dQ = scale * dS K, dK = scale * dS^T Q,
// dV = P^T dO.  All products run on v_mfma_f32_32x32x16 with fp32
// accumulation; P and dS are rounded to the input type for their products.
//
// dK/dV kernel (bwd_dkv_kernel): a workgroup owns 32*NW keys of one
// (batch, KV head), 32 per wave, and walks every query head of that KV
// head's group and every query tile that can see its keys, so the GQA sum
// happens in registers (deterministic, no atomics).  The wave computes
// S = Q K^T and dP = dO V^T with K and V held in registers as the B operand:
// each lane then owns one key (its l%32) and 16 queries per 32-query block.
// P and dS feed dV^T += dO^T P and dK^T += Q^T dS straight from registers,
// with dO^T / Q^T read transposed from the row-major LDS tiles by
// ds_read_b64_tr_b16 (the contraction over queries is permuted identically
// on both operands).  Q / dO tiles and their row statistics stream through
// double-buffered LDS.  At D = 256 the output head dim is split over two
// workgroups to keep the accumulators inside the register file.
//
// dQ kernel (bwd_dq_kernel): the forward kernel's organisation -- a
// workgroup owns 32*NW query rows, K/V tiles stream through double-buffered
// LDS, S^T = K Q^T and dP^T = V dO^T have one query per lane, and
// dQ^T += K^T dS^T reads K^T transposed from LDS.
#include "sk_common.h"
#include "sk_kernels.h"

namespace sk {

template <int DP, int ROWS>
struct RowTile {
  static constexpr int kStride = DP + 16;             // 16-bit words per LDS row
  static constexpr int kWords = ROWS * kStride;       // one tile
  static constexpr int kChunksPerRow = DP / 8;        // 16-byte chunks per row
  static constexpr int kChunks = ROWS * kChunksPerRow;
};

// A-operand offset of the transposed 4x16 read pattern: lane j of each
// 16-lane group points at row 4*(l/32) + (j/4), column 16*((l/16)%2) + 4*(j%4).
__device__ __forceinline__ int tr_offset(int lane, int stride) {
  const int j16 = lane & 15;
  return (4 * (lane >> 5) + j16 / 4) * stride + 16 * ((lane >> 4) & 1) + 4 * (j16 & 3);
}

template <class T, int DP, int DO, int BMQ, int NW, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64, 1) bwd_dkv_kernel(BwdParams p) {
  using Tile = RowTile<DP, BMQ>;
  constexpr int NT = NW * 64;
  constexpr int BNK = 32 * NW;
  constexpr int KD = DP / 16;   // k-steps over the head dim (S, dP)
  constexpr int QB = BMQ / 32;  // 32-query blocks per tile
  constexpr int KM = BMQ / 16;  // k-steps over queries (dV, dK)
  constexpr int DB = DO / 32;   // 32-wide output head-dim blocks
  constexpr int LOADS = (Tile::kChunks + NT - 1) / NT;
  constexpr bool kRagged = Tile::kChunks % NT != 0;
  static_assert(BMQ <= NT, "one thread per row loads the row statistics");

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * 2 * Tile::kWords];
  __shared__ __attribute__((aligned(16))) float stat[2][2][BMQ];  // [buf][lse2 | delta][row]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  constexpr int kDSplit = DP / DO;
  int bid = blockIdx.x;
  const int dsp = bid % kDSplit;
  bid /= kDSplit;
  const int bk_count = p.B * p.Hkv;
  const int bk = bid % bk_count;
  const int nblk = bid / bk_count;
  const int b = bk / p.Hkv;
  const int hkv = bk % p.Hkv;
  const int n0 = nblk * BNK;
  const int nw = n0 + 32 * wave;
  const int key = nw + l32;
  const int diag = p.Sk - p.Sq;
  const int d_out0 = dsp * DO;

  // K and V rows of this lane's key as the B operand: k[key][16*s + 8*hl .. +7].
  u32x4 kreg[KD], vreg[KD];
  {
    const int64_t krow = ((int64_t)bk * p.Sk + key) * p.D;
    const uint16_t* kp = (const uint16_t*)p.k + krow;
    const uint16_t* vp = (const uint16_t*)p.v + krow;
#pragma unroll
    for (int s = 0; s < KD; ++s) {
      const int d0 = 16 * s + 8 * hl;
      u32x4 kx = {0u, 0u, 0u, 0u}, vx = {0u, 0u, 0u, 0u};
      if (key < p.Sk && d0 < p.D) {
        kx = ldg_b128_cached(kp + d0);
        vx = ldg_b128_cached(vp + d0);
      }
      kreg[s] = kx;
      vreg[s] = vx;
    }
  }

  // Query tiles that can see a key of this block: i >= n0 - diag.
  int m_begin = 0;
  if (CAUSAL) m_begin = max(0, n0 - diag) / BMQ * BMQ;
  const int n_mt = m_begin < p.Sq ? (p.Sq - m_begin + BMQ - 1) / BMQ : 0;
  const int n_it = p.group * n_mt;

  u32x4 qld[LOADS], gld[LOADS];
  float st_l = 0.f, st_d = 0.f;
  auto load_tile = [&](int it) {
    const int gi = it / n_mt;
    const int m0 = m_begin + (it - gi * n_mt) * BMQ;
    const int64_t bh = (int64_t)b * p.Hq + hkv * p.group + gi;
    const uint16_t* qb = (const uint16_t*)p.q + bh * p.Sq * p.D;
    const uint16_t* gb = (const uint16_t*)p.dout + bh * p.Sq * p.D;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * NT;
      const int r = c / Tile::kChunksPerRow;
      const int d = (c % Tile::kChunksPerRow) * 8;
      const int m = m0 + r;
      u32x4 qx = {0u, 0u, 0u, 0u}, gx = {0u, 0u, 0u, 0u};
      if ((!kRagged || c < Tile::kChunks) && m < p.Sq && d < p.D) {
        qx = ldg_b128_cached(qb + (int64_t)m * p.D + d);
        gx = ldg_b128_cached(gb + (int64_t)m * p.D + d);
      }
      qld[i] = qx;
      gld[i] = gx;
    }
    if (tid < BMQ) {
      const int m = m0 + tid;
      st_l = m < p.Sq ? p.lse_log2[bh * p.Sq + m] : __builtin_inff();
      st_d = m < p.Sq ? p.delta[bh * p.Sq + m] : 0.f;
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* qs = smem + buf * 2 * Tile::kWords;
    uint16_t* gs = qs + Tile::kWords;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * NT;
      if (kRagged && c >= Tile::kChunks) continue;
      const int r = c / Tile::kChunksPerRow;
      const int d = (c % Tile::kChunksPerRow) * 8;
      *reinterpret_cast<u32x4*>(qs + r * Tile::kStride + d) = qld[i];
      *reinterpret_cast<u32x4*>(gs + r * Tile::kStride + d) = gld[i];
    }
    if (tid < BMQ) {
      stat[buf][0][tid] = st_l;
      stat[buf][1][tid] = st_d;
    }
  };

  f32x16 dkacc[DB], dvacc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) {
    dkacc[c] = f32x16{};
    dvacc[c] = f32x16{};
  }

  if (n_it > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  const int a_off = l32 * Tile::kStride + 8 * hl;
  const int t_off = tr_offset(lane, Tile::kStride) + d_out0;

  for (int it = 0; it < n_it; ++it) {
    const int buf = it & 1;
    if (it + 1 < n_it) load_tile(it + 1);
    const int gi = it / n_mt;
    const int m0 = m_begin + (it - gi * n_mt) * BMQ;
    const uint16_t* qs = smem + buf * 2 * Tile::kWords;
    const uint16_t* gs = qs + Tile::kWords;
    const float* lsp = stat[buf][0];
    const float* dlp = stat[buf][1];

    bool active = nw < p.Sk;
    if (CAUSAL) active = active && (m0 + BMQ - 1 + diag >= nw);
    if (active) {
      // S = Q K^T and dP = dO V^T: lane holds [query 32*qb + 8*(r/4) + 4*hl + r%4][key l32].
      f32x16 sacc[QB], pacc[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        sacc[qb] = f32x16{};
        pacc[qb] = f32x16{};
#pragma unroll
        for (int s = 0; s < KD; ++s) {
          const u32x4 a = lds_read_b128(qs + a_off + 32 * qb * Tile::kStride + 16 * s);
          sacc[qb] = mfma32<T>(a, kreg[s], sacc[qb]);
        }
#pragma unroll
        for (int s = 0; s < KD; ++s) {
          const u32x4 a = lds_read_b128(gs + a_off + 32 * qb * Tile::kStride + 16 * s);
          pacc[qb] = mfma32<T>(a, vreg[s], pacc[qb]);
        }
      }

      const bool straddle = CAUSAL && (nw + 31 > m0 + diag);
      u32x4 pk[KM], dsk[KM];
#pragma unroll
      for (int s2 = 0; s2 < KM; ++s2) {
        const int qb = s2 >> 1;
        const int base = 8 * (s2 & 1);
        const int q0 = 32 * qb + 2 * base + 4 * hl;  // first query of register group base/4
        const f32x4 l0 = *reinterpret_cast<const f32x4*>(lsp + q0);
        const f32x4 l1 = *reinterpret_cast<const f32x4*>(lsp + q0 + 8);
        const f32x4 d0 = *reinterpret_cast<const f32x4*>(dlp + q0);
        const f32x4 d1 = *reinterpret_cast<const f32x4*>(dlp + q0 + 8);
        float pv[8], dv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = base + j;
          const float lj = j < 4 ? l0[j & 3] : l1[j & 3];
          const float dj = j < 4 ? d0[j & 3] : d1[j & 3];
          float pe = fast_exp2(fmaf(sacc[qb][r], p.scale_log2, -lj));
          if (straddle) {
            const int query = m0 + q0 + 8 * (j >> 2) + (j & 3);
            if (key > query + diag) pe = 0.f;
          }
          pv[j] = pe;
          dv[j] = pe * (pacc[qb][r] - dj);
        }
        pk[s2] = u32x4{pack2<T>(pv[0], pv[1]), pack2<T>(pv[2], pv[3]), pack2<T>(pv[4], pv[5]),
                       pack2<T>(pv[6], pv[7])};
        dsk[s2] = u32x4{pack2<T>(dv[0], dv[1]), pack2<T>(dv[2], dv[3]), pack2<T>(dv[4], dv[5]),
                        pack2<T>(dv[6], dv[7])};
      }

      // dV^T += dO^T P and dK^T += Q^T dS: lane holds [d 32*c + 8*(r/4) + 4*hl + r%4][key l32].
#pragma unroll
      for (int c = 0; c < DB; ++c) {
#pragma unroll
        for (int s2 = 0; s2 < KM; ++s2) {
          const int off = t_off + 16 * s2 * Tile::kStride + 32 * c;
          const u32x2 glo = lds_read_tr(gs + off);
          const u32x2 ghi = lds_read_tr(gs + off + 8 * Tile::kStride);
          dvacc[c] = mfma32<T>(u32x4{glo[0], glo[1], ghi[0], ghi[1]}, pk[s2], dvacc[c]);
          const u32x2 qlo = lds_read_tr(qs + off);
          const u32x2 qhi = lds_read_tr(qs + off + 8 * Tile::kStride);
          dkacc[c] = mfma32<T>(u32x4{qlo[0], qlo[1], qhi[0], qhi[1]}, dsk[s2], dkacc[c]);
        }
      }
    }

    if (it + 1 < n_it) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (key >= p.Sk) return;
  const int64_t krow = ((int64_t)bk * p.Sk + key) * p.D;
  uint16_t* dkp = (uint16_t*)p.dk + krow;
  uint16_t* dvp = (uint16_t*)p.dv + krow;
#pragma unroll
  for (int c = 0; c < DB; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = d_out0 + 32 * c + 8 * i + 4 * hl;
      if (d < p.D) {
        const f32x16& kk = dkacc[c];
        const f32x16& vv = dvacc[c];
        *reinterpret_cast<u32x2*>(dkp + d) =
            u32x2{pack2<T>(kk[4 * i] * p.scale, kk[4 * i + 1] * p.scale),
                  pack2<T>(kk[4 * i + 2] * p.scale, kk[4 * i + 3] * p.scale)};
        *reinterpret_cast<u32x2*>(dvp + d) =
            u32x2{pack2<T>(vv[4 * i], vv[4 * i + 1]), pack2<T>(vv[4 * i + 2], vv[4 * i + 3])};
      }
    }
}

template <class T, int DP, int BN, int NW, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64, 1) bwd_dq_kernel(BwdParams p) {
  using Tile = RowTile<DP, BN>;
  constexpr int BM = 32 * NW;
  constexpr int NT = NW * 64;
  constexpr int LOADS = Tile::kChunks / NT;
  static_assert(Tile::kChunks % NT == 0, "tile chunks must divide over the workgroup");
  constexpr int KD = DP / 16;
  constexpr int KB = BN / 32;
  constexpr int DB = DP / 32;
  constexpr int KN = BN / 16;

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * 2 * Tile::kWords];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  const int bh_count = p.B * p.Hq;
  const int mblk = p.n_mblocks - 1 - (int)blockIdx.x / bh_count;
  const int bh = blockIdx.x % bh_count;
  const int b = bh / p.Hq;
  const int hq = bh % p.Hq;
  const int hkv = hq / p.group;
  const int m0 = mblk * BM;
  const int mw = m0 + 32 * wave;
  const int row = mw + l32;
  const int diag = p.Sk - p.Sq;

  const uint16_t* kbase = (const uint16_t*)p.k + ((int64_t)b * p.Hkv + hkv) * p.Sk * p.D;
  const uint16_t* vbase = (const uint16_t*)p.v + ((int64_t)b * p.Hkv + hkv) * p.Sk * p.D;

  u32x4 qreg[KD], greg[KD];
  {
    const int64_t qrow = ((int64_t)bh * p.Sq + row) * p.D;
#pragma unroll
    for (int s = 0; s < KD; ++s) {
      const int d0 = 16 * s + 8 * hl;
      u32x4 qx = {0u, 0u, 0u, 0u}, gx = {0u, 0u, 0u, 0u};
      if (row < p.Sq && d0 < p.D) {
        qx = ldg_b128_cached((const uint16_t*)p.q + qrow + d0);
        gx = ldg_b128_cached((const uint16_t*)p.dout + qrow + d0);
      }
      qreg[s] = qx;
      greg[s] = gx;
    }
  }
  const float lse2 = row < p.Sq ? p.lse_log2[(int64_t)bh * p.Sq + row] : __builtin_inff();
  const float dl = row < p.Sq ? p.delta[(int64_t)bh * p.Sq + row] : 0.f;

  int n_end = p.Sk;
  if (CAUSAL) n_end = min(p.Sk, m0 + BM + diag);
  const int n_tiles = n_end > 0 ? (n_end + BN - 1) / BN : 0;

  u32x4 kld[LOADS], vld[LOADS];
  auto load_tile = [&](int t) {
    const int nn = t * BN;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * NT;
      const int r = c / Tile::kChunksPerRow;
      const int d = (c % Tile::kChunksPerRow) * 8;
      const int n = nn + r;
      u32x4 kx = {0u, 0u, 0u, 0u}, vx = {0u, 0u, 0u, 0u};
      if (n < p.Sk && d < p.D) {
        kx = ldg_b128_cached(kbase + (int64_t)n * p.D + d);
        vx = ldg_b128_cached(vbase + (int64_t)n * p.D + d);
      }
      kld[i] = kx;
      vld[i] = vx;
    }
  };
  auto store_tile = [&](int buf) {
    uint16_t* ks = smem + buf * 2 * Tile::kWords;
    uint16_t* vs = ks + Tile::kWords;
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * NT;
      const int r = c / Tile::kChunksPerRow;
      const int d = (c % Tile::kChunksPerRow) * 8;
      *reinterpret_cast<u32x4*>(ks + r * Tile::kStride + d) = kld[i];
      *reinterpret_cast<u32x4*>(vs + r * Tile::kStride + d) = vld[i];
    }
  };

  f32x16 dqacc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) dqacc[c] = f32x16{};

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  const int a_off = l32 * Tile::kStride + 8 * hl;
  const int t_off = tr_offset(lane, Tile::kStride);
  const bool wave_has_rows = mw < p.Sq;

  for (int t = 0; t < n_tiles; ++t) {
    const int buf = t & 1;
    if (t + 1 < n_tiles) load_tile(t + 1);
    const uint16_t* ks = smem + buf * 2 * Tile::kWords;
    const uint16_t* vs = ks + Tile::kWords;
    const int nn = t * BN;

    bool active = wave_has_rows;
    if (CAUSAL) active = active && (nn <= mw + 31 + diag);
    if (active) {
      // S^T = K Q^T, dP^T = V dO^T: lane holds [key nn + 32*kb + 8*(r/4) + 4*hl + r%4][query row].
      f32x16 sacc[KB], pacc[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        sacc[kb] = f32x16{};
        pacc[kb] = f32x16{};
#pragma unroll
        for (int s = 0; s < KD; ++s) {
          const u32x4 a = lds_read_b128(ks + a_off + 32 * kb * Tile::kStride + 16 * s);
          sacc[kb] = mfma32<T>(a, qreg[s], sacc[kb]);
        }
#pragma unroll
        for (int s = 0; s < KD; ++s) {
          const u32x4 a = lds_read_b128(vs + a_off + 32 * kb * Tile::kStride + 16 * s);
          pacc[kb] = mfma32<T>(a, greg[s], pacc[kb]);
        }
      }

      const bool edge = (nn + BN > p.Sk) || (CAUSAL && (nn + BN - 1 > mw + diag));
      int lim = p.Sk - 1;
      if (CAUSAL) lim = min(lim, row + diag);
      u32x4 dsk[KN];
#pragma unroll
      for (int s2 = 0; s2 < KN; ++s2) {
        const int kb = s2 >> 1;
        const int base = 8 * (s2 & 1);
        float dv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int r = base + j;
          float pe = fast_exp2(fmaf(sacc[kb][r], p.scale_log2, -lse2));
          if (edge) {
            const int kk = nn + 32 * kb + 8 * (r >> 2) + 4 * hl + (r & 3);
            if (kk > lim) pe = 0.f;
          }
          dv[j] = pe * (pacc[kb][r] - dl);
        }
        dsk[s2] = u32x4{pack2<T>(dv[0], dv[1]), pack2<T>(dv[2], dv[3]), pack2<T>(dv[4], dv[5]),
                        pack2<T>(dv[6], dv[7])};
      }

      // dQ^T += K^T dS^T: lane holds [d 32*c + 8*(r/4) + 4*hl + r%4][query row].
#pragma unroll
      for (int c = 0; c < DB; ++c) {
#pragma unroll
        for (int s2 = 0; s2 < KN; ++s2) {
          const int off = t_off + 16 * s2 * Tile::kStride + 32 * c;
          const u32x2 lo = lds_read_tr(ks + off);
          const u32x2 hi = lds_read_tr(ks + off + 8 * Tile::kStride);
          dqacc[c] = mfma32<T>(u32x4{lo[0], lo[1], hi[0], hi[1]}, dsk[s2], dqacc[c]);
        }
      }
    }

    if (t + 1 < n_tiles) store_tile(buf ^ 1);
    __syncthreads();
  }

  if (row >= p.Sq) return;
  uint16_t* dqp = (uint16_t*)p.dq + ((int64_t)bh * p.Sq + row) * p.D;
#pragma unroll
  for (int c = 0; c < DB; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = 32 * c + 8 * i + 4 * hl;
      if (d < p.D) {
        const f32x16& a = dqacc[c];
        *reinterpret_cast<u32x2*>(dqp + d) =
            u32x2{pack2<T>(a[4 * i] * p.scale, a[4 * i + 1] * p.scale),
                  pack2<T>(a[4 * i + 2] * p.scale, a[4 * i + 3] * p.scale)};
      }
    }
}

// gfx950 tile table for the backward: (padded head dim) ->
//   dK/dV: output head-dim width DO per workgroup, query tile BMQ, waves NW;
//   dQ:    key tile BN, waves NW.
// Four waves per workgroup, one workgroup per CU: the K/V (or Q/dO) operands
// in registers plus the fp32 accumulators need most of the 512 VGPR+AGPR
// file of a one-wave-per-SIMD launch.
template <class T, int DP, int DO, int BMQ, int BN>
static hipError_t launch_bwd_t(const BwdParams& p, bool causal, hipStream_t s) {
  constexpr int NW = 4;
  const int nb = (p.Sk + 32 * NW - 1) / (32 * NW);
  const int64_t g_kv = (int64_t)nb * p.B * p.Hkv * (DP / DO);
  BwdParams q = p;
  q.n_mblocks = (p.Sq + 32 * NW - 1) / (32 * NW);
  const int64_t g_q = (int64_t)q.n_mblocks * p.B * p.Hq;
  if (g_kv > 0x7fffffffLL || g_q > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  if (g_kv > 0) {
    if (causal)
      hipLaunchKernelGGL((bwd_dkv_kernel<T, DP, DO, BMQ, NW, true>), dim3((unsigned)g_kv),
                         dim3(NW * 64), 0, s, q);
    else
      hipLaunchKernelGGL((bwd_dkv_kernel<T, DP, DO, BMQ, NW, false>), dim3((unsigned)g_kv),
                         dim3(NW * 64), 0, s, q);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (g_q > 0) {
    if (causal)
      hipLaunchKernelGGL((bwd_dq_kernel<T, DP, BN, NW, true>), dim3((unsigned)g_q), dim3(NW * 64),
                         0, s, q);
    else
      hipLaunchKernelGGL((bwd_dq_kernel<T, DP, BN, NW, false>), dim3((unsigned)g_q), dim3(NW * 64),
                         0, s, q);
  }
  return hipGetLastError();
}

template <class T>
static hipError_t launch_bwd_dt(const BwdParams& p, bool causal, hipStream_t s) {
  switch (padded_head_dim(p.D)) {
    case 64:
      return launch_bwd_t<T, 64, 64, 64, 64>(p, causal, s);
    case 96:
      return launch_bwd_t<T, 96, 96, 64, 64>(p, causal, s);
    case 128:
      return launch_bwd_t<T, 128, 128, 64, 64>(p, causal, s);
    case 256:
      return launch_bwd_t<T, 256, 128, 32, 32>(p, causal, s);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_bwd_mfma(int dtype, const BwdParams& p, bool causal, hipStream_t s) {
  if (dtype == BF16::code) return launch_bwd_dt<BF16>(p, causal, s);
  if (dtype == F16::code) return launch_bwd_dt<F16>(p, causal, s);
  return hipErrorInvalidValue;
}

}  // namespace sk
