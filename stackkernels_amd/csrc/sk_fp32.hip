// fp32 attention kernels (forward, backward) and the backward row-statistics
// pass shared by every dtype.
//
// fp32 inputs are computed in true fp32 (no reduced-precision MFMA inputs),
// which is what the reference path does (_reference/torch/attention.py:56-61).
// The forward of padded head dims up to 128 runs on the matrix cores
// (fwd_f32_mfma_kernel, v_mfma_f32_32x32x2_f32: fp32 products, fp32
// accumulation).  The other kernels here run on the vector ALUs: four lanes
// share one row, each holding a quarter of the head dimension, and q.k
// partial sums are combined with two cross-lane adds; K/V (or Q/dO) tiles of
// 16 rows are staged in LDS and the online softmax is updated once per tile.
#include "sk_common.h"
#include "sk_kernels.h"
#include "sk_rope.h"

namespace sk {

constexpr int kF32Rows = 64;  // rows per workgroup (4 lanes per row)
constexpr int kF32Tile = 16;  // keys (or queries) per LDS tile

__device__ __forceinline__ float quad_sum(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  return x;
}

// Forward: O = softmax(scale q k^T + mask) v, LSE in natural log.
template <int DP, bool CAUSAL>
__global__ void __launch_bounds__(256) fwd_f32_kernel(FwdParams p) {
  constexpr int DC = DP / 4;  // head-dim slice per lane
  __shared__ float ks[kF32Tile][DP];
  __shared__ float vs[kF32Tile][DP];
  __shared__ int kok[kF32Tile];  // paged decode: the key's page lies in the pool

  const int tid = threadIdx.x;
  const int part = tid & 3;
  const int rloc = tid >> 2;
  const int bh_count = p.B * p.Hq;
  const int mblk = p.n_mblocks - 1 - blockIdx.x / bh_count;
  const int bh = blockIdx.x % bh_count;
  const int b = bh / p.Hq, hq = bh % p.Hq, hkv = hq / p.group;
  const int m0 = mblk * kF32Rows;
  const int row = m0 + rloc;
  const int diag = p.Sk - p.Sq;
  const bool row_ok = row < p.Sq;

  const float* qp = (const float*)p.q + b * p.q_sb + hq * p.q_sh + (int64_t)row * p.q_ss;
  const float* kbase = (const float*)p.k + b * p.k_sb + hkv * p.k_sh;
  const float* vbase = (const float*)p.v + b * p.v_sb + hkv * p.v_sh;
  const float sgn = p.q_sign ? -1.f : 1.f;

  // q, rotated when the call carries RoPE tables (query row i is token i).
  const int rrow = row_ok ? rope_row(p.rope, b, row) : -1;
  const int half = p.D >> 1;
  float q[DC], acc[DC];
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int d = part * DC + i;
    float x = 0.f;
    if (row_ok && d < p.D) x = rrow >= 0 ? rope1(qp, d, half, p.rope, rrow) : qp[d];
    q[i] = x * sgn;
    acc[i] = 0.f;
  }
  float m_run = kNegInf, l_run = 0.f;
  // Keys this batch row sees: all S_k, or its cache length (decode).
  const int sk_b = p.seqlens ? min(max(p.seqlens[b], 0), p.Sk) : p.Sk;
  int n_end = sk_b;
  if (CAUSAL) n_end = min(sk_b, m0 + kF32Rows + diag);
  const int lim = CAUSAL ? min(sk_b - 1, row + diag) : sk_b - 1;

  // Key n's K and V rows: contiguous, or in-page row n % page_size of page
  // block_table[b][n / page_size] of a paged pool (decode only).
  auto key_rows = [&](int n, const float*& kr, const float*& vr) {
    if (!p.block_table) {
      kr = kbase + (int64_t)n * p.k_ss;
      vr = vbase + (int64_t)n * p.v_ss;
      return true;
    }
    const int page = p.block_table[(int64_t)b * p.max_pages + n / p.page_size];
    const bool ok = page >= 0 && page < p.num_pages;
    const int64_t pg = ok ? page : 0, off = n % p.page_size;
    kr = (const float*)p.k + pg * p.k_sb + (int64_t)hkv * p.k_sh + off * p.k_ss;
    vr = (const float*)p.v + pg * p.v_sb + (int64_t)hkv * p.v_sh + off * p.v_ss;
    return ok;
  };

  for (int n0 = 0; n0 < n_end; n0 += kF32Tile) {
    __syncthreads();
    for (int e = tid; e < kF32Tile * DP; e += 256) {
      const int r = e / DP, d = e % DP, n = n0 + r;
      const float* kr = nullptr;
      const float* vr = nullptr;
      const bool page_ok = n < sk_b && key_rows(n, kr, vr);
      const bool ok = page_ok && d < p.D;
      ks[r][d] = ok ? kr[d] : 0.f;
      vs[r][d] = ok ? vr[d] : 0.f;
      if (d == 0) kok[r] = page_ok;
    }
    __syncthreads();
    float s[kF32Tile];
    float mt = kNegInf;
#pragma unroll
    for (int j = 0; j < kF32Tile; ++j) {
      float x = 0.f;
#pragma unroll
      for (int i = 0; i < DC; ++i) x = fmaf(q[i], ks[j][part * DC + i], x);
      x = quad_sum(x) * p.scale;
      if (n0 + j > lim || !kok[j]) x = kNegInf;
      s[j] = x;
      mt = fmaxf(mt, x);
    }
    const float m_new = fmaxf(m_run, mt);
    const float m_sub = m_new == kNegInf ? 0.f : m_new;
    const float alpha = __expf(m_run - m_sub);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int i = 0; i < DC; ++i) acc[i] *= alpha;
#pragma unroll
    for (int j = 0; j < kF32Tile; ++j) {
      const float pj = expf(s[j] - m_sub);
      l_run += pj;
#pragma unroll
      for (int i = 0; i < DC; ++i) acc[i] = fmaf(pj, vs[j][part * DC + i], acc[i]);
    }
  }
  if (!row_ok) return;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  float* op = (float*)p.o + b * p.o_sb + hq * p.o_sh + (int64_t)row * p.o_ss;
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int d = part * DC + i;
    if (d < p.D) op[d] = acc[i] * inv;
  }
  if (part == 0) p.lse[(int64_t)bh * p.Sq + row] = l_run > 0.f ? m_run + logf(l_run) : kNegInf;
}

// Forward on the matrix cores (padded head dim 64 or 128, at least 32 query
// rows).  v_mfma_f32_32x32x2_f32 multiplies and accumulates in fp32: lane l
// supplies A[l%32][l/32] and B[l/32][l%32], and holds D[8*(r/4) + 4*(l/32) +
// r%4][l%32] in register r, as for the 16-bit 32x32 products.  A workgroup
// of 8 waves (two per SIMD) owns 256 query rows of one (batch, head), 32 per
// wave with q in registers; 64-key K/V tiles go through a 2-deep LDS ring
// written by buffer_load ... lds, one barrier per tile (a tile is about 16k
// MFMA cycles per wave, so one tile of load look-ahead is ample).
// * S^T = K Q^T: k-step s contracts head-dim column s in lanes 0-31 and
//   DP/2 + s in lanes 32-63 (the same permutation on both operands), so one
//   16-byte LDS read gives a lane four k-steps of K.  K rows are stored with
//   16-byte chunk c at c ^ (row % 16), which puts the 16 rows a read touches
//   in distinct bank quads.  Two 32-key score blocks per tile are two
//   independent MFMA chains.
// * O^T += V^T P^T: P^T is the score registers themselves (k-step r
//   contracts the keys the two lane halves hold in register r), and output
//   block c holds head-dim columns DB*m + c (m its row), so one 16-byte read
//   of a V row serves all DB blocks and the epilogue writes whole 16-byte
//   pieces of each output row.
// * Online softmax in base 2 with |sm_scale| * log2(e) folded into one FMA;
//   the running maximum moves every tile (the VALU work is small beside the
//   MFMAs).  Masking and the rows without a visible key follow the reference
//   path as in fwd_f32_kernel.
constexpr int kF32MmaRows = 256;

template <int DP, bool CAUSAL>
__global__ void __launch_bounds__(512, 1) fwd_f32_mfma_kernel(FwdParams p) {
  constexpr int NW = 8;
  constexpr int BN = 64;
  constexpr int KS = DP / 2;              // k-steps of S^T (per lane half: DP/2 columns)
  constexpr int DB = DP / 32;             // output blocks of 32 head-dim columns
  constexpr int RB = DP * 4;              // row bytes
  constexpr int KT = BN * RB;             // tile bytes
  constexpr int CPR = RB / 16;            // 16-byte chunks per row
  constexpr int SEGR = 1024 / RB;         // rows per 1 KiB DMA segment
  constexpr int LK = KT / 1024 / NW;      // segments per wave per tile (K, and V)
  static_assert(DP == 64 || DP == 128, "padded head dim 64 or 128");
  static_assert((KT / 1024) % NW == 0, "tile segments must divide over the waves");
  typedef float vrow_t __attribute__((ext_vector_type(DB)));

  __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * KT];  // K stages, then V stages

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  // Heaviest query block first under the causal mask; XCD-aware order.
  const int w = xcd_work_index(blockIdx.x, gridDim.x);
  const int bh = w / p.n_mblocks;
  const int mblk = p.n_mblocks - 1 - (w - bh * p.n_mblocks);
  const int b = bh / p.Hq, hq = bh % p.Hq, hkv = hq / p.group;
  const int m0 = mblk * kF32MmaRows;
  const int mw = m0 + 32 * wave;
  const int row = mw + l32;
  const bool row_ok = row < p.Sq;
  const int diag = p.Sk - p.Sq;

  // Q^T operand: lane holds q[row][hl * KS + s] at k-step s (rotated when
  // the call carries RoPE tables; zero past S_q and D; negated for a
  // negative scale).
  float qv[KS];
  {
    const float* qp = (const float*)p.q + b * p.q_sb + hq * p.q_sh + (int64_t)row * p.q_ss;
    const int rrow = row_ok ? rope_row(p.rope, b, row) : -1;
    if (rrow >= 0) {
      const int half = p.D >> 1;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int d = hl * KS + s;
        qv[s] = d < p.D ? rope1(qp, d, half, p.rope, rrow) : 0.f;
      }
    } else {
#pragma unroll
      for (int j = 0; j < KS / 4; ++j) {
        const int d = hl * KS + 4 * j;
        f32x4 x = {0.f, 0.f, 0.f, 0.f};
        if (row_ok && d < p.D) x = *reinterpret_cast<const f32x4*>(qp + d);
#pragma unroll
        for (int e = 0; e < 4; ++e) qv[4 * j + e] = x[e];
      }
    }
    if (p.q_sign) {
#pragma unroll
      for (int s = 0; s < KS; ++s) qv[s] = -qv[s];
    }
  }

  // DMA: segment j of this wave is segment wave + 8 j of the tile; the
  // lane's global byte offset of the chunk that lands at its LDS slot.
  const float* kbase = (const float*)p.k + b * p.k_sb + hkv * p.k_sh;
  const float* vbase = (const float*)p.v + b * p.v_sb + hkv * p.v_sh;
  uint32_t koff[LK], voff[LK];
#pragma unroll
  for (int j = 0; j < LK; ++j) {
    const int r = (wave + j * NW) * SEGR + lane / CPR;
    const int pc = lane % CPR;
    const int kc = pc ^ (r & 15);
    koff[j] = kc * 4 < p.D ? (uint32_t)((r * p.k_ss + kc * 4) * 4) : kBufferOob;
    voff[j] = pc * 4 < p.D ? (uint32_t)((r * p.v_ss + pc * 4) * 4) : kBufferOob;
  }
  const uint32_t lds0 = lds_addr(smem);
  auto range = [&](int rows, int64_t stride) {
    return rows > 0 ? (int)(((int64_t)(rows - 1) * stride + p.D) * 4) : 0;
  };
  auto issue = [&](int t) {
    const int n0 = t * BN;
    const int rows = min(BN, p.Sk - n0);
    const int st = t & 1;
    const i32x4 kr = make_rsrc_words(kbase + (int64_t)n0 * p.k_ss, range(rows, p.k_ss));
    const i32x4 vr = make_rsrc_words(vbase + (int64_t)n0 * p.v_ss, range(rows, p.v_ss));
#pragma unroll
    for (int j = 0; j < LK; ++j)
      buffer_load_lds_b128(kr, lds0 + st * KT + (wave + j * NW) * 1024, koff[j]);
#pragma unroll
    for (int j = 0; j < LK; ++j)
      buffer_load_lds_b128(vr, lds0 + (2 + st) * KT + (wave + j * NW) * 1024, voff[j]);
  };

  int n_end = p.Sk;
  if (CAUSAL) n_end = min(p.Sk, m0 + kF32MmaRows + diag);
  const int n_tiles = n_end > 0 ? (n_end + BN - 1) / BN : 0;
  // Tiles [0, vis) hold keys this wave's rows can see.
  int vis = mw < p.Sq ? n_tiles : 0;
  if (CAUSAL) {
    const int last_key = mw + 31 + diag;
    vis = last_key < 0 ? 0 : min(vis, last_key / BN + 1);
  }

  // Lane-constant LDS byte offsets: K chunk j of this lane's half (row l32
  // of key block kb adds kb * 32 rows, which keeps the swizzle), and this
  // lane's V piece (columns DB*m .. DB*m + DB-1, m = l32) in row 4*hl.
  int k_lds[KS / 4];
#pragma unroll
  for (int j = 0; j < KS / 4; ++j) k_lds[j] = l32 * RB + (((hl * (KS / 4) + j) ^ (l32 & 15)) * 16);
  const int v_lds = 2 * KT + 4 * hl * RB + l32 * DB * 4;

  f32x16 oacc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) oacc[c] = f32x16{};
  float m_run = kNegInf, l_run = 0.f;

  if (n_tiles > 0) issue(0);
  for (int t = 0; t < n_tiles; ++t) {
    wait_vmcnt<0>();  // tile t (the only one in flight) landed for this wave ...
    __syncthreads();  // ... and for all; every read of tile t-1 retired
    if (t + 1 < n_tiles) issue(t + 1);  // into tile t-1's stage
    if (t >= vis) continue;
    const int st = t & 1;
    const uint8_t* kt = smem + st * KT;
    f32x16 sc[2] = {f32x16{}, f32x16{}};
#pragma unroll
    for (int j = 0; j < KS / 4; ++j) {
      const f32x4 a0 = *reinterpret_cast<const f32x4*>(kt + k_lds[j]);
      const f32x4 a1 = *reinterpret_cast<const f32x4*>(kt + 32 * RB + k_lds[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[e], qv[4 * j + e], sc[0], 0, 0, 0);
        sc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[e], qv[4 * j + e], sc[1], 0, 0, 0);
      }
    }
    // Register r of block kb: key n0 + 32 kb + 8 (r/4) + 4 hl + r%4.
    const int n0 = t * BN;
    if (n0 + BN > p.Sk || (CAUSAL && n0 + BN - 1 > mw + diag)) {
      int lim = p.Sk - 1;
      if (CAUSAL) lim = min(lim, row + diag);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (n0 + 32 * kb + 8 * (r >> 2) + 4 * hl + (r & 3) > lim) sc[kb][r] = kNegInf;
    }
    float mt = kNegInf;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sc[kb][r]);
    mt = xhalf_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const float alpha = m_new == kNegInf ? 1.f : fast_exp2((m_run - m_new) * p.scale_log2);
    const float neg_m = m_new == kNegInf ? 0.f : -m_new * p.scale_log2;
    m_run = m_new;
    float ps = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sc[kb][r] = fast_exp2(fmaf(sc[kb][r], p.scale_log2, neg_m));
        ps += sc[kb][r];
      }
    l_run = l_run * alpha + ps;
#pragma unroll
    for (int c = 0; c < DB; ++c) oacc[c] *= alpha;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int krow = 32 * kb + 8 * (r >> 2) + (r & 3);
        const vrow_t x = *reinterpret_cast<const vrow_t*>(smem + st * KT + v_lds + krow * RB);
#pragma unroll
        for (int c = 0; c < DB; ++c)
          oacc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(x[c], sc[kb][r], oacc[c], 0, 0, 0);
      }
  }

  const float l_tot = xhalf_sum(l_run);
  if (!row_ok) return;
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  float* op = (float*)p.o + b * p.o_sb + hq * p.o_sh + (int64_t)row * p.o_ss;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int d = DB * (8 * (r >> 2) + 4 * hl + (r & 3));
    if (d < p.D) {
      vrow_t x;
#pragma unroll
      for (int c = 0; c < DB; ++c) x[c] = oacc[c][r] * inv;
      *reinterpret_cast<vrow_t*>(op + d) = x;
    }
  }
  if (hl == 0)
    p.lse[(int64_t)bh * p.Sq + row] = l_tot > 0.f ? m_run * p.scale + logf(l_tot) : kNegInf;
}

// Row statistics for the backward, any dtype:
//   delta[r]    = sum_d dO[r,d] * O[r,d]          (reference flash_bwd.py:15-55)
//   lse_log2[r] = lse[r] * log2(e), or +inf where lse = -inf so that
//                 exp2(s - lse_log2) is exactly 0 on rows that see no key.
// Sixteen lanes per row, each reading 16-byte chunks of dO and O (D is a
// multiple of 8 and rows start 16-byte aligned), so a wave's loads cover
// four whole rows; the lanes' partial sums meet in a butterfly.
template <class T>
__device__ __forceinline__ float dot_chunk(u32x4 a, u32x4 b, float x);
template <>
__device__ __forceinline__ float dot_chunk<float>(u32x4 a, u32x4 b, float x) {
#pragma unroll
  for (int e = 0; e < 4; ++e) x = fmaf(__uint_as_float(a[e]), __uint_as_float(b[e]), x);
  return x;
}
template <class T>
__device__ __forceinline__ float dot_chunk(u32x4 a, u32x4 b, float x) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x = fmaf(to_f32<T>((uint16_t)(a[e] & 0xffffu)), to_f32<T>((uint16_t)(b[e] & 0xffffu)), x);
    x = fmaf(to_f32<T>((uint16_t)(a[e] >> 16)), to_f32<T>((uint16_t)(b[e] >> 16)), x);
  }
  return x;
}

template <class T>
constexpr int kElemBytes = 2;
template <>
constexpr int kElemBytes<float> = 4;

template <class T>
__global__ void __launch_bounds__(256) bwd_prep_kernel(BwdParams p) {
  constexpr int kRowLanes = 16;
  constexpr int esize = kElemBytes<T>;
  const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
  const int64_t r = (int64_t)blockIdx.x * (256 / kRowLanes) + (threadIdx.x / kRowLanes);
  const int j = threadIdx.x % kRowLanes;
  float x = 0.f;
  if (r < rows) {
    const int64_t base = r * p.D * esize;
    const uint8_t* g = (const uint8_t*)p.dout + base;
    const uint8_t* o = (const uint8_t*)p.o + base;
    const int chunks = p.D * esize / 16;
    for (int c = j; c < chunks; c += kRowLanes)
      x = dot_chunk<T>(*reinterpret_cast<const u32x4*>(g + 16 * c),
                       *reinterpret_cast<const u32x4*>(o + 16 * c), x);
  }
#pragma unroll
  for (int m = kRowLanes / 2; m > 0; m >>= 1) x += __shfl_xor(x, m);
  if (r < rows && j == 0) {
    p.delta[r] = x;
    const float l = p.lse[r];
    p.lse_log2[r] = l == kNegInf ? __builtin_inff() : l * kLog2e;
  }
}

// dQ for fp32: rows of queries, loop over keys.
template <int DP, bool CAUSAL>
__global__ void __launch_bounds__(256) bwd_dq_f32_kernel(BwdParams p) {
  constexpr int DC = DP / 4;
  __shared__ float ks[kF32Tile][DP];
  __shared__ float vs[kF32Tile][DP];
  const int tid = threadIdx.x, part = tid & 3, rloc = tid >> 2;
  const int bh_count = p.B * p.Hq;
  const int mblk = p.n_mblocks - 1 - blockIdx.x / bh_count;
  const int bh = blockIdx.x % bh_count;
  const int b = bh / p.Hq, hq = bh % p.Hq, hkv = hq / p.group;
  const int row = mblk * kF32Rows + rloc;
  const bool row_ok = row < p.Sq;
  const int diag = p.Sk - p.Sq;
  const int64_t qrow = ((int64_t)bh * p.Sq + row) * p.D;
  const float* kbase = (const float*)p.k + ((int64_t)b * p.Hkv + hkv) * p.Sk * p.D;
  const float* vbase = (const float*)p.v + ((int64_t)b * p.Hkv + hkv) * p.Sk * p.D;

  float q[DC], g[DC], acc[DC];
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int d = part * DC + i;
    const bool ok = row_ok && d < p.D;
    q[i] = ok ? ((const float*)p.q)[qrow + d] : 0.f;
    g[i] = ok ? ((const float*)p.dout)[qrow + d] : 0.f;
    acc[i] = 0.f;
  }
  const float lse2 = row_ok ? p.lse_log2[(int64_t)bh * p.Sq + row] : __builtin_inff();
  const float dl = row_ok ? p.delta[(int64_t)bh * p.Sq + row] : 0.f;
  int n_end = p.Sk;
  if (CAUSAL) n_end = min(p.Sk, mblk * kF32Rows + kF32Rows + diag);
  const int lim = CAUSAL ? min(p.Sk - 1, row + diag) : p.Sk - 1;
  for (int n0 = 0; n0 < n_end; n0 += kF32Tile) {
    __syncthreads();
    for (int e = tid; e < kF32Tile * DP; e += 256) {
      const int r = e / DP, d = e % DP, n = n0 + r;
      const bool ok = n < p.Sk && d < p.D;
      ks[r][d] = ok ? kbase[(int64_t)n * p.D + d] : 0.f;
      vs[r][d] = ok ? vbase[(int64_t)n * p.D + d] : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int j = 0; j < kF32Tile; ++j) {
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int i = 0; i < DC; ++i) {
        s = fmaf(q[i], ks[j][part * DC + i], s);
        dp = fmaf(g[i], vs[j][part * DC + i], dp);
      }
      s = quad_sum(s);
      dp = quad_sum(dp);
      const float pj = (n0 + j > lim) ? 0.f : exp2f(s * p.scale_log2 - lse2);
      const float ds = pj * (dp - dl);
#pragma unroll
      for (int i = 0; i < DC; ++i) acc[i] = fmaf(ds, ks[j][part * DC + i], acc[i]);
    }
  }
  if (!row_ok) return;
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int d = part * DC + i;
    if (d < p.D) ((float*)p.dq)[qrow + d] = acc[i] * p.scale;
  }
}

// dK, dV for fp32: rows of keys of one KV head; loop over the group's query
// heads and their queries (the GQA sum happens in registers, no atomics).
template <int DP, bool CAUSAL>
__global__ void __launch_bounds__(256) bwd_dkv_f32_kernel(BwdParams p) {
  constexpr int DC = DP / 4;
  __shared__ float qs[kF32Tile][DP];
  __shared__ float gs[kF32Tile][DP];
  __shared__ float ls[kF32Tile], dls[kF32Tile];
  const int tid = threadIdx.x, part = tid & 3, rloc = tid >> 2;
  const int bk_count = p.B * p.Hkv;
  const int nblk = blockIdx.x / bk_count;
  const int bk = blockIdx.x % bk_count;
  const int b = bk / p.Hkv, hkv = bk % p.Hkv;
  const int n = nblk * kF32Rows + rloc;
  const bool key_ok = n < p.Sk;
  const int diag = p.Sk - p.Sq;
  const int64_t krow = ((int64_t)bk * p.Sk + n) * p.D;

  float k[DC], v[DC], dk[DC], dv[DC];
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int d = part * DC + i;
    const bool ok = key_ok && d < p.D;
    k[i] = ok ? ((const float*)p.k)[krow + d] : 0.f;
    v[i] = ok ? ((const float*)p.v)[krow + d] : 0.f;
    dk[i] = dv[i] = 0.f;
  }
  // Query rows that can see some key of this block: i >= n0 - diag.
  int m_begin = 0;
  if (CAUSAL) m_begin = max(0, nblk * kF32Rows - diag);
  for (int gi = 0; gi < p.group; ++gi) {
    const int hq = hkv * p.group + gi;
    const int64_t bh = (int64_t)b * p.Hq + hq;
    for (int m0 = m_begin; m0 < p.Sq; m0 += kF32Tile) {
      __syncthreads();
      for (int e = tid; e < kF32Tile * DP; e += 256) {
        const int r = e / DP, d = e % DP, m = m0 + r;
        const bool ok = m < p.Sq && d < p.D;
        const int64_t idx = (bh * p.Sq + m) * p.D + d;
        qs[r][d] = ok ? ((const float*)p.q)[idx] : 0.f;
        gs[r][d] = ok ? ((const float*)p.dout)[idx] : 0.f;
      }
      if (tid < kF32Tile) {
        const int m = m0 + tid;
        ls[tid] = m < p.Sq ? p.lse_log2[bh * p.Sq + m] : __builtin_inff();
        dls[tid] = m < p.Sq ? p.delta[bh * p.Sq + m] : 0.f;
      }
      __syncthreads();
#pragma unroll 4
      for (int j = 0; j < kF32Tile; ++j) {
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int i = 0; i < DC; ++i) {
          s = fmaf(k[i], qs[j][part * DC + i], s);
          dp = fmaf(v[i], gs[j][part * DC + i], dp);
        }
        s = quad_sum(s);
        dp = quad_sum(dp);
        const int m = m0 + j;
        const bool vis = m < p.Sq && (!CAUSAL || n <= m + diag);
        const float pj = vis ? exp2f(s * p.scale_log2 - ls[j]) : 0.f;
        const float ds = pj * (dp - dls[j]);
#pragma unroll
        for (int i = 0; i < DC; ++i) {
          dv[i] = fmaf(pj, gs[j][part * DC + i], dv[i]);
          dk[i] = fmaf(ds, qs[j][part * DC + i], dk[i]);
        }
      }
    }
  }
  if (!key_ok) return;
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int d = part * DC + i;
    if (d < p.D) {
      ((float*)p.dk)[krow + d] = dk[i] * p.scale;
      ((float*)p.dv)[krow + d] = dv[i];
    }
  }
}

template <int DP>
static KernelPlan plan_fwd_f32_dp(const FwdParams& p, bool causal) {
  KernelPlan k;
  k.fn = causal ? (const void*)fwd_f32_kernel<DP, true> : (const void*)fwd_f32_kernel<DP, false>;
  k.grid = dim3((unsigned)(p.n_mblocks * p.B * p.Hq));
  k.block = dim3(256);
  k.kernel = "fwd_f32_kernel";
  k.elem = 0;
  k.head_dim = DP;
  k.block_m = kF32Rows;
  k.block_n = kF32Tile;
  k.causal = causal;
  k.paged = p.block_table != nullptr;
  k.rope = p.rope.cos != nullptr;
  return k;
}

// The matrix-core kernel for padded head dims up to 128 and at least 32
// query rows (no paged or per-row-length decode: those have one query row);
// the vector kernel otherwise.  A tile-study build with -DSK_F32_MFMA=0
// sends every fp32 forward and backward to the vector kernels.
#ifndef SK_F32_MFMA
#define SK_F32_MFMA 1
#endif
static bool fwd_f32_on_mfma(int d, int sq) {
  const int dp = padded_head_dim(d);
  return SK_F32_MFMA && dp > 0 && dp <= 128 && sq >= 32;
}

int fwd_f32_rows_per_block(int d, int sq) { return fwd_f32_on_mfma(d, sq) ? kF32MmaRows : kF32Rows; }

template <int DP>
static KernelPlan plan_fwd_f32_mfma(const FwdParams& p, bool causal) {
  KernelPlan k;
  k.fn = causal ? (const void*)fwd_f32_mfma_kernel<DP, true> : (const void*)fwd_f32_mfma_kernel<DP, false>;
  k.grid = dim3((unsigned)(p.n_mblocks * p.B * p.Hq));
  k.block = dim3(512);
  k.kernel = "fwd_f32_mfma_kernel";
  k.elem = 0;
  k.head_dim = DP;
  k.block_m = kF32MmaRows;
  k.block_n = 64;
  k.stages = 2;
  k.causal = causal;
  k.rope = p.rope.cos != nullptr;
  return k;
}

KernelPlan plan_fwd_f32(const FwdParams& p, bool causal) {
  if (fwd_f32_on_mfma(p.D, p.Sq) && !p.block_table && !p.seqlens)
    return padded_head_dim(p.D) <= 64 ? plan_fwd_f32_mfma<64>(p, causal)
                                      : plan_fwd_f32_mfma<128>(p, causal);
  switch (padded_head_dim(p.D)) {
    case 64: return plan_fwd_f32_dp<64>(p, causal);
    case 96: return plan_fwd_f32_dp<96>(p, causal);
    case 128: return plan_fwd_f32_dp<128>(p, causal);
    case 256: return plan_fwd_f32_dp<256>(p, causal);
    default: return KernelPlan{};
  }
}

hipError_t launch_fwd_f32(const FwdParams& p, bool causal, hipStream_t s) {
  const KernelPlan k = plan_fwd_f32(p, causal);
  if (!k.fn) return hipErrorInvalidValue;
  return run_plan(k, &p, s);
}

hipError_t launch_bwd_prep(int dtype, const BwdParams& p, hipStream_t s) {
  const int64_t rows = (int64_t)p.B * p.Hq * p.Sq;
  const dim3 grid((unsigned)((rows + 15) / 16));
  if (dtype == 0)
    hipLaunchKernelGGL((bwd_prep_kernel<float>), grid, dim3(256), 0, s, p);
  else if (dtype == BF16::code)
    hipLaunchKernelGGL((bwd_prep_kernel<BF16>), grid, dim3(256), 0, s, p);
  else if (dtype == F16::code)
    hipLaunchKernelGGL((bwd_prep_kernel<F16>), grid, dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// Backward on the matrix cores (padded head dim 64 or 128), the same fp32
// products as the forward's matrix-core kernel and its operand layouts: the
// k-steps of a product over the head dim contract column s in lanes 0-31 and
// DP/2 + s in lanes 32-63; a product over keys or queries contracts the two
// rows the lane halves hold in score register r (8 (r/4) + 4 hl + r%4); an
// output block c holds head-dim columns DB*m + c.  Streamed tiles (32 rows)
// keep 16-byte chunk c of row r at c ^ (r % 16), so the row-wise operand
// reads (16 rows, one chunk each) and the column-piece reads (one row, 32
// chunks) both hit distinct bank quads.  A workgroup is 4 waves, one per SIMD
// (the resident operands and two accumulator sets exceed 256 registers), and
// its tiles go through a 2-deep ring written by buffer_load ... lds, one
// barrier per step; a step is 192 (dQ) or 256 (dK/dV) MFMAs of 64 cycles per
// wave, so one step of load look-ahead is ample.  P = exp2(S * scale * log2 e
// - lse * log2 e) is set to 0 where the key is masked, past S_k, or the query
// past S_q; dS = P (dP - delta).
constexpr int kF32MmaTile = 32;

// Byte offset, in a swizzled tile of DP fp32 columns, of the DB-column piece
// m (columns DB*m .. DB*m + DB - 1) of row r.
template <int DP>
__device__ __forceinline__ int f32_piece(int r, int m) {
  constexpr int DB = DP / 32;
  const int chunk = (DB * m) >> 2, sub = (DB * m) & 3;
  return r * DP * 4 + ((chunk ^ (r & 15)) << 4) + 4 * sub;
}

// dQ: a wave owns 32 queries of one (batch, query head), q and dO resident;
// 32-key K and V tiles stream.  S^T = K Q^T and dP^T = V dO^T (two chains),
// then dQ^T += K^T dS^T.
template <int DP, bool CAUSAL>
__global__ void __launch_bounds__(256, 1) bwd_dq_f32_mfma_kernel(BwdParams p) {
  constexpr int NW = 4, BN = kF32MmaTile, BM = 32 * NW;
  constexpr int KS = DP / 2, DB = DP / 32, RB = DP * 4, KT = BN * RB;
  constexpr int CPR = RB / 16, SEGR = 1024 / RB, LK = KT / 1024 / NW;
  static_assert(DP == 64 || DP == 128, "padded head dim 64 or 128");
  static_assert(LK >= 1 && (KT / 1024) % NW == 0, "tile segments must divide over the waves");
  typedef float vrow_t __attribute__((ext_vector_type(DB)));
  __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * KT];  // K stages, then V stages

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hl = lane >> 5;
  const int w = xcd_work_index(blockIdx.x, gridDim.x);
  const int bh = w / p.n_mblocks;
  const int mblk = p.n_mblocks - 1 - (w - bh * p.n_mblocks);
  const int b = bh / p.Hq, hq = bh % p.Hq, hkv = hq / p.group;
  const int m0 = mblk * BM;
  const int mw = m0 + 32 * wave;
  const int row = mw + l32;
  const bool row_ok = row < p.Sq;
  const int diag = p.Sk - p.Sq;

  const int64_t qrow = ((int64_t)bh * p.Sq + row) * p.D;
  float qv[KS], gv[KS];
#pragma unroll
  for (int j = 0; j < KS / 4; ++j) {
    const int d = hl * KS + 4 * j;
    f32x4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
    if (row_ok && d < p.D) {
      x = *reinterpret_cast<const f32x4*>((const float*)p.q + qrow + d);
      y = *reinterpret_cast<const f32x4*>((const float*)p.dout + qrow + d);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[4 * j + e] = x[e], gv[4 * j + e] = y[e];
  }
  const float lse2 = row_ok ? p.lse_log2[(int64_t)bh * p.Sq + row] : __builtin_inff();
  const float dl = row_ok ? p.delta[(int64_t)bh * p.Sq + row] : 0.f;

  const float* kbase = (const float*)p.k + ((int64_t)b * p.Hkv + hkv) * p.Sk * p.D;
  const float* vbase = (const float*)p.v + ((int64_t)b * p.Hkv + hkv) * p.Sk * p.D;
  uint32_t goff[LK];
#pragma unroll
  for (int j = 0; j < LK; ++j) {
    const int r = (wave + j * NW) * SEGR + lane / CPR;
    const int c = (lane % CPR) ^ (r & 15);
    goff[j] = c * 4 < p.D ? (uint32_t)((r * p.D + c * 4) * 4) : kBufferOob;
  }
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int t) {
    const int n0 = t * BN;
    const int bytes = min(BN, p.Sk - n0) * p.D * 4;
    const i32x4 kr = make_rsrc_words(kbase + (int64_t)n0 * p.D, bytes);
    const i32x4 vr = make_rsrc_words(vbase + (int64_t)n0 * p.D, bytes);
    const int st = t & 1;
#pragma unroll
    for (int j = 0; j < LK; ++j) buffer_load_lds_b128(kr, lds0 + st * KT + (wave + j * NW) * 1024, goff[j]);
#pragma unroll
    for (int j = 0; j < LK; ++j)
      buffer_load_lds_b128(vr, lds0 + (2 + st) * KT + (wave + j * NW) * 1024, goff[j]);
  };

  int n_end = p.Sk;
  if (CAUSAL) n_end = min(p.Sk, m0 + BM + diag);
  const int n_tiles = n_end > 0 ? (n_end + BN - 1) / BN : 0;
  int vis = mw < p.Sq ? n_tiles : 0;
  if (CAUSAL) {
    const int last_key = mw + 31 + diag;
    vis = last_key < 0 ? 0 : min(vis, last_key / BN + 1);
  }
  // Row-wise operand chunk j of key row l32; column piece of key row
  // 8 (r/4) + 4 hl + r%4 for the K^T operand of k-step r.
  int k_lds[KS / 4], kt_lds[16];
#pragma unroll
  for (int j = 0; j < KS / 4; ++j) k_lds[j] = l32 * RB + (((hl * (KS / 4) + j) ^ (l32 & 15)) << 4);
#pragma unroll
  for (int r = 0; r < 16; ++r) kt_lds[r] = f32_piece<DP>(8 * (r >> 2) + 4 * hl + (r & 3), l32);

  f32x16 acc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) acc[c] = f32x16{};
  if (n_tiles > 0) issue(0);
  for (int t = 0; t < n_tiles; ++t) {
    wait_vmcnt<0>();  // tile t landed for this wave ...
    __syncthreads();  // ... and for all; every read of tile t-1 retired
    if (t + 1 < n_tiles) issue(t + 1);
    if (t >= vis) continue;
    const uint8_t* kt = smem + (t & 1) * KT;
    const uint8_t* vt = smem + (2 + (t & 1)) * KT;
    f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int j = 0; j < KS / 4; ++j) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(kt + k_lds[j]);
      const f32x4 g = *reinterpret_cast<const f32x4*>(vt + k_lds[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], qv[4 * j + e], s, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x2f32(g[e], gv[4 * j + e], dp, 0, 0, 0);
      }
    }
    // Register r: key t*BN + 8 (r/4) + 4 hl + r%4 of query row `row`.
    int lim = p.Sk - 1;
    if (CAUSAL) lim = min(lim, row + diag);
    const int n0 = t * BN + 4 * hl;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pr =
          n0 + 8 * (r >> 2) + (r & 3) <= lim ? fast_exp2(fmaf(s[r], p.scale_log2, -lse2)) : 0.f;
      s[r] = pr * (dp[r] - dl);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const vrow_t x = *reinterpret_cast<const vrow_t*>(kt + kt_lds[r]);
#pragma unroll
      for (int c = 0; c < DB; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(x[c], s[r], acc[c], 0, 0, 0);
    }
  }
  if (!row_ok) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int d = DB * (8 * (r >> 2) + 4 * hl + (r & 3));
    if (d < p.D) {
      vrow_t x;
#pragma unroll
      for (int c = 0; c < DB; ++c) x[c] = acc[c][r] * p.scale;
      *reinterpret_cast<vrow_t*>((float*)p.dq + qrow + d) = x;
    }
  }
}

// dK, dV: a wave owns 32 keys of one (batch, KV head), K and V resident; the
// group's query heads and their 32-query tiles stream (Q, dO and the row
// statistics), so the GQA sum happens in registers.  S = Q K^T and dP = dO
// V^T (two chains), then dV^T += dO^T P and dK^T += Q^T dS.
template <int DP, bool CAUSAL>
__global__ void __launch_bounds__(256, 1) bwd_dkv_f32_mfma_kernel(BwdParams p) {
  constexpr int NW = 4, BMQ = kF32MmaTile, BNK = 32 * NW;
  constexpr int KS = DP / 2, DB = DP / 32, RB = DP * 4, QT = BMQ * RB;
  constexpr int CPR = RB / 16, SEGR = 1024 / RB, LQ = QT / 1024 / NW;
  constexpr int kStat = 4 * QT;         // per stage: 64 lse*log2e, then 64 delta
  static_assert(DP == 64 || DP == 128, "padded head dim 64 or 128");
  static_assert(LQ >= 1 && (QT / 1024) % NW == 0, "tile segments must divide over the waves");
  typedef float vrow_t __attribute__((ext_vector_type(DB)));
  __shared__ __attribute__((aligned(1024))) uint8_t smem[4 * QT + 2 * 512];  // Q, dO stages; stats

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hl = lane >> 5;
  // Lowest key block first: under the causal mask it sees the most queries.
  const int w = xcd_work_index(blockIdx.x, gridDim.x);
  const int bk = w / p.n_nblocks;
  const int nblk = w - bk * p.n_nblocks;
  const int b = bk / p.Hkv, hkv = bk % p.Hkv;
  const int n0 = nblk * BNK;
  const int nw = n0 + 32 * wave;
  const int key = nw + l32;
  const bool key_ok = key < p.Sk;
  const int diag = p.Sk - p.Sq;

  const int64_t krow = ((int64_t)bk * p.Sk + key) * p.D;
  float kv[KS], vv[KS];
#pragma unroll
  for (int j = 0; j < KS / 4; ++j) {
    const int d = hl * KS + 4 * j;
    f32x4 x = {0.f, 0.f, 0.f, 0.f}, y = {0.f, 0.f, 0.f, 0.f};
    if (key_ok && d < p.D) {
      x = *reinterpret_cast<const f32x4*>((const float*)p.k + krow + d);
      y = *reinterpret_cast<const f32x4*>((const float*)p.v + krow + d);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) kv[4 * j + e] = x[e], vv[4 * j + e] = y[e];
  }

  // Query tiles that can see a key of this block: rows i >= n0 - diag.
  int m_begin = 0;
  if (CAUSAL) m_begin = max(0, n0 - diag) / BMQ * BMQ;
  const int n_mt = m_begin < p.Sq ? (p.Sq - m_begin + BMQ - 1) / BMQ : 0;
  const int n_it = n0 < p.Sk ? p.group * n_mt : 0;

  uint32_t goff[LQ];
#pragma unroll
  for (int j = 0; j < LQ; ++j) {
    const int r = (wave + j * NW) * SEGR + lane / CPR;
    const int c = (lane % CPR) ^ (r & 15);
    goff[j] = c * 4 < p.D ? (uint32_t)((r * p.D + c * 4) * 4) : kBufferOob;
  }
  const uint32_t lds0 = lds_addr(smem);
  const int64_t bh0 = (int64_t)b * p.Hq + hkv * p.group;
  auto issue = [&](int it) {
    const int gi = it / n_mt;
    const int m = m_begin + (it - gi * n_mt) * BMQ;
    const int rows = min(BMQ, p.Sq - m);
    const int64_t r0 = (bh0 + gi) * p.Sq + m;
    const i32x4 qr = make_rsrc_words((const float*)p.q + r0 * p.D, rows * p.D * 4);
    const i32x4 gr = make_rsrc_words((const float*)p.dout + r0 * p.D, rows * p.D * 4);
    const int st = it & 1;
#pragma unroll
    for (int j = 0; j < LQ; ++j) buffer_load_lds_b128(qr, lds0 + st * QT + (wave + j * NW) * 1024, goff[j]);
#pragma unroll
    for (int j = 0; j < LQ; ++j)
      buffer_load_lds_b128(gr, lds0 + (2 + st) * QT + (wave + j * NW) * 1024, goff[j]);
    if (wave < 2) {  // wave 0: lse * log2 e, wave 1: delta (64 slots; the first 32 used)
      const i32x4 sr = make_rsrc_words((wave == 0 ? p.lse_log2 : p.delta) + r0, rows * 4);
      buffer_load_lds_b32(sr, lds0 + kStat + st * 512 + wave * 256, lane * 4);
    }
  };

  // Row-wise operand chunk j of query row l32; column piece of query row
  // 8 (r/4) + 4 hl + r%4 for the dO^T / Q^T operands of k-step r.
  int q_lds[KS / 4], qt_lds[16];
#pragma unroll
  for (int j = 0; j < KS / 4; ++j) q_lds[j] = l32 * RB + (((hl * (KS / 4) + j) ^ (l32 & 15)) << 4);
#pragma unroll
  for (int r = 0; r < 16; ++r) qt_lds[r] = f32_piece<DP>(8 * (r >> 2) + 4 * hl + (r & 3), l32);

  f32x16 dk[DB], dv[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) dk[c] = f32x16{}, dv[c] = f32x16{};
  if (n_it > 0) issue(0);
  for (int it = 0; it < n_it; ++it) {
    wait_vmcnt<0>();  // step it's tiles landed for this wave ...
    __syncthreads();  // ... and for all; every read of step it-1 retired
    if (it + 1 < n_it) issue(it + 1);
    const int m = m_begin + (it % n_mt) * BMQ;
    // Skip a tile none of this wave's keys can see (or keys past S_k).
    if (nw >= p.Sk || (CAUSAL && m + BMQ - 1 + diag < nw)) continue;
    const uint8_t* qt = smem + (it & 1) * QT;
    const uint8_t* gt = smem + (2 + (it & 1)) * QT;
    const float* stl = reinterpret_cast<const float*>(smem + kStat + (it & 1) * 512);
    f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
    for (int j = 0; j < KS / 4; ++j) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(qt + q_lds[j]);
      const f32x4 g = *reinterpret_cast<const f32x4*>(gt + q_lds[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(a[e], kv[4 * j + e], s, 0, 0, 0);
        dp = __builtin_amdgcn_mfma_f32_32x32x2f32(g[e], vv[4 * j + e], dp, 0, 0, 0);
      }
    }
    // Register r: query m + 8 (r/4) + 4 hl + r%4 against key `key`.
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 l4 = *reinterpret_cast<const f32x4*>(stl + 8 * i + 4 * hl);
      const f32x4 d4 = *reinterpret_cast<const f32x4*>(stl + 64 + 8 * i + 4 * hl);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * i + e;
        const int q = m + 8 * i + 4 * hl + e;
        const bool ok = key_ok && q < p.Sq && (!CAUSAL || key <= q + diag);
        const float pr = ok ? fast_exp2(fmaf(s[r], p.scale_log2, -l4[e])) : 0.f;
        s[r] = pr;
        dp[r] = pr * (dp[r] - d4[e]);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const vrow_t g = *reinterpret_cast<const vrow_t*>(gt + qt_lds[r]);
      const vrow_t x = *reinterpret_cast<const vrow_t*>(qt + qt_lds[r]);
#pragma unroll
      for (int c = 0; c < DB; ++c) {
        dv[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(g[c], s[r], dv[c], 0, 0, 0);
        dk[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(x[c], dp[r], dk[c], 0, 0, 0);
      }
    }
  }
  if (!key_ok) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int d = DB * (8 * (r >> 2) + 4 * hl + (r & 3));
    if (d < p.D) {
      vrow_t x, y;
#pragma unroll
      for (int c = 0; c < DB; ++c) x[c] = dk[c][r] * p.scale, y[c] = dv[c][r];
      *reinterpret_cast<vrow_t*>((float*)p.dk + krow + d) = x;
      *reinterpret_cast<vrow_t*>((float*)p.dv + krow + d) = y;
    }
  }
}

template <int DP>
static KernelPlan plan_bwd_f32_mfma(BwdParams& p, bool causal, bool dq) {
  KernelPlan k;
  if (dq) {
    p.n_mblocks = (p.Sq + 127) / 128;
    k.fn = causal ? (const void*)bwd_dq_f32_mfma_kernel<DP, true>
                  : (const void*)bwd_dq_f32_mfma_kernel<DP, false>;
    k.grid = dim3((unsigned)((int64_t)p.n_mblocks * p.B * p.Hq));
    k.kernel = "bwd_dq_f32_mfma_kernel";
    k.block_m = 128;
    k.block_n = kF32MmaTile;
  } else {
    p.n_nblocks = (p.Sk + 127) / 128;
    k.fn = causal ? (const void*)bwd_dkv_f32_mfma_kernel<DP, true>
                  : (const void*)bwd_dkv_f32_mfma_kernel<DP, false>;
    k.grid = dim3((unsigned)((int64_t)p.n_nblocks * p.B * p.Hkv));
    k.kernel = "bwd_dkv_f32_mfma_kernel";
    k.block_m = kF32MmaTile;
    k.block_n = 128;
  }
  k.block = dim3(256);
  k.elem = 0;
  k.head_dim = DP;
  k.stages = 2;
  k.causal = causal;
  return k;
}

template <int DP>
static KernelPlan plan_bwd_f32_dp(BwdParams& p, bool causal, bool dq) {
  p.n_mblocks = (p.Sq + kF32Rows - 1) / kF32Rows;
  const int nb = (p.Sk + kF32Rows - 1) / kF32Rows;
  KernelPlan k;
  if (dq) {
    k.fn = causal ? (const void*)bwd_dq_f32_kernel<DP, true>
                  : (const void*)bwd_dq_f32_kernel<DP, false>;
    k.grid = dim3((unsigned)(p.n_mblocks * p.B * p.Hq));
    k.kernel = "bwd_dq_f32_kernel";
  } else {
    k.fn = causal ? (const void*)bwd_dkv_f32_kernel<DP, true>
                  : (const void*)bwd_dkv_f32_kernel<DP, false>;
    k.grid = dim3((unsigned)(nb * p.B * p.Hkv));
    k.kernel = "bwd_dkv_f32_kernel";
  }
  k.block = dim3(256);
  k.elem = 0;
  k.head_dim = DP;
  k.block_m = kF32Rows;
  k.block_n = kF32Tile;
  k.causal = causal;
  return k;
}

static KernelPlan plan_bwd_f32(BwdParams& p, bool causal, bool dq) {
  const int dp = padded_head_dim(p.D);
  if (SK_F32_MFMA && dp > 0 && dp <= 64) return plan_bwd_f32_mfma<64>(p, causal, dq);
  if (SK_F32_MFMA && dp > 64 && dp <= 128) return plan_bwd_f32_mfma<128>(p, causal, dq);
  switch (dp) {
    case 64: return plan_bwd_f32_dp<64>(p, causal, dq);
    case 96: return plan_bwd_f32_dp<96>(p, causal, dq);
    case 128: return plan_bwd_f32_dp<128>(p, causal, dq);
    case 256: return plan_bwd_f32_dp<256>(p, causal, dq);
    default: return KernelPlan{};
  }
}

KernelPlan plan_bwd_dq_f32(BwdParams& p, bool causal) { return plan_bwd_f32(p, causal, true); }
KernelPlan plan_bwd_dkv_f32(BwdParams& p, bool causal) { return plan_bwd_f32(p, causal, false); }

hipError_t launch_bwd_f32(const BwdParams& p, bool causal, hipStream_t s) {
  BwdParams q = p;
  const KernelPlan dq = plan_bwd_dq_f32(q, causal);
  const KernelPlan kv = plan_bwd_dkv_f32(q, causal);
  if (!dq.fn || !kv.fn) return hipErrorInvalidValue;
  hipError_t e = run_plan(dq, &q, s);
  if (e != hipSuccess) return e;
  return run_plan(kv, &q, s);
}

}  // namespace sk
