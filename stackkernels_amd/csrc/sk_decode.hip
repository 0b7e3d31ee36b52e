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
//   16-wide column dimension of v_mfma_f32_16x16x32: S^T = K Q^T for a tile
//   of 32 or 64 keys, then O^T += V^T P^T with V^T read transposed from LDS by
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
#include "sk_rope.h"

namespace sk {

template <int DP, int BN = 32>
struct DecTile {
  static constexpr int kBN = BN;                      // keys per tile
  static constexpr int kStride = DP + 16;             // 16-bit words per LDS row
  static constexpr int kWords = kBN * kStride;
  static constexpr int kChunksPerRow = DP / 8;
  static constexpr int kChunks = kBN * kChunksPerRow;
};

// Rows of the tile that starts at key n0 of batch row b (a tile never
// straddles a page): contiguous caches, or the tile's page of a paged cache.
// ok is false when the page index lies outside the pool; such a tile reads as
// zeros and its keys are masked.
struct TileRows {
  const uint16_t* k;
  const uint16_t* v;
  bool ok;
};
// The same, for a tile whose block-table entry the caller has read.
template <bool PAGED>
__device__ __forceinline__ TileRows tile_rows_in(const DecParams& p, const uint16_t* kbase,
                                                 const uint16_t* vbase, int hkv, int n0,
                                                 int page_entry) {
  if (!PAGED) return {kbase + (int64_t)n0 * p.k_ss, vbase + (int64_t)n0 * p.v_ss, true};
  // (readfirstlane: the table entry is the same for every lane, and the
  // DMA resource built from it must sit in scalar registers.)
  const int page = __builtin_amdgcn_readfirstlane(page_entry);
  const bool ok = page >= 0 && page < p.num_pages;
  const int64_t pg = ok ? page : 0;
  const int64_t off = n0 % p.page_size;
  return {(const uint16_t*)p.k + pg * p.k_sb + (int64_t)hkv * p.k_sh + off * p.k_ss,
          (const uint16_t*)p.v + pg * p.v_sb + (int64_t)hkv * p.v_sh + off * p.v_ss, ok};
}

template <bool PAGED>
__device__ __forceinline__ TileRows tile_rows(const DecParams& p, const uint16_t* kbase,
                                              const uint16_t* vbase, int b, int hkv, int n0) {
  return tile_rows_in<PAGED>(
      p, kbase, vbase, hkv, n0,
      PAGED ? p.block_table[(int64_t)b * p.max_pages + n0 / p.page_size] : 0);
}

// Block-table entries of one batch row read by vector loads (counted by
// vmcnt, like the tile loads), so a kernel can fetch a tile's page a tile
// ahead of use without a scalar-load wait inside the tile loop.
struct PageTable {
  buf_rsrc rsrc;
  int first_key, page_size;
  __device__ __forceinline__ int entry(int n0) const {
    return (int)__builtin_amdgcn_raw_buffer_load_b32(
        rsrc, (uint32_t)(((n0 - first_key) / page_size) * 4), 0, 0);
  }
};

// Batch row with the r-th longest cache length (ties by row index), for
// workgroup row r of the grid.  Workgroups are dispatched in grid order, so
// handing rows out longest first lets the short rows fill in behind the long
// ones (list scheduling, longest first) instead of leaving a few long rows to
// run alone at the end.  Lane i ranks row c + i of each 64-row chunk against
// every row, reading the lengths of the other rows with readlane; one ballot
// per chunk finds the row of rank r.  O(B^2 / 64) steps per workgroup, which
// is why the host enables it for B <= 256 only.
__device__ __forceinline__ int row_of_rank(const DecParams& p, int r) {
  const int lane = threadIdx.x & 63;
  auto len = [&](int i) { return min(max(p.seqlens[i], 0), p.Sk); };
  for (int c = 0; c < p.B; c += 64) {
    const int i = c + lane;
    const int li = i < p.B ? len(i) : -1;
    int rank = 0;
    for (int c2 = 0; c2 < p.B; c2 += 64) {
      const int lj_v = c2 + lane < p.B ? len(c2 + lane) : -1;
      const int n = min(64, p.B - c2);
      for (int j = 0; j < n; ++j) {
        const int lj = __builtin_amdgcn_readlane(lj_v, j);
        rank += (lj > li) || (lj == li && c2 + j < i);
      }
    }
    const uint64_t hit = __ballot(i < p.B && rank == r);
    if (hit) return c + (int)__builtin_ctzll(hit);
  }
  return r;  // every r < B has a row
}

// Q^T operand: lane holds q[hq][32*s + 8*g .. +7] (zeros past D and for
// lanes without a head), rotated when the call carries RoPE tables and
// sign-flipped when sm_scale < 0 (the rotation is linear, so the order of the
// two does not matter).
template <class T, int KD>
__device__ __forceinline__ void load_q(const DecParams& p, int b, int hq, bool head_ok, int g,
                                       u32x4 (&qreg)[KD]) {
  const uint16_t* qp = (const uint16_t*)p.q + b * p.q_sb + hq * p.q_sh;
  const int row = rope_row(p.rope, b, 0);
  const int half = p.D >> 1;
#pragma unroll
  for (int s = 0; s < KD; ++s) {
    const int d0 = 32 * s + 8 * g;
    u32x4 x = {0u, 0u, 0u, 0u};
    if (head_ok && d0 < p.D) {
      x = ldg_b128_cached(qp + d0);
      if (row >= 0)
        x = rope8_at<T>(x, ldg_b128_cached(qp + (d0 < half ? d0 + half : d0 - half)), d0, half,
                     p.rope, row);
    }
    qreg[s] = x ^ p.q_sign;
  }
}

// Keys per tile of decode_split_kernel.  The four-wave kernel (groups of 33
// to 64 query heads, MQA) takes 64 keys per barrier pair: each tile's serial
// chain (LDS store, barrier, score MFMAs, row maximum, exp2, output MFMAs,
// barrier) has a fixed latency that 64 keys amortise over twice the bytes,
// which made the C5 decode 3-10% faster and a 48-head group 3.5% faster.
// 32 keys elsewhere: with two waves the 64-key staging takes the kernel from
// 148 to 208 VGPRs and measured 3% slower (groups of 32), one-wave
// workgroups gained nothing (C4), a page of a paged pool may hold only 32
// keys, and the D = 256 tile is already twice the bytes.
// (SK_DEC_BN_W4=32 builds the 32-key candidate of the tile study.)
#ifndef SK_DEC_BN_W4
#define SK_DEC_BN_W4 64
#endif
template <int DP, int NWH, bool PAGED>
constexpr int dec_split_bn() {
  return NWH == 4 && !PAGED && DP <= 128 ? SK_DEC_BN_W4 : 32;
}

template <class T, int DP, int NWH, bool PAGED>
__global__ void __launch_bounds__(NWH * 64) decode_split_kernel(DecParams p) {
  constexpr int BN = dec_split_bn<DP, NWH, PAGED>();
  using Tile = DecTile<DP, BN>;
  constexpr int NKB = BN / 16;  // 16-key blocks of S^T per tile
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
  const int b = p.longest_first ? row_of_rank(p, bk / p.Hkv) : bk / p.Hkv;
  const int hkv = bk % p.Hkv;
  // Keys this row sees: all S_k, or its cache length.  With per-row lengths
  // the row's keys are spread over all its splits (32-key multiples), so a
  // short row does not leave most of its workgroups empty.
  const int sk_b =
      p.seqlens ? min(max(__builtin_amdgcn_readfirstlane(p.seqlens[b]), 0), p.Sk) : p.Sk;
  const int kps = p.seqlens ? max(32, ((sk_b + p.num_splits - 1) / p.num_splits + 31) / 32 * 32)
                            : p.keys_per_split;
  const int k_lo = split * kps;
  const int k_hi = min(sk_b, k_lo + kps);
  const int n_tiles = k_hi > k_lo ? (k_hi - k_lo + BN - 1) / BN : 0;

  const int hd = 16 * wave + c16;  // head within the group for this lane's column
  const bool head_ok = hd < p.group;
  const int hq = hkv * p.group + (head_ok ? hd : 0);

  const uint16_t* kbase = (const uint16_t*)p.k + b * p.k_sb + hkv * p.k_sh;
  const uint16_t* vbase = (const uint16_t*)p.v + b * p.v_sb + hkv * p.v_sh;

  u32x4 qreg[KD];
  load_q<T>(p, b, hq, head_ok, g, qreg);

  // Paged: the page of tile t + 2 is read (vector load) while tile t runs,
  // and used when tile t + 2's loads are issued, one iteration later.
  PageTable ptab{};
  if constexpr (PAGED) {
    const int first = k_lo / p.page_size * p.page_size;
    ptab.rsrc = make_rsrc(p.block_table + (int64_t)b * p.max_pages + first / p.page_size,
                          max(0, p.max_pages - first / p.page_size) * 4);
    ptab.first_key = first;
    ptab.page_size = p.page_size;
  }
  auto page_of = [&](int t) { return PAGED ? ptab.entry(k_lo + t * BN) : 0; };

  u32x4 kreg[LOADS], vreg[LOADS];
  auto load_tile = [&](int t, int page_entry) {
    const int n0 = k_lo + t * BN;
    const TileRows tr = tile_rows_in<PAGED>(p, kbase, vbase, hkv, n0, page_entry);
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
      const int c = tid + i * NT;
      const int r = c / Tile::kChunksPerRow;
      const int d = (c % Tile::kChunksPerRow) * 8;
      const int n = n0 + r;
      u32x4 kx = {0u, 0u, 0u, 0u}, vx = {0u, 0u, 0u, 0u};
      if (tr.ok && n < k_hi && d < p.D && (!kRagged || c < Tile::kChunks)) {
        kx = ldg_b128(tr.k + (int64_t)r * p.k_ss + d);
        vx = ldg_b128(tr.v + (int64_t)r * p.v_ss + d);
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

  int pg_cur = 0, pg_nxt = 0;  // block-table entries of tiles t and t + 1 (paged)
  if (n_tiles > 0) {
    pg_cur = page_of(0);
    if (n_tiles > 1) pg_nxt = page_of(1);
    load_tile(0, pg_cur);
  }
  for (int t = 0; t < n_tiles; ++t) {
    store_tile();
    __syncthreads();
    const int pg_far = (PAGED && t + 2 < n_tiles) ? page_of(t + 2) : 0;
    if (t + 1 < n_tiles) load_tile(t + 1, pg_nxt);
    const int n0 = k_lo + t * BN;

    f32x4 sacc[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      sacc[kb] = f32x4{};
#pragma unroll
      for (int s = 0; s < KD; ++s) {
        const u32x4 a = lds_read_b128(ks + k_off + 16 * kb * Tile::kStride + 32 * s);
        sacc[kb] = mfma16<T>(a, qreg[s], sacc[kb]);
      }
    }
    bool tile_ok = true;
    if constexpr (PAGED) {
      const int page = __builtin_amdgcn_readfirstlane(pg_cur);
      tile_ok = page >= 0 && page < p.num_pages;
      pg_cur = pg_nxt;
      pg_nxt = pg_far;
    }
    if (!tile_ok || n0 + BN > k_hi) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (!tile_ok || n0 + 16 * kb + 4 * g + r >= k_hi) sacc[kb][r] = kNegInf;
    }
    float mt = fmaxf(fmaxf(fmaxf(sacc[0][0], sacc[0][1]), fmaxf(sacc[0][2], sacc[0][3])),
                     fmaxf(fmaxf(sacc[1][0], sacc[1][1]), fmaxf(sacc[1][2], sacc[1][3])));
#pragma unroll
    for (int kb = 2; kb < NKB; ++kb)
      mt = fmaxf(mt, fmaxf(fmaxf(sacc[kb][0], sacc[kb][1]), fmaxf(sacc[kb][2], sacc[kb][3])));
    mt = fmaxf(mt, __shfl_xor(mt, 16));
    mt = xhalf_max(mt);
    const float m_new = fmaxf(m_run, mt);
    const float m_sub = (m_new == kNegInf) ? 0.f : m_new;
    const float alpha = fast_exp2((m_run - m_sub) * p.scale_log2);
    const float neg_m = -m_sub * p.scale_log2;
    m_run = m_new;
    float e[4 * NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j) e[4 * kb + j] = fast_exp2(fmaf(sacc[kb][j], p.scale_log2, neg_m));
    l_run *= alpha;
#pragma unroll
    for (int j = 0; j < 4 * NKB; j += 4) l_run += (e[j] + e[j + 1]) + (e[j + 2] + e[j + 3]);
    // O^T += V^T P^T, one 32-key k-step per 32 keys of the tile; the
    // rescale by alpha rides on the first.
#pragma unroll
    for (int s2 = 0; s2 < BN / 32; ++s2) {
      const float* es = e + 8 * s2;
      const u32x4 pk = {pack2<T>(es[0], es[1]), pack2<T>(es[2], es[3]), pack2<T>(es[4], es[5]),
                        pack2<T>(es[6], es[7])};
#pragma unroll
      for (int c = 0; c < DB; ++c) {
        const uint16_t* vp = vs + v_off + 16 * c + 32 * s2 * Tile::kStride;
        const u32x2 lo = lds_read_tr(vp);
        const u32x2 hi = lds_read_tr(vp + 16 * Tile::kStride);
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        oacc[c] = mfma16<T>(a, pk, s2 == 0 ? oacc[c] * alpha : oacc[c]);
      }
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

// Merge split partials: one 256-thread workgroup per (batch, query head).
// Split weights exp(LSE_s - max) go to LDS; then 8 groups of 32 lanes each
// sum a strided subset of the splits with 16-byte loads (4 head-dim values
// per lane) and the 8 partial sums are added through LDS.
template <class T>
__global__ void __launch_bounds__(256) decode_combine_kernel(DecParams p) {
  __shared__ float w[1024];
  __shared__ float red[8][2];
  __shared__ __attribute__((aligned(16))) float part[8][256];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int bh = blockIdx.x;
  const int b = bh / p.Hq;
  const int hq = bh % p.Hq;
  const int ns = p.num_splits;
  const float* lse = p.part_lse + (int64_t)bh * ns;
  const float* po = p.part_o + (int64_t)bh * ns * p.dpad;
  const int sg = tid >> 5;        // split group 0..7: splits sg, sg + 8, ...
  const int d4 = (tid & 31) * 4;  // head-dim quad

  // The first 64 splits' partials of head-dim block 0 are loaded before the
  // LSE pass, so their latency overlaps it (the weights are not needed to
  // issue them).  Summation order is the same as without the prefetch.
  constexpr int kPre = 8;
  f32x4 pre[kPre];
#pragma unroll
  for (int k = 0; k < kPre; ++k) {
    const int s = sg + 8 * k;
    pre[k] = s < ns && d4 < p.D ? *reinterpret_cast<const f32x4*>(po + (int64_t)s * p.dpad + d4)
                                : f32x4{0.f, 0.f, 0.f, 0.f};
  }

  float mx = kNegInf;
  for (int s = tid; s < ns; s += 256) mx = fmaxf(mx, lse[s]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) red[wv][0] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0][0], red[1][0]), fmaxf(red[2][0], red[3][0]));
  float den = 0.f;
  for (int s = tid; s < ns; s += 256) {
    const float x = mx == kNegInf ? 0.f : __expf(lse[s] - mx);
    w[s] = x;
    den += x;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o);
  if (lane == 0) red[wv][1] = den;
  __syncthreads();
  den = (red[0][1] + red[1][1]) + (red[2][1] + red[3][1]);
  const float inv = den > 0.f ? 1.f / den : 0.f;

  uint16_t* op = (uint16_t*)p.o + b * p.o_sb + hq * p.o_sh;
  for (int d0 = 0; d0 < p.D; d0 += 128) {
    const int d = d0 + d4;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (d < p.D) {
      int s = sg;
      if (d0 == 0) {
#pragma unroll
        for (int k = 0; k < kPre; ++k, s += 8)
          if (s < ns) acc += w[s] * pre[k];
      }
      for (; s < ns; s += 8)
        acc += w[s] * *reinterpret_cast<const f32x4*>(po + (int64_t)s * p.dpad + d);
    }
    *reinterpret_cast<f32x4*>(&part[sg][d4]) = acc;
    __syncthreads();
    if (tid < 64) {
      const int dd = 2 * tid;  // two values per thread
      if (d0 + dd < p.D) {
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          a0 += part[k][dd];
          a1 += part[k][dd + 1];
        }
        *reinterpret_cast<uint32_t*>(op + d0 + dd) = pack2<T>(a0 * inv, a1 * inv);
      }
    }
    __syncthreads();
  }
}

// Split kernel selection (the gfx950 decode table's kernel half; the split
// count half is plan_splits in sk_abi.hip): one register-staged kernel for
// every group size, with 1, 2 or 4 waves per workgroup (16 query heads per
// wave) sharing each K/V tile through LDS.  An LDS-ring variant (tiles by
// buffer_load ... lds, 3 to 8 stages of 16 KB) measured 5-10% slower at C5
// (MQA, 64 heads) with the same bytes in flight per CU.
template <class T, int DP, bool PAGED>
static KernelPlan plan_decode_dp(const DecParams& p) {
  KernelPlan k;
  k.grid = dim3((unsigned)p.num_splits, (unsigned)(p.B * p.Hkv));
  k.elem = T::code;
  k.head_dim = DP;
  k.paged = PAGED;
  k.rope = p.rope.cos != nullptr;
  int nwh = 0;
  if (p.group <= 16) {
    nwh = 1;
    k.fn = (const void*)decode_split_kernel<T, DP, 1, PAGED>;
  } else if (p.group <= 32) {
    nwh = 2;
    k.fn = (const void*)decode_split_kernel<T, DP, 2, PAGED>;
  } else if (p.group <= 64) {
    nwh = 4;
    k.fn = (const void*)decode_split_kernel<T, DP, 4, PAGED>;
  } else {
    return KernelPlan{};
  }
  k.kernel = "decode_split_kernel";
  k.stages = 0;
  k.block = dim3(64 * nwh);
  k.block_m = 16 * nwh;
  k.block_n = nwh == 1 ? dec_split_bn<DP, 1, PAGED>()
                       : nwh == 2 ? dec_split_bn<DP, 2, PAGED>() : dec_split_bn<DP, 4, PAGED>();
  return k;
}

template <class T, bool PAGED>
static KernelPlan plan_decode_tp(const DecParams& p) {
  switch (padded_head_dim(p.D)) {
    case 64:
      return plan_decode_dp<T, 64, PAGED>(p);
    case 96:
      return plan_decode_dp<T, 96, PAGED>(p);
    case 128:
      return plan_decode_dp<T, 128, PAGED>(p);
    case 256:
      return plan_decode_dp<T, 256, PAGED>(p);
    default:
      return KernelPlan{};
  }
}

template <class T>
static KernelPlan plan_decode_t(const DecParams& p) {
  return p.block_table ? plan_decode_tp<T, true>(p) : plan_decode_tp<T, false>(p);
}

KernelPlan plan_decode_mfma(int dtype, const DecParams& p) {
  if (dtype == BF16::code) return plan_decode_t<BF16>(p);
  if (dtype == F16::code) return plan_decode_t<F16>(p);
  return KernelPlan{};
}

hipError_t launch_decode_mfma(int dtype, const DecParams& p, hipStream_t s) {
  const KernelPlan k = plan_decode_mfma(dtype, p);
  if (!k.fn) return hipErrorInvalidValue;
  return run_plan(k, &p, s);
}

KernelPlan plan_decode_combine(int dtype, const DecParams& p) {
  KernelPlan k;
  if (dtype == BF16::code)
    k.fn = (const void*)decode_combine_kernel<BF16>;
  else if (dtype == F16::code)
    k.fn = (const void*)decode_combine_kernel<F16>;
  else
    return k;
  k.grid = dim3((unsigned)(p.B * p.Hq));
  k.block = dim3(256);
  k.kernel = "decode_combine_kernel";
  k.elem = dtype;
  k.head_dim = p.dpad;
  k.block_m = 1;
  return k;
}

hipError_t launch_decode_combine(int dtype, const DecParams& p, hipStream_t s) {
  const KernelPlan k = plan_decode_combine(dtype, p);
  if (!k.fn) return hipErrorInvalidValue;
  return run_plan(k, &p, s);
}

}  // namespace sk
