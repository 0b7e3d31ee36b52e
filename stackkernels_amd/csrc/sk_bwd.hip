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
// A negative sm_scale is applied by flipping the sign bits of the register
// operand of the score product (q in the dQ kernel, k in the dK/dV kernel),
// so the exponent always uses |sm_scale| and a masked score is simply -inf.
//
// Shared organisation (the forward kernel's, adapted):
// * Two waves per SIMD (256 registers each; the dQ kernel at D = 256 runs
//   one), so every MFMA accumulates in VGPRs and the two waves of a SIMD
//   overlap one's VALU work with the other's MFMAs.
// * The streamed tiles go through a 4-deep LDS ring written by
//   buffer_load ... lds (direct to LDS), two tiles ahead of the math, one
//   barrier per tile.  Rows past the sequence end and head-dim padding come
//   back as zeros from the buffer range check.
// * Streamed tiles are read both row-wise (ds_read_b128, 16 consecutive rows
//   per 16-lane group) and transposed (ds_read_b64_tr_b16, 4 aligned rows x 4
//   chunks per 32-lane group).  One XOR swizzle on the 16-byte chunk index
//   serves both: chunk c of row r sits at c ^ f(r) with f a bijection on
//   r % 16 whose top two bits differ across every aligned group of 4 rows,
//   so both read shapes hit 16 distinct bank quads of the 64-bank LDS.
// * XCD-aware order: the 8 XCDs each walk a contiguous range of work items,
//   head-major, so the workgroups that share a head's streamed operand share
//   an L2.
//
// dK/dV kernel (bwd_dkv_kernel): a workgroup of 8 waves owns 128 keys of one
// (batch, KV head) and walks every query head of that KV head's group and
// every 32-query tile that can see its keys, so the GQA sum happens in
// registers (deterministic, no atomics).  The two waves of a SIMD share a
// 32-key group and split the work by role: one holds K and computes
// S = Q K^T, P and dV^T += dO^T P; the other holds V and computes
// dP = dO V^T, dS and dK^T += Q^T dS, reading P from LDS.  With K or V as
// the B operand each lane owns one key (its l%32) and 16 queries per
// 32-query block; dO^T / Q^T are read transposed from the ring (the
// contraction over queries is permuted identically on both operands).  At
// D = 256 the output head dim is split over two workgroups to keep the
// accumulators in the register file.
//
// dQ kernel (bwd_dq_kernel): a workgroup of 4 waves owns 128 query rows, 32
// per wave, with Q and dO in registers, two workgroups per CU (one at
// D = 256); 32-key K/V tiles stream through the ring; S^T = K Q^T and
// dP^T = V dO^T give one query per lane, and dQ^T += K^T dS^T reads K^T
// transposed from the ring.
#include <algorithm>
#include <mutex>

#include "sk_common.h"

// dQ schedule 2: row-operand and transposed-operand read leads (MFMA slots).
#ifndef SK_DQ_KL
#define SK_DQ_KL 3
#endif
#ifndef SK_DQ_XL
#define SK_DQ_XL 4
#endif
// dK/dV ring depth at D = 128: 6 (pipelined schedule) or 4.
#ifndef SK_BWD_DKV_STAGES
#define SK_BWD_DKV_STAGES 6
#endif
// The D = 64 dK/dV ring: 6 (the pipelined schedule, the table), or 4 for the
// one-tile-per-step schedule in a tile-study build.  Against 4, bit-identical:
// C3 shape at D = 64 9.9% faster, causal MHA S = 8192 7.1%, causal S = 2048
// 6.2%, non-causal S = 2048 / 4096 1.2% / 2.0%; causal S = 1024 2.1% slower
// and causal S = 4096 even (one box, alternating libraries).
#ifndef SK_BWD_DKV_STAGES_D64
#define SK_BWD_DKV_STAGES_D64 6
#endif
// Output head-dim columns per dK/dV workgroup at D = 256: 128 (two
// workgroups per key block, the table) or 256 in a tile-study build.
#ifndef SK_BWD_DKV_DO_D256
#define SK_BWD_DKV_DO_D256 128
#endif
// Five-GEMM backward at D = 128 (1, the table) or seven GEMMs everywhere (0):
// the dK/dV kernel stores dS and bwd_dq_ds_kernel computes dQ from it.
#ifndef SK_BWD_FIVE_GEMM
#define SK_BWD_FIVE_GEMM 1
#endif
// Non-temporal hint on the dS tiles: bit 0 on the dK/dV kernel's stores,
// bit 1 on the dQ kernel's loads.  The tiles are written once and read once,
// and the hint keeps them from evicting the Q/dO and K tiles the kernels
// re-read from L2: with both bits the C3 backward is 4.6% faster and MHA
// S = 4096 2.0% faster (bit-identical results).
#ifndef SK_BWD_DS_NT
#define SK_BWD_DS_NT 3
#endif
#include "sk_kernels.h"

namespace sk {

// One streamed tile of ROWS rows x DP 16-bit words in LDS, unpadded, moved
// in 1 KiB segments (one wave-wide 16-byte-per-lane DMA each).
template <int DP, int ROWS>
struct BwdTile {
  static constexpr int kCpr = DP / 8;  // 16-byte chunks per row
  static constexpr int kRowBytes = DP * 2;
  static constexpr int kTileBytes = ROWS * kRowBytes;
  static constexpr int kSegRows = 1024 / kRowBytes;
  static constexpr int kSegs = kTileBytes / 1024;
};

// Chunk swizzle for tiles read both row-wise and transposed (see the file
// comment).  D >= 128 (rows of whole 64-bank lines): f(r) swaps the two bit
// pairs of r % 16.  D = 64 (two rows per bank line, alternating halves):
// f depends on r / 2 so that rows of one parity get distinct values.  In
// both, f(r + 16) = f(r).
template <int DP>
__device__ __forceinline__ int swz_rt(int r) {
  return DP == 64 ? (((r >> 1) & 1) << 2) | ((r >> 2) & 3) : ((r & 3) << 2) | ((r >> 2) & 3);
}

// Lane-constant byte offsets of a transposed (ds_read_b64_tr_b16) operand
// read: A[m = l%32 -> head-dim column 32c + m][k = 8*(l/32) + j -> tile rows
// 4*(l/32) + j (j < 4) and 8 + 4*(l/32) + j - 4 (j >= 4)].  Lane j16 of each
// 16-lane group addresses row 4*(l/32) + j16/4 (+8 for the upper half),
// chunk chunk0 + 4c + 2*((l/16)%2) + (j16%4)/2, 8-byte half j16%2.  The
// upper half needs its own offsets because f(r + 8) != f(r).
template <int DP, int NC>
__device__ __forceinline__ void tr_offsets(int lane, int chunk0, int (&lo)[NC], int (&hi)[NC]) {
  const int j16 = lane & 15;
  const int r = 4 * (lane >> 5) + j16 / 4;
  const int g = 2 * ((lane >> 4) & 1) + (j16 & 3) / 2;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int ch = chunk0 + 4 * c + g;
    lo[c] = r * DP * 2 + ((ch ^ swz_rt<DP>(r)) * 16) + 8 * (j16 & 1);
    hi[c] = (r + 8) * DP * 2 + ((ch ^ swz_rt<DP>(r + 8)) * 16) + 8 * (j16 & 1);
  }
}

__device__ __forceinline__ u32x4 lds_b128(const uint8_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

__device__ __forceinline__ u32x4 lds_tr_pair(const uint8_t* lo, const uint8_t* hi) {
  const u32x2 a = lds_read_tr((const uint16_t*)lo);
  const u32x2 b = lds_read_tr((const uint16_t*)hi);
  return __builtin_shufflevector(a, b, 0, 1, 2, 3);
}

// ---------------------------------------------------------------------------
// dK / dV
// ---------------------------------------------------------------------------
// Eight waves: key group kg = wave % 4 (32 keys) and role = wave / 4, so the
// two waves of a key group share a SIMD.  Role 0 holds K and computes
// S = Q K^T, P and dV^T += dO^T P for query tile j; role 1 holds V and
// finishes tile j - 1 (dS = P (dP - delta) with the P role 0 left in LDS,
// dK^T += Q^T dS) before computing dP = dO V^T of tile j, so the two waves of
// a SIMD alternate VALU and MFMA phases.  Each wave keeps half of a key
// group's accumulators, so both fit the 256 registers of a two-waves-per-SIMD
// launch and every MFMA result lands in VGPRs.
//
// LDS is region-major -- all Q tiles, all dO tiles, the row statistics, the
// P exchange -- and the step loop is unrolled by the ring depth, so every
// LDS access is a lane-constant register plus a compile-time offset.
//
// Two schedules: a 4-deep ring where a step is one tile's S, P and dV (role
// 0) or dS, dK and the next dP (role 1), each phase a block of MFMAs or of
// VALU work; and, at D = 64 and D = 128, a 6-deep ring where role 0 computes S one tile
// ahead so that every step interleaves MFMAs with the VALU work of the
// previous tile in the same wave (a wave overlaps MFMA and VALU issue only
// with its own instructions).
template <class T, int DP, int DO, int STAGES, bool CAUSAL>
__global__ void __launch_bounds__(512, 1) bwd_dkv_kernel(BwdParams p) {
  constexpr int NW = 8;   // waves: two roles per key group
  constexpr int NKG = 4;  // key groups of 32 keys
  constexpr int BMQ = 32;  // queries per tile (one 32x32 score block per wave)
  using L = BwdTile<DP, BMQ>;  // Q and dO tiles
  constexpr int BNK = 128;
  constexpr int KD = DP / 16;  // k-steps over the head dim (S, dP)
  constexpr int DB = DO / 32;  // 32-wide output head-dim blocks
  constexpr int LS = 2 * L::kSegs / NW;  // Q + dO segments per wave per tile
  constexpr int QT = L::kTileBytes;
  constexpr int RB = L::kRowBytes;
  constexpr int kStatStage = NW * 256;  // per stage: each wave's 64 floats
  constexpr bool kPF32 = DP <= 128;  // P exchanged in fp32 (else 16-bit)
  constexpr int kPBlock = kPF32 ? 4096 : 2048;  // one key group's 32x32 P
  constexpr int kQReg = 0;
  constexpr int kDReg = STAGES * QT;
  constexpr int kSReg = 2 * STAGES * QT;
  constexpr int kPReg = kSReg + STAGES * kStatStage;
  constexpr int kLds = kPReg + 2 * 4 * kPBlock;
  constexpr int kLoads = LS + 1;  // DMAs per wave per tile
  constexpr int PD = 2;  // tiles issued ahead
  constexpr int kDSplit = DP / DO;
  // 4 stages: S and P of a tile in one step (any D).  6 stages (D <= 128):
  // the pipelined schedule below, S one step ahead of P.
  constexpr bool kV2 = STAGES == 6;
  static_assert(STAGES == 4 || (kV2 && DP <= 128), "a 4-deep ring, or 6-deep at D <= 128");
  static_assert((2 * L::kSegs) % NW == 0, "tile segments must divide over the waves");
  static_assert((STAGES - 1) * QT + 16 * RB < 65536, "stage offsets must fit the ds immediate");

  __shared__ __attribute__((aligned(1024))) uint8_t smem[kLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kg = wave % NKG;
  const int role = wave / NKG;
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  // Work item: (batch, KV head) major, then key block (lowest first: under
  // the causal mask it sees the most queries), then head-dim half.
  const int w = xcd_work_index(blockIdx.x, gridDim.x);
  const int per_head = p.n_nblocks * kDSplit;
  const int bkl = w / per_head;  // pair within this launch
  const int bk = p.bk0 + bkl;
  const int rem = w - bkl * per_head;
  const int nblk = rem / kDSplit;
  const int dsp = rem - nblk * kDSplit;
  const int b = bk / p.Hkv;
  const int hkv = bk - b * p.Hkv;
  const int n0 = nblk * BNK;
  const int nw = n0 + 32 * kg;  // first key of this wave
  const int key = nw + l32;
  const int diag = p.Sk - p.Sq;
  const int d_out0 = dsp * DO;

  // Resident B operand, rows of this lane's key: K (sign-flipped for a
  // negative scale) for role 0, V for role 1: x[key][16*s + 8*hl .. +7].
  u32x4 kv[KD];
  {
    const int krows = max(0, min(32, p.Sk - nw));
    const int64_t k0 = ((int64_t)bk * p.Sk + min(nw, p.Sk)) * p.D;
    const int bytes = __builtin_amdgcn_readfirstlane(tile_bytes(krows, p.D, p.D));
    const uint16_t* src = (const uint16_t*)(role == 0 ? p.k : p.v) + k0;
    const uint32_t sgn = role == 0 ? p.op_sign : 0u;
    const buf_rsrc r = make_rsrc(src, bytes);
#pragma unroll
    for (int s = 0; s < KD; ++s) {
      const int d0 = 16 * s + 8 * hl;
      const uint32_t off = d0 < p.D ? (uint32_t)((l32 * p.D + d0) * 2) : kBufferOob;
      kv[s] = buffer_load_b128(r, off) ^ sgn;
    }
  }

  // Query tiles that can see a key of this block: i >= n0 - diag.
  int m_begin = 0;
  if (CAUSAL) m_begin = max(0, n0 - diag) / BMQ * BMQ;
  const int n_mt = m_begin < p.Sq ? (p.Sq - m_begin + BMQ - 1) / BMQ : 0;
  const int n_it = p.group * n_mt;

  // DMA: segment j of this wave is segment wave + 8j of the tile pair (Q
  // segments first, then dO); its LDS target and lane source offsets.
  uint32_t goff[LS];
#pragma unroll
  for (int j = 0; j < LS; ++j) {
    const int seg = (wave + j * NW) % L::kSegs;
    const int r = seg * L::kSegRows + lane / L::kCpr;
    const int c = (lane % L::kCpr) ^ swz_rt<DP>(r);
    goff[j] = c * 8 < p.D ? (uint32_t)((r * p.D + c * 8) * 2) : kBufferOob;
  }
  // Issue cursor: query head, first row, and that row's index in [B*Hq*Sq].
  const int64_t bh0 = (int64_t)b * p.Hq + hkv * p.group;
  int iss_gi = 0, iss_m0 = m_begin;
  int64_t iss_row = bh0 * p.Sq + m_begin;
  const float* stat_src = role == 0 ? p.lse_log2 : p.delta;  // role 0: lse*log2e
  const uint32_t lds0 = lds_addr(smem);
  auto issue = [&](int stg) {
    const int bytes = tile_bytes(min(BMQ, p.Sq - iss_m0), p.D, p.D);
    const int64_t e0 = iss_row * p.D;
    const i32x4 qr = make_rsrc_words((const uint16_t*)p.q + e0, bytes);
    const i32x4 gr = make_rsrc_words((const uint16_t*)p.dout + e0, bytes);
#pragma unroll
    for (int j = 0; j < LS; ++j) {
      const int seg = wave + j * NW;
      const bool is_do = seg >= L::kSegs;  // wave-uniform
      const int sseg = is_do ? seg - L::kSegs : seg;
      buffer_load_lds_b128(is_do ? gr : qr,
                           lds0 + (is_do ? kDReg : kQReg) + stg * QT + sseg * 1024, goff[j]);
    }
    const i32x4 sr = make_rsrc_words(stat_src + iss_row, min(64, p.Sq - iss_m0) * 4);
    buffer_load_lds_b32(sr, lds0 + kSReg + stg * kStatStage + wave * 256, lane * 4);
    iss_m0 += BMQ;
    iss_row += BMQ;
    if (iss_m0 >= p.Sq) {
      iss_m0 = m_begin;
      ++iss_gi;
      iss_row = (bh0 + iss_gi) * p.Sq + m_begin;
    }
  };

  f32x16 acc[DB];  // role 0: dV^T, role 1: dK^T
#pragma unroll
  for (int c = 0; c < DB; ++c) acc[c] = f32x16{};

  // Lane-constant LDS byte addresses.  Row-wise A operand (query row l32,
  // chunk 2s + hl) of S (role 0: Q region) or dP (role 1: dO region);
  // transposed operand of dV (role 0: dO region) or dK (role 1: Q region).
  const int row_reg = role == 0 ? kQReg : kDReg;
  const int tr_reg = role == 0 ? kDReg : kQReg;
  int row_lds[KD];
#pragma unroll
  for (int s = 0; s < KD; ++s)
    row_lds[s] = row_reg + l32 * RB + (((2 * s + hl) ^ swz_rt<DP>(l32)) * 16);
  int tr_lo[DB], tr_hi[DB];
  tr_offsets<DP, DB>(lane, d_out0 / 8, tr_lo, tr_hi);
#pragma unroll
  for (int c = 0; c < DB; ++c) {
    tr_lo[c] += tr_reg;
    tr_hi[c] += tr_reg;
  }
  // This wave's statistics copy (queries 8*i + 4*hl .. +3 at +32*i) and its
  // key group's P block (16-byte chunk k of every lane at +1024*k).
  const int stat_lds = kSReg + wave * 256 + 16 * hl;
  const int p_lds = kPReg + kg * kPBlock + lane * 16;
  const float c_log2 = p.abs_scale_log2;

  auto ld128 = [&](int addr) { return *reinterpret_cast<const u32x4*>(smem + addr); };
  auto ldf4 = [&](int addr) { return *reinterpret_cast<const f32x4*>(smem + addr); };
  // x[query][key] = X Y^T over the row-wise operand of stage stg and the
  // register operand: lane holds [query 8*(r/4) + 4*hl + r%4][key l32].
  auto score = [&](int stg) {
    u32x4 a[KD];
#pragma unroll
    for (int s = 0; s < KD; ++s) a[s] = ld128(row_lds[s] + stg * QT);
    f32x16 sc = f32x16{};
#pragma unroll
    for (int s = 0; s < KD; ++s) sc = mfma32<T>(a[s], kv[s], sc);
    return sc;
  };
  // acc^T += X^T G, X^T read transposed from stage stg, G the packed B
  // operand (P or dS) of the two 16-query k-steps.
  auto accumulate = [&](int stg, const u32x4 (&g)[2]) {
    u32x4 x[2][DB];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int c = 0; c < DB; ++c) {
        const int o = stg * QT + 16 * s2 * RB;
        x[s2][c] = lds_tr_pair(smem + tr_lo[c] + o, smem + tr_hi[c] + o);
      }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int c = 0; c < DB; ++c) acc[c] = mfma32<T>(x[s2][c], g[s2], acc[c]);
  };
  auto pack16 = [&](const float (&v)[16], u32x4 (&g)[2]) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
      g[s2] = u32x4{pack2<T>(v[8 * s2], v[8 * s2 + 1]), pack2<T>(v[8 * s2 + 2], v[8 * s2 + 3]),
                    pack2<T>(v[8 * s2 + 4], v[8 * s2 + 5]), pack2<T>(v[8 * s2 + 6], v[8 * s2 + 7])};
  };

  // Role 0, tile in stage stg (P buffer pb): S, causal mask, P =
  // exp2(S*scale*log2e - lse*log2e), published for role 1, dV^T += dO^T P.
  int cur_gi = 0, cur_m0 = m_begin;  // role 0's tile
  // Five-GEMM backward: role 1 stores each tile's dS (32 keys x 32 queries,
  // 16-bit) for the dQ kernel.  A lane holds key l32 and, as pieces of 4
  // queries, P_m = queries 8 m + 4 hl + {0..3}: P_0, P_1 = g[0].xy, .zw and
  // P_2, P_3 = g[1].xy, .zw.  Chunk (key r, m) -- queries 8 m .. 8 m + 7, the
  // pieces of lanes r and r + 32 -- is formed by one lane-half swap per
  // dword and stored at byte 1024 (m % 2) + 16 (r + 32 (m / 2)) of the 2 KiB
  // tile, so each wave writes the tile with two contiguous 1 KiB stores.
  // Key groups past S_k store nothing; in the group that holds the last key,
  // the rows of keys past S_k are stored as zeros (their P is not masked, and
  // exp2(-lse * log2 e) * delta can overflow to inf, which the dQ kernel's
  // zero K rows would turn into NaN).  Tile (query head, key tile, query
  // tile) sits where the dS tile layout (DsLayout) puts it, counted from the
  // launch's first pair.
  int ds_gi = 0, ds_m0 = m_begin;  // role 1's dS tile
  const int64_t ds_t0 =
      (int64_t)bkl * p.group * p.ds_head_tiles + 4 * ds_off(nblk, p.ds_nqt, p.ds_c, CAUSAL) +
      (int64_t)kg * ds_cnt(nblk, p.ds_nqt, p.ds_c, CAUSAL) - ds_qb(nblk, p.ds_c, CAUSAL);
  auto store_ds = [&](const u32x4 (&gin)[2]) SK_INLINE {
    if constexpr (SK_BWD_FIVE_GEMM) {
      if (p.ds != nullptr) {
        if (nw < p.Sk) {
          const int64_t tile = ds_t0 + (int64_t)ds_gi * p.ds_head_tiles + (ds_m0 >> 5);
          u32x4 g[2] = {gin[0], gin[1]};
          if (nw + 32 > p.Sk) {
            const uint32_t keep = key < p.Sk ? ~0u : 0u;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
              for (int e = 0; e < 4; ++e) g[h][e] &= keep;
          }
          // lane r < 32 gets chunks (r, 0), (r, 1); lane r + 32 chunks (r, 2), (r, 3)
          const auto a0 = __builtin_amdgcn_permlane32_swap(g[0][0], g[1][0], false, false);
          const auto a1 = __builtin_amdgcn_permlane32_swap(g[0][1], g[1][1], false, false);
          const auto b0 = __builtin_amdgcn_permlane32_swap(g[0][2], g[1][2], false, false);
          const auto b1 = __builtin_amdgcn_permlane32_swap(g[0][3], g[1][3], false, false);
          uint8_t* dst = (uint8_t*)p.ds + tile * 2048 + 16 * lane;
          const u32x4 c0{(uint32_t)a0[0], (uint32_t)a1[0], (uint32_t)a0[1], (uint32_t)a1[1]};
          const u32x4 c1{(uint32_t)b0[0], (uint32_t)b1[0], (uint32_t)b0[1], (uint32_t)b1[1]};
          if constexpr (SK_BWD_DS_NT & 1) {
            __builtin_nontemporal_store(c0, reinterpret_cast<u32x4*>(dst));
            __builtin_nontemporal_store(c1, reinterpret_cast<u32x4*>(dst + 1024));
          } else {
            *reinterpret_cast<u32x4*>(dst) = c0;
            *reinterpret_cast<u32x4*>(dst + 1024) = c1;
          }
        }
        ds_m0 += BMQ;
        if (ds_m0 >= p.Sq) {
          ds_m0 = m_begin;
          ++ds_gi;
        }
      }
    }
  };
  auto step0 = [&](int stg, int pbi) {
    f32x16 sc = score(stg);
    if (CAUSAL && nw + 31 > cur_m0 + diag) {
      const int lim = key - diag - cur_m0 - 4 * hl;  // masked iff 8*(r/4) + r%4 < lim
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + (r & 3) < lim) sc[r] = kNegInf;
    }
    float pe[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 lv = ldf4(stat_lds + stg * kStatStage + 32 * i);
#pragma unroll
      for (int k = 0; k < 4; ++k) pe[4 * i + k] = fast_exp2(fmaf(sc[4 * i + k], c_log2, -lv[k]));
    }
    u32x4 pk[2];
    pack16(pe, pk);
    uint8_t* pb = smem + p_lds + pbi * 4 * kPBlock;
    if constexpr (kPF32) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        *reinterpret_cast<f32x4*>(pb + 1024 * k) = f32x4{pe[4 * k], pe[4 * k + 1], pe[4 * k + 2], pe[4 * k + 3]};
    } else {
      *reinterpret_cast<u32x4*>(pb) = pk[0];
      *reinterpret_cast<u32x4*>(pb + 1024) = pk[1];
    }
    accumulate(stg, pk);
    cur_m0 += BMQ;
    if (cur_m0 >= p.Sq) {
      cur_m0 = m_begin;
      ++cur_gi;
    }
  };
  // Role 1, tile in stage stg (P buffer pbi): dS = P (dP - delta) with the
  // dP of that tile (computed one step earlier, or here at D = 256 where
  // registers are short), then dK^T += Q^T dS.
  constexpr bool kSkew = DP <= 128;
  f32x16 dp = f32x16{};
  auto step1 = [&](int stg, int pbi) {
    if constexpr (!kSkew) dp = score(stg);
    const uint8_t* pb = smem + p_lds + pbi * 4 * kPBlock;
    float pr[16];
    if constexpr (kPF32) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(pb + 1024 * k);
#pragma unroll
        for (int e = 0; e < 4; ++e) pr[4 * k + e] = v[e];
      }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(pb + 1024 * h);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pr[8 * h + e] = to_f32<T>((uint16_t)((e & 1) ? (v[e >> 1] >> 16) : (v[e >> 1] & 0xffffu)));
      }
    }
    float de[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4 dv = ldf4(stat_lds + stg * kStatStage + 32 * i);
#pragma unroll
      for (int k = 0; k < 4; ++k) de[4 * i + k] = pr[4 * i + k] * (dp[4 * i + k] - dv[k]);
    }
    u32x4 dsk[2];
    pack16(de, dsk);
    accumulate(stg, dsk);
  };

  // Step j: role 0 works on tile j; role 1 finishes tile j - 1 and computes
  // dP of tile j.  At the start of a step, tile j has landed (vmcnt, then the
  // barrier, which also publishes role 0's P of tile j - 1 and retires every
  // read of tile j - 2), and tile j + 2 is issued into tile j - 2's stage.
  // Tile t lives in stage t % 4 and its P in buffer t % 2.  Steps 0 and n_it
  // (one role idle) are peeled; the steps in between run unconditionally in
  // a loop unrolled by 4, so stages and buffers are compile-time constants
  // and no accumulator moves between registers.
  auto begin_step = [&](int j, int issue_stage) {
    if (j + 1 < n_it)
      wait_vmcnt<kLoads>();
    else
      wait_vmcnt<0>();
    __syncthreads();
    if (j + PD < n_it) issue(issue_stage);
  };
  // ---- Pipelined schedule (6-deep ring, D <= 128) ----------------------
  // Step j: role 0 computes S(j+1) and, between those MFMAs, P(j) from the
  // S(j) of the previous step (mask, exp2, pack, publish to LDS), then
  // dV^T += dO(j)^T P(j); role 1 computes dP(j) and, between those MFMAs,
  // dS(j-1) = P(j-1) (dP(j-1) - delta(j-1)), then dK^T += Q(j-1)^T dS(j-1).
  // Each wave thus keeps its own MFMA and VALU work interleaved (a wave
  // overlaps MFMA and VALU only with its own instructions).  Barrier j makes
  // role 0's P(j-1) visible, retires every read of tile j-2 (role 1 reads
  // Q(j-2) in step j-1), and makes tile j+2 visible (the furthest-ahead tile
  // read in step j: the preload of S(j+2)'s first operands; tile j+1 without
  // the preload); tile j+4 then goes into tile j-2's stage, so every load
  // has two steps to land (three without the preload).
  //
  // A step is a list of MFMA slots, each closed by a scheduling barrier:
  // NS score slots (k-step s, key block kb; one read of each A operand for
  // all key blocks), then NA accumulate slots in the order k-step s2, key
  // block kb, head-dim block c (one transposed read per (s2, c) for all key
  // blocks).  Operand reads run KL / XL slots ahead of their first use; the
  // VALU work on element pairs is spread over the slots in the order the
  // accumulate slots consume the packed operands.
  constexpr int NS = KD;               // score MFMAs per step
  constexpr int NA = 2 * DB;           // accumulate MFMAs per step
  constexpr int NX = 2 * DB;           // transposed reads per step
  constexpr int NM = NS + NA;
  constexpr int NP = 8;                // element pairs per step
  constexpr int KL = 3;                // row-operand read lead (MFMA slots)
  constexpr int XL = 4;                // transposed-operand read lead
  constexpr int SL = 2;                // statistics / P read lead
  constexpr int F0 = NS >= 8 ? 1 : 0;  // first softmax / dS slot
  // Preloaded step start: barrier j waits for tile j+2, so at the end of
  // step j a wave already reads the first KLP row operands of step j+1 (role
  // 0: Q(j+2), role 1: dO(j+1)) and its MFMAs start right after the next
  // barrier; the DMA of tile j+4 is issued at slot kIssSlot, after the
  // step's first MFMAs, instead of right after the barrier.  (Reading them
  // after the barrier, and the statistics by one 4-byte read per lane with
  // DPP row broadcasts, were slower candidates of the tile study.)
  constexpr int KLP = KL;  // row operands read before slot 0
  constexpr int kIssSlot = 2;
  constexpr int kPreSlot = NS + 1;
  u32x4 pre[KLP];
  // Element pair g (elements 2g, 2g+1; k-step g / 4 of the accumulate
  // operand) starts (FMA) at slot pf(g), exponentiates at pf(g) + 1 and
  // packs at pf(g) + 2; pairs 4u .. 4u+3 feed accumulate slot NS + u DB.
  auto pf = [](int g) {
    return g < 4 ? F0 + g * (NS - 3 - F0) / 3 : NS - 2 + (g - 4) * (DB - 1) / 3;
  };
  static_assert(
      [] {
        for (int g = 0; g < NP; ++g)
          if ((g < 4 ? F0 + g * (NS - 3 - F0) / 3 : NS - 2 + (g - 4) * (DB - 1) / 3) + 3 >
              NS + (g / 4) * DB)
            return false;
        return true;
      }(),
      "every pair is packed before its accumulate slot");
  auto begin_v2 = [&](int j) {
    wait_tiles<kLoads, 1>(min(1, max(0, n_it - j - 3)));  // tile j+2 landed
    __syncthreads();
  };
  // Role 0, tile j in stage st, tile j+1 in stage st1, P buffer pbi; sc holds
  // S(j), nx receives S(j+1).
  auto body0 = [&](int j, int st, int st1, int pbi, f32x16& sc, f32x16& nx) SK_INLINE {
    if (CAUSAL && nw + 31 > cur_m0 + diag) {
      // masked iff 8*(r/4) + r%4 < lim
      const int lim = key - diag - cur_m0 - 4 * hl;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + (r & 3) < lim) sc[r] = kNegInf;
    }
    // statistics of elements 4q..4q+3, read SL slots before the first pair
    // that uses them
    f32x4 lv[4];
    auto lv_slot = [&](int q) { return pf(2 * q) - SL; };
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (lv_slot(q) < 0) lv[q] = ldf4(stat_lds + st * kStatStage + 32 * q);
    // statistic of result register r
    auto lse_r = [&](int r) { return lv[r / 4][r % 4]; };
    u32x4 aq[KD];
    u32x4 xt[NX];
    float pe[16];
    u32x4 pk[2];
    uint8_t* pb = smem + p_lds + pbi * 4 * kPBlock;
    auto read_xt = [&](int x) {
      const int s2 = x / DB, c = x % DB;
      const int o = st * QT + 16 * s2 * RB;
      xt[x] = lds_tr_pair(smem + tr_lo[c] + o, smem + tr_hi[c] + o);
    };
    auto xt_slot = [&](int x) { return NS + x - XL; };
#pragma unroll
    for (int s = 0; s < KD; ++s)
      if (s - KL < 0) aq[s] = pre[s];
#pragma unroll
    for (int x = 0; x < NX; ++x)
      if (xt_slot(x) < 0) read_xt(x);
    nx = f32x16{};
#pragma unroll
    for (int i = 0; i < NM; ++i) {
#pragma unroll
      for (int s = 0; s < KD; ++s)
        if (s - KL == i && i >= 0) aq[s] = ld128(row_lds[s] + st1 * QT);
      if (i == kIssSlot && j + 4 < n_it) issue((st + 4) % STAGES);
      if (i == kPreSlot) {
#pragma unroll
        for (int s = 0; s < KLP; ++s) pre[s] = ld128(row_lds[s] + ((st1 + 1) % STAGES) * QT);
      }
#pragma unroll
      for (int x = 0; x < NX; ++x)
        if (xt_slot(x) == i) read_xt(x);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (lv_slot(q) == i) lv[q] = ldf4(stat_lds + st * kStatStage + 32 * q);
      if (i < NS) {
        nx = mfma32<T>(aq[i], kv[i], nx);
      } else {
        const int a = i - NS;
        acc[a % DB] = mfma32<T>(xt[a], pk[a / DB], acc[a % DB]);
      }
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const int f = pf(g);
        float* e = pe;
        if (f == i) {
          e[2 * g] = fmaf(sc[2 * g], c_log2, -lse_r(2 * g));
          e[2 * g + 1] = fmaf(sc[2 * g + 1], c_log2, -lse_r(2 * g + 1));
        }
        if (f + 1 == i) {
          e[2 * g] = fast_exp2(e[2 * g]);
          e[2 * g + 1] = fast_exp2(e[2 * g + 1]);
        }
        if (f + 2 == i) pk[g >> 2][g & 3] = pack2<T>(e[2 * g], e[2 * g + 1]);
        // P (fp32) of elements 4k..4k+3 goes to LDS for role 1 once both
        // pairs are exponentiated.
        if ((g & 1) && f + 2 == i)
          *reinterpret_cast<f32x4*>(pb + 1024 * (g >> 1)) =
              f32x4{e[2 * g - 2], e[2 * g - 1], e[2 * g], e[2 * g + 1]};
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    cur_m0 += BMQ;
    if (cur_m0 >= p.Sq) {
      cur_m0 = m_begin;
      ++cur_gi;
    }
  };
  // Role 1: tile j in stage st (dO(j) rows: dP(j) into dn), tile j-1 in
  // stage stp (Q(j-1)^T, delta(j-1)), P(j-1) in buffer pbp; dpv holds dP(j-1).
  // dprev: the packed dS of tile j-2, stored here before this step's DMA
  // issue (so no store is issued after a tile load whose wait comes first:
  // one counter covers loads and stores, and they may complete out of
  // order); receives dS(j-1).
  auto body1 = [&](int j, int st, int stp, int pbp, const f32x16& dpv, f32x16& dn,
                   u32x4 (&dprev)[2]) SK_INLINE {
    if (SK_BWD_FIVE_GEMM && j >= 2) store_ds(dprev);
    const uint8_t* pb = smem + p_lds + pbp * 4 * kPBlock;
    f32x4 pr[4], dv[4];
    auto pr_slot = [&](int q) { return pf(2 * q) + 1 - SL; };
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (pr_slot(q) < 0) dv[q] = ldf4(stat_lds + stp * kStatStage + 32 * q);
    auto delta_r = [&](int r) { return dv[r / 4][r % 4]; };
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (pr_slot(q) < 0) pr[q] = *reinterpret_cast<const f32x4*>(pb + 1024 * q);
    u32x4 ad[KD];
    u32x4 xq[NX];
    float de[16];
    u32x4 dsk[2];
    auto read_xq = [&](int x) {
      const int s2 = x / DB, c = x % DB;
      const int o = stp * QT + 16 * s2 * RB;
      xq[x] = lds_tr_pair(smem + tr_lo[c] + o, smem + tr_hi[c] + o);
    };
    auto xq_slot = [&](int x) { return NS + x - XL; };
#pragma unroll
    for (int s = 0; s < KD; ++s)
      if (s - KL < 0) ad[s] = pre[s];
#pragma unroll
    for (int x = 0; x < NX; ++x)
      if (xq_slot(x) < 0) read_xq(x);
    dn = f32x16{};
#pragma unroll
    for (int i = 0; i < NM; ++i) {
#pragma unroll
      for (int s = 0; s < KD; ++s)
        if (s - KL == i && i >= 0) ad[s] = ld128(row_lds[s] + st * QT);
      if (i == kIssSlot && j + 4 < n_it) issue((st + 4) % STAGES);
      if (i == kPreSlot) {
#pragma unroll
        for (int s = 0; s < KLP; ++s) pre[s] = ld128(row_lds[s] + ((st + 1) % STAGES) * QT);
      }
#pragma unroll
      for (int x = 0; x < NX; ++x)
        if (xq_slot(x) == i) read_xq(x);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (pr_slot(q) == i) dv[q] = ldf4(stat_lds + stp * kStatStage + 32 * q);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (pr_slot(q) == i) pr[q] = *reinterpret_cast<const f32x4*>(pb + 1024 * q);
      if (i < NS) {
        dn = mfma32<T>(ad[i], kv[i], dn);
      } else {
        const int a = i - NS;
        acc[a % DB] = mfma32<T>(xq[a], dsk[a / DB], acc[a % DB]);
      }
#pragma unroll
      for (int g = 0; g < 8; ++g) {
        const int f = pf(g) + 1;
        if (f == i) {
#pragma unroll
          for (int e = 0; e < 2; ++e) {
            const int x = 2 * g + e;
            de[x] = pr[x >> 2][x & 3] * (dpv[x] - delta_r(x));
          }
        }
        if (f + 1 == i) dsk[g >> 2][g & 3] = pack2<T>(de[2 * g], de[2 * g + 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (SK_BWD_FIVE_GEMM) {
      dprev[0] = dsk[0];
      dprev[1] = dsk[1];
    }
  };
  // Each role runs its own copy of the step loop (the same barriers in the
  // same order).  role_body(st, par) runs step j >= 1 with tile j in stage
  // st and par = j & 1.
  f32x16 sv[2];  // role 0: S of even / odd tiles; role 1: dP of even / odd tiles
  auto run_v2 = [&](auto role_body) SK_INLINE {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (t < n_it) issue(t);
    begin_v2(0);
    sv[0] = score(0);
    // first row operands of the next body: role 0's S(1) reads Q(1), role
    // 1's dP(1) reads dO(1), both in stage 1
#pragma unroll
    for (int s = 0; s < KLP; ++s) pre[s] = ld128(row_lds[s] + QT);
    if (role == 0)
      body0(0, 0, 1, 0, sv[0], sv[1]);
    else if (4 < n_it)
      issue(4);
    for (int j0 = 1; j0 < n_it; j0 += STAGES) {
#pragma unroll
      for (int u = 0; u < STAGES; ++u) {
        const int j = j0 + u;
        if (j >= n_it) break;
        begin_v2(j);
        role_body(j, (1 + u) % STAGES, (1 + u) & 1);  // j % 6, j & 1
      }
    }
    __syncthreads();  // role 0's P of the last tile
  };
  auto run_v2_roles = [&]() {
    if (role == 0) {
      run_v2([&](int j, int st, int par) SK_INLINE {
        body0(j, st, (st + 1) % STAGES, par, sv[par], sv[par ^ 1]);
      });
      return;
    }
    u32x4 dprev[2];
    run_v2([&](int j, int st, int par) SK_INLINE {
      body1(j, st, (st + STAGES - 1) % STAGES, par ^ 1, sv[par ^ 1], sv[par], dprev);
    });
    if (SK_BWD_FIVE_GEMM && n_it >= 2) store_ds(dprev);  // dS of tile n_it - 2
    // dS and dK^T of the last tile (stage chosen at run time; the dP
    // register set by a branch, so both sets stay in registers)
    const int jl = n_it - 1;
    const int stp = jl % STAGES;
    auto tail = [&](f32x16& dpv, int pbi) SK_INLINE {
      const uint8_t* pb = smem + p_lds + pbi * 4 * kPBlock;
      f32x4 dv[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) dv[k] = ldf4(stat_lds + stp * kStatStage + 32 * k);
      float de[16];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const f32x4 pr = *reinterpret_cast<const f32x4*>(pb + 1024 * k);
#pragma unroll
        for (int e = 0; e < 4; ++e) de[4 * k + e] = pr[e] * (dpv[4 * k + e] - dv[k][e]);
      }
      u32x4 dsk[2];
      pack16(de, dsk);
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
        for (int c = 0; c < DB; ++c) {
          const int o = stp * QT + 16 * s2 * RB;
          const u32x4 x = lds_tr_pair(smem + tr_lo[c] + o, smem + tr_hi[c] + o);
          acc[c] = mfma32<T>(x, dsk[s2], acc[c]);
        }
      if (SK_BWD_FIVE_GEMM) store_ds(dsk);
    };
    if (jl & 1)
      tail(sv[1], 1);
    else
      tail(sv[0], 0);
  };

  // 4-deep schedule: each role runs its own copy of the step loop (the same
  // barriers in the same order), so its accumulators stay in place.
  auto run = [&](auto role_step) {
    issue(0);
    if (n_it > 1) issue(1);
    begin_step(0, PD);
    role_step(0, -1);
    for (int j0 = 1; j0 < n_it; j0 += STAGES) {
#pragma unroll
      for (int u = 0; u < STAGES; ++u) {
        const int j = j0 + u;
        if (j >= n_it) break;
        const int stg = (1 + u) % STAGES;  // j % 4
        begin_step(j, (stg + PD) % STAGES);
        role_step(stg, (stg + STAGES - 1) % STAGES);
      }
    }
    __syncthreads();  // role 0's P of the last tile
  };
  if constexpr (kV2) {
    if (n_it > 0) run_v2_roles();
  } else if (n_it > 0) {
    if (role == 0) {
      run([&](int stg, int) { step0(stg, stg & 1); });
    } else {
      run([&](int stg, int prev) {
        if (prev >= 0) step1(prev, prev & 1);
        if (kSkew) dp = score(stg);
      });
      step1((n_it - 1) % STAGES, (n_it - 1) & 1);
    }
  }

  const float osc = role == 0 ? 1.f : p.scale;
  if (key >= p.Sk) return;
  const int64_t krow = ((int64_t)bk * p.Sk + key) * p.D;
  uint16_t* outp = (uint16_t*)(role == 0 ? p.dv : p.dk) + krow;
#pragma unroll
  for (int c = 0; c < DB; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = d_out0 + 32 * c + 8 * i + 4 * hl;
      if (d < p.D) {
        const f32x16& a = acc[c];
        *reinterpret_cast<u32x2*>(outp + d) =
            u32x2{pack2<T>(a[4 * i] * osc, a[4 * i + 1] * osc),
                  pack2<T>(a[4 * i + 2] * osc, a[4 * i + 3] * osc)};
      }
    }
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
template <class T, int DP, int BN, int NW, int STAGES, int OCC, int MODE, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64, OCC) bwd_dq_kernel(BwdParams p) {
  static_assert(MODE == 0 || MODE == 2, "dQ schedule: 0 (tiles in order) or 2");
  using L = BwdTile<DP, BN>;  // K and V tiles
  constexpr int BM = 32 * NW;
  constexpr int KD = DP / 16;  // k-steps over the head dim (S^T, dP^T)
  constexpr int KB = BN / 32;  // 32-key blocks per tile
  constexpr int DB = DP / 32;  // 32-wide head-dim blocks of dQ^T
  constexpr int KN = BN / 16;  // k-steps over keys (dQ^T)
  constexpr int LK = L::kSegs / NW;
  constexpr int kStageBytes = 2 * L::kTileBytes;  // K tile, then V tile
  constexpr int PD = STAGES - 2;
  constexpr int RB = L::kRowBytes;
  static_assert(L::kSegs % NW == 0, "tile segments must divide over the waves");
  static_assert(PD >= 1 && PD <= 2, "prefetch distance");
  static_assert((STAGES & (STAGES - 1)) == 0, "the ring index is a mask");

  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * kStageBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  // Work item: (batch, query head) major, heaviest query block first.
  const int w = xcd_work_index(blockIdx.x, gridDim.x);
  const int bh = w / p.n_mblocks;
  const int mblk = p.n_mblocks - 1 - (w - bh * p.n_mblocks);
  const int b = bh / p.Hq;
  const int hkv = (bh - b * p.Hq) / p.group;
  const int m0 = mblk * BM;
  const int mw = m0 + 32 * wave;
  const int row = mw + l32;
  const int diag = p.Sk - p.Sq;

  const int64_t kv0 = ((int64_t)b * p.Hkv + hkv) * p.Sk * p.D;
  const uint16_t* kbase = (const uint16_t*)p.k + kv0;
  const uint16_t* vbase = (const uint16_t*)p.v + kv0;

  uint32_t goff[LK];
#pragma unroll
  for (int j = 0; j < LK; ++j) {
    const int seg = wave + j * NW;
    const int r = seg * L::kSegRows + lane / L::kCpr;
    const int c = (lane % L::kCpr) ^ swz_rt<DP>(r);
    goff[j] = c * 8 < p.D ? (uint32_t)((r * p.D + c * 8) * 2) : kBufferOob;
  }
  auto issue_tile = [&](int t) {
    const int n0 = t * BN;
    const int bytes = tile_bytes(min(BN, p.Sk - n0), p.D, p.D);
    const i32x4 kr = make_rsrc_words(kbase + (int64_t)n0 * p.D, bytes);
    const i32x4 vr = make_rsrc_words(vbase + (int64_t)n0 * p.D, bytes);
    const uint32_t st = lds_addr(smem) + (t & (STAGES - 1)) * kStageBytes;
#pragma unroll
    for (int j = 0; j < LK; ++j) {
      const int seg = wave + j * NW;
      buffer_load_lds_b128(kr, st + seg * 1024, goff[j]);
      buffer_load_lds_b128(vr, st + L::kTileBytes + seg * 1024, goff[j]);
    }
  };

  // Q (sign-flipped for a negative scale) and dO rows as the B operand:
  // lane holds q[row][16*s + 8*hl .. +7] (zero past S_q and D).
  u32x4 qreg[KD], greg[KD];
  {
    const int qrows = max(0, min(32, p.Sq - mw));
    const int64_t q0 = ((int64_t)bh * p.Sq + min(mw, p.Sq)) * p.D;
    // Wave-uniform; readfirstlane keeps the resource in SGPRs (no waterfall loop).
    const int bytes = __builtin_amdgcn_readfirstlane(tile_bytes(qrows, p.D, p.D));
    const buf_rsrc qr = make_rsrc((const uint16_t*)p.q + q0, bytes);
    const buf_rsrc gr = make_rsrc((const uint16_t*)p.dout + q0, bytes);
#pragma unroll
    for (int s = 0; s < KD; ++s) {
      const int d0 = 16 * s + 8 * hl;
      const uint32_t off = d0 < p.D ? (uint32_t)((l32 * p.D + d0) * 2) : kBufferOob;
      qreg[s] = buffer_load_b128(qr, off) ^ p.op_sign;
      greg[s] = buffer_load_b128(gr, off);
    }
  }
  float lse2 = __builtin_inff(), dl = 0.f;
  if (row < p.Sq) {
    lse2 = p.lse_log2[(int64_t)bh * p.Sq + row];
    dl = p.delta[(int64_t)bh * p.Sq + row];
  }

  int n_end = p.Sk;
  if (CAUSAL) n_end = min(p.Sk, m0 + BM + diag);
  const int n_tiles = n_end > 0 ? (n_end + BN - 1) / BN : 0;

#pragma unroll
  for (int t = 0; t <= PD; ++t)
    if (t < n_tiles) issue_tile(t);

  f32x16 dqacc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) dqacc[c] = f32x16{};

  // Row-wise A operand of S^T / dP^T: key row l32 (+32 kb), chunk 2s + hl.
  int k_lds[KD];
#pragma unroll
  for (int s = 0; s < KD; ++s) k_lds[s] = l32 * RB + (((2 * s + hl) ^ swz_rt<DP>(l32)) * 16);
  int kt_lo[DB], kt_hi[DB];
  tr_offsets<DP, DB>(lane, 0, kt_lo, kt_hi);

  const float c_log2 = p.abs_scale_log2;
  auto stage = [&](int t) { return smem + (t & (STAGES - 1)) * kStageBytes; };
  auto sync_tile = [&](int t, int max_ahead) {
    wait_tiles<2 * LK, PD>(min(max_ahead, n_tiles - 1 - t));
    __syncthreads();
  };

  // S^T = K Q^T and dP^T = V dO^T of tile t (no interleave): lane holds
  // [key t*BN + 32*kb + 8*(r/4) + 4*hl + r%4][query row].
  auto gemm_sdp = [&](int t, f32x16 (&sd)[KB], f32x16 (&pd)[KB]) {
    const uint8_t* st = stage(t);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      sd[kb] = f32x16{};
      pd[kb] = f32x16{};
    }
#pragma unroll
    for (int s = 0; s < KD; ++s)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        sd[kb] = mfma32<T>(lds_b128(st + k_lds[s] + kb * 32 * RB), qreg[s], sd[kb]);
        pd[kb] = mfma32<T>(lds_b128(st + L::kTileBytes + k_lds[s] + kb * 32 * RB), greg[s], pd[kb]);
      }
  };

  // Keys past S_k and, under the causal mask, keys past row + diag -> -inf.
  auto premask = [&](int t, f32x16 (&sd)[KB]) {
    const int n0 = t * BN;
    const bool tail = n0 + BN > p.Sk;
    const bool straddle = CAUSAL && (n0 + BN - 1 > mw + diag);
    if (!(tail || straddle)) return;
    int lim = p.Sk - 1;
    if (CAUSAL) lim = min(lim, row + diag);
    lim -= n0 + 4 * hl;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (32 * kb + 8 * (r >> 2) + (r & 3) > lim) sd[kb][r] = kNegInf;
  };

  // dS^T of one element, packed eight at a time into the B operand of k-step
  // x / 8 (keys permuted as the transposed K reads are).
  u32x4 dsk[KN];
  float de[KN * 8];
  auto elem = [&](int x, const f32x16 (&sd)[KB], const f32x16 (&pd)[KB]) {
    const int kb = x >> 4, r = x & 15;
    const float pe = fast_exp2(fmaf(sd[kb][r], c_log2, -lse2));
    de[x] = pe * (pd[kb][r] - dl);
    if ((x & 7) == 7) {
      const int b8 = x - 7;
      dsk[x >> 3] = u32x4{pack2<T>(de[b8], de[b8 + 1]), pack2<T>(de[b8 + 2], de[b8 + 3]),
                          pack2<T>(de[b8 + 4], de[b8 + 5]), pack2<T>(de[b8 + 6], de[b8 + 7])};
    }
  };
  auto tile_valu = [&](const f32x16 (&sd)[KB], const f32x16 (&pd)[KB]) {
#pragma unroll
    for (int x = 0; x < KN * 8; ++x) elem(x, sd, pd);
  };

  // Stage B: dQ^T += K^T dS^T for tile t: lane holds
  // [d 32*c + 8*(r/4) + 4*hl + r%4][query row].
  auto gemm_dq = [&](int t) {
    const uint8_t* st = stage(t);
    constexpr int NM = DB * KN;
    constexpr int OLEAD = NM < 5 ? NM : 5;
    u32x4 kt[KN][DB];
#pragma unroll
    for (int s2 = 0; s2 < KN; ++s2)
#pragma unroll
      for (int c = 0; c < DB; ++c)
        kt[s2][c] = lds_tr_pair(st + 16 * s2 * RB + kt_lo[c], st + 16 * s2 * RB + kt_hi[c]);
#pragma unroll
    for (int s2 = 0; s2 < KN; ++s2)
#pragma unroll
      for (int c = 0; c < DB; ++c) dqacc[c] = mfma32<T>(kt[s2][c], dsk[s2], dqacc[c]);
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * OLEAD, 0);
#pragma unroll
    for (int i = 0; i < NM - OLEAD; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, OLEAD, 0);
  };

  // Every tile runs the same straight-line code.  Keys a wave cannot see
  // (past its rows' diagonal or past S_k) are masked, not skipped: their dS
  // is exactly zero.  Waves with no rows (past S_q) compute unused values.
  f32x16 s0[KB], p0[KB], s1[KB], p1[KB];
  if constexpr (MODE == 2) {
    // S^T one tile ahead, dP^T in step: step t runs the dP^T MFMAs of tile t
    // with P(t) = exp2(S^T(t)...) between them, then the S^T MFMAs of tile
    // t+1 with dS(t) = P(t) (dP(t) - delta) between them, then dQ^T += K^T
    // dS^T of tile t, its transposed K reads XL slots ahead.  Three score
    // tiles are live (S^T of t and t+1, dP^T of t) instead of four.
    static_assert(KB == 1, "one 32-key block per tile");
    constexpr int NP = KD;           // dP^T MFMAs (slots 0 .. NP-1)
    constexpr int NSN = KD;          // S^T MFMAs of the next tile
    constexpr int NQ = DB * KN;      // dQ^T MFMAs
    constexpr int KL = SK_DQ_KL, XL = SK_DQ_XL;
    constexpr int NE = KN * 8;       // elements per lane and tile
    // element x: FMA at pa(x), exp2 at pa(x) + 1; dS at pb(x); pack of
    // elements 8g..8g+7 one slot after the last of them
    auto pa = [](int x) { return (x * NP) / NE; };
    auto pb = [](int x) { return NP + 1 + (x * (NSN + DB - 5)) / NE; };
    auto pk_slot = [&](int g) { return pb(8 * g + 7) + 1; };
    static_assert(NE == 16 && KN == 2, "two packed k-steps per tile");
    // P(t) overwrites S^T(t) and dS(t) overwrites dP^T(t) in place.
    // su = t % STAGES, a compile-time constant in the unrolled loop, so every
    // LDS address is a lane-constant register plus an immediate.
    auto body = [&](int su, f32x16& cs, f32x16& ns, bool next) SK_INLINE {
      const uint8_t* st = smem + su * kStageBytes;
      const uint8_t* sn = smem + ((su + 1) & (STAGES - 1)) * kStageBytes;
      f32x16 dp = f32x16{};
      u32x4 a[NP + NSN];
      u32x4 kt[NQ];
      auto addr = [&](int i) {
        return i < NP ? st + L::kTileBytes + k_lds[i] : sn + k_lds[i - NP];
      };
      auto read_kt = [&](int m) {
        const int s2 = m / DB, c = m % DB;
        kt[m] = lds_tr_pair(st + 16 * s2 * RB + kt_lo[c], st + 16 * s2 * RB + kt_hi[c]);
      };
#pragma unroll
      for (int i = 0; i < KL; ++i) a[i] = lds_b128(addr(i));
      ns = f32x16{};
#pragma unroll
      for (int i = 0; i < NP + NSN + NQ; ++i) {
        if (i + KL < NP + NSN && (next || i + KL < NP)) a[i + KL] = lds_b128(addr(i + KL));
#pragma unroll
        for (int m = 0; m < NQ; ++m)
          if (NP + NSN + m - XL == i) read_kt(m);
        if (i < NP) {
          dp = mfma32<T>(a[i], greg[i], dp);
        } else if (i < NP + NSN) {
          if (next) ns = mfma32<T>(a[i], qreg[i - NP], ns);
        } else {
          const int m = i - NP - NSN, s2 = m / DB, c = m % DB;
          dqacc[c] = mfma32<T>(kt[m], dsk[s2], dqacc[c]);
        }
#pragma unroll
        for (int x = 0; x < NE; ++x) {
          if (pa(x) == i) cs[x] = fmaf(cs[x], c_log2, -lse2);
          if (pa(x) + 1 == i) cs[x] = fast_exp2(cs[x]);
          if (pb(x) == i) dp[x] = cs[x] * (dp[x] - dl);
        }
#pragma unroll
        for (int g = 0; g < 2; ++g)
          if (pk_slot(g) == i)
            dsk[g] = u32x4{pack2<T>(dp[8 * g], dp[8 * g + 1]), pack2<T>(dp[8 * g + 2], dp[8 * g + 3]),
                           pack2<T>(dp[8 * g + 4], dp[8 * g + 5]), pack2<T>(dp[8 * g + 6], dp[8 * g + 7])};
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    static_assert(pb(7) + 1 < NP + NSN && pb(15) + 1 < NP + NSN + DB,
                  "dS^T packed before its dQ^T MFMAs");
    if (n_tiles > 0) {
      sync_tile(0, PD);
      s0[0] = f32x16{};
#pragma unroll
      for (int s = 0; s < KD; ++s) s0[0] = mfma32<T>(lds_b128(stage(0) + k_lds[s]), qreg[s], s0[0]);
    }
    // Tiles with a successor run in a loop unrolled by the ring depth; the
    // last tile (no S^T ahead) runs once after it, its stage and score
    // registers chosen at run time.
    auto iteration = [&](int t, int su, f32x16 (&cs)[KB], f32x16 (&ns)[KB]) SK_INLINE {
      premask(t, cs);
      sync_tile(t + 1, PD - 1);
      if (t + 1 + PD < n_tiles) issue_tile(t + 1 + PD);
      body(su, cs[0], ns[0], true);
    };
    const int n_main = n_tiles - 1;
    for (int t0 = 0; t0 < n_main; t0 += STAGES) {
#pragma unroll
      for (int u = 0; u < STAGES; ++u) {
        if (t0 + u >= n_main) break;
        if (u & 1)
          iteration(t0 + u, u, s1, s0);
        else
          iteration(t0 + u, u, s0, s1);
      }
    }
    if (n_main >= 0) {
      auto last = [&](f32x16 (&cs)[KB], f32x16 (&ns)[KB]) SK_INLINE {
        premask(n_main, cs);
        body(n_main & (STAGES - 1), cs[0], ns[0], false);
      };
      if (n_main & 1)
        last(s1, s0);
      else
        last(s0, s1);
    }
  } else {
    // Tiles in order without the interleave: the other resident wave of the
    // SIMD (two workgroups per CU), or at D = 256 nothing, overlaps the VALU
    // work with MFMAs; one score tile is live.  Loads run PD + 1 tiles ahead.
    (void)s1;
    (void)p1;
    for (int t = 0; t < n_tiles; ++t) {
      sync_tile(t, PD);
      if (t + PD + 1 < n_tiles) issue_tile(t + PD + 1);
      gemm_sdp(t, s0, p0);
      premask(t, s0);
      tile_valu(s0, p0);
      gemm_dq(t);
    }
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

// dQ of the five-GEMM backward (bwd_dq_ds_kernel): dQ^T += K^T dS^T over the
// dS tiles the dK/dV kernel stored, so S and dP are computed once per
// (query tile, key tile) instead of twice.  A workgroup of 4 waves owns
// 32 x QW x 4 query rows of one (b, h_q), QW query tiles of 32 per wave;
// 32-key K tiles and each wave's 2 KiB dS tiles of the same keys stream
// through an LDS ring, STAGES - 2 tiles ahead.  K^T is read transposed from
// the K tile and dS^T transposed from the key-major dS tile with the same key
// order in the MFMA's k-slots (keys 4 hl + {0..3} and 8 + 4 hl + {0..3} of
// each 16-key step), so the lane of query l32 holds its 8 dS values of a
// k-step as the B operand, and each K^T read feeds QW MFMAs.  The dK/dV
// kernel writes the dS tiles of every 128-key block from the first query
// tile that can see the block (the dS tile layout); a wave reads a tile only
// if its query tile lies in that range (else the DMA is empty and the tile
// reads as zeros).  dS of keys past S_k is stored as zeros and meets K rows
// that read as zeros.
// dQ-from-dS tile: query tiles of 32 per wave, ring depth, workgroups per
// CU.  Two query tiles per wave let each K^T operand read feed two MFMAs and
// halve the steps (each closed by a workgroup barrier) per query: at C3 the
// backward ran 1.549 ms with 2,3,2, 1.555 with 2,6,1, 1.645 with 1,5,2.
#ifndef SK_BWD_DQDS_TILE
#define SK_BWD_DQDS_TILE 2, 3, 2
#endif
struct DqDsTile {
  int qw, stages, occ;
};
constexpr DqDsTile kDqDs{SK_BWD_DQDS_TILE};

template <class T, int DP, int QW, int STAGES, int OCC, bool CAUSAL>
__global__ void __launch_bounds__(256, OCC) bwd_dq_ds_kernel(BwdParams p) {
  constexpr int NW = 4;
  constexpr int BN = 32;
  constexpr int PD = STAGES - 2 >= 1 ? STAGES - 2 : 1;  // tiles issued ahead
  static_assert(STAGES >= 3, "a ring of at least three stages");
  using L = BwdTile<DP, BN>;  // K tiles
  constexpr int BM = 32 * QW * NW;
  constexpr int DB = DP / 32;  // 32-wide head-dim blocks of dQ^T
  constexpr int KN = BN / 16;  // k-steps over keys
  constexpr int LK = L::kSegs / NW;
  constexpr int kDs = 2048;  // one 32-query dS tile
  constexpr int kStageBytes = L::kTileBytes + NW * QW * kDs;
  constexpr int kLoads = LK + 2 * QW;  // DMAs per wave per tile
  constexpr int RB = L::kRowBytes;
  static_assert(L::kSegs % NW == 0, "tile segments must divide over the waves");
  static_assert(KN == 2 && DB <= 4, "32-key tiles, D <= 128");
  static_assert(STAGES * kStageBytes * OCC <= 160 * 1024, "workgroups per CU must fit the LDS");
  static_assert(kLoads * (PD - 1) < 64, "vmcnt range");

  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * kStageBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hl = lane >> 5;

  // Work item: (batch, query head) major, heaviest query block first, over
  // the query heads of the launch's (batch, KV head) pairs.
  const int w = xcd_work_index(blockIdx.x, gridDim.x);
  const int bhl = w / p.n_mblocks;  // query head within this launch
  const int bh = p.bk0 * p.group + bhl;
  const int mblk = p.n_mblocks - 1 - (w - bhl * p.n_mblocks);
  const int b = bh / p.Hq;
  const int hkv = (bh - b * p.Hq) / p.group;
  const int m0 = mblk * BM;
  const int mw = m0 + 32 * QW * wave;  // first query row of this wave
  const int diag = p.Sk - p.Sq;

  const uint16_t* kbase = (const uint16_t*)p.k + ((int64_t)b * p.Hkv + hkv) * p.Sk * p.D;
  uint32_t goff[LK];
#pragma unroll
  for (int j = 0; j < LK; ++j) {
    const int seg = wave + j * NW;
    const int r = seg * L::kSegRows + lane / L::kCpr;
    const int c = (lane % L::kCpr) ^ swz_rt<DP>(r);
    goff[j] = c * 8 < p.D ? (uint32_t)((r * p.D + c * 8) * 2) : kBufferOob;
  }
  // This wave's dS tiles: query tile qt = mw / 32 + q; key tile t = 4 kb + j
  // of it at tile 4 off(kb) + j cnt(kb) + qt - qb(kb) of the head (the dS
  // tile layout), written iff qt >= qb(kb), i.e. iff a row of the query tile
  // sees key 128 kb.  The key block's terms are scalars, recomputed by
  // issue_tile when t enters a new key block (it is called for t = 0, 1, 2,
  // ... in order).
  const uint8_t* ds_head = (const uint8_t*)p.ds + (int64_t)bhl * p.ds_head_tiles * kDs;
  const int qt0 = mw >> 5;
  const int q_rows = mw < p.Sq ? min(QW, (p.Sq - mw + 31) >> 5) : 0;  // query tiles in range
  int cur_kb = -1, cur_cnt = 0, cur_qb = 0;
  int64_t cur_off = 0;
  // The dS tile lands in LDS key-major (row r, queries 8 m .. 8 m + 7 at byte
  // 64 r + 16 m); DMA h, lane i fills chunk c = 64 h + i, i.e. (r, m) =
  // (c / 4, c % 4), stored by the dK/dV kernel at 1024 (m % 2) + 16 (r + 32
  // (m / 2)).
  uint32_t ds_goff[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = 16 * h + (lane >> 2), m = lane & 3;
    ds_goff[h] = (uint32_t)(1024 * (m & 1) + 16 * (r + 32 * (m >> 1)));
  }
  const uint32_t lds0 = lds_addr(smem);
  auto issue_tile = [&](int t) {
    const int n0 = t * BN;
    const int bytes = tile_bytes(min(BN, p.Sk - n0), p.D, p.D);
    const i32x4 kr = make_rsrc_words(kbase + (int64_t)n0 * p.D, bytes);
    const uint32_t st = lds0 + (t % STAGES) * kStageBytes;
#pragma unroll
    for (int j = 0; j < LK; ++j) buffer_load_lds_b128(kr, st + (wave + j * NW) * 1024, goff[j]);
    if ((t >> 2) != cur_kb) {
      cur_kb = t >> 2;
      cur_off = 4 * ds_off(cur_kb, p.ds_nqt, p.ds_c, CAUSAL);
      cur_cnt = ds_cnt(cur_kb, p.ds_nqt, p.ds_c, CAUSAL);
      cur_qb = ds_qb(cur_kb, p.ds_c, CAUSAL);
    }
#pragma unroll
    for (int q = 0; q < QW; ++q) {
      const int rel = qt0 + q - cur_qb;
      const bool ok = q < q_rows && rel >= 0;
      const int64_t tile = ok ? cur_off + (int64_t)(t & 3) * cur_cnt + rel : 0;
      const i32x4 dr = make_rsrc_words(ds_head + tile * kDs, ok ? kDs : 0);
      const uint32_t sd = st + L::kTileBytes + (wave * QW + q) * kDs;
      if constexpr (SK_BWD_DS_NT & 2) {
        buffer_load_lds_b128_nt(dr, sd, ds_goff[0]);
        buffer_load_lds_b128_nt(dr, sd + 1024, ds_goff[1]);
      } else {
        buffer_load_lds_b128(dr, sd, ds_goff[0]);
        buffer_load_lds_b128(dr, sd + 1024, ds_goff[1]);
      }
    }
  };

  int n_end = p.Sk;
  if (CAUSAL) n_end = min(p.Sk, m0 + BM + diag);
  const int n_tiles = n_end > 0 ? (n_end + BN - 1) / BN : 0;
#pragma unroll
  for (int t = 0; t < PD; ++t)
    if (t < n_tiles) issue_tile(t);

  f32x16 dqacc[QW][DB];
#pragma unroll
  for (int q = 0; q < QW; ++q)
#pragma unroll
    for (int c = 0; c < DB; ++c) dqacc[q][c] = f32x16{};
  // K^T: transposed reads of the K tile (head-dim block c); dS^T: transposed
  // reads of each dS tile, rows 4 hl + j16 / 4 (+8), columns lane % 32.
  int kt_lo[DB], kt_hi[DB];
  tr_offsets<DP, DB>(lane, 0, kt_lo, kt_hi);
  const int j16 = lane & 15;
  const int ds_lo = L::kTileBytes + wave * QW * kDs + (4 * hl + (j16 >> 2)) * 64 +
                    32 * ((lane >> 4) & 1) + 8 * (j16 & 3);

  for (int t = 0; t < n_tiles; ++t) {
    wait_tiles<kLoads, PD - 1>(min(PD - 1, n_tiles - 1 - t));  // tile t landed
    __syncthreads();  // ... for every wave; every read of the stage refilled next retired
    if (t + PD < n_tiles) issue_tile(t + PD);
    const uint8_t* st = smem + (t % STAGES) * kStageBytes;
    u32x4 kt[KN][DB], dst[QW][KN];
#pragma unroll
    for (int s2 = 0; s2 < KN; ++s2) {
#pragma unroll
      for (int q = 0; q < QW; ++q)
        dst[q][s2] = lds_tr_pair(st + ds_lo + q * kDs + 1024 * s2, st + ds_lo + q * kDs + 512 + 1024 * s2);
#pragma unroll
      for (int c = 0; c < DB; ++c)
        kt[s2][c] = lds_tr_pair(st + 16 * s2 * RB + kt_lo[c], st + 16 * s2 * RB + kt_hi[c]);
    }
#pragma unroll
    for (int s2 = 0; s2 < KN; ++s2)
#pragma unroll
      for (int c = 0; c < DB; ++c)
#pragma unroll
        for (int q = 0; q < QW; ++q) dqacc[q][c] = mfma32<T>(kt[s2][c], dst[q][s2], dqacc[q][c]);
  }

#pragma unroll
  for (int q = 0; q < QW; ++q) {
    const int row = mw + 32 * q + (lane & 31);
    if (row < p.Sq) {
      uint16_t* dqp = (uint16_t*)p.dq + ((int64_t)bh * p.Sq + row) * p.D;
#pragma unroll
      for (int c = 0; c < DB; ++c)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 32 * c + 8 * i + 4 * hl;
          if (d < p.D) {
            const f32x16& a = dqacc[q][c];
            *reinterpret_cast<u32x2*>(dqp + d) =
                u32x2{pack2<T>(a[4 * i] * p.scale, a[4 * i + 1] * p.scale),
                      pack2<T>(a[4 * i + 2] * p.scale, a[4 * i + 3] * p.scale)};
          }
        }
    }
  }
}

// gfx950 tile table for the backward, by head dim (padded to 64, 128 or 256;
// other dims run zero-padded in the next size up):
//   dK/dV: 8 waves, one workgroup per CU, 128 keys per workgroup, 32-query
//          tiles (at D = 256 the output head dim is split over two
//          workgroups); LDS ring 6 x (Q + dO + stats) + P exchange
//          = 92 / 140 KiB at D = 64 / 128 (the pipelined schedule),
//          4 x (Q + dO + stats) + P exchange = 152 KiB at D = 256.
//   dQ:    4 waves, 128 query rows per workgroup, 32-key tiles; ring
//          4 x (K + V) = 32 / 64 / 128 KiB, so two workgroups fit a CU at
//          D <= 128.
// dQ kernel table by padded head dim: key tile, workgroups per CU, and the
// schedule of a wave's MFMA and VALU work.
// SK_BWD_DQ_TILE (key tile, workgroups per CU, schedule) overrides the
// D <= 128 row for candidate builds.  Schedules: 0 tiles in order (the other
// wave of the SIMD overlaps the VALU work), 2 S^T one tile ahead and dP^T in
// step.  (Schedule 1, S^T and dP^T both one tile ahead, was a slower
// candidate of the tile study and is no longer in the sources.)
#ifndef SK_BWD_DQ_TILE
#define SK_BWD_DQ_TILE 32, 2, 2
#endif
struct DqTile {
  int bn, occ, mode;
};
constexpr DqTile kDqSmall{SK_BWD_DQ_TILE};
template <int DP>
struct DqConfig {
  static constexpr int kBn = kDqSmall.bn;
  static constexpr int kOcc = kDqSmall.occ;
  static constexpr int kMode = kDqSmall.mode;
};
// SK_BWD_DQ_TILE_D256 overrides the D = 256 row (32 keys, one workgroup per
// CU, schedule 0) for candidate builds.
#ifndef SK_BWD_DQ_TILE_D256
#define SK_BWD_DQ_TILE_D256 32, 1, 0
#endif
constexpr DqTile kDq256{SK_BWD_DQ_TILE_D256};
template <>
struct DqConfig<256> {
  static constexpr int kBn = kDq256.bn;
  static constexpr int kOcc = kDq256.occ;
  static constexpr int kMode = kDq256.mode;
};

// (Batch, KV head) pairs a dK/dV or dQ-from-dS launch covers: a chunk of the
// five-GEMM backward, else all of them.
static int64_t launch_pairs(const BwdParams& p) {
  return p.n_pairs > 0 ? p.n_pairs : (int64_t)p.B * p.Hkv;
}

template <class T, int DP, int DO>
static KernelPlan plan_dkv_t(BwdParams& p, bool causal) {
  // D = 128 and D = 64: the 6-deep pipelined schedule (S one step ahead of
  // P; 3%-7% faster at D = 128, up to 10% at D = 64); SK_BWD_DKV_STAGES=4
  // and SK_BWD_DKV_STAGES_D64=4 build the 4-deep one-tile-per-step schedule
  // instead.  D = 256 keeps the 4-deep one (the 6-deep ring does not fit).
  constexpr int STAGES = DP == 128 ? SK_BWD_DKV_STAGES : DP == 64 ? SK_BWD_DKV_STAGES_D64 : 4;
  p.n_nblocks = (p.Sk + 127) / 128;
  KernelPlan k;
  k.fn = causal ? (const void*)bwd_dkv_kernel<T, DP, DO, STAGES, true>
                : (const void*)bwd_dkv_kernel<T, DP, DO, STAGES, false>;
  k.grid = dim3((unsigned)((int64_t)p.n_nblocks * launch_pairs(p) * (DP / DO)));
  k.block = dim3(512);
  k.kernel = "bwd_dkv_kernel";
  k.elem = T::code;
  k.head_dim = DP;
  k.block_m = 32;   // queries per streamed tile
  k.block_n = 128;  // keys per workgroup
  k.stages = STAGES;
  k.causal = causal;
  return k;
}

template <class T, int DP>
static KernelPlan plan_dq_t(BwdParams& p, bool causal) {
  constexpr int NW = 4;  // dQ waves per workgroup
  constexpr int STAGES = 4;
  using QC = DqConfig<DP>;
  p.n_mblocks = (p.Sq + 32 * NW - 1) / (32 * NW);
  KernelPlan k;
  k.fn = causal ? (const void*)bwd_dq_kernel<T, DP, QC::kBn, NW, STAGES, QC::kOcc, QC::kMode, true>
                : (const void*)bwd_dq_kernel<T, DP, QC::kBn, NW, STAGES, QC::kOcc, QC::kMode, false>;
  k.grid = dim3((unsigned)((int64_t)p.n_mblocks * p.B * p.Hq));
  k.block = dim3(NW * 64);
  k.kernel = "bwd_dq_kernel";
  k.elem = T::code;
  k.head_dim = DP;
  k.block_m = 32 * NW;
  k.block_n = QC::kBn;
  k.stages = STAGES;
  k.causal = causal;
  return k;
}

template <class T>
static KernelPlan plan_dkv_dt(BwdParams& p, bool causal) {
  if (p.D <= 64) return plan_dkv_t<T, 64, 64>(p, causal);
  if (p.D <= 128) return plan_dkv_t<T, 128, 128>(p, causal);
  if (p.D <= 256) return plan_dkv_t<T, 256, SK_BWD_DKV_DO_D256>(p, causal);
  return KernelPlan{};
}

template <class T>
static KernelPlan plan_dq_dt(BwdParams& p, bool causal) {
  if (p.D <= 64) return plan_dq_t<T, 64>(p, causal);
  if (p.D <= 128) return plan_dq_t<T, 128>(p, causal);
  if (p.D <= 256) return plan_dq_t<T, 256>(p, causal);
  return KernelPlan{};
}

KernelPlan plan_bwd_dkv(int dtype, BwdParams& p, bool causal) {
  if (dtype == BF16::code) return plan_dkv_dt<BF16>(p, causal);
  if (dtype == F16::code) return plan_dkv_dt<F16>(p, causal);
  if (dtype == 0) return plan_bwd_dkv_f32(p, causal);
  return KernelPlan{};
}

// The five-GEMM backward (dS tiles in the workspace) runs where the dK/dV
// kernel's pipelined schedule stores them: 16-bit inputs, padded head dim
// 128, 32 keys per wave.  Its tiles take 2 KiB per 32 x 32 (key, query)
// tile that a visible key block writes (the dS tile layout: about
// B * H_q * S_q * S_k bytes under a square causal mask, twice that without
// it); the caller's workspace sets how many (batch, KV head) pairs' tiles
// one dK/dV + dQ launch pair holds, and the pairs run in chunks of that size.
// It gives the seven-GEMM results bit for bit (the same dS values, summed
// into dQ in the same key order), whatever the chunking: the dS stores cost
// the dK/dV kernel about 8%, and the dQ pass, which no longer recomputes S
// and dP, runs after it instead of beside it.  C3 backward 4.7% faster, MHA
// S = 4096 1.8% faster (one box, alternating libraries).
size_t bwd_ds_pair_bytes(int dtype, int Hq, int Hkv, int Sq, int Sk, int D, bool causal) {
  if (!SK_BWD_FIVE_GEMM) return 0;
  if (dtype != BF16::code && dtype != F16::code) return 0;
  if (D <= 64 || D > 128 || SK_BWD_DKV_STAGES != 6) return 0;
  if (Hkv <= 0 || Sq <= 0 || Sk <= 0) return 0;
  const int nqt = (Sq + 31) / 32;
  const int c = ds_causal_c(Sq, Sk);
  const int64_t tiles = ds_head_tiles((Sk + 127) / 128, nqt, c, causal);
  return (size_t)(Hq / Hkv) * (size_t)tiles * 2048;
}

template <class T>
static KernelPlan plan_dq_ds_t(BwdParams& p, bool causal) {
  constexpr int NW = 4, QW = kDqDs.qw;
  p.n_mblocks = (p.Sq + 32 * QW * NW - 1) / (32 * QW * NW);
  KernelPlan k;
  k.fn = causal ? (const void*)bwd_dq_ds_kernel<T, 128, QW, kDqDs.stages, kDqDs.occ, true>
                : (const void*)bwd_dq_ds_kernel<T, 128, QW, kDqDs.stages, kDqDs.occ, false>;
  k.grid = dim3((unsigned)((int64_t)p.n_mblocks * launch_pairs(p) * p.group));
  k.block = dim3(NW * 64);
  k.kernel = "bwd_dq_ds_kernel";
  k.elem = T::code;
  k.head_dim = 128;
  k.block_m = 32 * QW * NW;
  k.block_n = 32;
  k.stages = kDqDs.stages;
  k.causal = causal;
  return k;
}

KernelPlan plan_bwd_dq(int dtype, BwdParams& p, bool causal) {
  if (p.ds != nullptr &&
      bwd_ds_pair_bytes(dtype, p.Hq, p.Hkv, p.Sq, p.Sk, p.D, causal) > 0)
    return dtype == BF16::code ? plan_dq_ds_t<BF16>(p, causal) : plan_dq_ds_t<F16>(p, causal);
  if (dtype == BF16::code) return plan_dq_dt<BF16>(p, causal);
  if (dtype == F16::code) return plan_dq_dt<F16>(p, causal);
  if (dtype == 0) return plan_bwd_dq_f32(p, causal);
  return KernelPlan{};
}

// Side streams for the dQ kernel, one per (device, caller stream), each with
// its own fork and join events, created on first use with the caller's device
// current (default priority) and kept until the process ends.  Keying by the
// caller's stream keeps callers apart: a backward launched on one stream
// never puts work on a side stream that another stream's call (possibly under
// graph capture, possibly on another thread) has pulled into its capture.
// Calls on one caller stream are already ordered by that stream; sharing its
// side stream and events among them is safe, because a wait on an event
// sees its latest record, which is at or after the calling thread's own.
namespace {
struct SideEntry {
  int dev = -1;
  hipStream_t caller = nullptr;
  hipStream_t side = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
constexpr int kMaxSides = 128;
std::mutex g_side_mu;
SideEntry g_side[kMaxSides];
int g_n_side = 0;
}  // namespace

// The side entry of caller stream s, or null (no fork: the one-stream order)
// when none exists and none can be made now: s is capturing (creating
// streams and events is not a stream operation, so a call under capture gets
// the one-stream order until an eager call on the same stream has made the
// entry), the table is full, or a HIP call fails.
static const SideEntry* side_entry(hipStream_t s) {
  hipDevice_t dev = -1;
  if (hipStreamGetDevice(s, &dev) != hipSuccess || dev < 0) return nullptr;
  std::lock_guard<std::mutex> lock(g_side_mu);
  for (int i = 0; i < g_n_side; ++i)
    if (g_side[i].dev == dev && g_side[i].caller == s) return &g_side[i];
  if (g_n_side == kMaxSides) return nullptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone)
    return nullptr;
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
  SideEntry e;
  e.dev = dev;
  e.caller = s;
  hipError_t err = hipStreamCreateWithFlags(&e.side, hipStreamNonBlocking);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&e.fork, hipEventDisableTiming);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&e.join, hipEventDisableTiming);
  if (err != hipSuccess) {
    if (e.join) (void)hipEventDestroy(e.join);
    if (e.fork) (void)hipEventDestroy(e.fork);
    if (e.side) (void)hipStreamDestroy(e.side);
  }
  if (cur != dev) (void)hipSetDevice(cur);
  if (err != hipSuccess) return nullptr;
  g_side[g_n_side] = e;
  return &g_side[g_n_side++];
}

// dK/dV and dQ only read what the preprocess pass and the caller wrote, and
// write disjoint outputs.  When the dK/dV grid runs more than one round of
// workgroups, dQ runs on the caller stream's side stream, forked from the
// caller's stream after the preprocess pass and joined back with events: the
// last, partly filled round of each kernel then overlaps the other kernel's
// work.  Once dQ is queued on the side stream, the caller's stream always
// waits for it, also when the dK/dV launch fails, so nothing queued after the
// call can reuse its buffers early and a capture stays joined.
//
// Five-GEMM backward (p.ds set, p.n_pairs the pairs per chunk): for each
// chunk of (batch, KV head) pairs in turn, the dK/dV kernel writes the
// chunk's dS tiles and the dQ kernel reads them, both on the caller's stream.
hipError_t launch_bwd_mfma(int dtype, const BwdParams& p, bool causal, hipStream_t s) {
  if (dtype != BF16::code && dtype != F16::code) return hipErrorInvalidValue;
  const int64_t pairs = (int64_t)p.B * p.Hkv;
  if (p.ds != nullptr) {
    if (bwd_ds_pair_bytes(dtype, p.Hq, p.Hkv, p.Sq, p.Sk, p.D, causal) == 0 || p.n_pairs <= 0)
      return hipErrorInvalidValue;
    if ((int64_t)((p.Sk + 127) / 128) * p.n_pairs > 0x7fffffffLL ||
        (int64_t)((p.Sq + 255) / 256) * p.n_pairs * p.group > 0x7fffffffLL)
      return hipErrorInvalidConfiguration;
    for (int64_t c0 = 0; c0 < pairs; c0 += p.n_pairs) {
      BwdParams q = p;
      q.bk0 = (int)c0;
      q.n_pairs = (int)std::min<int64_t>(p.n_pairs, pairs - c0);
      const KernelPlan kv = plan_bwd_dkv(dtype, q, causal);
      const KernelPlan dq = plan_bwd_dq(dtype, q, causal);
      if (!kv.fn || !dq.fn) return hipErrorInvalidValue;
      hipError_t e = run_plan(kv, &q, s);
      if (e != hipSuccess) return e;
      if ((e = run_plan(dq, &q, s)) != hipSuccess) return e;
    }
    return hipSuccess;
  }
  BwdParams q = p;
  q.bk0 = 0;
  q.n_pairs = (int)pairs;
  const KernelPlan kv = plan_bwd_dkv(dtype, q, causal);
  const KernelPlan dq = plan_bwd_dq(dtype, q, causal);
  if (!kv.fn || !dq.fn) return hipErrorInvalidValue;
  const int64_t g_kv = (int64_t)q.n_nblocks * p.B * p.Hkv * (kv.head_dim == 256 ? 2 : 1);
  const int64_t g_q = (int64_t)q.n_mblocks * p.B * p.Hq;
  if (g_kv > 0x7fffffffLL || g_q > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  const SideEntry* se = g_kv > 256 && g_q > 0 ? side_entry(s) : nullptr;
  if (!se) {
    hipError_t e = run_plan(kv, &q, s);
    if (e != hipSuccess) return e;
    return run_plan(dq, &q, s);
  }
  hipError_t e = hipEventRecord(se->fork, s);
  if (e == hipSuccess) e = hipStreamWaitEvent(se->side, se->fork, 0);
  if (e != hipSuccess) return e;
  // From here on the side stream depends on s (under capture it has joined
  // s's capture), so it is joined back whatever fails.
  const hipError_t e_dq = run_plan(dq, &q, se->side);
  const hipError_t e_kv = e_dq == hipSuccess ? run_plan(kv, &q, s) : hipSuccess;
  hipError_t e_join = hipEventRecord(se->join, se->side);
  if (e_join == hipSuccess) e_join = hipStreamWaitEvent(s, se->join, 0);
  if (e_dq != hipSuccess) return e_dq;
  return e_kv != hipSuccess ? e_kv : e_join;
}

}  // namespace sk
