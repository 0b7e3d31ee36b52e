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
// * Four waves per workgroup, one per SIMD, one workgroup per CU: each wave
//   keeps its 32 rows of the resident operands in registers and has the
//   whole 512-entry VGPR+AGPR file for operands, two score blocks in flight
//   and the fp32 accumulators.
// * The streamed tiles go through a STAGES-deep LDS ring written by
//   buffer_load ... lds (direct to LDS), two tiles ahead of the math, one
//   barrier per tile.  Rows past the sequence end and head-dim padding come
//   back as zeros from the buffer range check.
// * Streamed tiles are read both row-wise (ds_read_b128, 16 consecutive rows
//   per 16-lane group) and transposed (ds_read_b64_tr_b16, 4 aligned rows x 4
//   chunks per 32-lane group).  One XOR swizzle on the 16-byte chunk index
//   serves both: chunk c of row r sits at c ^ f(r) with f a bijection on
//   r % 16 whose top two bits differ across every aligned group of 4 rows,
//   so both read shapes hit 16 distinct bank quads of the 64-bank LDS.
// * Software pipeline per wave: the score and dP MFMAs of the next block are
//   interleaved, MFMA by MFMA, with the exp / dS / pack VALU work of the
//   current block (the MFMA unit runs asynchronously to the VALU), then the
//   gradient MFMAs of the current block run with their transposed operand
//   reads issued a few MFMAs ahead.
// * XCD-aware order: the 8 XCDs each walk a contiguous range of work items,
//   head-major, so the workgroups that share a head's streamed operand share
//   an L2.
//
// dK/dV kernel (bwd_dkv_kernel): a workgroup owns 128 keys of one
// (batch, KV head), 32 per wave, and walks every query head of that KV
// head's group and every 64-query tile that can see its keys, so the GQA sum
// happens in registers (deterministic, no atomics).  S = Q K^T and
// dP = dO V^T use K and V from registers as the B operand: each lane then
// owns one key (its l%32) and 16 queries per 32-query block; P and dS feed
// dV^T += dO^T P and dK^T += Q^T dS straight from registers, with dO^T / Q^T
// read transposed from the ring (the contraction over queries is permuted
// identically on both operands).  Every wave keeps its own copy of the
// tile's row statistics in the ring.  At D = 256 the output head dim is
// split over two workgroups to keep the accumulators in the register file.
//
// dQ kernel (bwd_dq_kernel): a workgroup owns 128 query rows, 32 per wave,
// with Q and dO in registers; K/V tiles stream through the ring;
// S^T = K Q^T and dP^T = V dO^T give one query per lane, and
// dQ^T += K^T dS^T reads K^T transposed from the ring.
#include "sk_common.h"
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
template <class T, int DP, int DO, int BMQ, int NW, int STAGES, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64, 1) bwd_dkv_kernel(BwdParams p) {
  using L = BwdTile<DP, BMQ>;  // Q and dO tiles
  constexpr int BNK = 32 * NW;
  constexpr int KD = DP / 16;  // k-steps over the head dim (S, dP)
  constexpr int QB = BMQ / 32;  // 32-query blocks per tile
  constexpr int DB = DO / 32;  // 32-wide output head-dim blocks
  constexpr int LQ = L::kSegs / NW;  // Q (and dO) segments per wave per tile
  constexpr int kStatBytes = 512;  // per wave: 64 lse*log2e, then 64 delta
  constexpr int kStageBytes = 2 * L::kTileBytes + NW * kStatBytes;
  constexpr int kLoads = 2 * LQ + 2;  // DMAs per wave per tile
  constexpr int PD = STAGES - 2;
  constexpr int kDSplit = DP / DO;
  constexpr int RB = L::kRowBytes;
  static_assert(L::kSegs % NW == 0, "tile segments must divide over the waves");
  static_assert(QB >= 1 && BMQ <= 64, "32 or 64 queries per tile");
  static_assert(PD >= 1 && PD <= 2, "prefetch distance");
  static_assert((STAGES & (STAGES - 1)) == 0, "the ring index is a mask");

  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * kStageBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  // Work item: (batch, KV head) major, then key block (lowest first: under
  // the causal mask it sees the most queries), then head-dim half.
  const int w = xcd_work_index(blockIdx.x, gridDim.x);
  const int per_head = p.n_nblocks * kDSplit;
  const int bk = w / per_head;
  const int rem = w - bk * per_head;
  const int nblk = rem / kDSplit;
  const int dsp = rem - nblk * kDSplit;
  const int b = bk / p.Hkv;
  const int hkv = bk - b * p.Hkv;
  const int n0 = nblk * BNK;
  const int nw = n0 + 32 * wave;
  const int key = nw + l32;
  const int diag = p.Sk - p.Sq;
  const int d_out0 = dsp * DO;

  // K (sign-flipped for a negative scale) and V rows of this lane's key as
  // the B operand: k[key][16*s + 8*hl .. +7].
  u32x4 kreg[KD], vreg[KD];
  {
    const int krows = max(0, min(32, p.Sk - nw));
    const int64_t k0 = ((int64_t)bk * p.Sk + min(nw, p.Sk)) * p.D;
    // Wave-uniform; readfirstlane keeps the resource in SGPRs (no waterfall loop).
    const int bytes = __builtin_amdgcn_readfirstlane(tile_bytes(krows, p.D, p.D));
    const buf_rsrc kr = make_rsrc((const uint16_t*)p.k + k0, bytes);
    const buf_rsrc vr = make_rsrc((const uint16_t*)p.v + k0, bytes);
#pragma unroll
    for (int s = 0; s < KD; ++s) {
      const int d0 = 16 * s + 8 * hl;
      const uint32_t off = d0 < p.D ? (uint32_t)((l32 * p.D + d0) * 2) : kBufferOob;
      kreg[s] = buffer_load_b128(kr, off) ^ p.op_sign;
      vreg[s] = buffer_load_b128(vr, off);
    }
  }

  // Query tiles that can see a key of this block: i >= n0 - diag.
  int m_begin = 0;
  if (CAUSAL) m_begin = max(0, n0 - diag) / BMQ * BMQ;
  const int n_mt = m_begin < p.Sq ? (p.Sq - m_begin + BMQ - 1) / BMQ : 0;
  const int n_it = p.group * n_mt;
  const int n_blk = n_it * QB;

  uint32_t goff[LQ];
#pragma unroll
  for (int j = 0; j < LQ; ++j) {
    const int seg = wave + j * NW;
    const int r = seg * L::kSegRows + lane / L::kCpr;
    const int c = (lane % L::kCpr) ^ swz_rt<DP>(r);
    goff[j] = c * 8 < p.D ? (uint32_t)((r * p.D + c * 8) * 2) : kBufferOob;
  }
  // Tile cursors, (query head gi, first row m0), advanced one tile at a time
  // (no divisions in the loop): the tile to issue next and the tile whose
  // blocks are being computed.
  int issue_gi = 0, issue_m0 = m_begin;
  int cur_gi = 0, cur_m0 = m_begin;
  auto advance = [&](int& gi, int& m0) {
    m0 += BMQ;
    if (m0 >= p.Sq) {
      m0 = m_begin;
      ++gi;
    }
  };
  auto stage = [&](int it) { return smem + (it & (STAGES - 1)) * kStageBytes; };
  auto issue_next = [&](int it) {
    const int64_t bh = (int64_t)b * p.Hq + hkv * p.group + issue_gi;
    const int m0 = issue_m0;
    const int bytes = tile_bytes(min(BMQ, p.Sq - m0), p.D, p.D);
    const int64_t q0 = (bh * p.Sq + m0) * p.D;
    const i32x4 qr = make_rsrc_words((const uint16_t*)p.q + q0, bytes);
    const i32x4 gr = make_rsrc_words((const uint16_t*)p.dout + q0, bytes);
    const uint32_t st = lds_addr(stage(it));
#pragma unroll
    for (int j = 0; j < LQ; ++j) {
      const int seg = wave + j * NW;
      buffer_load_lds_b128(qr, st + seg * 1024, goff[j]);
      buffer_load_lds_b128(gr, st + L::kTileBytes + seg * 1024, goff[j]);
    }
    const int sbytes = min(64, p.Sq - m0) * 4;
    const i32x4 lr = make_rsrc_words(p.lse_log2 + bh * p.Sq + m0, sbytes);
    const i32x4 dr = make_rsrc_words(p.delta + bh * p.Sq + m0, sbytes);
    const uint32_t sb = st + 2 * L::kTileBytes + wave * kStatBytes;
    buffer_load_lds_b32(lr, sb, lane * 4);
    buffer_load_lds_b32(dr, sb + 256, lane * 4);
    advance(issue_gi, issue_m0);
  };

#pragma unroll
  for (int t = 0; t <= PD; ++t)
    if (t < n_it) issue_next(t);

  f32x16 dkacc[DB], dvacc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) {
    dkacc[c] = f32x16{};
    dvacc[c] = f32x16{};
  }

  // Row-wise A operand of S / dP: query row l32 (+32 per block), chunk 2s + hl.
  int qa_lds[KD];
#pragma unroll
  for (int s = 0; s < KD; ++s) qa_lds[s] = l32 * RB + (((2 * s + hl) ^ swz_rt<DP>(l32)) * 16);
  int tr_lo[DB], tr_hi[DB];
  tr_offsets<DP, DB>(lane, d_out0 / 8, tr_lo, tr_hi);

  const float c_log2 = p.abs_scale_log2;
  auto sync_tile = [&](int it, int max_ahead) {
    wait_tiles<kLoads, PD>(min(max_ahead, n_it - 1 - it));
    __syncthreads();
  };

  // Every block runs the same straight-line code.  Under the causal mask a
  // block the wave cannot see at all, or sees in part, is masked instead of
  // skipped: its P and dS are exactly zero, so it adds nothing.  Waves whose
  // keys all lie past S_k compute unused values.

  // S = Q K^T and dP = dO V^T of the block whose rows start at `rows` (no
  // interleave): lane holds [query 8*(r/4) + 4*hl + r%4][key l32].
  auto block_sdp = [&](const uint8_t* rows, f32x16& sc, f32x16& pc) {
    sc = f32x16{};
    pc = f32x16{};
#pragma unroll
    for (int s = 0; s < KD; ++s) {
      sc = mfma32<T>(lds_b128(rows + qa_lds[s]), kreg[s], sc);
      pc = mfma32<T>(lds_b128(rows + L::kTileBytes + qa_lds[s]), vreg[s], pc);
    }
  };

  // Causal mask of the block of queries mq..mq+31: key > query + diag -> -inf.
  auto premask = [&](int mq, f32x16& sc) {
    if (!CAUSAL || nw + 31 <= mq + diag) return;
    const int lim = key - diag - mq - 4 * hl;  // masked iff 8*(r/4) + r%4 < lim
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (8 * (r >> 2) + (r & 3) < lim) sc[r] = kNegInf;
  };

  // Row statistics of a block (stats = its tile's stat area + 128 * block)
  // for this lane's 16 queries.
  auto load_stats = [&](const uint8_t* stats, f32x4 (&lv)[4], f32x4 (&dv)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lv[i] = *reinterpret_cast<const f32x4*>(stats + 4 * (8 * i + 4 * hl));
      dv[i] = *reinterpret_cast<const f32x4*>(stats + 256 + 4 * (8 * i + 4 * hl));
    }
  };
  auto stats_of = [&](int it, int blk) {
    return stage(it) + 2 * L::kTileBytes + wave * kStatBytes + 128 * blk;
  };

  // P and dS of one element, packed eight at a time into the B operands of
  // the k-step s2 = r / 8 (queries permuted as the transposed reads are).
  u32x4 pk[2], dsk[2];
  float pe[16], de[16];
  auto elem = [&](int r, const f32x16& sc, const f32x16& pc, const f32x4 (&lv)[4],
                  const f32x4 (&dv)[4]) {
    pe[r] = fast_exp2(fmaf(sc[r], c_log2, -lv[r >> 2][r & 3]));
    de[r] = pe[r] * (pc[r] - dv[r >> 2][r & 3]);
    if ((r & 7) == 7) {
      const int b8 = r - 7;
      pk[r >> 3] = u32x4{pack2<T>(pe[b8], pe[b8 + 1]), pack2<T>(pe[b8 + 2], pe[b8 + 3]),
                         pack2<T>(pe[b8 + 4], pe[b8 + 5]), pack2<T>(pe[b8 + 6], pe[b8 + 7])};
      dsk[r >> 3] = u32x4{pack2<T>(de[b8], de[b8 + 1]), pack2<T>(de[b8 + 2], de[b8 + 3]),
                          pack2<T>(de[b8 + 4], de[b8 + 5]), pack2<T>(de[b8 + 6], de[b8 + 7])};
    }
  };
  auto block_valu = [&](const uint8_t* stats, const f32x16& sc, const f32x16& pc) {
    f32x4 lv[4], dv[4];
    load_stats(stats, lv, dv);
#pragma unroll
    for (int r = 0; r < 16; ++r) elem(r, sc, pc, lv, dv);
  };

  // Stage A: S / dP MFMAs of the next block (alternating, so each
  // accumulator's chain has one independent MFMA between its links)
  // interleaved with the P / dS elements of the current block; fenced per
  // MFMA so the in-order issue keeps the LDS read KLEAD MFMAs ahead and EPM
  // elements between MFMAs.
  auto stage_a = [&](const uint8_t* rows_n, f32x16& sn, f32x16& pn, const uint8_t* stats,
                     const f32x16& sc, const f32x16& pc) {
    constexpr int NM = 2 * KD;
    constexpr int KLEAD = 3;
    constexpr int EPM = (16 + NM - 1) / NM;
    f32x4 lv[4], dv[4];
    load_stats(stats, lv, dv);
    u32x4 a[NM];
#pragma unroll
    for (int i = 0; i < KLEAD; ++i)
      a[i] = lds_b128(rows_n + (i & 1) * L::kTileBytes + qa_lds[i >> 1]);
    sn = f32x16{};
    pn = f32x16{};
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (i + KLEAD < NM) {
        const int n = i + KLEAD;
        a[n] = lds_b128(rows_n + (n & 1) * L::kTileBytes + qa_lds[n >> 1]);
      }
      if (i & 1)
        pn = mfma32<T>(a[i], vreg[i >> 1], pn);
      else
        sn = mfma32<T>(a[i], kreg[i >> 1], sn);
#pragma unroll
      for (int k = 0; k < EPM; ++k)
        if (i * EPM + k < 16) elem(i * EPM + k, sc, pc, lv, dv);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Stage B: dV^T += dO^T P and dK^T += Q^T dS for the block whose rows
  // start at `rows`: lane holds [d d_out0 + 32*c + 8*(r/4) + 4*hl + r%4][key l32].
  auto stage_b = [&](const uint8_t* rows) {
    constexpr int NM = 2 * 2 * DB;
    constexpr int OLEAD = NM < 4 ? NM : 4;
    u32x4 go[2][DB], qo[2][DB];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int c = 0; c < DB; ++c) {
        const uint8_t* r0 = rows + 16 * s2 * RB;
        go[s2][c] = lds_tr_pair(r0 + L::kTileBytes + tr_lo[c], r0 + L::kTileBytes + tr_hi[c]);
        qo[s2][c] = lds_tr_pair(r0 + tr_lo[c], r0 + tr_hi[c]);
      }
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int c = 0; c < DB; ++c) {
        dvacc[c] = mfma32<T>(go[s2][c], pk[s2], dvacc[c]);
        dkacc[c] = mfma32<T>(qo[s2][c], dsk[s2], dkacc[c]);
      }
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * OLEAD, 0);
#pragma unroll
    for (int i = 0; i < NM - OLEAD; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, OLEAD, 0);
  };

  // Crossing into tile it: its loads landed (vmcnt, then barrier; the barrier
  // also retires every wave's reads of tile it - 2's stage), then tile
  // it + PD is issued into that stage.
  auto enter_tile = [&](int it) {
    sync_tile(it, PD - 1);
    if (it + PD < n_it) issue_next(it + PD);
  };

  f32x16 sA, pA, sB, pB;
  if constexpr (QB == 2) {
    // Block pipeline with fixed register roles: block 0 of a tile (rows
    // 0-31) in (sA, pA), block 1 in (sB, pB), so no scores move between
    // registers.  One tile per iteration.
    if (n_it > 0) {
      sync_tile(0, PD);
      block_sdp(stage(0), sA, pA);
    }
    for (int it = 0; it < n_it; ++it) {
      const uint8_t* st = stage(it);
      premask(cur_m0, sA);
      stage_a(st + 32 * RB, sB, pB, stats_of(it, 0), sA, pA);
      stage_b(st);
      premask(cur_m0 + 32, sB);
      if (it + 1 < n_it) {
        enter_tile(it + 1);
        stage_a(stage(it + 1), sA, pA, stats_of(it, 1), sB, pB);
      } else {
        block_valu(stats_of(it, 1), sB, pB);
      }
      stage_b(st + 32 * RB);
      advance(cur_gi, cur_m0);
    }
  } else {
    // One 32-query block per tile (D = 256), run in order without the
    // interleave: the register file holds one score block next to the
    // larger K/V operands.  Loads run PD + 1 tiles ahead.
    (void)sB;
    (void)pB;
    for (int it = 0; it < n_it; ++it) {
      sync_tile(it, PD);
      if (it + PD + 1 < n_it) issue_next(it + PD + 1);
      block_sdp(stage(it), sA, pA);
      premask(cur_m0, sA);
      block_valu(stats_of(it, 0), sA, pA);
      stage_b(stage(it));
      advance(cur_gi, cur_m0);
    }
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

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
template <class T, int DP, int BN, int NW, int STAGES, int OCC, bool PIPE, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64, OCC) bwd_dq_kernel(BwdParams p) {
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

  // Stage A: S^T / dP^T MFMAs of tile tn interleaved with the dS elements of
  // the current tile, fenced per MFMA (see the dK/dV kernel).  MFMA order
  // cycles over the 2*KB accumulators so consecutive links of one chain are
  // 2*KB MFMAs apart.
  auto stage_a = [&](int tn, f32x16 (&sn)[KB], f32x16 (&pn)[KB], const f32x16 (&sd)[KB],
                     const f32x16 (&pd)[KB]) {
    constexpr int NM = 2 * KD * KB;
    constexpr int KLEAD = 3;
    constexpr int NE = KN * 8;
    constexpr int EPM = (NE + NM - 1) / NM;
    const uint8_t* st = stage(tn);
    auto addr = [&](int i) {
      const int j = i % (2 * KB);
      return st + (j / KB) * L::kTileBytes + k_lds[i / (2 * KB)] + (j % KB) * 32 * RB;
    };
    u32x4 a[NM];
#pragma unroll
    for (int i = 0; i < KLEAD; ++i) a[i] = lds_b128(addr(i));
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      sn[kb] = f32x16{};
      pn[kb] = f32x16{};
    }
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (i + KLEAD < NM) a[i + KLEAD] = lds_b128(addr(i + KLEAD));
      const int j = i % (2 * KB), s = i / (2 * KB);
      if (j / KB == 0)
        sn[j % KB] = mfma32<T>(a[i], qreg[s], sn[j % KB]);
      else
        pn[j % KB] = mfma32<T>(a[i], greg[s], pn[j % KB]);
#pragma unroll
      for (int k = 0; k < EPM; ++k)
        if (i * EPM + k < NE) elem(i * EPM + k, sd, pd);
      __builtin_amdgcn_sched_barrier(0);
    }
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
  if constexpr (PIPE) {
    // Fixed register roles: even tiles in s0/p0, odd tiles in s1/p1.
    if (n_tiles > 0) {
      sync_tile(0, PD);
      gemm_sdp(0, s0, p0);
    }
    auto iteration = [&](int t, f32x16 (&cs)[KB], f32x16 (&cp)[KB], f32x16 (&ns)[KB],
                         f32x16 (&np)[KB]) {
      premask(t, cs);
      if (t + 1 < n_tiles) {
        sync_tile(t + 1, PD - 1);
        if (t + 1 + PD < n_tiles) issue_tile(t + 1 + PD);
        stage_a(t + 1, ns, np, cs, cp);
      } else {
        tile_valu(cs, cp);
      }
      gemm_dq(t);
    };
    for (int t = 0; t < n_tiles; t += 2) {
      iteration(t, s0, p0, s1, p1);
      if (t + 1 < n_tiles) iteration(t + 1, s1, p1, s0, p0);
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

// gfx950 tile table for the backward, by head dim (padded to 64, 128 or 256;
// other dims run zero-padded in the next size up).  Four waves (one per
// SIMD), 4 ring stages, one workgroup per CU:
//   dK/dV: 128 keys per workgroup; query tiles of 64 rows (32 at D = 256,
//          where the output head dim is also split over two workgroups);
//          ring 4 x (Q + dO + stats) = 72 / 136 / 136 KiB.
//   dQ:    128 query rows per workgroup; key tiles of 64 rows (32 at
//          D = 256); ring 4 x (K + V) = 64 / 128 / 128 KiB.
// dQ kernel table by padded head dim: key tile, workgroups per CU, and
// whether a wave interleaves its own softmax with the next tile's MFMAs.
template <int DP>
struct DqConfig {
  static constexpr int kBn = 32;
  static constexpr int kOcc = 2;
  static constexpr bool kPipe = false;
};
template <>
struct DqConfig<256> {
  static constexpr int kBn = 32;
  static constexpr int kOcc = 1;
  static constexpr bool kPipe = false;
};

template <class T, int DP, int DO, int BMQ>
static hipError_t launch_bwd_t(const BwdParams& p, bool causal, hipStream_t s) {
  constexpr int NW = 4;
  constexpr int STAGES = 4;
  using QC = DqConfig<DP>;
  BwdParams q = p;
  q.n_nblocks = (p.Sk + 32 * NW - 1) / (32 * NW);
  q.n_mblocks = (p.Sq + 32 * NW - 1) / (32 * NW);
  const int64_t g_kv = (int64_t)q.n_nblocks * p.B * p.Hkv * (DP / DO);
  const int64_t g_q = (int64_t)q.n_mblocks * p.B * p.Hq;
  if (g_kv > 0x7fffffffLL || g_q > 0x7fffffffLL) return hipErrorInvalidConfiguration;
  if (g_kv > 0) {
    if (causal)
      hipLaunchKernelGGL((bwd_dkv_kernel<T, DP, DO, BMQ, NW, STAGES, true>), dim3((unsigned)g_kv),
                         dim3(NW * 64), 0, s, q);
    else
      hipLaunchKernelGGL((bwd_dkv_kernel<T, DP, DO, BMQ, NW, STAGES, false>), dim3((unsigned)g_kv),
                         dim3(NW * 64), 0, s, q);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (g_q > 0) {
    if (causal)
      hipLaunchKernelGGL((bwd_dq_kernel<T, DP, QC::kBn, NW, STAGES, QC::kOcc, QC::kPipe, true>),
                         dim3((unsigned)g_q), dim3(NW * 64), 0, s, q);
    else
      hipLaunchKernelGGL((bwd_dq_kernel<T, DP, QC::kBn, NW, STAGES, QC::kOcc, QC::kPipe, false>),
                         dim3((unsigned)g_q), dim3(NW * 64), 0, s, q);
  }
  return hipGetLastError();
}

template <class T>
static hipError_t launch_bwd_dt(const BwdParams& p, bool causal, hipStream_t s) {
  if (p.D <= 64) return launch_bwd_t<T, 64, 64, 64>(p, causal, s);
  if (p.D <= 128) return launch_bwd_t<T, 128, 128, 64>(p, causal, s);
  if (p.D <= 256) return launch_bwd_t<T, 256, 128, 32>(p, causal, s);
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_mfma(int dtype, const BwdParams& p, bool causal, hipStream_t s) {
  if (dtype == BF16::code) return launch_bwd_dt<BF16>(p, causal, s);
  if (dtype == F16::code) return launch_bwd_dt<F16>(p, causal, s);
  return hipErrorInvalidValue;
}

}  // namespace sk
