// FlashAttention-2 forward for bf16 / fp16 on gfx950 MFMA.
//
// Replaces the reference's _flash_fwd_kernel
// (src/stackkernels/_core/attention/flash_fwd.py:15-179); same math, a
// gfx950-first organisation:
//
// * A workgroup of NW waves owns BM = 32*NW query rows of one (batch, query
//   head); each wave owns 32 of them, with its Q rows held in registers.
//   At D <= 128 a workgroup is 8 waves (two per SIMD) and fills a CU alone,
//   or, for short work, 4 waves with two workgroups per CU (the tile table
//   at the end of this file).
// * K/V tiles of BN keys stream through two 4-deep LDS rings (all K stages,
//   then all V stages), written by buffer_load ... lds (direct to LDS, no
//   register staging).  Each wave issues whole 1 KiB segments; rows past S_k
//   and head-dim padding come back as zeros from the buffer range check.
//   One barrier per two tiles, each issuing the next two K and V tiles into
//   the stages the two previous tiles freed, so every load has two tiles'
//   time to land.  (The two-workgroup entry has 2-deep rings: one barrier
//   per tile, issuing the next K and V tiles, which get one tile's time.)
//   The tile loop is unrolled by the ring depth, so every LDS address is a
//   lane-constant register plus a compile-time offset.
// * One tile body per tile and wave: the score MFMAs of tile t+1, then the
//   O MFMAs of tile t, with the softmax of tile t (scale/exp2, row sum,
//   pack) and the row maximum of tile t+1 spread evenly between all of
//   them.  A wave overlaps MFMA and VALU work only with its own
//   instructions (an MFMA-bound wave starves the other wave of its SIMD),
//   so every wave keeps both busy itself.
// * LDS tiles are unpadded with a 16-byte-chunk XOR swizzle: chunk c of row r
//   sits at c ^ (r % 16) in K tiles (the 16-byte row reads of 16 consecutive
//   rows hit disjoint bank quads) and at c ^ 4 (r % 4) in V tiles (the four
//   rows x four chunks a 32-lane ds_read_b64_tr_b16 group touches hit
//   disjoint banks).
// * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16:
//   every lane then holds one query column (its l%32) and 16 keys per 32-key
//   block, so the softmax row max needs one v_permlane32_swap per tile and
//   the row sum none until the end.
// * The output is accumulated transposed as well, O^T += V^T P^T.  The P^T
//   operand comes straight from the score registers (the contraction order
//   over keys is permuted consistently on both sides), and V^T is read from
//   the row-major V tile with ds_read_b64_tr_b16.
// * Online softmax in base 2 with |sm_scale|*log2(e) folded into one FMA per
//   score; a negative sm_scale is applied by negating q's sign bits.
//   Rescaling is lazy: the exponent offset moves only when a tile's maximum
//   exceeds it by more than 2^8, so the O rescale runs on a few tiles.
// * Bottom-right causal masking (key j visible to query i iff
//   j <= i + Sk - Sq, reference flash_fwd.py:122-128) is applied only on the
//   tiles that straddle the diagonal or the end of the keys; tiles a wave
//   cannot see are skipped.  Rows that see no key end with O = 0 and
//   LSE = -inf, as the reference path does (_reference/torch/attention.py:70-73).
// * XCD-aware order: each of the 8 XCDs walks a contiguous range of
//   (head, query block) items, head-major, heaviest query block first, so
//   the heads an XCD has in flight share its L2 and the causal triangle's
//   long rows do not trail at the end of the grid.  Under the causal mask a
//   workgroup runs query blocks j and n-1-j back to back when the grid
//   stays at two or more workgroups per CU, which evens out the work per
//   workgroup and halves the per-item fixed cost.
#include <type_traits>

#include "sk_common.h"
#include "sk_kernels.h"
#include "sk_rope.h"

// Tiles between two workgroup barriers of the forward's tile loop (1 or 2).
#ifndef SK_FWD_SYNC_TILES
#define SK_FWD_SYNC_TILES 2
#endif

namespace sk {

// Geometry of one K or V tile in LDS: BN rows of DP 16-bit words, unpadded.
template <int DP, int BN>
struct FwdLds {
  static constexpr int kCpr = DP / 8;                     // 16-byte chunks per row
  static constexpr int kRowBytes = DP * 2;
  static constexpr int kTileBytes = BN * kRowBytes;
  static constexpr int kStageBytes = 2 * kTileBytes;      // K tile, then V tile
  static constexpr int kSegRows = 1024 / kRowBytes;       // rows per 1 KiB segment
  static constexpr int kSegs = kTileBytes / 1024;         // segments per tile
};

// Chunk swizzles (XOR on the 16-byte chunk index of a row) for the 64-bank
// LDS, which serves a 16-byte read for 16 lanes and an 8-byte read for 32
// lanes per cycle.  K: the 16 rows of a 16-lane ds_read_b128 group (same
// logical chunk) land on 16 distinct bank quads.  V: the 4 rows x 4 chunks a
// 32-lane ds_read_b64_tr_b16 group touches land on 16 distinct bank quads.
// (128-byte rows, D = 64, alternate bank halves, hence the r/2 terms.)
template <int DP>
__device__ __forceinline__ int swz_k(int r) {
  return DP == 64 ? (r >> 1) & 7 : r & 15;
}
template <int DP>
__device__ __forceinline__ int swz_v(int r) {
  return DP == 64 ? 4 * ((r >> 1) & 1) : 4 * (r & 3);
}

// Forward tile body schedule check: softmax pair g (FMA at slot g*fl/(ng-1),
// pack two slots later) is packed at least one slot before the first O MFMA
// that reads its k-step, O MFMA j sitting at slot ns + j with k-step j / db.
constexpr bool softmax_pairs_fit(int ns, int db, int fl, int ng) {
  for (int g = 0; g < ng; ++g)
    if (g * fl / (ng - 1) + 2 > ns + (g / 4) * db - 2) return false;
  return true;
}

template <class T, int DP, int BN, int NW, int STAGES, int OCC, bool CAUSAL, bool ROPE>
__global__ void __launch_bounds__(NW * 64, OCC) fwd_mfma_kernel(FwdParams p) {
  using L = FwdLds<DP, BN>;
  constexpr int BM = 32 * NW;
  constexpr int KD = DP / 16;  // k-steps over the head dim for S^T
  constexpr int KB = BN / 32;  // 32-key blocks per tile
  constexpr int DB = DP / 32;  // 32-wide head-dim blocks of O^T
  constexpr int KN = BN / 16;  // k-steps over keys for O^T
  constexpr int LK = L::kSegs / NW;  // K (and V) segments each wave loads per tile
  constexpr int KT = L::kTileBytes;
  constexpr int RB = L::kRowBytes;
  constexpr int kVReg = STAGES * KT;  // LDS: all K stages, then all V stages
  static_assert(L::kSegs % NW == 0, "tile segments must divide over the waves");
  static_assert(STAGES == 4 || STAGES == 2, "a 4-deep ring (two groups ahead) or 2-deep (one ahead)");
  static_assert(3 * KT + (BN - 8) * RB < 65536, "stage offsets must fit the ds immediate");

  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGES * KT];
  // Tiles per workgroup barrier.  The 2-deep ring (two workgroups per CU)
  // synchronises every tile and keeps one load group in flight.
  constexpr int kSync = STAGES == 2 ? 1 : SK_FWD_SYNC_TILES;
  static_assert(kSync == 1 || kSync == 2, "one barrier per tile or per two tiles");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  // Work item: a (batch, head) and either one query block or, when the host
  // pairs them (causal), blocks j and n_mblocks-1-j run back to back, so every
  // workgroup carries the same causal work and the per-item fixed cost is
  // paid half as often.
  const int w = xcd_work_index(blockIdx.x, gridDim.x);
  const int bh = w / p.n_items;
  const int item = w - bh * p.n_items;
  const int b = bh / p.Hq;
  const int hq = bh % p.Hq;
  const int hkv = hq / p.group;
  const int diag = p.Sk - p.Sq;  // causal offset

  const uint16_t* kbase = (const uint16_t*)p.k + b * p.k_sb + hkv * p.k_sh;
  const uint16_t* vbase = (const uint16_t*)p.v + b * p.v_sb + hkv * p.v_sh;
  const uint32_t lds0 = lds_addr(smem);

  // Per-lane global byte offsets of the chunks this lane loads (tile-relative).
  uint32_t koff[LK], voff[LK];
#pragma unroll
  for (int j = 0; j < LK; ++j) {
    const int seg = wave + j * NW;
    const int r = seg * L::kSegRows + lane / L::kCpr;
    const int pc = lane % L::kCpr;
    const int kc = pc ^ swz_k<DP>(r);
    const int vc = pc ^ swz_v<DP>(r);
    koff[j] = kc * 8 < p.D ? (uint32_t)((r * p.k_ss + kc * 8) * 2) : kBufferOob;
    voff[j] = vc * 8 < p.D ? (uint32_t)((r * p.v_ss + vc * 8) * 2) : kBufferOob;
  }

  // Lane-constant LDS byte addresses (stage 0).  K operand of k-step s: row
  // l32 (+32 kb), chunk 2s + hl.  V^T operand of head-dim block c: rows
  // 4*hl + j16/4 (+16 s2, +8 for the upper half, neither of which changes the
  // row's swizzle), chunk 4c + 2*((lane/16)%2) + (j16%4)/2, and the 8-byte
  // half (j16%2) of that chunk.  Stage st adds st * KT.
  int k_lds[KD], v_lds[DB];
#pragma unroll
  for (int s = 0; s < KD; ++s) k_lds[s] = l32 * RB + (((2 * s + hl) ^ swz_k<DP>(l32)) * 16);
  {
    const int j16 = lane & 15;
    const int vr = 4 * hl + j16 / 4;
    const int g = 2 * ((lane >> 4) & 1) + (j16 & 3) / 2;
#pragma unroll
    for (int c = 0; c < DB; ++c)
      v_lds[c] = kVReg + vr * RB + (((4 * c + g) ^ swz_v<DP>(vr)) * 16) + 8 * (j16 & 1);
  }
  auto ld128 = [&](int addr) { return *reinterpret_cast<const u32x4*>(smem + addr); };

  auto run_item = [&](int mblk) {
  const int m0 = mblk * BM;
  const int mw = m0 + wave * 32;
  const int row = mw + l32;
  int n_end = p.Sk;
  if (CAUSAL) n_end = min(p.Sk, m0 + BM + diag);
  const int n_tiles = n_end > 0 ? (n_end + BN - 1) / BN : 0;

  // Q^T operand: lane holds q[row][16*s + 8*hl .. +7] (zero past S_q and D).
  u32x4 qreg[KD];
  {
    const int qrows = max(0, min(32, p.Sq - mw));
    const buf_rsrc qr = make_rsrc((const uint16_t*)p.q + b * p.q_sb + hq * p.q_sh +
                                      (int64_t)min(mw, p.Sq) * p.q_ss,
                                  tile_bytes(qrows, p.q_ss, p.D));
#pragma unroll
    for (int s = 0; s < KD; ++s) {
      const int d0 = 16 * s + 8 * hl;
      const uint32_t off = d0 < p.D ? (uint32_t)((l32 * p.q_ss + d0) * 2) : kBufferOob;
      qreg[s] = buffer_load_b128(qr, off);
    }
    if constexpr (ROPE) {
      // RoPE on load: query row i is token i of its batch row.  Rows past
      // S_q read zeros and stay zero.
      const int rrow = rope_row(p.rope, b, row);
      const int half = p.D >> 1;
#pragma unroll
      for (int s = 0; s < KD; ++s) {
        const int d0 = 16 * s + 8 * hl;
        const int dq = d0 < half ? d0 + half : d0 - half;
        const uint32_t off = d0 < p.D ? (uint32_t)((l32 * p.q_ss + dq) * 2) : kBufferOob;
        const u32x4 y = buffer_load_b128(qr, off);
        if (rrow >= 0 && d0 < p.D) qreg[s] = rope8_at<T>(qreg[s], y, d0, half, p.rope, rrow);
      }
    }
#pragma unroll
    for (int s = 0; s < KD; ++s) qreg[s] ^= p.q_sign;
  }

  // Issue cursors of K and V (first key, base pointer).  K and V tiles are
  // issued on separate schedules: group g carries K(g+1) and V(g).  A K
  // tile past the end is issued with an empty range (zeros), so every group
  // has the same number of loads.
  int k_n0 = 0, v_n0 = 0;
  const uint16_t* iss_k = kbase;
  const uint16_t* iss_v = vbase;
  auto issue_k = [&](int stg) {
    const int bytes = tile_bytes(max(0, min(BN, p.Sk - k_n0)), p.k_ss, p.D);
    const i32x4 kr = make_rsrc_words(iss_k, bytes);
#pragma unroll
    for (int j = 0; j < LK; ++j)
      buffer_load_lds_b128(kr, lds0 + stg * KT + (wave + j * NW) * 1024, koff[j]);
    k_n0 += BN;
    iss_k += (int64_t)BN * p.k_ss;
  };
  auto issue_v = [&](int stg) {
    const int bytes = tile_bytes(max(0, min(BN, p.Sk - v_n0)), p.v_ss, p.D);
    const i32x4 vr = make_rsrc_words(iss_v, bytes);
#pragma unroll
    for (int j = 0; j < LK; ++j)
      buffer_load_lds_b128(vr, lds0 + kVReg + stg * KT + (wave + j * NW) * 1024, voff[j]);
    v_n0 += BN;
    iss_v += (int64_t)BN * p.v_ss;
  };

  f32x16 oacc[DB];
#pragma unroll
  for (int c = 0; c < DB; ++c) oacc[c] = f32x16{};
  float m_run = kNegInf;
  float l_run = 0.f;

  const bool wave_has_rows = mw < p.Sq;
  // Tiles [0, vis_tiles) hold keys this wave can see.
  int vis_tiles = wave_has_rows ? n_tiles : 0;
  if (CAUSAL) {
    const int last_key = mw + 31 + diag;  // last key the wave's last row sees
    vis_tiles = last_key < 0 ? 0 : min(vis_tiles, last_key / BN + 1);
  }
  auto active = [&](int t) { return t < vis_tiles; };
  // Group g landed for this wave (vmcnt, with group g + 1 possibly still in
  // flight), then for all (barrier); the barrier also retires every wave's
  // reads of the stages the next issue refills.
  auto sync_group = [&](int g) {
    if (STAGES == 4 && g + 1 < n_tiles)
      wait_vmcnt<2 * LK>();
    else
      wait_vmcnt<0>();  // 2-deep ring: group g is the only one in flight
    __syncthreads();
  };

  // S^T = K Q^T of the tile in stage stg: lane holds
  // [key n0 + 32*kb + 8*(r/4) + 4*hl + r%4][query row].
  auto gemm0 = [&](int stg, f32x16 (&sd)[KB]) {
    u32x4 a[KD][KB];
#pragma unroll
    for (int s = 0; s < KD; ++s)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) a[s][kb] = ld128(k_lds[s] + stg * KT + kb * 32 * RB);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) sd[kb] = f32x16{};
#pragma unroll
    for (int s = 0; s < KD; ++s)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) sd[kb] = mfma32<T>(a[s][kb], qreg[s], sd[kb]);
  };

  // Mask tile t's scores where needed; returns the tile's row maximum.
  auto mask_max = [&](int t, f32x16 (&sc)[KB]) {
    const int n0 = t * BN;
    const bool tail = n0 + BN > p.Sk;
    const bool straddle = CAUSAL && (n0 + BN - 1 > mw + diag);
    if (tail || straddle) {
      int lim = p.Sk - 1;
      if (CAUSAL) lim = min(lim, row + diag);
      // Element offset o (32*kb + 8*(r/4) + r%4) is masked iff o > lim - n0 - 4*hl.
      // keep = all-ones iff visible; one bitfield insert per element selects
      // the score or -inf (no per-element condition registers).
      const int nlim = n0 + 4 * hl - lim - 1;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int o = 32 * kb + 8 * (r >> 2) + (r & 3);
          const uint32_t keep = (uint32_t)((o + nlim) >> 31);
          // (Copy the element out first: a bit_cast of a vector-element
          // lvalue reads the vector's first element.)
          const float x = sc[kb][r];
          sc[kb][r] = __builtin_bit_cast(
              float, (keep & __builtin_bit_cast(uint32_t, x)) | (~keep & 0xff800000u));
        }
    }
    float mt = kNegInf;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = __builtin_elementwise_maximum(mt, sc[kb][r]);
    return xhalf_max(mt);
  };

  // Lazy rescaling: the exponent offset m_run only moves when a score exceeds
  // it by more than kRescaleLog2 (in log2 units), so P <= 2^8.  Lanes that do
  // not grow keep alpha = 1 (their offset may still be -inf on a row that has
  // seen no key yet).  Returns -m_run * scale * log2(e) for the exponent.
  auto rescale = [&](float mt) {
    const bool grow = (mt - m_run) * p.scale_log2 > kRescaleLog2;
    if (__any(grow)) {
      const float alpha = grow ? fast_exp2((m_run - mt) * p.scale_log2) : 1.f;
      m_run = grow ? mt : m_run;
      l_run *= alpha;
#pragma unroll
      for (int c = 0; c < DB; ++c) oacc[c] *= alpha;
    }
    return (m_run == kNegInf) ? 0.f : -m_run * p.scale_log2;
  };

  // P^T = exp2(S^T * scale * log2 e - offset), packed by stage A as the B
  // operand of the O^T product.
  u32x4 pk[KN];

  // Tile body for tile t, one MFMA per slot: S(t+1) = K(t+1) Q^T in slots
  // 0..NS-1, then O^T += V(t)^T P(t)^T in slots NS..NM-1.  The softmax of
  // tile t runs between the MFMAs, spread over all of them, so every slot
  // carries about the same VALU work and the MFMA unit never waits for a
  // long VALU stretch; a wave keeps MFMAs and VALU work overlapped by
  // interleaving them itself.  Element pair g (elements 2g, 2g+1) takes its
  // FMA at slot F(g), its exp2 at F(g)+1 and its row sum and 16-bit pack at
  // F(g)+2; F spreads the pairs evenly so that P(t)'s k-step s2 is packed at
  // least one slot before the first O MFMA that reads it.  The raw row maximum
  // of S(t+1) is taken in the last slots, after its MFMAs have completed.
  // The operand reads run KLEAD (K) and OLEAD (V^T) MFMAs ahead.  Each slot
  // is fenced with sched_barrier so the in-order issue keeps this order.
  // next: std::true_type, or std::false_type for the block's last tile,
  // whose body leaves out the score MFMAs, their K reads and the row maximum
  // of a tile past the end.
  auto body = [&](int stg_k, int stg_v, f32x16 (&nx)[KB], const f32x16 (&sc)[KB],
                  float neg_m, auto next) {
    constexpr bool kNext = decltype(next)::value;
    constexpr int NS = KD * KB;
    constexpr int NO = DB * KN;
    constexpr int NM = NS + NO;
    constexpr int KLEAD = NS < 3 ? NS : 3;
    constexpr int OLEAD = NO < 5 ? NO : 5;
    constexpr int NE = KN * 8;  // softmax elements per lane (pairs 4*s2 .. 4*s2+3 form pk[s2])
    constexpr int NG = NE / 2;
    constexpr int FL = NS + ((NG - 1) / 4) * DB - 4;  // F of the last pair
    constexpr int MS = NS + 2;                         // first slot of the row maximum
    constexpr int NX = 16 * KB;                        // S(t+1) elements per lane
    static_assert(FL >= 0 && softmax_pairs_fit(NS, DB, FL, NG),
                  "every pair is packed at least one slot before the first O MFMA that reads it");
    static_assert(MS < NM, "row maximum slots");
    auto fslot = [](int g) { return g * FL / (NG - 1); };
    auto kaddr = [&](int i) { return k_lds[i / KB] + stg_k * KT + (i % KB) * 32 * RB; };
    auto score = [&](int x) { return sc[x >> 4][x & 15]; };
    auto read_vt = [&](int j) {
      const int s2 = j / DB, c = j % DB;
      const int ad = v_lds[c] + stg_v * KT + 16 * s2 * RB;
      const u32x2 lo = lds_read_tr((const uint16_t*)(smem + ad));
      const u32x2 hi = lds_read_tr((const uint16_t*)(smem + ad + 8 * RB));
      return u32x4(__builtin_shufflevector(lo, hi, 0, 1, 2, 3));
    };
    // A result that nothing reads until the end of the body would otherwise
    // be computed wherever the instruction selector puts it (at the end);
    // an empty asm statement with side effects pins it into its slot.
    u32x4 a[NS];
    u32x4 vt[NO];
    float y[NE], e[NE];
    float psum[2] = {0.f, 0.f};
    float mx = kNegInf;
    if constexpr (kNext) {
#pragma unroll
      for (int i = 0; i < KLEAD; ++i) a[i] = ld128(kaddr(i));
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) nx[kb] = f32x16{};
    }
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (kNext && i + KLEAD < NS) a[i + KLEAD] = ld128(kaddr(i + KLEAD));
      if (i + OLEAD >= NS && i + OLEAD - NS < NO) vt[i + OLEAD - NS] = read_vt(i + OLEAD - NS);
      if (i < NS) {
        if constexpr (kNext) nx[i % KB] = mfma32<T>(a[i], qreg[i / KB], nx[i % KB]);
      } else {
        const int j = i - NS;
        oacc[j % DB] = mfma32<T>(vt[j], pk[j / DB], oacc[j % DB]);
      }
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const int f = fslot(g);
        if (f == i) {
          y[2 * g] = fmaf(score(2 * g), p.scale_log2, neg_m);
          y[2 * g + 1] = fmaf(score(2 * g + 1), p.scale_log2, neg_m);
        }
        if (f + 1 == i) {
          e[2 * g] = fast_exp2(y[2 * g]);
          e[2 * g + 1] = fast_exp2(y[2 * g + 1]);
        }
        if (f + 2 == i) {
          psum[0] += e[2 * g];
          psum[1] += e[2 * g + 1];
          pk[g >> 2][g & 3] = pack2<T>(e[2 * g], e[2 * g + 1]);
          asm volatile("" : "+v"(psum[0]), "+v"(psum[1]));
        }
      }
      if constexpr (kNext) {
#pragma unroll
        for (int q = 0; q < NX / 2; ++q)
          if (i == MS + q * (NM - MS) / (NX / 2))
            mx = __builtin_elementwise_maximum(
                mx, __builtin_elementwise_maximum(nx[q >> 3][(2 * q) & 15], nx[q >> 3][(2 * q + 1) & 15]));
        if (i >= MS) asm volatile("" : "+v"(mx));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    l_run += psum[0] + psum[1];
    return xhalf_max(mx);
  };

  // Pipeline.  Stage indices are tile % STAGES and the loop is unrolled by
  // STAGES, so they are compile-time constants.  Even tiles' scores live in
  // s0, odd in s1.  A wave that sees tile t computes S(t+1) in its body; on
  // a visible tile before the block's last, when t+1 is past the wave's
  // causal limit, that result (from a stale stage) is never read.
  //
  // kSync == 2 (one barrier per two tiles): barrier k (k even) makes K(k+1),
  // K(k+2), V(k), V(k+1) visible to every wave (issued at barrier k-2, so all
  // of this wave's loads are waited for) and retires every wave's reads of
  // bodies k-2 and k-1 (K(k-1), K(k), V(k-2), V(k-1)); K(k+3), K(k+4),
  // V(k+2), V(k+3) then go into exactly those stages.  Bodies k and k+1 run
  // between barriers, and every load still has two tiles' time to land.
  //
  // kSync == 1 (one barrier per tile): barrier t makes group t (K(t+1), V(t))
  // visible and retires body t-1's reads (K(t), V(t-1)); group t+2 (K(t+3),
  // V(t+2)) is then issued into the stages K(t-1) and V(t-2) used.
  f32x16 s0[KB], s1[KB];
  auto masked = [&](int t) {
    const int n0 = t * BN;
    return n0 + BN > p.Sk || (CAUSAL && (n0 + BN - 1 > mw + diag));
  };
  auto barrier_issue = [&](int k, int u_k) {  // before body k; u_k = k % 4
    if constexpr (kSync == 2) {
      if (u_k & 1) {
        // No barrier.  The visible-tile count goes through an empty asm so
        // the compiler cannot tell that a skipped body k-1 implies a skipped
        // body k and thread the two bodies' control flow together (which
        // raises register pressure past the budget).
        asm volatile("" : "+s"(vis_tiles));
        __builtin_amdgcn_sched_barrier(0);
        return;
      }
      wait_vmcnt<0>();
      __syncthreads();
      if (k + 3 < n_tiles) issue_k((u_k + 3) % STAGES);
      if (k + 4 < n_tiles) issue_k(u_k);
      if (k + 2 < n_tiles) issue_v((u_k + 2) % STAGES);
      if (k + 3 < n_tiles) issue_v((u_k + 3) % STAGES);
    } else if constexpr (STAGES == 4) {
      sync_group(k);
      if (k + 2 < n_tiles) {
        issue_k((u_k + 3) % STAGES);
        issue_v((u_k + 2) % STAGES);
      }
    } else {
      // 2-deep: barrier k retires body k-1's reads (K(k), V(k-1)); group
      // k+1 (K(k+2), V(k+1)) goes into exactly those stages and has body
      // k's time to land.
      sync_group(k);
      if (k + 1 < n_tiles) {
        issue_k((u_k + 2) % STAGES);
        issue_v((u_k + 1) % STAGES);
      }
    }
  };
  float neg_m = 0.f;
  if (n_tiles > 0) {
    if constexpr (kSync == 2) {
      issue_k(0);
      issue_k(1);
      issue_v(0);
      issue_k(2);
      issue_v(1);
      wait_vmcnt<4 * LK>();  // K(0)
    } else if constexpr (STAGES == 2) {
      issue_k(0);
      issue_k(1);
      issue_v(0);  // group 0
      wait_vmcnt<2 * LK>();  // K(0)
    } else {
      issue_k(0);
      issue_k(1);
      issue_v(0);  // group 0
      if (n_tiles > 1) {
        issue_k(2);
        issue_v(1);  // group 1
        wait_vmcnt<2 * 2 * LK>();
      } else {
        wait_vmcnt<2 * LK>();
      }
    }
    __syncthreads();  // K(0)
    gemm0(0, s0);
    if (active(0)) neg_m = rescale(mask_max(0, s0));
  }
  // Every tile but the last in a loop unrolled by the ring depth; the last
  // tile (stage known only at run time, scores in s0 or s1 by its parity)
  // without the look-ahead score tile.  (At D = 256 the peeled copy does not
  // fit the register budget: all tiles run in the loop.)
  constexpr bool kPeel = DP <= 128;
  const int n_main = kPeel ? n_tiles - 1 : n_tiles;
  for (int t0 = 0; t0 < n_main; t0 += STAGES) {
#pragma unroll
    for (int u = 0; u < STAGES; ++u) {
      const int t = t0 + u;
      if (t >= n_main) break;
      f32x16(&cur)[KB] = (u & 1) ? s1 : s0;
      f32x16(&nxt)[KB] = (u & 1) ? s0 : s1;
      barrier_issue(t, u);
      if (active(t)) {
        float mt = body((u + 1) % STAGES, u, nxt, cur, neg_m, std::true_type{});
        if (active(t + 1)) {
          if (masked(t + 1)) mt = mask_max(t + 1, nxt);
          neg_m = rescale(mt);
        }
      }
    }
  }
  if (kPeel && n_main >= 0) {
    const int t = n_main;
    const int u = t % STAGES;
    barrier_issue(t, u);
    if (active(t)) {
      if (t & 1)
        body(0, u, s0, s1, neg_m, std::false_type{});
      else
        body(0, u, s1, s0, neg_m, std::false_type{});
    }
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
          u32x2 v = {pack2<T>(oacc[c][4 * i] * inv, oacc[c][4 * i + 1] * inv),
                     pack2<T>(oacc[c][4 * i + 2] * inv, oacc[c][4 * i + 3] * inv)};
          *reinterpret_cast<u32x2*>(ob + d) = v;
        }
      }
    if (hl == 0) {
      const float lse = l_tot > 0.f ? m_run * p.scale + __logf(l_tot) : kNegInf;
      p.lse[(int64_t)bh * p.Sq + row] = lse;
    }
  }
  };  // run_item

  const int first = p.n_mblocks - 1 - item;  // heaviest block first
  run_item(first);
  const int second = item;
  if (p.pair_items && second != first) {
    __syncthreads();  // every wave is done with the LDS ring before it is refilled
    run_item(second);
  }
}

// gfx950 tile table for the forward kernel, by head dim (padded to 64, 128
// or 256; other dims run zero-padded in the next size up) and, at D <= 128,
// by the amount of work:
//   D <= 64,  long work:  BN 64, 8 waves (2 per SIMD), 4 stages, 1 WG/CU (64 KiB LDS)
//   D <= 64,  short work: BN 64, 4 waves, 4 stages, 2 WGs/CU (64 KiB LDS each)
//   D <= 128, long work:  BN 64, 8 waves (2 per SIMD), 4 stages, 1 WG/CU (128 KiB LDS)
//   D <= 128, short work: BN 64, 4 waves, 2 stages, 2 WGs/CU (64 KiB LDS each)
//   D <= 256: BN 32, 4 waves (1 per SIMD), 4 stages, 1 WG/CU  (128 KiB LDS)
// BN = 64 keeps two 32x32 score blocks per wave per tile (two independent
// MFMA chains) while the score, operand and O registers fit the
// 256-register budget of two waves per SIMD.  The two-workgroup entries
// halve the rows per workgroup (128) and let one workgroup's prologue,
// epilogue and causal-diagonal idle waves overlap the other's tiles, at the
// price of twice the L2-to-LDS traffic per MFMA (and, at D = 128, where two
// 4-deep rings do not fit the LDS, one barrier per tile and one tile of load
// look-ahead).  They are taken for short work: a query length of at most
// 2,048 (4,096 under the causal mask, whose diagonal idles waves) or an
// 8-wave grid of fewer than 2,048 blocks (8 per CU).  Measured against the
// 8-wave entries, D = 128 bf16: 2-6% faster at S <= 2,048, 0.5-2.3% at
// causal S = 4,096, up to 31% on small grids; 0.3-1.1% slower non-causal at
// S = 4,096 and 0.7-2% slower at S = 8,192-16,384 with 2,048 or more 8-wave
// blocks.  D = 64 bf16: 6.5-9.6% faster at S <= 2,048 and causal S = 4,096,
// 49% on a small grid; even non-causal at S = 4,096, 0.9% slower causal at
// S = 16,384.
// A tile-study build fixes one D <= 128 entry for every shape (keys per
// tile, waves, workgroups per CU, ring depth): -DSK_FWD_D128_TILE=64,8,1,4,
// 64,4,2,2, 32,4,2,4 or 32,8,1,4.
struct FwdConfig {
  int dp, bn, nw, occ, stages;
};
struct FwdTile {
  int bn, nw, occ, stages;
};
#ifdef SK_FWD_D128_TILE
constexpr FwdTile kFwdD128Long{SK_FWD_D128_TILE};
constexpr FwdTile kFwdD128Short{SK_FWD_D128_TILE};
#else
constexpr FwdTile kFwdD128Long{64, 8, 1, 4};
constexpr FwdTile kFwdD128Short{64, 4, 2, 2};
#endif
static_assert(kFwdD128Long.stages == 4 || kFwdD128Long.stages == 2, "ring depth 4 or 2");
static_assert(kFwdD128Short.stages == 4 || kFwdD128Short.stages == 2, "ring depth 4 or 2");
// -DSK_FWD_D64_TILE=64,4,2,4 or 64,8,1,4 fixes one D <= 64 entry for every
// shape (tile study).
#ifdef SK_FWD_D64_TILE
constexpr FwdTile kFwdD64Long{SK_FWD_D64_TILE};
constexpr FwdTile kFwdD64Short{SK_FWD_D64_TILE};
#else
constexpr FwdTile kFwdD64Long{64, 8, 1, 4};
constexpr FwdTile kFwdD64Short{64, 4, 2, 4};
#endif

// Whether a D <= 128 forward over bh (batch, head) pairs of sq queries
// against sk keys takes the short-work entry: short query sequences or a
// small grid, unless the query blocks see long runs of keys (on average at
// least SK_FWD_LONG_KEYS, so the per-block fixed cost the short entry halves
// is small) and the long entry's workgroups fill whole rounds of the 256 CUs
// (a multiple of 256, or 2,048 or more).
static bool fwd_short(int d, int64_t bh, int sq, int sk, bool causal) {
  const int64_t n8 = (sq + 255) / 256;  // 256-row blocks of the long entry
  const int64_t blocks8 = n8 * bh;
  if (!(sq <= (causal ? 4096 : 2048) || blocks8 < 2048)) return false;
  // Keys a query row sees on average (bottom-right causal: row i sees
  // i + 1 + sk - sq of them, clamped to [0, sk]).
  const int64_t keys = !causal ? sk
                       : sk >= sq ? (int64_t)sk - sq / 2
                                  : (int64_t)sk * sk / (2 * (int64_t)sq);
  const int occ8 = d <= 64 ? kFwdD64Long.occ : kFwdD128Long.occ;
  const bool paired = causal && n8 >= 2 && (n8 + 1) / 2 * bh >= 256LL * occ8 * SK_FWD_PAIR_ROUNDS;
  const int64_t g8 = paired ? (n8 + 1) / 2 * bh : blocks8;  // long-entry workgroups
  const bool even = g8 % 256 == 0 || g8 >= 2048;
  return !(SK_FWD_LONG_KEYS > 0 && keys >= SK_FWD_LONG_KEYS && even);
}

static FwdConfig fwd_config(int d, int64_t bh, int sq, int sk, bool causal) {
  if (d <= 128) {
    const bool sh = fwd_short(d, bh, sq, sk, causal);
    const FwdTile t = d <= 64 ? (sh ? kFwdD64Short : kFwdD64Long)
                              : (sh ? kFwdD128Short : kFwdD128Long);
    return {d <= 64 ? 64 : 128, t.bn, t.nw, t.occ, t.stages};
  }
  return {256, 32, 4, 1, 4};
}

int fwd_rows_per_block(int dtype, int d, int64_t bh, int sq, int sk, bool causal) {
  (void)dtype;
  return 32 * fwd_config(d, bh, sq, sk, causal).nw;
}

int fwd_pair_min(int dtype, int d, int64_t bh, int sq, int sk, bool causal) {
  (void)dtype;
  return 256 * fwd_config(d, bh, sq, sk, causal).occ * SK_FWD_PAIR_ROUNDS;
}

template <class T, int DP, int BN, int NW, int OCC, int STAGES = 4>
static KernelPlan plan_fwd_t(const FwdParams& p, bool causal) {
  KernelPlan k;
  const bool rope = p.rope.cos != nullptr;
  if (causal && !rope)
    k.fn = (const void*)fwd_mfma_kernel<T, DP, BN, NW, STAGES, OCC, true, false>;
  else if (!rope)
    k.fn = (const void*)fwd_mfma_kernel<T, DP, BN, NW, STAGES, OCC, false, false>;
  else if (causal)
    k.fn = (const void*)fwd_mfma_kernel<T, DP, BN, NW, STAGES, OCC, true, true>;
  else
    k.fn = (const void*)fwd_mfma_kernel<T, DP, BN, NW, STAGES, OCC, false, true>;
  k.grid = dim3((unsigned)(p.n_items * p.B * p.Hq));
  k.block = dim3(NW * 64);
  k.kernel = "fwd_mfma_kernel";
  k.elem = T::code;
  k.head_dim = DP;
  k.block_m = 32 * NW;
  k.block_n = BN;
  k.stages = STAGES;
  k.causal = causal;
  k.rope = rope;
  return k;
}

template <class T>
static KernelPlan plan_fwd_dt(const FwdParams& p, bool causal) {
  const bool sh = fwd_short(p.D, (int64_t)p.B * p.Hq, p.Sq, p.Sk, causal);
  switch (fwd_config(p.D, (int64_t)p.B * p.Hq, p.Sq, p.Sk, causal).dp) {
    case 64:
      if (sh)
        return plan_fwd_t<T, 64, kFwdD64Short.bn, kFwdD64Short.nw, kFwdD64Short.occ,
                          kFwdD64Short.stages>(p, causal);
      return plan_fwd_t<T, 64, kFwdD64Long.bn, kFwdD64Long.nw, kFwdD64Long.occ,
                        kFwdD64Long.stages>(p, causal);
    case 128:
      if (sh)
        return plan_fwd_t<T, 128, kFwdD128Short.bn, kFwdD128Short.nw, kFwdD128Short.occ,
                          kFwdD128Short.stages>(p, causal);
      return plan_fwd_t<T, 128, kFwdD128Long.bn, kFwdD128Long.nw, kFwdD128Long.occ,
                        kFwdD128Long.stages>(p, causal);
    default:
      return plan_fwd_t<T, 256, 32, 4, 1>(p, causal);
  }
}

KernelPlan plan_fwd_mfma(int dtype, const FwdParams& p, bool causal) {
  if (p.D > 256) return KernelPlan{};
  if (dtype == BF16::code) return plan_fwd_dt<BF16>(p, causal);
  if (dtype == F16::code) return plan_fwd_dt<F16>(p, causal);
  return KernelPlan{};
}

hipError_t launch_fwd_mfma(int dtype, const FwdParams& p, bool causal, hipStream_t s) {
  const KernelPlan k = plan_fwd_mfma(dtype, p, causal);
  if (!k.fn) return hipErrorInvalidValue;
  return run_plan(k, &p, s);
}

hipError_t run_plan(const KernelPlan& k, const void* params, hipStream_t s) {
  if (!k.fn) return hipErrorInvalidValue;
  if ((uint64_t)k.grid.x * k.grid.y * k.grid.z == 0) return hipSuccess;
  void* args[] = {const_cast<void*>(params)};
  const hipError_t e = hipLaunchKernel(k.fn, k.grid, k.block, args, 0, s);
  return e != hipSuccess ? e : hipGetLastError();
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
