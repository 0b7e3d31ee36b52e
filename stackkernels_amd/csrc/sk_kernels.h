// Kernel parameter blocks and host-side launcher declarations shared by the
// kernel translation units and the C-ABI layer (sk_abi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

// Causal forward: blocks j and n_mblocks-1-j run in one workgroup when the
// paired workgroups still fill SK_FWD_PAIR_ROUNDS rounds of the 256 CUs at
// the table entry's workgroups per CU (a tile-study build can raise it to
// keep every block on its own).
#ifndef SK_FWD_PAIR_ROUNDS
#define SK_FWD_PAIR_ROUNDS 1
#endif
// Forward tile table: average visible keys per query row from which the
// long-work entry is taken when its workgroups fill whole rounds of the CUs
// (0: query length and grid size alone decide).
#ifndef SK_FWD_LONG_KEYS
#define SK_FWD_LONG_KEYS 4096
#endif

namespace sk {

// Rotary position embedding (rotate-half form) applied to a vector as it is
// loaded.  Token t of batch row b sits at position
// pos = (pos_b ? pos_b[b] : 0) + start + t, and element d of its rotated
// head vector is
//   x[d] * cos[pos][d] - x[d + D/2] * sin[pos][d]   for d <  D/2,
//   x[d] * cos[pos][d] + x[d - D/2] * sin[pos][d]   for d >= D/2,
// each product and the sum rounded to fp32 (no fused multiply-add), then
// rounded to the tensor's element type.  A position outside [0, rows) leaves
// the vector as it is.  cos == nullptr switches the rotation off.
struct RopeParams {
  const void* cos;  // (rows, >= D) tables, element stride `stride` between rows
  const void* sin;
  int64_t stride;
  int rows;
  int dtype;  // SK_F32 / SK_F16 / SK_BF16 element type of both tables
  const int* pos_b;
  int start;
};

// Forward attention, prefill shape.  Strides are element strides.
struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int B, Hq, Hkv, Sq, Sk, D, group;
  int n_mblocks;     // ceil(Sq / rows per workgroup)
  int n_items;       // work items per (batch, head): n_mblocks, or ceil(n_mblocks/2) if paired
  int pair_items;    // 1: item j runs query blocks n_mblocks-1-j and j
  float scale;       // |sm_scale|
  float scale_log2;  // |sm_scale| * log2(e)
  uint32_t q_sign;   // 0, or the sign-bit mask that negates q when sm_scale < 0
  // Decode only (fp32 path, non-causal): null, or per-batch-row key counts;
  // row b sees keys [0, clamp(seqlens[b], 0, Sk)).
  const int* seqlens;
  // Decode only: null, or a paged cache (see DecParams).
  const int* block_table;
  int page_size, max_pages, num_pages;
  // Rotation of q on load; query row i of batch row b is token i.
  RopeParams rope;
};

// Split-KV decode (Sq == 1).
struct DecParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* part_o;    // [B*Hq][num_splits][dpad] fp32, normalised per split
  float* part_lse;  // [B*Hq][num_splits]
  int64_t q_sb, q_sh;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh;
  int B, Hq, Hkv, Sk, D, group;
  int num_splits, keys_per_split, dpad;
  float scale, scale_log2;
  uint32_t q_sign;
  // Null, or per-batch-row key counts: row b sees keys [0, clamp(seqlens[b], 0, Sk)).
  const int* seqlens;
  // With seqlens: 1 hands batch rows to workgroups longest first (the
  // kernels rank the lengths themselves; the host sets it for B <= 256).
  int longest_first;
  // Null (k/v are (B, Hkv, Sk, D)), or a paged cache: k/v are pools of
  // num_pages pages (k_sb / v_sb is the page stride) of page_size keys, and
  // key n of row b is in-page row n % page_size of page
  // block_table[b * max_pages + n / page_size] (Sk = max_pages * page_size).
  // page_size is a multiple of 32; a page index outside the pool masks its keys.
  const int* block_table;
  int page_size, max_pages, num_pages;
  // Rotation of q on load (the query is token 0 of its batch row).
  RopeParams rope;
};

// Backward attention; every tensor contiguous BHSD.
struct BwdParams {
  const void* dout;
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const float* lse;
  void* dq;
  void* dk;
  void* dv;
  float* delta;     // [B*Hq*Sq] fp32 scratch: rowsum(dO * O)
  float* lse_log2;  // [B*Hq*Sq] fp32 scratch: lse * log2(e) (+inf for empty rows)
  float* dq_acc;    // [B*Hq*Sq*D] fp32 scratch (dQ accumulator) or null
  // dS tiles of 32 keys x 32 queries (16-bit, key-major rows of 64 bytes) of
  // the launch's (batch, KV head) pairs, in the DsLayout order below, written
  // by the dK/dV kernel and read by the dQ kernel of the five-GEMM backward;
  // null for the seven-GEMM backward.
  void* ds;
  int ds_nqt;             // query tiles per head: ceil(Sq / 32)
  int ds_c;               // causal: ceil((Sk - Sq) / 32); else unused
  int64_t ds_head_tiles;  // tiles per query head
  // First (batch, KV head) pair, b * Hkv + h_kv, of this launch and the pair
  // count: the five-GEMM backward runs the pairs in chunks whose dS tiles
  // fit the workspace; every other launch covers all B * Hkv pairs.
  int bk0, n_pairs;
  int B, Hq, Hkv, Sq, Sk, D, group;
  float scale, scale_log2;  // signed sm_scale and sm_scale * log2(e)
  // MFMA kernels: the score exponent uses |sm_scale| * log2(e) (never 0, so a
  // masked -inf score stays -inf), and op_sign flips the sign bits of the
  // register-resident score operand when sm_scale < 0.
  float abs_scale_log2;
  uint32_t op_sign;
  int n_mblocks, n_nblocks;
};

// dS tile layout of the five-GEMM backward, per query head.  The dK/dV
// workgroup of key block kb (keys 128 kb .. 128 kb + 127) walks the query
// tiles [qb(kb), nqt): under the bottom-right causal mask the first tile
// whose last row sees key 128 kb, qb(kb) = max(0, 4 kb - c) with
// c = ceil((Sk - Sq) / 32); without the mask 0.  Block kb holds
// cnt(kb) = max(0, nqt - qb(kb)) tiles for each of its four 32-key tiles,
// key tile kt = 4 kb + j at tile 4 off(kb) + j cnt(kb) + (qt - qb(kb)) of the
// head, off(kb) = cnt(0) + ... + cnt(kb - 1): only the tiles some visible
// key block writes are allocated (about half of the rectangle for a square
// causal shape).
__host__ __device__ inline int ds_causal_c(int Sq, int Sk) {
  const int d = Sk - Sq;
  return d >= 0 ? (d + 31) / 32 : -((-d) / 32);  // ceil(d / 32)
}
__host__ __device__ inline int ds_qb(int kb, int c, bool causal) {
  return causal ? (4 * kb - c > 0 ? 4 * kb - c : 0) : 0;
}
__host__ __device__ inline int ds_cnt(int kb, int nqt, int c, bool causal) {
  const int r = nqt - ds_qb(kb, c, causal);
  return r > 0 ? r : 0;
}
// off(kb) in closed form: cnt(k) = nqt while 4 k <= c, nqt + c - 4 k while
// c < 4 k < nqt + c, then 0.
__host__ __device__ inline int64_t ds_off(int kb, int nqt, int c, bool causal) {
  if (!causal) return (int64_t)kb * nqt;
  const int64_t a = (int64_t)nqt + c;
  const int64_t full = c >= 0 ? c / 4 + 1 : 0;   // k with 4 k <= c
  const int64_t live = a > 0 ? (a + 3) / 4 : 0;  // k with 4 k < nqt + c
  const int64_t k1 = kb < full ? kb : full;
  int64_t s = k1 * nqt;
  const int64_t hi = kb < live ? kb : live;
  if (hi > full) s += (hi - full) * a - 2 * (hi - full) * (hi + full - 1);
  return s;
}
// Tiles per query head for nkb key blocks.
__host__ __device__ inline int64_t ds_head_tiles(int nkb, int nqt, int c, bool causal) {
  return 4 * ds_off(nkb, nqt, c, causal);
}

// KV-cache append: k_cache[b, h, slots[b*T + t], :] = k[b, h, t, :], same for v.
// Strides are element strides (b, h, s); the head dim is contiguous.
struct CacheParams {
  const void* k;
  const void* v;
  void* kc;
  void* vc;
  const int64_t* slots;  // [B*T]; a slot outside [0, S) skips that token
  // 0: the caches are (B, Hkv, S, D) and a slot is a row of batch row b's cache.
  // > 0: the caches are pools of S / page_size pages (kc_sb / vc_sb is the page
  // stride) and slot s is in-page row s % page_size of page s / page_size.
  int page_size;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t kc_sb, kc_sh, kc_ss;
  int64_t vc_sb, vc_sh, vc_ss;
  int B, Hkv, T;
  int64_t S;      // slots: rows per batch row's cache, or num_pages * page_size
  int esize;      // bytes per element
  int row_bytes;  // D * esize
  int dtype;      // SK_F32 / SK_F16 / SK_BF16 (used by the rotating kernel)
  int D;
  // Rotation of the new keys before they are written (new token t of batch
  // row b is token t); values are copied unchanged.
  RopeParams rope;
};

// Rotation of a (B, H, S, D) tensor by its RoPE angles (inverse = 0) or by
// their negatives, the adjoint (inverse = 1): token t of batch row b at the
// position RopeParams gives it.  out may be x (in place).  Strides are
// element strides (b, h, s); the head dim is contiguous.
struct RotateParams {
  const void* x;
  void* out;
  int64_t x_sb, x_sh, x_ss;
  int64_t o_sb, o_sh, o_ss;
  int B, H, S, D;
  int dtype;  // SK_F32 / SK_F16 / SK_BF16
  int inverse;
  RopeParams rope;
};

// What a launcher runs for given parameters: the kernel, its grid and block,
// and the tile configuration of that instantiation.  Each launcher builds its
// plan with the plan_* function below and launches exactly that plan, and
// sk_kernel_config reports the same plan, so the introspection cannot drift
// from what runs.
struct KernelPlan {
  const void* fn = nullptr;  // the __global__ function; null: nothing to launch
  dim3 grid = dim3(0), block = dim3(0);
  const char* kernel = "";   // kernel family name
  int elem = -1;             // element type it is compiled for (SK_F32/F16/BF16)
  int head_dim = 0;          // padded head dim it is compiled for
  int block_m = 0;           // query rows per workgroup (decode: query heads)
  int block_n = 0;           // keys per tile (dK/dV: keys per workgroup)
  int stages = 0;            // tile ring depth (0: tiles staged in registers)
  bool causal = false, paged = false, rope = false;
};
// Launch plan k with the kernel's single parameter block.
hipError_t run_plan(const KernelPlan& k, const void* params, hipStream_t s);

KernelPlan plan_fwd_mfma(int dtype, const FwdParams& p, bool causal);
KernelPlan plan_fwd_f32(const FwdParams& p, bool causal);
// Query rows per workgroup of the fp32 forward for head dim d and sq queries.
int fwd_f32_rows_per_block(int d, int sq);
KernelPlan plan_decode_mfma(int dtype, const DecParams& p);
KernelPlan plan_decode_combine(int dtype, const DecParams& p);
// The backward plans fill the block counts of p they derive.
KernelPlan plan_bwd_dkv(int dtype, BwdParams& p, bool causal);
KernelPlan plan_bwd_dq(int dtype, BwdParams& p, bool causal);
// Bytes of dS tiles the five-GEMM backward needs per (batch, KV head) pair
// (its query heads' tiles), or 0 where the seven-GEMM backward runs (head
// dims other than 65-128, fp32).
size_t bwd_ds_pair_bytes(int dtype, int Hq, int Hkv, int Sq, int Sk, int D, bool causal);
KernelPlan plan_bwd_dkv_f32(BwdParams& p, bool causal);
KernelPlan plan_bwd_dq_f32(BwdParams& p, bool causal);

// Launchers: return hipSuccess or the launch error.  dtype is SK_F32/F16/BF16.
hipError_t launch_fwd_mfma(int dtype, const FwdParams& p, bool causal, hipStream_t s);
hipError_t launch_fwd_f32(const FwdParams& p, bool causal, hipStream_t s);
hipError_t launch_decode_mfma(int dtype, const DecParams& p, hipStream_t s);
hipError_t launch_decode_combine(int dtype, const DecParams& p, hipStream_t s);
hipError_t launch_bwd_prep(int dtype, const BwdParams& p, hipStream_t s);
hipError_t launch_bwd_mfma(int dtype, const BwdParams& p, bool causal, hipStream_t s);
hipError_t launch_bwd_f32(const BwdParams& p, bool causal, hipStream_t s);
hipError_t launch_kv_cache_update(const CacheParams& p, hipStream_t s);
hipError_t launch_rope_rotate(const RotateParams& p, hipStream_t s);

// Rows of queries one forward workgroup covers for (dtype, head dim, batch x
// query heads, query length, key length, causal mask).
int fwd_rows_per_block(int dtype, int d, int64_t bh, int sq, int sk, bool causal);
// Fewest paired workgroups for which a causal forward of that shape pairs
// its query blocks.
int fwd_pair_min(int dtype, int d, int64_t bh, int sq, int sk, bool causal);
// Padded head dim the kernels are compiled for (64, 96, 128 or 256), or 0.
int padded_head_dim(int d);

}  // namespace sk
