// extern "C" entry points of libsk_attn.so (declared in include/sk_attn.h).
//
// This layer validates arguments, fills the kernel parameter blocks, applies
// the gfx950 split table for decode, and launches on the caller's stream.  It
// never allocates device memory and never synchronises the host.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <cmath>
#include <mutex>

#include "sk_attn.h"
#include "sk_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
  return (int)e;
}

int elem_bytes(int dtype) { return dtype == SK_F32 ? 4 : 2; }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Common shape checks; messages follow the reference's
// validate_attention_layout (src/stackkernels/_opt/memory/layout.py:19-39).
int check_dims(int dtype, int B, int Hq, int Hkv, int Sq, int Sk, int D) {
  if (dtype != SK_F32 && dtype != SK_F16 && dtype != SK_BF16)
    return fail(SK_EUNSUPPORTED, "unsupported dtype code %d", dtype);
  if (B < 0 || Hq < 0 || Hkv <= 0 || Sq < 0 || Sk < 0 || D <= 0)
    return fail(SK_EINVAL, "invalid sizes B=%d Hq=%d Hkv=%d Sq=%d Sk=%d D=%d", B, Hq, Hkv, Sq, Sk, D);
  if (Hq % Hkv != 0)
    return fail(SK_EINVAL, "Query heads (%d) must be divisible by KV heads (%d) for GQA/MQA", Hq, Hkv);
  if (sk::padded_head_dim(D) == 0)
    return fail(SK_EUNSUPPORTED, "head dim %d unsupported: need a multiple of 8 in [8, 256]", D);
  return SK_OK;
}

int check_strides(int dtype, const char* name, const int64_t* st) {
  if (!st) return fail(SK_EINVAL, "%s strides pointer is NULL", name);
  const int64_t unit = dtype == SK_F32 ? 4 : 8;  // 16 bytes in elements
  for (int i = 0; i < 3; ++i)
    if (st[i] < 0 || st[i] % unit != 0)
      return fail(SK_EINVAL, "%s stride[%d]=%lld must be a non-negative multiple of %lld elements",
                  name, i, (long long)st[i], (long long)unit);
  return SK_OK;
}

int check_ptr(const char* name, const void* p) {
  if (!p) return fail(SK_EINVAL, "%s pointer is NULL", name);
  if (!aligned16(p)) return fail(SK_EINVAL, "%s pointer is not 16-byte aligned", name);
  return SK_OK;
}

// gfx950 decode split table.  A split is one workgroup per (batch, KV head);
// the table sizes the split count to the workgroups the chip holds at once,
// counted as eight waves per CU (16 query heads per wave: 1, 2 or 4 waves per
// workgroup):
// * groups of up to 16 heads (one-wave workgroups): one round with a
//   uniform cache length (every split the same size; C4: 4 splits, 1.7%
//   faster than two rounds), about two rounds with per-row lengths and over
//   paged pools (per_row), whose rows spread their keys over their splits so
//   a row shorter than the longest leaves a one-round grid uneven (8
//   splits: 6.9% and 7.7% faster than 4 at the C4 shape with lengths U[1, Sk]);
// * 32- and 64-head groups: exactly one round, so no split waits for a second
//   round; a 64-head group writes 32 KB of partials per split, so fewer,
//   longer splits also keep that traffic small (C5: 64 splits; 32 and 128
//   splits measured 15% and 10% slower).
// Every split keeps at least 256 keys (8 tiles) and the count is capped at
// 1024 (the combine kernel's LDS weight array).
int plan_splits(int B, int Hq, int Hkv, int Sk, int D, bool per_row) {
  (void)D;
  if (Sk <= 0 || B <= 0 || Hkv <= 0) return 1;
  const int group = Hq / Hkv;
  const int waves = group <= 16 ? 1 : group <= 32 ? 2 : 4;
  const int64_t slots = 256LL * 8 / waves;
  const int rounds = group <= 16 && per_row ? 2 : 1;
  const int64_t units = (int64_t)B * Hkv;
  int64_t splits = (rounds * slots + units - 1) / units;
  splits = std::min<int64_t>(splits, std::max(1, Sk / 256));
  splits = std::max<int64_t>(1, std::min<int64_t>(splits, 1024));
  return (int)splits;
}

int keys_per_split_for(int Sk, int splits) {
  int kps = (Sk + splits - 1) / splits;
  kps = (kps + 31) / 32 * 32;
  return std::max(kps, 32);
}

size_t decode_ws_bytes(int dtype, int B, int Hq, int D, int splits) {
  if (dtype == SK_F32) return (size_t)B * Hq * sizeof(float);  // LSE of the fp32 forward
  if (splits <= 1) return 0;
  const size_t dpad = (size_t)sk::padded_head_dim(D);
  return (size_t)B * Hq * splits * (dpad + 1) * sizeof(float);
}

// RoPE arguments of the *_rope entry points -> r.  `tokens` is the number of
// consecutive positions each batch row uses from its base (1 for decode, T
// for the cache append, Sq for the forward).  With one base for the whole
// batch (rope_pos NULL) the positions [rope_start, rope_start + tokens) must
// lie in the table, as the reference's table slice
// cos[start_pos : start_pos + seq_len] requires
// (src/stackkernels/_reference/torch/rope.py:49-50).
int make_rope(const void* cos, const void* sin, int rope_dtype, int rope_rows,
              int64_t rope_stride, const int32_t* rope_pos, int rope_start, int D, int tokens,
              sk::RopeParams* r) {
  if (!cos || !sin) return fail(SK_EINVAL, "rope cos/sin pointer is NULL");
  if (rope_dtype != SK_F32 && rope_dtype != SK_F16 && rope_dtype != SK_BF16)
    return fail(SK_EUNSUPPORTED, "unsupported rope table dtype code %d", rope_dtype);
  if (D % 16 != 0)
    return fail(SK_EUNSUPPORTED, "RoPE needs a head dim that is a multiple of 16, got %d", D);
  if (rope_rows <= 0 || rope_stride < D)
    return fail(SK_EINVAL, "rope table of %d rows with row stride %lld for head dim %d", rope_rows,
                (long long)rope_stride, D);
  if (!aligned16(cos) || !aligned16(sin) || (rope_stride * elem_bytes(rope_dtype)) % 16 != 0)
    return fail(SK_EINVAL, "rope tables must be 16-byte aligned with a row stride that is a "
                "multiple of 16 bytes");
  if (!rope_pos && tokens > 0 &&
      (rope_start < 0 || (int64_t)rope_start + tokens > (int64_t)rope_rows))
    return fail(SK_EINVAL, "positions [%d, %lld) lie outside the rope table of %d rows", rope_start,
                (long long)rope_start + tokens, rope_rows);
  r->cos = cos, r->sin = sin;
  r->stride = rope_stride;
  r->rows = rope_rows;
  r->dtype = rope_dtype;
  r->pos_b = rope_pos;
  r->start = rope_start;
  return SK_OK;
}

// Backward scratch: delta and lse * log2(e) (fp32 per query row, each array
// rounded up to 256 bytes), then, for the five-GEMM backward, the dS tiles of
// one chunk of (batch, KV head) pairs.
size_t bwd_rows_bytes(int B, int Hq, int Sq) {
  const size_t rows = (size_t)B * Hq * Sq;
  return 2 * ((rows * sizeof(float) + 255) / 256 * 256);
}

// Pairs per chunk of the five-GEMM backward when at most `budget` bytes of
// dS tiles fit (0: the seven-GEMM backward runs).  The chunks are as even as
// the budget allows: ceil(pairs / chunks) with the fewest chunks that fit.
int64_t bwd_chunk_pairs(int64_t pairs, size_t pair_bytes, size_t budget) {
  if (pairs <= 0 || pair_bytes == 0 || budget < pair_bytes) return 0;
  const int64_t fit = std::min<int64_t>(pairs, (int64_t)(budget / pair_bytes));
  const int64_t chunks = (pairs + fit - 1) / fit;
  return (pairs + chunks - 1) / chunks;
}

// Bytes sk_attn_bwd_workspace reports: the row statistics plus one chunk of
// dS tiles under SK_BWD_DS_CAP_BYTES.
size_t bwd_ws_bytes(int dtype, int B, int Hq, int Hkv, int Sq, int Sk, int D, bool causal) {
  const size_t pair = sk::bwd_ds_pair_bytes(dtype, Hq, Hkv, Sq, Sk, D, causal);
  const int64_t chunk = bwd_chunk_pairs((int64_t)B * Hkv, pair, (size_t)SK_BWD_DS_CAP_BYTES);
  return bwd_rows_bytes(B, Hq, Sq) + (size_t)chunk * pair;
}

}  // namespace

extern "C" {

int sk_abi_version(void) { return SK_ABI_VERSION; }

const char* sk_last_error(void) { return g_err; }

}  // extern "C"

// Sizes and work split of the forward: query blocks per (b, h) and, under
// the causal mask, whether blocks j and n_mblocks-1-j are paired in one
// workgroup (when that still leaves enough workgroups: fwd_pair_min).
static int fwd_shape(int dtype, int B, int Hq, int Hkv, int Sq, int Sk, int D, int is_causal,
                     sk::FwdParams* p) {
  p->B = B, p->Hq = Hq, p->Hkv = Hkv, p->Sq = Sq, p->Sk = Sk, p->D = D, p->group = Hq / Hkv;
  const int rows = dtype == SK_F32 ? sk::fwd_f32_rows_per_block(D, Sq)
                                   : sk::fwd_rows_per_block(dtype, D, (int64_t)B * Hq, Sq, Sk, is_causal != 0);
  p->n_mblocks = (Sq + rows - 1) / rows;
  if ((int64_t)p->n_mblocks * B * Hq > 0x7fffffffLL)
    return fail(SK_EINVAL, "grid too large: %lld workgroups", (long long)p->n_mblocks * B * Hq);
  p->pair_items = dtype != SK_F32 && is_causal && p->n_mblocks >= 2 &&
                  (int64_t)((p->n_mblocks + 1) / 2) * B * Hq >=
                      sk::fwd_pair_min(dtype, D, (int64_t)B * Hq, Sq, Sk, is_causal != 0);
  p->n_items = p->pair_items ? (p->n_mblocks + 1) / 2 : p->n_mblocks;
  return SK_OK;
}

// Split count and keys per split of a decode call (num_splits 0: the gfx950
// table's pick).  fp32 decode runs unsplit.
static int decode_splits(int dtype, int B, int Hq, int Hkv, int Sk, int D, bool per_row, int num_splits,
                         int* splits, int* kps) {
  if (dtype == SK_F32) num_splits = 1;
  if (num_splits == 0) num_splits = plan_splits(B, Hq, Hkv, Sk, D, per_row);
  if (num_splits < 1 || num_splits > 1024)
    return fail(SK_EINVAL, "num_splits=%d outside [1, 1024]", num_splits);
  *kps = keys_per_split_for(Sk, num_splits);
  if (Sk > 0) num_splits = std::min(num_splits, (Sk + *kps - 1) / *kps);
  *splits = num_splits;
  return SK_OK;
}

// sk_attn_fwd and sk_attn_fwd_rope.
static int fwd_impl(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                    int B, int Hq, int Hkv, int Sq, int Sk, int D, const int64_t* q_strides,
                    const int64_t* k_strides, const int64_t* v_strides,
                    const int64_t* o_strides, int is_causal, const sk::RopeParams& rope,
                    float sm_scale, void* stream) {
  int rc = check_dims(dtype, B, Hq, Hkv, Sq, Sk, D);
  if (rc) return rc;
  if ((rc = check_strides(dtype, "q", q_strides)) || (rc = check_strides(dtype, "k", k_strides)) ||
      (rc = check_strides(dtype, "v", v_strides)) || (rc = check_strides(dtype, "o", o_strides)))
    return rc;
  if ((int64_t)B * Hq * Sq == 0) return SK_OK;
  if ((rc = check_ptr("q", q)) || (rc = check_ptr("o", o)) || (rc = check_ptr("lse", lse)))
    return rc;
  if (Sk > 0 && ((rc = check_ptr("k", k)) || (rc = check_ptr("v", v)))) return rc;

  sk::FwdParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.lse = lse;
  p.q_sb = q_strides[0], p.q_sh = q_strides[1], p.q_ss = q_strides[2];
  p.k_sb = k_strides[0], p.k_sh = k_strides[1], p.k_ss = k_strides[2];
  p.v_sb = v_strides[0], p.v_sh = v_strides[1], p.v_ss = v_strides[2];
  p.o_sb = o_strides[0], p.o_sh = o_strides[1], p.o_ss = o_strides[2];
  p.scale = std::fabs(sm_scale);
  p.scale_log2 = p.scale * 1.4426950408889634f;
  const bool neg = sm_scale < 0.f;
  if ((rc = fwd_shape(dtype, B, Hq, Hkv, Sq, Sk, D, is_causal, &p))) return rc;
  p.rope = rope;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  if (dtype == SK_F32) {
    p.q_sign = neg ? 1u : 0u;
    e = sk::launch_fwd_f32(p, is_causal != 0, s);
  } else {
    p.q_sign = neg ? 0x80008000u : 0u;
    e = sk::launch_fwd_mfma(dtype, p, is_causal != 0, s);
  }
  if (e != hipSuccess) return hip_fail(e, "sk_attn_fwd launch");
  return SK_OK;
}

extern "C" {

int sk_attn_fwd(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                int B, int Hq, int Hkv, int Sq, int Sk, int D, const int64_t* q_strides,
                const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
                int is_causal, float sm_scale, void* stream) {
  g_err[0] = 0;
  return fwd_impl(dtype, q, k, v, o, lse, B, Hq, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides,
                  o_strides, is_causal, sk::RopeParams{}, sm_scale, stream);
}

int sk_attn_fwd_rope(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                     int B, int Hq, int Hkv, int Sq, int Sk, int D, const int64_t* q_strides,
                     const int64_t* k_strides, const int64_t* v_strides,
                     const int64_t* o_strides, int is_causal, const void* rope_cos,
                     const void* rope_sin, int rope_dtype, int rope_rows, int64_t rope_stride,
                     const int32_t* rope_pos, int rope_start, float sm_scale, void* stream) {
  g_err[0] = 0;
  sk::RopeParams r{};
  const int rc = make_rope(rope_cos, rope_sin, rope_dtype, rope_rows, rope_stride, rope_pos,
                           rope_start, D, (int64_t)B * Hq > 0 ? Sq : 0, &r);
  if (rc) return rc;
  return fwd_impl(dtype, q, k, v, o, lse, B, Hq, Hkv, Sq, Sk, D, q_strides, k_strides, v_strides,
                  o_strides, is_causal, r, sm_scale, stream);
}

int sk_attn_bwd_workspace(int dtype, int B, int Hq, int Hkv, int Sq, int Sk, int D, int is_causal,
                          size_t* bytes) {
  g_err[0] = 0;
  int rc = check_dims(dtype, B, Hq, Hkv, Sq, Sk, D);
  if (rc) return rc;
  if (!bytes) return fail(SK_EINVAL, "bytes pointer is NULL");
  *bytes = bwd_ws_bytes(dtype, B, Hq, Hkv, Sq, Sk, D, is_causal != 0);
  return SK_OK;
}

int sk_attn_bwd_workspace_min(int dtype, int B, int Hq, int Hkv, int Sq, int Sk, int D,
                              int is_causal, size_t* bytes) {
  g_err[0] = 0;
  (void)is_causal;
  int rc = check_dims(dtype, B, Hq, Hkv, Sq, Sk, D);
  if (rc) return rc;
  if (!bytes) return fail(SK_EINVAL, "bytes pointer is NULL");
  *bytes = bwd_rows_bytes(B, Hq, Sq);
  return SK_OK;
}

int sk_attn_bwd(int dtype, const void* dout, const void* q, const void* k, const void* v,
                const void* o, const float* lse, void* dq, void* dk, void* dv, void* workspace,
                size_t workspace_bytes, int B, int Hq, int Hkv, int Sq, int Sk, int D,
                int is_causal, float sm_scale, void* stream) {
  g_err[0] = 0;
  int rc = check_dims(dtype, B, Hq, Hkv, Sq, Sk, D);
  if (rc) return rc;
  if ((int64_t)B * Hq * Sq == 0 && (int64_t)B * Hkv * Sk == 0) return SK_OK;
  const size_t need = bwd_rows_bytes(B, Hq, Sq);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(SK_EWORKSPACE, "workspace of %zu bytes given, at least %zu needed",
                workspace_bytes, need);
  if ((int64_t)B * Hq * Sq > 0 &&
      ((rc = check_ptr("dout", dout)) || (rc = check_ptr("q", q)) || (rc = check_ptr("o", o)) ||
       (rc = check_ptr("lse", lse)) || (rc = check_ptr("dq", dq))))
    return rc;
  if ((int64_t)B * Hkv * Sk > 0 && ((rc = check_ptr("k", k)) || (rc = check_ptr("v", v)) ||
                                    (rc = check_ptr("dk", dk)) || (rc = check_ptr("dv", dv))))
    return rc;
  if (need > 0 && (rc = check_ptr("workspace", workspace))) return rc;

  sk::BwdParams p{};
  p.dout = dout, p.q = q, p.k = k, p.v = v, p.o = o, p.lse = lse;
  p.dq = dq, p.dk = dk, p.dv = dv;
  const size_t rows = (size_t)B * Hq * Sq;
  const size_t rows_bytes = (rows * sizeof(float) + 255) / 256 * 256;
  p.delta = (float*)workspace;
  p.lse_log2 = (float*)((char*)workspace + rows_bytes);
  p.dq_acc = nullptr;
  // The five-GEMM backward where its dS tiles for at least one (batch, KV
  // head) pair fit the workspace past the row statistics (at most
  // SK_BWD_DS_CAP_BYTES of it used); else the seven-GEMM backward.
  const size_t pair_bytes = sk::bwd_ds_pair_bytes(dtype, Hq, Hkv, Sq, Sk, D, is_causal != 0);
  const size_t ds_budget =
      std::min<size_t>(workspace_bytes - std::min(workspace_bytes, need), (size_t)SK_BWD_DS_CAP_BYTES);
  const int64_t chunk = bwd_chunk_pairs((int64_t)B * Hkv, pair_bytes, ds_budget);
  p.ds = chunk > 0 ? (char*)workspace + need : nullptr;
  p.n_pairs = (int)chunk;
  p.bk0 = 0;
  p.ds_nqt = (Sq + 31) / 32;
  p.ds_c = sk::ds_causal_c(Sq, Sk);
  p.ds_head_tiles = sk::ds_head_tiles((Sk + 127) / 128, p.ds_nqt, p.ds_c, is_causal != 0);
  p.B = B, p.Hq = Hq, p.Hkv = Hkv, p.Sq = Sq, p.Sk = Sk, p.D = D, p.group = Hq / Hkv;
  p.scale = sm_scale;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  // |s| * 1e-30 * log2(e) rounds to 0 next to any finite score, so a zero
  // scale still gives P = exp2(-lse * log2 e) exactly while -inf stays -inf.
  p.abs_scale_log2 = std::max(std::fabs(sm_scale), 1e-30f) * 1.4426950408889634f;
  p.op_sign = sm_scale < 0.f ? 0x80008000u : 0u;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipSuccess;
  if (rows > 0) e = sk::launch_bwd_prep(dtype, p, s);
  if (e != hipSuccess) return hip_fail(e, "sk_attn_bwd preprocess launch");
  if (dtype == SK_F32)
    e = sk::launch_bwd_f32(p, is_causal != 0, s);
  else
    e = sk::launch_bwd_mfma(dtype, p, is_causal != 0, s);
  if (e != hipSuccess) return hip_fail(e, "sk_attn_bwd launch");
  return SK_OK;
}

static int decode_plan_impl(int dtype, int B, int Hq, int Hkv, int Sk, int D, bool per_row,
                            int* num_splits, size_t* workspace_bytes) {
  int rc = check_dims(dtype, B, Hq, Hkv, 1, Sk, D);
  if (rc) return rc;
  if (!num_splits || !workspace_bytes) return fail(SK_EINVAL, "output pointer is NULL");
  int splits = dtype == SK_F32 ? 1 : plan_splits(B, Hq, Hkv, Sk, D, per_row);
  if (splits > 1) splits = (Sk + keys_per_split_for(Sk, splits) - 1) / keys_per_split_for(Sk, splits);
  *num_splits = splits;
  *workspace_bytes = decode_ws_bytes(dtype, B, Hq, D, splits);
  return SK_OK;
}

int sk_decode_plan(int dtype, int B, int Hq, int Hkv, int Sk, int D, int* num_splits,
                   size_t* workspace_bytes) {
  g_err[0] = 0;
  return decode_plan_impl(dtype, B, Hq, Hkv, Sk, D, false, num_splits, workspace_bytes);
}

int sk_decode_plan_varlen(int dtype, int B, int Hq, int Hkv, int Sk, int D, int* num_splits,
                          size_t* workspace_bytes) {
  g_err[0] = 0;
  return decode_plan_impl(dtype, B, Hq, Hkv, Sk, D, true, num_splits, workspace_bytes);
}

int sk_decode_workspace(int dtype, int B, int Hq, int Hkv, int Sk, int D, int num_splits,
                        size_t* workspace_bytes) {
  g_err[0] = 0;
  int rc = check_dims(dtype, B, Hq, Hkv, 1, Sk, D);
  if (rc) return rc;
  if (!workspace_bytes) return fail(SK_EINVAL, "output pointer is NULL");
  if (num_splits < 1 || num_splits > 1024)
    return fail(SK_EINVAL, "num_splits=%d outside [1, 1024]", num_splits);
  *workspace_bytes = decode_ws_bytes(dtype, B, Hq, D, num_splits);
  return SK_OK;
}

}  // extern "C"

// Paged cache of the decode entry points (block_table null: contiguous).
struct PagedCache {
  const int32_t* block_table = nullptr;
  int page_size = 0, max_pages = 0, num_pages = 0;
};

// Paged-pool arguments of sk_decode_paged / sk_decode_paged_rope -> pc.
static int paged_args(int B, int num_pages, int page_size, int max_pages,
                      const int32_t* block_table, const int32_t* cache_seqlens, PagedCache* pc) {
  if (page_size <= 0 || page_size % 32 != 0)
    return fail(SK_EINVAL, "page_size=%d must be a positive multiple of 32", page_size);
  if (num_pages < 0 || max_pages < 0)
    return fail(SK_EINVAL, "invalid num_pages=%d max_pages=%d", num_pages, max_pages);
  if ((int64_t)max_pages * page_size > 0x7fffffffLL)
    return fail(SK_EINVAL, "max_pages * page_size overflows int");
  if (B > 0 && max_pages > 0 && (!block_table || !cache_seqlens))
    return fail(SK_EINVAL, "block_table and cache_seqlens are required");
  if (max_pages > 0 && num_pages == 0) return fail(SK_EINVAL, "empty page pool");
  pc->block_table = block_table;
  pc->page_size = page_size, pc->max_pages = max_pages, pc->num_pages = num_pages;
  return SK_OK;
}

// sk_decode, sk_decode_varlen and sk_decode_paged: seqlens is null (every row
// sees all Sk keys) or a device array of B per-row key counts; pc describes a
// paged cache (then Sk = max_pages * page_size).
static int decode_impl(int dtype, const void* q, const void* k, const void* v, void* o,
                       void* workspace, size_t workspace_bytes, int num_splits, int B, int Hq,
                       int Hkv, int Sk, int D, const int64_t* q_strides, const int64_t* k_strides,
                       const int64_t* v_strides, const int64_t* o_strides,
                       const int32_t* seqlens, const PagedCache& pc,
                       const sk::RopeParams& rope, float sm_scale, void* stream) {
  int rc = check_dims(dtype, B, Hq, Hkv, 1, Sk, D);
  if (rc) return rc;
  if ((rc = check_strides(dtype, "q", q_strides)) || (rc = check_strides(dtype, "k", k_strides)) ||
      (rc = check_strides(dtype, "v", v_strides)) || (rc = check_strides(dtype, "o", o_strides)))
    return rc;
  if ((int64_t)B * Hq == 0) return SK_OK;
  if ((rc = check_ptr("q", q)) || (rc = check_ptr("o", o))) return rc;
  if (Sk > 0 && ((rc = check_ptr("k", k)) || (rc = check_ptr("v", v)))) return rc;
  if (Hq / Hkv > 64 && dtype != SK_F32)
    return fail(SK_EUNSUPPORTED, "decode supports up to 64 query heads per KV head, got %d", Hq / Hkv);

  int kps = 0;
  if ((rc = decode_splits(dtype, B, Hq, Hkv, Sk, D, seqlens != nullptr, num_splits, &num_splits,
                          &kps)))
    return rc;
  const size_t need = decode_ws_bytes(dtype, B, Hq, D, num_splits);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(SK_EWORKSPACE, "workspace of %zu bytes given, %zu needed", workspace_bytes, need);
  if (need > 0 && (rc = check_ptr("workspace", workspace))) return rc;
  hipStream_t s = (hipStream_t)stream;

  if (dtype == SK_F32) {
    // fp32 decode is the fp32 forward with one query row (reference:
    // src/stackkernels/torch/attention.py:154 computes it the same way).
    sk::FwdParams p{};
    p.q = q, p.k = k, p.v = v, p.o = o, p.lse = (float*)workspace;
    p.q_sb = q_strides[0], p.q_sh = q_strides[1], p.q_ss = q_strides[2];
    p.k_sb = k_strides[0], p.k_sh = k_strides[1], p.k_ss = k_strides[2];
    p.v_sb = v_strides[0], p.v_sh = v_strides[1], p.v_ss = v_strides[2];
    p.o_sb = o_strides[0], p.o_sh = o_strides[1], p.o_ss = o_strides[2];
    p.B = B, p.Hq = Hq, p.Hkv = Hkv, p.Sq = 1, p.Sk = Sk, p.D = D, p.group = Hq / Hkv;
    p.scale = std::fabs(sm_scale);
    p.scale_log2 = p.scale * 1.4426950408889634f;
    p.q_sign = sm_scale < 0.f ? 1u : 0u;
    p.n_mblocks = 1;
    p.seqlens = seqlens;
    p.block_table = pc.block_table;
    p.page_size = pc.page_size, p.max_pages = pc.max_pages, p.num_pages = pc.num_pages;
    p.rope = rope;
    hipError_t e = sk::launch_fwd_f32(p, false, s);
    if (e != hipSuccess) return hip_fail(e, "sk_decode launch");
    return SK_OK;
  }

  sk::DecParams p{};
  p.q = q, p.k = k, p.v = v, p.o = o;
  p.q_sb = q_strides[0], p.q_sh = q_strides[1];
  p.k_sb = k_strides[0], p.k_sh = k_strides[1], p.k_ss = k_strides[2];
  p.v_sb = v_strides[0], p.v_sh = v_strides[1], p.v_ss = v_strides[2];
  p.o_sb = o_strides[0], p.o_sh = o_strides[1];
  p.B = B, p.Hq = Hq, p.Hkv = Hkv, p.Sk = Sk, p.D = D, p.group = Hq / Hkv;
  p.num_splits = num_splits;
  p.keys_per_split = kps;
  p.dpad = sk::padded_head_dim(D);
  p.scale = std::fabs(sm_scale);
  p.scale_log2 = p.scale * 1.4426950408889634f;
  p.q_sign = sm_scale < 0.f ? 0x80008000u : 0u;
  p.seqlens = seqlens;
  p.longest_first = seqlens != nullptr && B <= 256;
  p.block_table = pc.block_table;
  p.page_size = pc.page_size, p.max_pages = pc.max_pages, p.num_pages = pc.num_pages;
  p.rope = rope;
  if (num_splits > 1) {
    p.part_o = (float*)workspace;
    p.part_lse = p.part_o + (size_t)B * Hq * num_splits * p.dpad;
  }
  hipError_t e = sk::launch_decode_mfma(dtype, p, s);
  if (e != hipSuccess) return hip_fail(e, "sk_decode split launch");
  if (num_splits > 1) {
    e = sk::launch_decode_combine(dtype, p, s);
    if (e != hipSuccess) return hip_fail(e, "sk_decode combine launch");
  }
  return SK_OK;
}

extern "C" {

int sk_decode(int dtype, const void* q, const void* k, const void* v, void* o, void* workspace,
              size_t workspace_bytes, int num_splits, int B, int Hq, int Hkv, int Sk, int D,
              const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
              const int64_t* o_strides, float sm_scale, void* stream) {
  g_err[0] = 0;
  return decode_impl(dtype, q, k, v, o, workspace, workspace_bytes, num_splits, B, Hq, Hkv, Sk, D,
                     q_strides, k_strides, v_strides, o_strides, nullptr, PagedCache{},
                     sk::RopeParams{}, sm_scale, stream);
}

}  // extern "C"

// Library-held scratch of sk_decode_noalloc: SK_NOALLOC_SCRATCH_BYTES of
// device memory, one copy on every GPU the library runs on, held until the
// process ends.  On the host the array's name is a stand-in, not a device
// address, so host code never passes it to a kernel or a copy: each device's
// address comes from hipGetSymbolAddress, taken once per device with that
// device current, and kept in g_scratch_ptr.  Every sk_decode_noalloc call on
// a GPU shares that GPU's copy; nothing in it must start at zero (each split
// writes its whole partial before the combine reads it), but calls that
// overlap on one GPU race.
static __device__ __align__(256) uint8_t scratch[SK_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];

// Device address of the scratch copy on the device of stream s.
int scratch_address(hipStream_t s, void** out) {
  hipDevice_t dev = -1;
  hipError_t e = hipStreamGetDevice(s, &dev);
  if (e != hipSuccess) return hip_fail(e, "sk_decode_noalloc: device of the stream");
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(SK_EINVAL, "sk_decode_noalloc: device %d outside [0, %d)", dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) != hipSuccess) return hip_fail(e, "sk_decode_noalloc: hipGetDevice");
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return hip_fail(e, "sk_decode_noalloc: hipSetDevice");
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess) return hip_fail(e, "sk_decode_noalloc: hipGetSymbolAddress(scratch)");
    if (!ptr) return fail(SK_EINVAL, "sk_decode_noalloc: no scratch address on device %d", dev);
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SK_OK;
}

}  // namespace

extern "C" {

int sk_decode_noalloc(int dtype, const void* q, const void* k, const void* v, void* o,
                      int num_splits, int B, int Hq, int Hkv, int Sk, int D,
                      const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* v_strides, const int64_t* o_strides, float sm_scale,
                      void* stream) {
  g_err[0] = 0;
  int rc = check_dims(dtype, B, Hq, Hkv, 1, Sk, D);
  if (rc) return rc;
  constexpr size_t kBytes = SK_NOALLOC_SCRATCH_BYTES;
  if (num_splits == 0 && dtype != SK_F32 && (int64_t)B * Hq > 0) {
    // the table's split count, lowered until the partials fit the scratch
    const size_t per_split = (size_t)B * Hq * (sk::padded_head_dim(D) + 1) * sizeof(float);
    const int64_t fit = std::max<int64_t>(1, (int64_t)(kBytes / per_split));
    num_splits = (int)std::min<int64_t>(plan_splits(B, Hq, Hkv, Sk, D, false), fit);
  }
  int splits = 0, kps = 0;
  if ((rc = decode_splits(dtype, B, Hq, Hkv, Sk, D, false, num_splits, &splits, &kps))) return rc;
  const size_t need = decode_ws_bytes(dtype, B, Hq, D, splits);
  if (need > kBytes)
    return fail(SK_EWORKSPACE,
                "sk_decode_noalloc: %d split(s) need %zu bytes of scratch, more than the "
                "library's %zu-byte static scratch (pass fewer splits, or use sk_decode)",
                splits, need, kBytes);
  void* ws = nullptr;
  if (need > 0 && (rc = scratch_address((hipStream_t)stream, &ws))) return rc;
  return decode_impl(dtype, q, k, v, o, ws, kBytes, splits, B, Hq, Hkv, Sk, D, q_strides,
                     k_strides, v_strides, o_strides, nullptr, PagedCache{}, sk::RopeParams{},
                     sm_scale, stream);
}

}  // extern "C"

// sk_kv_cache_update (page_size 0: S_cache rows per batch row) and
// sk_kv_cache_update_paged (S_cache = num_pages * page_size pool slots).
static int cache_update_impl(int dtype, const void* k, const void* v, void* k_cache,
                             void* v_cache, const int64_t* slots, int B, int Hkv, int T,
                             int64_t S_cache, int page_size, int D, const int64_t* k_strides,
                             const int64_t* v_strides, const int64_t* kc_strides,
                             const int64_t* vc_strides, const sk::RopeParams& rope,
                             void* stream) {
  if (dtype != SK_F32 && dtype != SK_F16 && dtype != SK_BF16)
    return fail(SK_EUNSUPPORTED, "unsupported dtype code %d", dtype);
  if (B < 0 || Hkv <= 0 || T < 0 || S_cache < 0 || D <= 0)
    return fail(SK_EINVAL, "invalid sizes B=%d Hkv=%d T=%d S_cache=%lld D=%d", B, Hkv, T,
                (long long)S_cache, D);
  const int64_t* sts[4] = {k_strides, v_strides, kc_strides, vc_strides};
  const char* names[4] = {"k", "v", "k_cache", "v_cache"};
  for (int i = 0; i < 4; ++i) {
    if (!sts[i]) return fail(SK_EINVAL, "%s strides pointer is NULL", names[i]);
    for (int j = 0; j < 3; ++j)
      if (sts[i][j] < 0)
        return fail(SK_EINVAL, "%s stride[%d]=%lld must be non-negative", names[i], j,
                    (long long)sts[i][j]);
  }
  if ((int64_t)B * T == 0) return SK_OK;
  const void* ptrs[5] = {k, v, k_cache, v_cache, slots};
  const char* pnames[5] = {"k", "v", "k_cache", "v_cache", "slot_indices"};
  for (int i = 0; i < 5; ++i)
    if (!ptrs[i]) return fail(SK_EINVAL, "%s pointer is NULL", pnames[i]);
  sk::CacheParams p{};
  p.k = k, p.v = v, p.kc = k_cache, p.vc = v_cache, p.slots = slots;
  p.k_sb = k_strides[0], p.k_sh = k_strides[1], p.k_ss = k_strides[2];
  p.v_sb = v_strides[0], p.v_sh = v_strides[1], p.v_ss = v_strides[2];
  p.kc_sb = kc_strides[0], p.kc_sh = kc_strides[1], p.kc_ss = kc_strides[2];
  p.vc_sb = vc_strides[0], p.vc_sh = vc_strides[1], p.vc_ss = vc_strides[2];
  p.B = B, p.Hkv = Hkv, p.T = T, p.S = S_cache;
  p.page_size = page_size;
  p.esize = elem_bytes(dtype);
  p.row_bytes = D * p.esize;
  p.dtype = dtype;
  p.D = D;
  p.rope = rope;
  if (rope.cos) {
    // The rotating kernel moves aligned 16-byte chunks.
    const void* rp[4] = {k, v, k_cache, v_cache};
    for (int i = 0; i < 4; ++i)
      if (!aligned16(rp[i])) return fail(SK_EINVAL, "%s pointer is not 16-byte aligned", names[i]);
    for (int i = 0; i < 4; ++i)
      for (int j = 0; j < 3; ++j)
        if ((sts[i][j] * p.esize) % 16 != 0)
          return fail(SK_EINVAL, "%s stride[%d]=%lld is not a multiple of 16 bytes", names[i], j,
                      (long long)sts[i][j]);
  }
  hipError_t e = sk::launch_kv_cache_update(p, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "sk_kv_cache_update launch");
  return SK_OK;
}

extern "C" {

int sk_kv_cache_update(int dtype, const void* k, const void* v, void* k_cache, void* v_cache,
                       const int64_t* slots, int B, int Hkv, int T, int S_cache, int D,
                       const int64_t* k_strides, const int64_t* v_strides,
                       const int64_t* kc_strides, const int64_t* vc_strides, void* stream) {
  g_err[0] = 0;
  return cache_update_impl(dtype, k, v, k_cache, v_cache, slots, B, Hkv, T, S_cache, 0, D,
                           k_strides, v_strides, kc_strides, vc_strides, sk::RopeParams{},
                           stream);
}

int sk_kv_cache_update_paged(int dtype, const void* k, const void* v, void* k_pool,
                             void* v_pool, const int64_t* slot_mapping, int B, int Hkv, int T,
                             int num_pages, int page_size, int D, const int64_t* k_strides,
                             const int64_t* v_strides, const int64_t* kp_strides,
                             const int64_t* vp_strides, void* stream) {
  g_err[0] = 0;
  if (page_size <= 0 || num_pages < 0)
    return fail(SK_EINVAL, "invalid page_size=%d num_pages=%d", page_size, num_pages);
  return cache_update_impl(dtype, k, v, k_pool, v_pool, slot_mapping, B, Hkv, T,
                           (int64_t)num_pages * page_size, page_size, D, k_strides, v_strides,
                           kp_strides, vp_strides, sk::RopeParams{}, stream);
}

int sk_decode_varlen(int dtype, const void* q, const void* k, const void* v, void* o,
                     void* workspace, size_t workspace_bytes, int num_splits, int B, int Hq,
                     int Hkv, int Sk, int D, const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides,
                     const int32_t* cache_seqlens, float sm_scale, void* stream) {
  g_err[0] = 0;
  if (B > 0 && !cache_seqlens) return fail(SK_EINVAL, "cache_seqlens is null");
  return decode_impl(dtype, q, k, v, o, workspace, workspace_bytes, num_splits, B, Hq, Hkv, Sk, D,
                     q_strides, k_strides, v_strides, o_strides, cache_seqlens, PagedCache{},
                     sk::RopeParams{}, sm_scale, stream);
}

int sk_decode_paged(int dtype, const void* q, const void* k_pool, const void* v_pool, void* o,
                    void* workspace, size_t workspace_bytes, int num_splits, int B, int Hq,
                    int Hkv, int num_pages, int page_size, int max_pages, int D,
                    const int64_t* q_strides, const int64_t* kp_strides,
                    const int64_t* vp_strides, const int64_t* o_strides,
                    const int32_t* block_table, const int32_t* cache_seqlens, float sm_scale,
                    void* stream) {
  g_err[0] = 0;
  PagedCache pc;
  const int rc = paged_args(B, num_pages, page_size, max_pages, block_table, cache_seqlens, &pc);
  if (rc) return rc;
  return decode_impl(dtype, q, k_pool, v_pool, o, workspace, workspace_bytes, num_splits, B, Hq,
                     Hkv, max_pages * page_size, D, q_strides, kp_strides, vp_strides, o_strides,
                     cache_seqlens, pc, sk::RopeParams{}, sm_scale, stream);
}

int sk_decode_rope(int dtype, const void* q, const void* k, const void* v, void* o,
                   void* workspace, size_t workspace_bytes, int num_splits, int B, int Hq,
                   int Hkv, int Sk, int D, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* o_strides,
                   const int32_t* cache_seqlens, const void* rope_cos, const void* rope_sin,
                   int rope_dtype, int rope_rows, int64_t rope_stride, const int32_t* rope_pos,
                   int rope_start, float sm_scale, void* stream) {
  g_err[0] = 0;
  sk::RopeParams r{};
  const int rc = make_rope(rope_cos, rope_sin, rope_dtype, rope_rows, rope_stride, rope_pos,
                           rope_start, D, B > 0 ? 1 : 0, &r);
  if (rc) return rc;
  return decode_impl(dtype, q, k, v, o, workspace, workspace_bytes, num_splits, B, Hq, Hkv, Sk, D,
                     q_strides, k_strides, v_strides, o_strides, cache_seqlens, PagedCache{}, r,
                     sm_scale, stream);
}

int sk_decode_paged_rope(int dtype, const void* q, const void* k_pool, const void* v_pool,
                         void* o, void* workspace, size_t workspace_bytes, int num_splits, int B,
                         int Hq, int Hkv, int num_pages, int page_size, int max_pages, int D,
                         const int64_t* q_strides, const int64_t* kp_strides,
                         const int64_t* vp_strides, const int64_t* o_strides,
                         const int32_t* block_table, const int32_t* cache_seqlens,
                         const void* rope_cos, const void* rope_sin, int rope_dtype,
                         int rope_rows, int64_t rope_stride, const int32_t* rope_pos,
                         int rope_start, float sm_scale, void* stream) {
  g_err[0] = 0;
  PagedCache pc;
  int rc = paged_args(B, num_pages, page_size, max_pages, block_table, cache_seqlens, &pc);
  if (rc) return rc;
  sk::RopeParams r{};
  rc = make_rope(rope_cos, rope_sin, rope_dtype, rope_rows, rope_stride, rope_pos, rope_start, D,
                 B > 0 ? 1 : 0, &r);
  if (rc) return rc;
  return decode_impl(dtype, q, k_pool, v_pool, o, workspace, workspace_bytes, num_splits, B, Hq,
                     Hkv, max_pages * page_size, D, q_strides, kp_strides, vp_strides, o_strides,
                     cache_seqlens, pc, r, sm_scale, stream);
}

int sk_kv_cache_update_rope(int dtype, const void* k, const void* v, void* k_cache, void* v_cache,
                            const int64_t* slots, int B, int Hkv, int T, int S_cache, int D,
                            const int64_t* k_strides, const int64_t* v_strides,
                            const int64_t* kc_strides, const int64_t* vc_strides,
                            const void* rope_cos, const void* rope_sin, int rope_dtype,
                            int rope_rows, int64_t rope_stride, const int32_t* rope_pos,
                            int rope_start, void* stream) {
  g_err[0] = 0;
  sk::RopeParams r{};
  const int rc = make_rope(rope_cos, rope_sin, rope_dtype, rope_rows, rope_stride, rope_pos,
                           rope_start, D, B > 0 ? T : 0, &r);
  if (rc) return rc;
  return cache_update_impl(dtype, k, v, k_cache, v_cache, slots, B, Hkv, T, S_cache, 0, D,
                           k_strides, v_strides, kc_strides, vc_strides, r, stream);
}

int sk_kv_cache_update_paged_rope(int dtype, const void* k, const void* v, void* k_pool,
                                  void* v_pool, const int64_t* slot_mapping, int B, int Hkv,
                                  int T, int num_pages, int page_size, int D,
                                  const int64_t* k_strides, const int64_t* v_strides,
                                  const int64_t* kp_strides, const int64_t* vp_strides,
                                  const void* rope_cos, const void* rope_sin, int rope_dtype,
                                  int rope_rows, int64_t rope_stride, const int32_t* rope_pos,
                                  int rope_start, void* stream) {
  g_err[0] = 0;
  if (page_size <= 0 || num_pages < 0)
    return fail(SK_EINVAL, "invalid page_size=%d num_pages=%d", page_size, num_pages);
  sk::RopeParams r{};
  const int rc = make_rope(rope_cos, rope_sin, rope_dtype, rope_rows, rope_stride, rope_pos,
                           rope_start, D, B > 0 ? T : 0, &r);
  if (rc) return rc;
  return cache_update_impl(dtype, k, v, k_pool, v_pool, slot_mapping, B, Hkv, T,
                           (int64_t)num_pages * page_size, page_size, D, k_strides, v_strides,
                           kp_strides, vp_strides, r, stream);
}

int sk_rope_rotate(int dtype, const void* x, void* out, int B, int H, int S, int D,
                   const int64_t* x_strides, const int64_t* out_strides, const void* rope_cos,
                   const void* rope_sin, int rope_dtype, int rope_rows, int64_t rope_stride,
                   const int32_t* rope_pos, int rope_start, int inverse, void* stream) {
  g_err[0] = 0;
  int rc = check_dims(dtype, B, H, 1, S, 0, D);
  if (rc) return rc;
  if ((rc = check_strides(dtype, "x", x_strides)) || (rc = check_strides(dtype, "out", out_strides)))
    return rc;
  sk::RopeParams r{};
  const int64_t rows = (int64_t)B * H * S;
  if ((rc = make_rope(rope_cos, rope_sin, rope_dtype, rope_rows, rope_stride, rope_pos,
                      rope_start, D, rows > 0 ? S : 0, &r)))
    return rc;
  if (rows == 0) return SK_OK;
  if ((rc = check_ptr("x", x)) || (rc = check_ptr("out", out))) return rc;
  {
    // out's rows must not overlap one another (else the writes race): sorted
    // by stride, each dimension of extent > 1 must step past the rows of the
    // dimensions below it.
    int64_t ext[3] = {B, H, S}, st[3] = {out_strides[0], out_strides[1], out_strides[2]};
    for (int i = 0; i < 3; ++i)
      for (int j = i + 1; j < 3; ++j)
        if (st[j] < st[i]) std::swap(st[i], st[j]), std::swap(ext[i], ext[j]);
    int64_t span = D;  // elements the dimensions below cover
    for (int i = 0; i < 3; ++i) {
      if (ext[i] <= 1) continue;
      if (st[i] < span) return fail(SK_EINVAL, "out strides make rows overlap");
      span = st[i] * ext[i];
    }
  }
  if (x == out && (x_strides[0] != out_strides[0] || x_strides[1] != out_strides[1] ||
                   x_strides[2] != out_strides[2]))
    return fail(SK_EINVAL, "in place (out == x) needs out's strides to equal x's");
  if (x != out) {
    // In place or disjoint: a partial overlap would let one row's write
    // reach another row's unread input.
    const int64_t es = elem_bytes(dtype);
    const int64_t span_x = ((int64_t)(B - 1) * x_strides[0] + (int64_t)(H - 1) * x_strides[1] +
                            (int64_t)(S - 1) * x_strides[2] + D) * es;
    const int64_t span_o = ((int64_t)(B - 1) * out_strides[0] + (int64_t)(H - 1) * out_strides[1] +
                            (int64_t)(S - 1) * out_strides[2] + D) * es;
    const uintptr_t xa = (uintptr_t)x, oa = (uintptr_t)out;
    if (xa < oa + (uintptr_t)span_o && oa < xa + (uintptr_t)span_x)
      return fail(SK_EINVAL, "out overlaps x without being x");
  }
  sk::RotateParams p{};
  p.x = x, p.out = out;
  p.x_sb = x_strides[0], p.x_sh = x_strides[1], p.x_ss = x_strides[2];
  p.o_sb = out_strides[0], p.o_sh = out_strides[1], p.o_ss = out_strides[2];
  p.B = B, p.H = H, p.S = S, p.D = D;
  p.dtype = dtype;
  p.inverse = inverse != 0;
  p.rope = r;
  const hipError_t e = sk::launch_rope_rotate(p, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "sk_rope_rotate launch");
  return SK_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- introspection

static const char* elem_name(int e) {
  return e == SK_BF16 ? "BF16" : e == SK_F16 ? "F16" : e == SK_F32 ? "F32" : "?";
}

extern "C" {

int sk_kernel_config(int op, int dtype, int B, int Hq, int Hkv, int Sq, int Sk, int D,
                     int is_causal, int num_splits, int variant, int query_device, int64_t* cfg,
                     char* kernel_name, size_t name_len) {
  g_err[0] = 0;
  if (!cfg) return fail(SK_EINVAL, "cfg pointer is NULL");
  for (int i = 0; i < SK_CFG_LEN; ++i) cfg[i] = 0;
  if (kernel_name && name_len) kernel_name[0] = 0;
  const bool decode = op == SK_OP_DECODE || op == SK_OP_DECODE_COMBINE;
  int rc = check_dims(dtype, B, Hq, Hkv, decode ? 1 : Sq, Sk, D);
  if (rc) return rc;
  if (decode && Hq / Hkv > 64 && dtype != SK_F32)
    return fail(SK_EUNSUPPORTED, "decode supports up to 64 query heads per KV head, got %d", Hq / Hkv);
  // Non-null stand-ins for the optional inputs a variant carries: the plan
  // only tests them for null, and nothing is launched here.
  static const int kStandIn = 0;
  const bool rope = (variant & SK_VARIANT_ROPE) != 0;
  const bool paged = (variant & SK_VARIANT_PAGED) != 0;
  sk::KernelPlan k;
  int64_t splits = 1, kps = 0, paired = 0, chunks = 1;
  size_t ws = 0;
  if (op == SK_OP_FWD || (decode && dtype == SK_F32)) {
    if (op == SK_OP_DECODE_COMBINE) {  // fp32 decode has no combine pass
      cfg[SK_CFG_SPLITS] = 1;
      return SK_OK;
    }
    sk::FwdParams p{};
    if ((rc = fwd_shape(dtype, B, Hq, Hkv, decode ? 1 : Sq, Sk, D, decode ? 0 : is_causal, &p)))
      return rc;
    if (rope) p.rope.cos = &kStandIn;
    if (paged && decode) p.block_table = &kStandIn;
    k = dtype == SK_F32 ? sk::plan_fwd_f32(p, !decode && is_causal)
                        : sk::plan_fwd_mfma(dtype, p, is_causal != 0);
    paired = p.pair_items;
    if (decode) ws = decode_ws_bytes(dtype, B, Hq, D, 1);
  } else if (op == SK_OP_BWD_DKV || op == SK_OP_BWD_DQ) {
    sk::BwdParams p{};
    p.B = B, p.Hq = Hq, p.Hkv = Hkv, p.Sq = Sq, p.Sk = Sk, p.D = D, p.group = Hq / Hkv;
    // The plan of one chunk at the workspace size sk_attn_bwd_workspace reports.
    const int64_t pairs = (int64_t)B * Hkv;
    const int64_t chunk = bwd_chunk_pairs(
        pairs, sk::bwd_ds_pair_bytes(dtype, Hq, Hkv, Sq, Sk, D, is_causal != 0),
        (size_t)SK_BWD_DS_CAP_BYTES);
    if (chunk > 0) {
      p.ds = const_cast<int*>(&kStandIn);
      p.n_pairs = (int)chunk;
      chunks = (pairs + chunk - 1) / chunk;
    }
    k = op == SK_OP_BWD_DKV ? sk::plan_bwd_dkv(dtype, p, is_causal != 0)
                            : sk::plan_bwd_dq(dtype, p, is_causal != 0);
    ws = bwd_ws_bytes(dtype, B, Hq, Hkv, Sq, Sk, D, is_causal != 0);
  } else if (decode) {
    int ns = 0, per = 0;
    const bool per_row = (variant & (SK_VARIANT_PAGED | SK_VARIANT_VARLEN)) != 0;
    if ((rc = decode_splits(dtype, B, Hq, Hkv, Sk, D, per_row, num_splits, &ns, &per))) return rc;
    sk::DecParams p{};
    p.B = B, p.Hq = Hq, p.Hkv = Hkv, p.Sk = Sk, p.D = D, p.group = Hq / Hkv;
    p.num_splits = ns, p.keys_per_split = per, p.dpad = sk::padded_head_dim(D);
    if (rope) p.rope.cos = &kStandIn;
    if (paged) p.block_table = &kStandIn;
    splits = ns, kps = per;
    ws = decode_ws_bytes(dtype, B, Hq, D, ns);
    if (op == SK_OP_DECODE_COMBINE && ns <= 1) {  // one split writes O directly
      cfg[SK_CFG_SPLITS] = splits;
      return SK_OK;
    }
    k = op == SK_OP_DECODE ? sk::plan_decode_mfma(dtype, p) : sk::plan_decode_combine(dtype, p);
  } else {
    return fail(SK_EINVAL, "unknown op %d", op);
  }
  if (!k.fn) return fail(SK_EUNSUPPORTED, "no kernel for op %d with these arguments", op);
  cfg[SK_CFG_GRID] = (int64_t)k.grid.x * k.grid.y * k.grid.z;
  cfg[SK_CFG_THREADS] = (int64_t)k.block.x * k.block.y * k.block.z;
  cfg[SK_CFG_BLOCK_M] = k.block_m;
  cfg[SK_CFG_BLOCK_N] = k.block_n;
  cfg[SK_CFG_STAGES] = k.stages;
  cfg[SK_CFG_HEAD_DIM] = k.head_dim;
  cfg[SK_CFG_SPLITS] = splits;
  cfg[SK_CFG_PAIRED] = paired;
  cfg[SK_CFG_WORKSPACE] = (int64_t)ws;
  cfg[SK_CFG_KEYS_PER_SPLIT] = kps;
  cfg[SK_CFG_CHUNKS] = chunks;
  cfg[SK_CFG_LDS_BYTES] = cfg[SK_CFG_VGPRS] = cfg[SK_CFG_WG_PER_CU] = -1;
  if (kernel_name && name_len)
    snprintf(kernel_name, name_len, "%s<%s, D=%d, BM=%d, BN=%d, stages=%d, causal=%d, paged=%d, rope=%d>",
             k.kernel, elem_name(k.elem), k.head_dim, k.block_m, k.block_n, k.stages, (int)k.causal,
             (int)k.paged, (int)k.rope);
  if (query_device) {
    hipFuncAttributes a{};
    hipError_t e = hipFuncGetAttributes(&a, k.fn);
    if (e != hipSuccess) return hip_fail(e, "sk_kernel_config attributes");
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k.fn, (int)cfg[SK_CFG_THREADS], 0);
    if (e != hipSuccess) return hip_fail(e, "sk_kernel_config occupancy");
    cfg[SK_CFG_LDS_BYTES] = (int64_t)a.sharedSizeBytes;
    cfg[SK_CFG_VGPRS] = a.numRegs;
    cfg[SK_CFG_WG_PER_CU] = per_cu;
  }
  return SK_OK;
}

}  // extern "C"
