/*
 * sk_attn.h -- C ABI of libsk_attn.so, the gfx950 (MI355X) attention kernels.
 *
 * Plain C: pointers, sizes and ints only.  No allocation happens inside the
 * library: every output, the backward scratch and the decode split buffer
 * are device memory that the caller owns and passes in.  All work is ordered
 * on the HIP stream the caller passes (NULL = the null stream): it starts
 * after the work queued there before the call and ends before the work
 * queued after it.  Every kernel goes on that stream except the backward's
 * dQ kernel, which sk_attn_bwd may fork onto a side stream that the library
 * keeps for each caller stream (created on the first call on that stream
 * that is not under graph capture) and join back with events.  No call
 * synchronises the host.  Calls are re-entrant and thread-safe: calls on
 * different streams share no stream, so one thread's graph capture never
 * picks up another caller's work.
 *
 * Tensor layout is (B, H, S, D) with D contiguous ("BHSD").  Where a call
 * takes strides they are ELEMENT strides, given as int64_t[3] = {b, h, s};
 * the D stride is always 1.  Device pointers to bf16/fp16/fp32 data must be
 * 16-byte aligned and every stride a multiple of 8 elements (16 bytes) for
 * bf16/fp16, 4 elements for fp32.
 *
 * Return value: SK_OK (0) on success; a negative SK_E* code for a rejected
 * argument (nothing launched); a positive hipError_t for a HIP launch
 * failure.  sk_last_error() gives the message of the last failure on the
 * calling thread.
 */
#ifndef SK_ATTN_H_
#define SK_ATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define SK_API __attribute__((visibility("default")))
#else
#define SK_API
#endif

#define SK_ABI_VERSION 7

/* Element type codes. */
#define SK_F32 0
#define SK_F16 1
#define SK_BF16 2

/* Error codes (negative: argument rejected before any launch). */
#define SK_OK 0
#define SK_EINVAL (-1)      /* bad shape, stride, alignment or pointer   */
#define SK_EUNSUPPORTED (-2) /* dtype / head dim this library has no kernel for */
#define SK_EWORKSPACE (-3)  /* workspace pointer NULL or smaller than required */

/* Version of this ABI; equals SK_ABI_VERSION of the header it was built with. */
SK_API int sk_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
SK_API const char* sk_last_error(void);

/*
 * Forward attention.  Replaces the launcher flash_attn_fwd
 * (reference: src/stackkernels/_core/attention/flash_fwd.py:182-264) and its
 * kernel _flash_fwd_kernel (:15-179).
 *
 *   q (B,Hq,Sq,D)  k, v (B,Hkv,Sk,D)  ->  o (B,Hq,Sq,D) in the input dtype,
 *   lse (B,Hq,Sq) fp32, contiguous.
 *
 * Hq % Hkv == 0; query head h reads KV head h / (Hq/Hkv).  With is_causal the
 * mask is bottom-right aligned: key j is visible to query i iff
 * j <= i + (Sk - Sq).  A row with no visible key gets o = 0, lse = -inf.
 * sm_scale multiplies q.k before the softmax.  D: any multiple of 8 up to 256.
 */
SK_API int sk_attn_fwd(int dtype, const void* q, const void* k, const void* v, void* o, float* lse,
                int B, int Hq, int Hkv, int Sq, int Sk, int D,
                const int64_t* q_strides, const int64_t* k_strides,
                const int64_t* v_strides, const int64_t* o_strides,
                int is_causal, float sm_scale, void* stream);

/*
 * Most bytes of dS tiles one sk_attn_bwd call uses (2 GiB), whatever the
 * shape and the workspace it is given.
 */
#define SK_BWD_DS_CAP_BYTES 2147483648ULL

/*
 * Preferred bytes of scratch for sk_attn_bwd with these dims: the two fp32
 * row statistics per query row (delta = rowsum(dO * O) and lse * log2(e),
 * each array rounded up to 256 bytes: the minimum,
 * sk_attn_bwd_workspace_min) and, where the five-GEMM backward runs (16-bit
 * inputs, head dim 65-128), its 16-bit 32 x 32 dS tiles for one chunk of
 * (batch, KV head) pairs.  Each pair needs 2048 bytes per tile that a
 * visible 128-key block writes, for each of its Hq / Hkv query heads: about
 * Sq * Sk * 2 bytes per query head, half that under a square causal mask
 * (117 MB per pair at B = 2, Hq = 32, Hkv = 8, Sq = 2048, Sk = 8192 causal,
 * so 1.88 GB for all 16 pairs).  The chunk is the whole batch where that
 * fits under SK_BWD_DS_CAP_BYTES, else the fewest even chunks that do; when
 * one pair's tiles exceed the cap the seven-GEMM backward runs and the
 * minimum is all it needs.  Replaces allocate_delta_buffer
 * (reference: src/stackkernels/_opt/memory/workspace.py:16-23).
 */
SK_API int sk_attn_bwd_workspace(int dtype, int B, int Hq, int Hkv, int Sq, int Sk, int D,
                          int is_causal, size_t* bytes);

/*
 * Minimum bytes of scratch for sk_attn_bwd: the two row statistics, with
 * which it runs the seven-GEMM backward.  The reference's counterpart is
 * the same delta buffer (src/stackkernels/_opt/memory/workspace.py:16-23).
 */
SK_API int sk_attn_bwd_workspace_min(int dtype, int B, int Hq, int Hkv, int Sq, int Sk, int D,
                              int is_causal, size_t* bytes);

/*
 * Backward attention.  Replaces flash_attn_bwd
 * (reference: src/stackkernels/_core/attention/flash_bwd.py:362-528) with its
 * three kernels _bwd_preprocess_kernel (:15-55), _flash_bwd_dq_kernel
 * (:58-198) and _flash_bwd_dkv_kernel (:201-359).
 *
 * All tensors contiguous BHSD: dout, q, o, dq (B,Hq,Sq,D); k, v, dk, dv
 * (B,Hkv,Sk,D); lse (B,Hq,Sq) fp32 as written by sk_attn_fwd.  dk and dv are
 * summed over the query heads that share a KV head.  Rows with lse = -inf
 * contribute nothing.  workspace: at least sk_attn_bwd_workspace_min()
 * bytes (SK_EWORKSPACE otherwise), any contents (the call initialises what
 * it uses).  Five-GEMM backward (head dim 65-128, 16-bit), when the bytes
 * past the row statistics hold one (batch, KV head) pair's dS tiles: the
 * pairs run in the fewest even chunks whose tiles fit those bytes (at most
 * SK_BWD_DS_CAP_BYTES of them); for each chunk the dK/dV kernel stores dS in
 * the workspace and the dQ kernel reads it, both on `stream`.  The results
 * are the same bit for bit for every chunking and equal the seven-GEMM
 * backward's.  Seven-GEMM backward (other head dims, fp32, or a workspace
 * too small for one pair's tiles): when the dK/dV grid runs more than one round of workgroups (more
 * than 256 workgroups), the dQ kernel runs on the library's side stream for
 * `stream`, forked from `stream` after the preprocess pass and joined back
 * into it (also when a launch fails); under graph capture the fork and the
 * join are recorded as graph edges.  A call under capture on a stream that
 * has never run an eager backward keeps the one-stream order.
 */
SK_API int sk_attn_bwd(int dtype, const void* dout, const void* q, const void* k, const void* v,
                const void* o, const float* lse, void* dq, void* dk, void* dv,
                void* workspace, size_t workspace_bytes,
                int B, int Hq, int Hkv, int Sq, int Sk, int D,
                int is_causal, float sm_scale, void* stream);

/*
 * Split-KV plan for single-token decode: the number of key splits the gfx950
 * table picks and the scratch bytes sk_decode (uniform cache length) then
 * needs; what sk_decode runs with num_splits = 0.  Replaces the split
 * heuristic chain decode_heuristic -> seed_configs
 * (reference: src/stackkernels/_opt/heuristics/flash_decode.py:9-12,
 * src/stackkernels/_opt/classes/decode.py:9-63) as used at
 * src/stackkernels/_core/attention/decode.py:220-226.
 */
SK_API int sk_decode_plan(int dtype, int B, int Hq, int Hkv, int Sk, int D,
                   int* num_splits, size_t* workspace_bytes);

/*
 * The same for per-row cache lengths and paged pools (sk_decode_varlen,
 * sk_decode_paged and their _rope forms with num_splits = 0): for groups of
 * up to 16 query heads about twice the uniform plan's splits, since rows
 * shorter than the longest leave a one-round grid uneven.  No counterpart in
 * the reference (its decode has one cache length).
 */
SK_API int sk_decode_plan_varlen(int dtype, int B, int Hq, int Hkv, int Sk, int D,
                          int* num_splits, size_t* workspace_bytes);

/*
 * Single-token decode (Sq == 1), non-causal over all Sk keys.  Replaces the
 * launcher flash_decode (reference: src/stackkernels/_core/attention/decode.py:192-312)
 * and its kernels _flash_decode_split_kernel (:15-121) and
 * _flash_decode_reduce_kernel (:124-189).
 *
 *   q (B,Hq,1,D), k/v (B,Hkv,Sk,D) with any b/h/s strides  ->  o (B,Hq,1,D).
 *
 * num_splits: as returned by sk_decode_plan, or any value in [1, Sk] (0 lets
 * the library plan).  workspace: >= the plan's bytes for that split count
 * (sk_decode_workspace), any contents.
 */
SK_API int sk_decode(int dtype, const void* q, const void* k, const void* v, void* o,
              void* workspace, size_t workspace_bytes, int num_splits,
              int B, int Hq, int Hkv, int Sk, int D,
              const int64_t* q_strides, const int64_t* k_strides,
              const int64_t* v_strides, const int64_t* o_strides,
              float sm_scale, void* stream);

/*
 * sk_decode without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The split
 * partials go to a static scratch array the library holds on each GPU it runs
 * on, SK_NOALLOC_SCRATCH_BYTES per GPU until the process ends; the call itself
 * allocates nothing.  num_splits 0 takes the gfx950 table's split count,
 * lowered until the partials fit; an explicit split count whose partials do
 * not fit (B * Hq * num_splits * (padded D + 1) * 4 bytes) is rejected with
 * SK_EWORKSPACE.  fp32 runs unsplit with its B * Hq LSE values in the scratch.
 * Every call on one GPU shares that GPU's scratch, which keeps the last call's
 * contents: calls that overlap on one GPU (concurrent streams, threads) race
 * and must be ordered by the caller.  Results equal sk_decode's for the same
 * split count.
 */
#define SK_NOALLOC_SCRATCH_BYTES (32u << 20)
SK_API int sk_decode_noalloc(int dtype, const void* q, const void* k, const void* v, void* o,
                      int num_splits, int B, int Hq, int Hkv, int Sk, int D,
                      const int64_t* q_strides, const int64_t* k_strides,
                      const int64_t* v_strides, const int64_t* o_strides,
                      float sm_scale, void* stream);

/* Scratch bytes sk_decode needs for an explicit split count. */
SK_API int sk_decode_workspace(int dtype, int B, int Hq, int Hkv, int Sk, int D, int num_splits,
                        size_t* workspace_bytes);

/*
 * sk_decode with a cache length per batch row: row b attends to keys
 * [0, clamp(cache_seqlens[b], 0, Sk)) of its cache; a row with no key gives
 * O = 0.  cache_seqlens is a device array of B int32.  Sk is the cache
 * capacity and sets the split plan (sk_decode_plan_varlen /
 * sk_decode_workspace with the same Sk; num_splits = 0 runs the
 * sk_decode_plan_varlen count).  The reference has no counterpart yet: it realises the
 * per-sequence cache lengths its decode roadmap names (stubs
 * src/stackkernels/_core/attention/varlen.py, paged.py; reference decode
 * src/stackkernels/_core/attention/decode.py:192-312 takes one S_k for all rows).
 */
SK_API int sk_decode_varlen(int dtype, const void* q, const void* k, const void* v, void* o,
                     void* workspace, size_t workspace_bytes, int num_splits,
                     int B, int Hq, int Hkv, int Sk, int D,
                     const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides,
                     const int32_t* cache_seqlens, float sm_scale, void* stream);

/*
 * sk_decode_varlen over a paged cache.  k_pool, v_pool hold num_pages pages of
 * page_size keys (element strides: page, head, in-page row; contiguous head
 * dim); key j of batch row b is in-page row j % page_size of page
 * block_table[b * max_pages + j / page_size], for j < cache_seqlens[b]
 * (clamped to max_pages * page_size).  page_size is a positive multiple of 32;
 * a page index outside [0, num_pages) masks its keys.  block_table (B x
 * max_pages int32) and cache_seqlens (B int32) live on the device.  Plan the
 * splits with sk_decode_plan_varlen at Sk = max_pages * page_size.  The reference has no counterpart
 * yet: it realises the paged KV decode of its roadmap (stub
 * src/stackkernels/_core/attention/paged.py).
 */
SK_API int sk_decode_paged(int dtype, const void* q, const void* k_pool, const void* v_pool,
                    void* o, void* workspace, size_t workspace_bytes, int num_splits,
                    int B, int Hq, int Hkv, int num_pages, int page_size, int max_pages, int D,
                    const int64_t* q_strides, const int64_t* kp_strides,
                    const int64_t* vp_strides, const int64_t* o_strides,
                    const int32_t* block_table, const int32_t* cache_seqlens,
                    float sm_scale, void* stream);

/*
 * KV-cache append: k_cache[b, h, slots[b*T + t], :] = k[b, h, t, :] and the
 * same for v, for b < B, h < Hkv, t < T.  k, v (B, Hkv, T, D); k_cache,
 * v_cache (B, Hkv, S_cache, D); element strides (b, h, s) with a contiguous
 * head dim; slots is a device array of B*T int64.  A slot outside
 * [0, S_cache) skips its token (pad value -1).  Slots must be distinct
 * within a batch row (tokens that share one race).  Realises the planned
 * kv_cache_update(k, v, k_cache, v_cache, slot_indices)
 * (reference: docs/user_guide/dropout_cache_sampling.md:66-72; stubs
 * src/stackkernels/torch/cache.py, src/stackkernels/_core/cache/kv_update.py).
 */
SK_API int sk_kv_cache_update(int dtype, const void* k, const void* v, void* k_cache,
                       void* v_cache, const int64_t* slots, int B, int Hkv, int T,
                       int S_cache, int D, const int64_t* k_strides,
                       const int64_t* v_strides, const int64_t* kc_strides,
                       const int64_t* vc_strides, void* stream);

/*
 * KV-cache append into a paged pool: token t of batch row b goes to in-page
 * row s % page_size of page s / page_size, s = slot_mapping[b*T + t], for
 * s in [0, num_pages * page_size) (other values skip the token).  Pool
 * element strides: page, head, in-page row.  Realises the planned
 * kv_cache_update for paged caches (reference:
 * docs/user_guide/dropout_cache_sampling.md:66-72, stub
 * src/stackkernels/_core/cache/kv_update.py).
 */
SK_API int sk_kv_cache_update_paged(int dtype, const void* k, const void* v, void* k_pool,
                             void* v_pool, const int64_t* slot_mapping, int B, int Hkv,
                             int T, int num_pages, int page_size, int D,
                             const int64_t* k_strides, const int64_t* v_strides,
                             const int64_t* kp_strides, const int64_t* vp_strides,
                             void* stream);

/*
 * RoPE fused into the attention prologue.  The *_rope entry points below take
 * the arguments of the call they extend plus a rotary position embedding that
 * the kernels apply to q (attention, decode) or to the new keys (cache
 * append) as they load them, so the rotated vectors never make a separate
 * trip through HBM.  The rotation is the reference's apply_rope
 * (src/stackkernels/torch/embedding.py:67-100; math in
 * src/stackkernels/_reference/torch/rope.py:32-58):
 *
 *   out[d] = x[d] cos[p][d] - x[d + D/2] sin[p][d]   (d <  D/2)
 *   out[d] = x[d] cos[p][d] + x[d - D/2] sin[p][d]   (d >= D/2)
 *
 * in fp32 (two products and a sum, each rounded; no fused multiply-add),
 * rounded to the tensor's type.  Arguments:
 *
 *   rope_cos, rope_sin  device tables of rope_rows rows (element stride
 *                       rope_stride >= D between rows; the first D columns are
 *                       read), element type rope_dtype (SK_F32/F16/BF16),
 *                       16-byte aligned with rows a multiple of 16 bytes apart
 *                       -- the (max_seq_len, D) tables of precompute_freqs
 *                       (src/stackkernels/_reference/torch/rope.py:6-29);
 *   rope_pos            NULL, or a device array of B int32 per-row base positions;
 *   rope_start          added to every position (the reference's start_pos).
 *
 * Token t of batch row b sits at p = (rope_pos ? rope_pos[b] : 0) + rope_start + t:
 * query row t for attention, t = 0 for the decode query, new token t for the
 * cache append.  With rope_pos NULL, [rope_start, rope_start + tokens) must lie
 * in the table (SK_EINVAL otherwise, as the reference's table slice fails);
 * with rope_pos given, a position outside [0, rope_rows) leaves that vector
 * unrotated.  D must be a multiple of 16 (SK_EUNSUPPORTED otherwise).  The
 * reference has no fused counterpart: it rotates q and k in a separate pass
 * (src/stackkernels/_core/positional/rope.py:12-222) before attention.
 */

/* sk_attn_fwd with q rotated on load (query row i is token i).  It does not
 * write the rotated q out: its backward is sk_rope_rotate(q) into a buffer,
 * sk_attn_bwd on that rotated q, then sk_rope_rotate(dq, inverse = 1) in
 * place. */
SK_API int sk_attn_fwd_rope(int dtype, const void* q, const void* k, const void* v, void* o,
                     float* lse, int B, int Hq, int Hkv, int Sq, int Sk, int D,
                     const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides, int is_causal,
                     const void* rope_cos, const void* rope_sin, int rope_dtype, int rope_rows,
                     int64_t rope_stride, const int32_t* rope_pos, int rope_start,
                     float sm_scale, void* stream);

/*
 * Rotate a (B, H, S, D) tensor by its RoPE angles (inverse = 0) or by their
 * negatives (inverse = 1, the adjoint: the gradient of the rotation), token t
 * of batch row b at the position given above (positions as in the other
 * *_rope calls, tokens = S).  Element strides {b, h, s} for x and out; out's
 * rows must not overlap one another; out may be x (in place, with the same
 * strides), otherwise it must not overlap it (SK_EINVAL).  The rotation is
 * the one the fused kernels apply, bit for bit, so it rebuilds the rotated q
 * that sk_attn_fwd_rope used and carries dq back through the rotation for
 * sk_attn_bwd.  Replaces rope_fwd / _rope_fwd_kernel and rope_bwd /
 * _rope_bwd_kernel (reference: src/stackkernels/_core/positional/rope.py:12-222;
 * the adjoint as in src/stackkernels/torch/embedding.py:46-66).
 */
SK_API int sk_rope_rotate(int dtype, const void* x, void* out, int B, int H, int S, int D,
                   const int64_t* x_strides, const int64_t* out_strides,
                   const void* rope_cos, const void* rope_sin, int rope_dtype, int rope_rows,
                   int64_t rope_stride, const int32_t* rope_pos, int rope_start, int inverse,
                   void* stream);

/* sk_decode (cache_seqlens NULL) or sk_decode_varlen with q rotated on load. */
SK_API int sk_decode_rope(int dtype, const void* q, const void* k, const void* v, void* o,
                   void* workspace, size_t workspace_bytes, int num_splits,
                   int B, int Hq, int Hkv, int Sk, int D,
                   const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* o_strides,
                   const int32_t* cache_seqlens, const void* rope_cos, const void* rope_sin,
                   int rope_dtype, int rope_rows, int64_t rope_stride, const int32_t* rope_pos,
                   int rope_start, float sm_scale, void* stream);

/* sk_decode_paged with q rotated on load. */
SK_API int sk_decode_paged_rope(int dtype, const void* q, const void* k_pool, const void* v_pool,
                         void* o, void* workspace, size_t workspace_bytes, int num_splits,
                         int B, int Hq, int Hkv, int num_pages, int page_size, int max_pages,
                         int D, const int64_t* q_strides, const int64_t* kp_strides,
                         const int64_t* vp_strides, const int64_t* o_strides,
                         const int32_t* block_table, const int32_t* cache_seqlens,
                         const void* rope_cos, const void* rope_sin, int rope_dtype,
                         int rope_rows, int64_t rope_stride, const int32_t* rope_pos,
                         int rope_start, float sm_scale, void* stream);

/* sk_kv_cache_update with the new keys rotated before they are written (new
 * token t is token t); values are copied unchanged.  k, v, the caches and all
 * their strides must be 16-byte aligned. */
SK_API int sk_kv_cache_update_rope(int dtype, const void* k, const void* v, void* k_cache,
                            void* v_cache, const int64_t* slots, int B, int Hkv, int T,
                            int S_cache, int D, const int64_t* k_strides,
                            const int64_t* v_strides, const int64_t* kc_strides,
                            const int64_t* vc_strides, const void* rope_cos,
                            const void* rope_sin, int rope_dtype, int rope_rows,
                            int64_t rope_stride, const int32_t* rope_pos, int rope_start,
                            void* stream);

/* sk_kv_cache_update_paged with the new keys rotated (as above). */
SK_API int sk_kv_cache_update_paged_rope(int dtype, const void* k, const void* v, void* k_pool,
                                  void* v_pool, const int64_t* slot_mapping, int B, int Hkv,
                                  int T, int num_pages, int page_size, int D,
                                  const int64_t* k_strides, const int64_t* v_strides,
                                  const int64_t* kp_strides, const int64_t* vp_strides,
                                  const void* rope_cos, const void* rope_sin, int rope_dtype,
                                  int rope_rows, int64_t rope_stride, const int32_t* rope_pos,
                                  int rope_start, void* stream);

/*
 * Introspection: the kernel and launch configuration a call would run, from
 * the same plan the launchers use.  Replaces what the reference's
 * pick(op, shape, ..., explain=True) reports for this path
 * (src/stackkernels/_opt/pick.py:18-226: the chosen BLOCK_M / BLOCK_N /
 * num_warps / num_stages / SPLIT_KV and the grid), for the gfx950 table of
 * this library instead of a Triton heuristic.
 *
 *   op       SK_OP_FWD, SK_OP_BWD_DKV, SK_OP_BWD_DQ, SK_OP_DECODE (the split
 *            pass; fp32: the fp32 forward kernel with one query row) or
 *            SK_OP_DECODE_COMBINE (grid 0 when one split writes O directly);
 *   Sq       ignored for decode; num_splits: decode only (0 = the table's pick);
 *   variant  SK_VARIANT_* bits: the decode over a paged pool, the RoPE
 *            prologue (forward and decode), per-row cache lengths (decode:
 *            the sk_decode_plan_varlen split count; paged implies it);
 *   query_device  0: no HIP call is made (works without a GPU) and the
 *            device-reported slots hold -1; 1: also ask the HIP runtime for
 *            the kernel's LDS bytes, registers per lane and resident
 *            workgroups per CU on the current device.
 *   cfg      int64_t[SK_CFG_LEN], slots below; kernel_name (optional) gets
 *            the kernel and its template configuration.
 */
#define SK_OP_FWD 0
#define SK_OP_BWD_DKV 1
#define SK_OP_BWD_DQ 2
#define SK_OP_DECODE 3
#define SK_OP_DECODE_COMBINE 4

#define SK_VARIANT_PAGED 1
#define SK_VARIANT_ROPE 2
#define SK_VARIANT_VARLEN 4  /* decode with per-row cache lengths (the paged pool implies it) */

#define SK_CFG_GRID 0           /* workgroups per launch                        */
#define SK_CFG_THREADS 1        /* threads per workgroup (64 per wavefront)     */
#define SK_CFG_BLOCK_M 2        /* query rows per workgroup (decode: query heads) */
#define SK_CFG_BLOCK_N 3        /* keys per tile (dK/dV: keys per workgroup)    */
#define SK_CFG_STAGES 4         /* tile ring depth; 0 = staged in registers     */
#define SK_CFG_HEAD_DIM 5       /* padded head dim the kernel is compiled for   */
#define SK_CFG_SPLITS 6         /* decode key splits (1 otherwise)              */
#define SK_CFG_PAIRED 7         /* forward: causal query blocks paired per workgroup */
#define SK_CFG_WORKSPACE 8      /* scratch bytes the call needs                 */
#define SK_CFG_KEYS_PER_SPLIT 9 /* decode                                       */
#define SK_CFG_LDS_BYTES 10     /* device-reported, or -1                       */
#define SK_CFG_VGPRS 11         /* device-reported registers per lane, or -1    */
#define SK_CFG_WG_PER_CU 12     /* device-reported resident workgroups per CU, or -1 */
#define SK_CFG_CHUNKS 13        /* backward: launches of the kernel per call (chunks of pairs) */
#define SK_CFG_LEN 16

SK_API int sk_kernel_config(int op, int dtype, int B, int Hq, int Hkv, int Sq, int Sk, int D,
                     int is_causal, int num_splits, int variant, int query_device,
                     int64_t* cfg, char* kernel_name, size_t name_len);

#ifdef __cplusplus
}
#endif

#endif /* SK_ATTN_H_ */
