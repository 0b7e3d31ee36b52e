"""CPU oracle for the StackKernels attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this module, and only as the checker.  The product path never
calls it: device tensors run the HIP library, and the library fails loudly
when it is missing.

What it restates (all arithmetic in float64 unless a caller asks otherwise):

* ``repeat_kv``            -- ``src/stackkernels/_reference/torch/attention.py:10-14``
* ``allowed_mask``         -- bottom-right causal rule, ``_core/attention/_masks.py:22-35``
                              and ``_reference/torch/attention.py:63-68``
* ``attention_forward``    -- ``_reference/torch/attention.py:17-76`` (scores, mask,
                              logsumexp, softmax, NaN->0 for fully masked rows, P.V)
* ``attention_backward``   -- the gradient of ``attention_forward``; the reference
                              obtains it by autograd through the same function
                              (``src/stackkernels/torch/attention.py:82-102``).  Written
                              here in closed form: dV = P^T dO, dP = dO V^T,
                              dS = P * (dP - rowsum(dO * O)), dQ = s dS K, dK = s dS^T Q,
                              with dK/dV summed over each KV head's query group.
* ``decode``               -- ``src/stackkernels/torch/attention.py:134-155`` (CPU branch
                              ``:154`` calls the non-causal reference with S_q = 1).
* ``split_partials`` / ``combine_partials`` -- the split-KV decomposition and the
                              LSE-weighted merge of ``_core/attention/decode.py:81-121,166-186``.
* ``decode_varlen``        -- decode with a cache length per batch row: row b is the
                              reference decode over its first ``min(L_b, S_k)`` keys
                              (zeros when none); the per-sequence cache lengths of the
                              reference's decode roadmap (stubs ``_core/attention/varlen.py``,
                              ``paged.py``), which has no implementation to follow.
* ``kv_cache_update``      -- ``k_cache[b, h, slot[b, t]] = k[b, h, t]`` (and v), slots outside
                              the cache skipped: the planned ``kv_cache_update``
                              (``docs/user_guide/dropout_cache_sampling.md:66-72``).
* ``gather_pages`` / ``decode_paged`` / ``kv_cache_update_paged`` -- the same two
                              operations on a paged pool (key j of row b in page
                              ``table[b, j // page_size]``, row ``j % page_size``; a page
                              outside the pool masks its keys): the paged KV decode of
                              the roadmap (stub ``_core/attention/paged.py``).
* ``rope_tables`` / ``rope_positions`` / ``rope_rotate`` / ``round_to`` -- RoPE:
                              ``precompute_freqs``, ``rotate_half`` and
                              ``apply_rope_single`` of ``_reference/torch/rope.py:6-58``
                              (fp32 products and sum, each rounded, then rounded
                              to the tensor type), with one position per (row,
                              token); the fused paths are these composed with
                              ``attention_forward`` / ``decode*`` / ``kv_cache_update*``.
* ``rope_rotate_adjoint``  -- the gradient of ``rope_rotate`` (its transpose per
                              (d, d + D/2) plane); for ``precompute_freqs`` tables the
                              reference's rotation by -theta,
                              ``src/stackkernels/torch/embedding.py:46-66`` and
                              ``_core/positional/rope.py:77-134``.  The fused-RoPE
                              backward is ``attention_backward`` at the rotated q
                              followed by it on dQ.

How each function is pinned (see ``tests/test_oracle.py``):

* against the committed golden vectors in ``tests/golden/`` (written by
  ``tests/golden/make_golden.py`` from torch's own
  ``scaled_dot_product_attention`` in float64 -- an independent library
  routine, with its autograd for the gradients);
* against a brute-force per-element loop on tiny shapes;
* against central finite differences of ``attention_forward`` (backward);
* through invariants a plausible slip would break: rows of P sum to one,
  GQA equals MHA on repeated K/V with grads summed per group, a causal row
  does not depend on keys it may not see, ``S_k = 1`` gives ``O = V`` and
  ``LSE = score``, ``q = 0`` gives the mean of the visible V rows and
  ``LSE = log(#visible)``, fully masked rows give ``O = 0`` and
  ``LSE = -inf`` and zero gradients, and the split-KV merge is invariant to
  the number of splits;
* ``decode_varlen`` against ``decode`` (all rows full), against
  ``attention_forward`` on each row's sliced cache, against a brute-force loop,
  and with empty and over-long rows; ``kv_cache_update`` against a
  per-element loop, including padded (-1) and out-of-range slots;
  ``decode_paged`` against ``decode_varlen`` on caches assembled page by page
  with a loop, and with a page index outside the pool against the same row
  cut at that page; ``kv_cache_update_paged`` against a per-element loop.
* RoPE: ``rope_tables`` against cos/sin of the angle written out per entry,
  with row 0 all (1, 0) and the two halves equal; ``rope_rotate`` against the
  rotation written as a complex product (x_d + i x_{d+D/2}) e^{i angle} in
  float64, which fixes the sign and the half that is negated, against a
  per-element loop, through the invariants it must keep (the norm of each
  (d, d + D/2) pair, identity at position 0, rotation by p1 then p2 equals
  rotation by p1 + p2), and with out-of-table positions; ``round_to`` against
  torch's own bfloat16 / float16 casts, ties included.  The reference's RoPE
  tests (``tests/ops/test_rope.py``) hold no fixed vectors: they compare its
  kernel with its torch restatement at start_pos 0, 15, 23, 31, 64, and the
  same start positions are used here.  ``rope_rotate_adjoint`` against the
  definition of a transpose, <R x, y> = <x, R^T y>, with tables whose halves
  differ (a sine from the wrong half or a wrong sign breaks it), against
  R^T R = I for real tables, and bit for bit against the reference's formula
  ``dy * cos - rotate_half(dy) * sin`` evaluated by torch.
"""

from __future__ import annotations

import math

import numpy as np

NEG_INF = float("-inf")


def repeat_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """(B, H_kv, S, D) -> (B, H_kv * n_rep, S, D), each KV head repeated in place.

    Follows ``_reference/torch/attention.py:10-14`` (``repeat_interleave`` on dim 1):
    query head ``h`` reads KV head ``h // n_rep``.
    """
    if n_rep == 1:
        return x
    return np.repeat(x, n_rep, axis=1)


def allowed_mask(s_q: int, s_k: int) -> np.ndarray:
    """Boolean (S_q, S_k): True where query i may attend key j, i.e. j <= i + (S_k - S_q).

    Bottom-right alignment, ``_core/attention/_masks.py:22-35``.
    """
    i = np.arange(s_q)[:, None]
    j = np.arange(s_k)[None, :]
    return j <= i + (s_k - s_q)


def _default_scale(d: int, sm_scale: float | None) -> float:
    # src/stackkernels/torch/attention.py:33-36
    return 1.0 / math.sqrt(d) if sm_scale is None else float(sm_scale)


def attention_forward(q, k, v, is_causal=False, sm_scale=None, dtype=np.float64):
    """Return (O, LSE) for BHSD inputs, following ``_reference/torch/attention.py:17-76``.

    O has shape (B, H_q, S_q, D), LSE (B, H_q, S_q).  Fully masked rows give
    O = 0 and LSE = -inf.  Inputs are upcast to ``dtype`` first, as the
    reference upcasts to float32 (``:56-59``); the default float64 is the
    checker's precision.
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    assert hq % hkv == 0
    scale = _default_scale(d, sm_scale)
    kk = repeat_kv(k, hq // hkv)
    vv = repeat_kv(v, hq // hkv)
    scores = np.matmul(q, np.swapaxes(kk, -1, -2)) * scale
    if is_causal:
        scores = np.where(allowed_mask(sq, sk)[None, None], scores, NEG_INF)
    if sk == 0:
        lse = np.full((b, hq, sq), NEG_INF, dtype=dtype)
        return np.zeros((b, hq, sq, d), dtype=dtype), lse
    m = scores.max(axis=-1, keepdims=True)
    finite = np.isfinite(m)
    m_safe = np.where(finite, m, 0.0)
    e = np.exp(scores - m_safe)
    l = e.sum(axis=-1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        lse = np.where(finite, m_safe + np.log(l), NEG_INF)[..., 0]
        p = np.where(finite, e / l, 0.0)
    out = np.matmul(p, vv)
    return out.astype(dtype), lse.astype(dtype)


def softmax_probs(q, k, is_causal=False, sm_scale=None):
    """P = softmax(scale Q K^T + mask) with fully masked rows set to 0, float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    hq, hkv = q.shape[1], k.shape[1]
    sq, sk, d = q.shape[2], k.shape[2], q.shape[3]
    scale = _default_scale(d, sm_scale)
    s = np.matmul(q, np.swapaxes(repeat_kv(k, hq // hkv), -1, -2)) * scale
    if is_causal:
        s = np.where(allowed_mask(sq, sk)[None, None], s, NEG_INF)
    m = s.max(axis=-1, keepdims=True) if sk else np.zeros(s.shape[:-1] + (1,))
    m = np.where(np.isfinite(m), m, 0.0)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        return np.where(l > 0, e / np.where(l > 0, l, 1.0), 0.0)


def attention_backward(q, k, v, do, is_causal=False, sm_scale=None):
    """Return (dQ, dK, dV) of ``sum(O * dO)`` w.r.t. q, k, v, float64.

    This is the gradient the reference computes by autograd through its
    reference forward (``src/stackkernels/torch/attention.py:82-102``).
    dK/dV come back in the KV-head shape: the ``repeat_kv`` copies of a head
    are summed over its query group.  Rows that see no key contribute zero.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    do = np.asarray(do, dtype=np.float64)
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    g = hq // hkv
    scale = _default_scale(d, sm_scale)
    kk = repeat_kv(k, g)
    vv = repeat_kv(v, g)
    p = softmax_probs(q, k, is_causal, sm_scale)  # (B, Hq, Sq, Sk)
    out = np.matmul(p, vv)
    dvv = np.matmul(np.swapaxes(p, -1, -2), do)
    dp = np.matmul(do, np.swapaxes(vv, -1, -2))
    delta = (do * out).sum(axis=-1, keepdims=True)
    ds = p * (dp - delta)
    dq = np.matmul(ds, kk) * scale
    dkk = np.matmul(np.swapaxes(ds, -1, -2), q) * scale
    dk = dkk.reshape(b, hkv, g, sk, d).sum(axis=2)
    dv = dvv.reshape(b, hkv, g, sk, d).sum(axis=2)
    return dq, dk, dv


def decode(q, k, v, sm_scale=None, dtype=np.float64):
    """Single-token decode: O of ``attention_forward(q, k, v, is_causal=False)``.

    ``src/stackkernels/torch/attention.py:134-155``; the reference asserts
    ``S_q == 1`` (``_core/attention/decode.py:212``).
    """
    assert np.asarray(q).shape[2] == 1, "flash_decode requires q_len == 1"
    out, _ = attention_forward(q, k, v, is_causal=False, sm_scale=sm_scale, dtype=dtype)
    return out


def split_partials(q, k, v, num_splits, sm_scale=None):
    """Per-split normalised partial outputs and LSEs for S_q = 1 decode.

    Split ``s`` covers keys ``[s*c, min((s+1)*c, S_k))`` with ``c = ceil(S_k / num_splits)``,
    the chunking of ``_core/attention/decode.py:228-230``.  Returns
    (O_s of shape (B, H_q, splits, D), LSE_s of shape (B, H_q, splits)); an
    empty split has O_s = 0 and LSE_s = -inf.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    b, hq, _, d = q.shape
    sk = k.shape[2]
    chunk = -(-sk // num_splits) if sk else 0
    outs = np.zeros((b, hq, num_splits, d))
    lses = np.full((b, hq, num_splits), NEG_INF)
    for s in range(num_splits):
        lo, hi = s * chunk, min((s + 1) * chunk, sk)
        if hi <= lo:
            continue
        o, l = attention_forward(q, k[:, :, lo:hi], v[:, :, lo:hi], False, sm_scale)
        outs[:, :, s] = o[:, :, 0]
        lses[:, :, s] = l[:, :, 0]
    return outs, lses


def combine_partials(outs, lses):
    """LSE-weighted merge of split partials, ``_core/attention/decode.py:166-186``.

    O = sum_s exp(LSE_s - M) O_s / sum_s exp(LSE_s - M), M = max_s LSE_s;
    all splits empty gives O = 0.  Returns (O of shape (B, H_q, 1, D), LSE).
    """
    outs = np.asarray(outs, dtype=np.float64)
    lses = np.asarray(lses, dtype=np.float64)
    m = lses.max(axis=-1, keepdims=True)
    finite = np.isfinite(m)
    w = np.where(finite, np.exp(lses - np.where(finite, m, 0.0)), 0.0)
    den = w.sum(axis=-1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        o = np.where(den[..., None] > 0, (w[..., None] * outs).sum(axis=-2, keepdims=True)
                     / np.where(den > 0, den, 1.0)[..., None], 0.0)
        lse = np.where(finite, m + np.log(np.where(den > 0, den, 1.0)), NEG_INF)[..., 0]
    return o, lse


def decode_varlen(q, k, v, seqlens, sm_scale=None):
    """Decode where batch row b attends to keys ``[0, clamp(seqlens[b], 0, S_k))``.

    Each row is ``decode`` over its sliced cache; a row with no key gives zeros.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    assert q.shape[2] == 1, "flash_decode requires q_len == 1"
    sk = k.shape[2]
    out = np.zeros(q.shape)
    for b, n in enumerate(np.asarray(seqlens).reshape(-1)):
        n = int(min(max(int(n), 0), sk))
        if n > 0:
            out[b:b + 1] = decode(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n], sm_scale)
    return out


def kv_cache_update(k, v, k_cache, v_cache, slots):
    """Return copies of the caches with ``cache[b, h, slots[b, t]] = new[b, h, t]``.

    A slot outside ``[0, S_cache)`` skips its token; slots are distinct per row.
    """
    kc = np.array(k_cache, copy=True)
    vc = np.array(v_cache, copy=True)
    k = np.asarray(k)
    v = np.asarray(v)
    slots = np.asarray(slots)
    s = kc.shape[2]
    for b in range(slots.shape[0]):
        keep = (slots[b] >= 0) & (slots[b] < s)
        kc[b][:, slots[b][keep]] = k[b][:, keep]
        vc[b][:, slots[b][keep]] = v[b][:, keep]
    return kc, vc


def gather_pages(pool, table):
    """(num_pages, H_kv, page_size, D) pool and (B, max_pages) table ->
    (B, H_kv, max_pages * page_size, D) caches, and a (B, max_pages * page_size)
    mask that is False for keys whose page lies outside the pool."""
    pool = np.asarray(pool, dtype=np.float64)
    table = np.asarray(table)
    n_pages, hkv, ps, d = pool.shape
    b, mp = table.shape
    valid = (table >= 0) & (table < n_pages)
    rows = pool[np.where(valid, table, 0)]  # (B, max_pages, H_kv, page_size, D)
    cache = rows.transpose(0, 2, 1, 3, 4).reshape(b, hkv, mp * ps, d)
    return cache, np.repeat(valid, ps, axis=1)


def decode_paged(q, k_pool, v_pool, table, seqlens, sm_scale=None):
    """Decode over a paged pool: row b sees keys j < clamp(seqlens[b], 0,
    max_pages * page_size) whose page is inside the pool."""
    q = np.asarray(q, dtype=np.float64)
    k, kv_ok = gather_pages(k_pool, table)
    v, _ = gather_pages(v_pool, table)
    sk = k.shape[2]
    out = np.zeros(q.shape)
    for b, n in enumerate(np.asarray(seqlens).reshape(-1)):
        n = int(min(max(int(n), 0), sk))
        keep = np.nonzero(kv_ok[b, :n])[0]
        if keep.size:
            out[b:b + 1] = decode(q[b:b + 1], k[b:b + 1][:, :, keep], v[b:b + 1][:, :, keep], sm_scale)
    return out


def kv_cache_update_paged(k, v, k_pool, v_pool, slots):
    """Return copies of the pools with ``pool[s // ps, h, s % ps] = new[b, h, t]``,
    s = slots[b, t]; a slot outside the pool skips its token."""
    kp = np.array(k_pool, copy=True)
    vp = np.array(v_pool, copy=True)
    k = np.asarray(k)
    v = np.asarray(v)
    slots = np.asarray(slots)
    n_pages, _, ps, _ = kp.shape
    for b in range(slots.shape[0]):
        for t in range(slots.shape[1]):
            s = int(slots[b, t])
            if 0 <= s < n_pages * ps:
                kp[s // ps, :, s % ps] = k[b, :, t]
                vp[s // ps, :, s % ps] = v[b, :, t]
    return kp, vp


def round_to(x, dtype: str) -> np.ndarray:
    """float32 values rounded to the element type ``dtype`` ("bf16", "f16",
    "f32"; round to nearest even), returned as float32.  bf16 is the upper
    half of the fp32 bit pattern after adding 0x7fff plus the lowest kept bit
    (finite inputs)."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype != "bf16":
        raise ValueError(dtype)
    u = x.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def rope_tables(dim: int, max_seq_len: int, base: float = 10000.0):
    """(cos, sin), each (max_seq_len, dim) float64: angle t * base^(-i / (dim/2))
    for column i < dim/2, the same angles again for the second half
    (``src/stackkernels/_reference/torch/rope.py:6-29``)."""
    half = dim // 2
    inv_freq = 1.0 / (base ** (np.arange(half, dtype=np.float64) / half))
    ang = np.outer(np.arange(max_seq_len, dtype=np.float64), inv_freq)
    ang = np.concatenate([ang, ang], axis=1)
    return np.cos(ang), np.sin(ang)


def rope_positions(start_pos, b: int, tokens: int) -> np.ndarray:
    """(B, tokens) positions: start_pos + t, or start_pos[b] + t per row
    (``start_pos`` of ``src/stackkernels/_reference/torch/rope.py:40-58``, per row)."""
    t = np.arange(tokens, dtype=np.int64)
    base = np.asarray(start_pos, dtype=np.int64).reshape(-1, 1)
    return np.broadcast_to(base + t, (b, tokens)).copy()


def rope_rotate(x, cos, sin, positions) -> np.ndarray:
    """RoPE of x (B, H, S, D) with token (b, s) at ``positions[b, s]``.

    ``apply_rope_single`` (``src/stackkernels/_reference/torch/rope.py:40-58``,
    ``rotate_half`` ``:32-37``): out = x * cos + rotate_half(x) * sin with
    rotate_half(x) = (-x2, x1), in float32 with each product and the sum
    rounded (numpy float32 arithmetic is IEEE round-to-nearest-even).  The
    caller rounds the float32 result to the tensor's type (``round_to``).  A
    position outside the table leaves its token as it is.
    """
    x = np.asarray(x, dtype=np.float32)
    c = np.asarray(cos, dtype=np.float32)
    s = np.asarray(sin, dtype=np.float32)
    pos = np.asarray(positions, dtype=np.int64)
    d = x.shape[-1]
    half = d // 2
    ok = (pos >= 0) & (pos < c.shape[0])
    idx = np.where(ok, pos, 0)
    cc = c[idx][:, None, :, :d]  # (B, 1, S, D)
    ss = s[idx][:, None, :, :d]
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    out = (x * cc) + (rot * ss)
    return np.where(ok[:, None, :, None], out, x).astype(np.float32)


def rope_rotate_adjoint(y, cos, sin, positions, dtype=np.float32) -> np.ndarray:
    """Adjoint (transpose) of ``rope_rotate``: the gradient with respect to its
    input.  Per plane (column d < D/2 and d + D/2) the rotation is
    y_lo = x_lo c_lo - x_hi s_lo, y_hi = x_hi c_hi + x_lo s_hi, so
    x_lo = y_lo c_lo + y_hi s_hi, x_hi = y_hi c_hi - y_lo s_lo.  With tables
    whose halves are equal (``precompute_freqs``) this is the reference's
    rotation by -theta, ``dx = dy * cos - rotate_half(dy) * sin``
    (``src/stackkernels/torch/embedding.py:46-66``; Triton
    ``_rope_bwd_kernel``, ``src/stackkernels/_core/positional/rope.py:77-134``).
    In ``dtype`` arithmetic (float32: each product and the sum rounded, as
    ``rope_rotate``; float64 for checks); positions outside the table leave
    the token as it is."""
    y = np.asarray(y, dtype=dtype)
    c = np.asarray(cos, dtype=dtype)
    s = np.asarray(sin, dtype=dtype)
    pos = np.asarray(positions, dtype=np.int64)
    d = y.shape[-1]
    half = d // 2
    ok = (pos >= 0) & (pos < c.shape[0])
    idx = np.where(ok, pos, 0)
    cc = c[idx][:, None, :, :d]  # (B, 1, S, D)
    ss = s[idx][:, None, :, :d]
    lo = y[..., :half] * cc[..., :half] + y[..., half:] * ss[..., half:]
    hi = y[..., half:] * cc[..., half:] - y[..., :half] * ss[..., :half]
    out = np.concatenate([lo, hi], axis=-1)
    return np.where(ok[:, None, :, None], out, y).astype(dtype)


def attention_forward_loops(q, k, v, is_causal=False, sm_scale=None):
    """Brute-force per-element restatement for tiny shapes (pins ``attention_forward``)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    g = hq // hkv
    scale = _default_scale(d, sm_scale)
    out = np.zeros((b, hq, sq, d))
    lse = np.full((b, hq, sq), NEG_INF)
    for bi in range(b):
        for h in range(hq):
            kh = h // g
            for i in range(sq):
                keys = [j for j in range(sk) if not is_causal or j <= i + sk - sq]
                if not keys:
                    continue
                s = [scale * sum(q[bi, h, i, t] * k[bi, kh, j, t] for t in range(d)) for j in keys]
                mx = max(s)
                w = [math.exp(x - mx) for x in s]
                tot = sum(w)
                lse[bi, h, i] = mx + math.log(tot)
                for wj, j in zip(w, keys):
                    out[bi, h, i] += (wj / tot) * v[bi, kh, j]
    return out, lse


__all__ = [
    "repeat_kv",
    "allowed_mask",
    "attention_forward",
    "attention_backward",
    "softmax_probs",
    "decode",
    "split_partials",
    "combine_partials",
    "decode_varlen",
    "kv_cache_update",
    "gather_pages",
    "decode_paged",
    "kv_cache_update_paged",
    "round_to",
    "rope_tables",
    "rope_positions",
    "rope_rotate",
    "attention_forward_loops",
]
