"""KV-cache in-place update: the reference's planned ``stackkernels.torch.cache``
API (``docs/user_guide/dropout_cache_sampling.md:66-72``; the reference module
``src/stackkernels/torch/cache.py`` is still a stub).

ROCm device tensors run the HIP kernel; CPU tensors and ``backend='reference'``
run the same update with torch indexing.
"""

from __future__ import annotations

import torch

from stackkernels_amd._core.cache.kv_update import kv_cache_update as _core_kv_cache_update
from stackkernels_amd._core.cache.kv_update import validate_cache_update
from stackkernels_amd.torch._dispatch import should_use_hip


def kv_cache_update(
    k: torch.Tensor,
    v: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_indices: torch.Tensor,
    paged: bool = False,
    *,
    rope_cos: torch.Tensor | None = None,
    rope_sin: torch.Tensor | None = None,
    start_pos: int | torch.Tensor = 0,
) -> None:
    """Insert new key/value rows into the caches in place.

    ``k_cache[b, h, slot_indices[b, t], :] = k[b, h, t, :]`` (and for v) for every
    batch row b, KV head h and new token t.

    Args:
        k, v: (B, H_kv, T, D) new keys and values.
        k_cache, v_cache: (B, H_kv, S_cache, D) caches (any b/h/s strides, contiguous D),
            updated in place.
        slot_indices: integer (B, T) cache positions.  A position outside
            ``[0, S_cache)`` skips its token (pad ragged batches with -1).  Positions
            must be distinct within a batch row (within the pool when paged).
        paged: the caches are page pools (num_pages, H_kv, page_size, D) shared by
            all rows, and a position s is row ``s % page_size`` of page
            ``s // page_size`` (S_cache = num_pages * page_size).
        rope_cos, rope_sin: optional (max_seq_len, D) RoPE tables: the new keys are
            rotated (the reference's ``apply_rope`` on k) as they are written, new
            token t of row b at position ``start_pos + t``; values are copied as
            they are.
        start_pos: int, or integer (B,) tensor of per-row positions of token 0.
    """
    rope = rope_cos is not None or rope_sin is not None
    if should_use_hip(k_cache):
        extra = dict(rope_cos=rope_cos, rope_sin=rope_sin, start_pos=start_pos) if rope else {}
        _core_kv_cache_update(k, v, k_cache, v_cache, slot_indices, paged, **extra)
        return
    b, _, t, s, _ = validate_cache_update(k, v, k_cache, v_cache, slot_indices, paged)
    if rope:
        from stackkernels_amd.torch.attention import _rope_reference

        k = _rope_reference(k, rope_cos, rope_sin, start_pos)
    slots = slot_indices.to("cpu", torch.int64)
    if paged:
        ps = k_cache.shape[2]
        for i in range(b):
            for j in range(t):
                pos = int(slots[i, j])
                if 0 <= pos < s:
                    k_cache[pos // ps, :, pos % ps] = k[i, :, j].to(k_cache.dtype)
                    v_cache[pos // ps, :, pos % ps] = v[i, :, j].to(v_cache.dtype)
        return
    for i in range(b):
        pos = slots[i]
        keep = (pos >= 0) & (pos < s)
        if bool(keep.any()):
            idx = pos[keep].to(k_cache.device)
            sel = keep.nonzero().flatten().to(k.device)
            k_cache[i][:, idx] = k[i][:, sel].to(k_cache.dtype)
            v_cache[i][:, idx] = v[i][:, sel].to(v_cache.dtype)


__all__ = ["kv_cache_update"]
