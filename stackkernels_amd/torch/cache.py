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
            must be distinct within a batch row.
    """
    if should_use_hip(k_cache):
        _core_kv_cache_update(k, v, k_cache, v_cache, slot_indices)
        return
    b, _, t, s, _ = validate_cache_update(k, v, k_cache, v_cache, slot_indices)
    slots = slot_indices.to("cpu", torch.int64)
    for i in range(b):
        pos = slots[i]
        keep = (pos >= 0) & (pos < s)
        if bool(keep.any()):
            idx = pos[keep].to(k_cache.device)
            sel = keep.nonzero().flatten().to(k.device)
            k_cache[i][:, idx] = k[i][:, sel].to(k_cache.dtype)
            v_cache[i][:, idx] = v[i][:, sel].to(v_cache.dtype)


__all__ = ["kv_cache_update"]
