"""KV-cache append launcher over the gfx950 HIP kernel ``sk_kv_cache_update``.

Realises the reference's planned ``kv_cache_update(k, v, k_cache, v_cache,
slot_indices)`` (``docs/user_guide/dropout_cache_sampling.md:66-72``; the
reference's ``src/stackkernels/_core/cache/kv_update.py`` is a stub):
``k_cache[b, h, slot_indices[b, t], :] = k[b, h, t, :]`` and the same for v,
in place, with no reallocation.  A slot outside ``[0, S_cache)`` skips its
token (pad ragged batches with -1).  With RoPE tables the new keys are
rotated on their way into the cache (the reference's ``apply_rope`` on k,
fused into the append; values are copied unchanged).
"""

from __future__ import annotations

import torch

from stackkernels_amd._core.attention import _lib
from stackkernels_amd._core.attention._common import check_device, stream_of
from stackkernels_amd._core.attention._rope import rope_args


def validate_cache_update(k, v, k_cache, v_cache, slot_indices,
                          paged: bool = False) -> tuple[int, int, int, int, int]:
    """Shapes (B, Hkv, T, S_cache, D) -- for a paged pool S_cache is the pool's
    num_pages * page_size slots; raises ValueError on a mismatch."""
    for name, t in (("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dim() != 4:
            raise ValueError(f"Expected 4D tensor for {name} (B, H, S, D), got {t.dim()}D")
    if k.shape != v.shape:
        raise ValueError(f"k and v shapes differ: {tuple(k.shape)} vs {tuple(v.shape)}")
    if k_cache.shape != v_cache.shape:
        raise ValueError(f"k_cache and v_cache shapes differ: {tuple(k_cache.shape)} vs "
                         f"{tuple(v_cache.shape)}")
    b, h, t, d = k.shape
    bc, hc, s, dc = k_cache.shape
    if paged:
        if (hc, dc) != (h, d):
            raise ValueError(f"pool (H, D) = {(hc, dc)} does not match new keys' {(h, d)}")
        s = bc * s  # pool slots: num_pages * page_size
    elif (bc, hc, dc) != (b, h, d):
        raise ValueError(f"cache (B, H, D) = {(bc, hc, dc)} does not match new keys' {(b, h, d)}")
    if tuple(slot_indices.shape) != (b, t):
        raise ValueError(f"slot_indices must have shape ({b}, {t}), got {tuple(slot_indices.shape)}")
    if slot_indices.dtype.is_floating_point or slot_indices.dtype == torch.bool:
        raise ValueError(f"slot_indices must be an integer tensor, got {slot_indices.dtype}")
    for name, x in (("k", k), ("v", v), ("k_cache", k_cache), ("v_cache", v_cache)):
        if x.stride(-1) != 1 and x.shape[-1] != 1:
            raise ValueError(f"{name} needs a contiguous head dim (stride(-1) == 1)")
    return b, h, t, s, d


def kv_cache_update(k, v, k_cache, v_cache, slot_indices, paged: bool = False,
                    rope_cos=None, rope_sin=None, start_pos=0) -> None:
    """Write k, v (B, Hkv, T, D) into k_cache, v_cache (B, Hkv, S_cache, D) at
    slot_indices (B, T); in place, on the caches' stream.  With ``paged`` the
    caches are page pools (num_pages, Hkv, page_size, D) and a slot s is row
    ``s % page_size`` of page ``s // page_size``.  With ``rope_cos`` /
    ``rope_sin`` ((max_seq_len, D) tables) new token t of row b is rotated to
    position ``start_pos + t`` (``start_pos``: int, or integer (B,) per row)
    before it is written."""
    b, h, t, s, d = validate_cache_update(k, v, k_cache, v_cache, slot_indices, paged)
    dev = check_device(k, v, k_cache, v_cache)
    slots = slot_indices.to(device=dev, dtype=torch.int64).contiguous()
    rope = rope_args(rope_cos, rope_sin, start_pos, b, d, dev)
    lib = _lib.load()
    sts = (_lib.strides3(k), _lib.strides3(v), _lib.strides3(k_cache), _lib.strides3(v_cache))
    with torch.cuda.device(dev):
        if rope is not None and paged:
            rc = lib.sk_kv_cache_update_paged_rope(
                _lib.dtype_code(k.dtype), k.data_ptr(), v.data_ptr(), k_cache.data_ptr(),
                v_cache.data_ptr(), slots.data_ptr(), b, h, t, k_cache.shape[0],
                k_cache.shape[2], d, *sts, *rope.args, stream_of(dev))
        elif rope is not None:
            rc = lib.sk_kv_cache_update_rope(
                _lib.dtype_code(k.dtype), k.data_ptr(), v.data_ptr(), k_cache.data_ptr(),
                v_cache.data_ptr(), slots.data_ptr(), b, h, t, s, d, *sts, *rope.args,
                stream_of(dev))
        elif paged:
            rc = lib.sk_kv_cache_update_paged(
                _lib.dtype_code(k.dtype), k.data_ptr(), v.data_ptr(), k_cache.data_ptr(),
                v_cache.data_ptr(), slots.data_ptr(), b, h, t, k_cache.shape[0],
                k_cache.shape[2], d, *sts, stream_of(dev))
        else:
            rc = lib.sk_kv_cache_update(
                _lib.dtype_code(k.dtype), k.data_ptr(), v.data_ptr(), k_cache.data_ptr(),
                v_cache.data_ptr(), slots.data_ptr(), b, h, t, s, d, *sts, stream_of(dev))
    _lib.check(rc, "kv_cache_update")


__all__ = ["kv_cache_update", "validate_cache_update"]
