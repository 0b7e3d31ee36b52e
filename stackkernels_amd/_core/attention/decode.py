"""Split-KV single-token decode launcher over the gfx950 HIP kernels.

Same contract as the reference's ``flash_decode``
(``src/stackkernels/_core/attention/decode.py:192-312``): q (B, H_q, 1, D),
k/v (B, H_kv, S_k, D) with any b/h/s strides (no copy when rows are
16-byte aligned), returns (B, H_q, 1, D) in q's dtype.  ``S_q != 1`` raises
``AssertionError`` as the reference does (``:212``).  The split count comes
from the library's gfx950 table (``plan``) unless ``num_splits`` is given.
``cache_seqlens`` gives each batch row its own cache length (decode over a
batch of sequences of different lengths sharing one cache capacity).
``rope_cos`` / ``rope_sin`` / ``start_pos`` rotate q in the kernel's
prologue (the reference's ``apply_rope`` on q, fused; see ``_rope``).
"""

from __future__ import annotations

import ctypes

import torch

from stackkernels_amd._core.attention import _lib
from stackkernels_amd._core.attention._rope import rope_args
from stackkernels_amd._core.attention._common import (
    check_device,
    default_scale,
    kernel_head_dim,
    kernel_operand,
    pad_head,
    stream_of,
)
from stackkernels_amd._core.attention.layout import validate_attention_layout
from stackkernels_amd._core.attention.workspace import decode_workspace


def plan(dtype: torch.dtype, b: int, hq: int, hkv: int, sk: int, d: int,
         per_row: bool = False) -> tuple[int, int]:
    """(num_splits, workspace bytes) the library picks for this decode shape
    (``per_row``: with per-row cache lengths or a paged pool)."""
    lib = _lib.load()
    ns = ctypes.c_int(0)
    nb = ctypes.c_size_t(0)
    fn = lib.sk_decode_plan_varlen if per_row else lib.sk_decode_plan
    _lib.check(fn(_lib.dtype_code(dtype), b, hq, hkv, sk, kernel_head_dim(d), ctypes.byref(ns),
                  ctypes.byref(nb)), "flash_decode plan")
    return ns.value, nb.value


def _seqlens_operand(cache_seqlens, b: int, dev) -> torch.Tensor:
    """cache_seqlens as the kernels read it: int32 (B,) on q's device."""
    if not isinstance(cache_seqlens, torch.Tensor):
        cache_seqlens = torch.as_tensor(cache_seqlens)
    if cache_seqlens.dim() != 1 or cache_seqlens.shape[0] != b:
        raise ValueError(f"cache_seqlens must have shape ({b},), got {tuple(cache_seqlens.shape)}")
    if cache_seqlens.dtype.is_floating_point or cache_seqlens.dtype == torch.bool:
        raise ValueError(f"cache_seqlens must be an integer tensor, got {cache_seqlens.dtype}")
    return cache_seqlens.to(device=dev, dtype=torch.int32).contiguous()


def flash_decode(q, k, v, sm_scale: float | None = None, num_splits: int | None = None,
                 cache_seqlens=None, rope_cos=None, rope_sin=None, start_pos=0):
    """Launch split + combine; see module docstring.

    ``cache_seqlens`` (optional, integer (B,)): row b attends to keys
    ``[0, min(cache_seqlens[b], S_k))`` of its cache (S_k is the capacity);
    a row with no key gives O = 0.  With ``rope_cos`` / ``rope_sin``
    ((max_seq_len, D) tables) q is rotated to position ``start_pos`` (int, or
    integer (B,) per row) before the scores."""
    b, hq, hkv, sq, sk, d = validate_attention_layout(q, k, v)
    assert sq == 1, f"flash_decode requires q_len == 1, got {sq}"
    dev = check_device(q, k, v)
    lens = None if cache_seqlens is None else _seqlens_operand(cache_seqlens, b, dev)
    rope = rope_args(rope_cos, rope_sin, start_pos, b, d, dev)
    scale = default_scale(d, sm_scale)
    dk = kernel_head_dim(d)
    qk, kk, vk = (kernel_operand(pad_head(t, dk)) for t in (q, k, v))
    lib = _lib.load()
    code = _lib.dtype_code(q.dtype)
    ws, ns = decode_workspace(q.dtype, b, hq, hkv, sk, dk, dev, num_splits,
                              per_row=lens is not None)
    out = torch.empty((b, hq, 1, dk), dtype=q.dtype, device=dev)
    with torch.cuda.device(dev):
        if rope is not None:
            rc = lib.sk_decode_rope(
                code, qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), out.data_ptr(), ws.data_ptr(),
                ws.numel(), ns, b, hq, hkv, sk, dk,
                _lib.strides3(qk), _lib.strides3(kk), _lib.strides3(vk), _lib.strides3(out),
                None if lens is None else lens.data_ptr(), *rope.args, scale, stream_of(dev),
            )
        elif lens is None:
            rc = lib.sk_decode(
                code, qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), out.data_ptr(), ws.data_ptr(),
                ws.numel(), ns, b, hq, hkv, sk, dk,
                _lib.strides3(qk), _lib.strides3(kk), _lib.strides3(vk), _lib.strides3(out),
                scale, stream_of(dev),
            )
        else:
            rc = lib.sk_decode_varlen(
                code, qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), out.data_ptr(), ws.data_ptr(),
                ws.numel(), ns, b, hq, hkv, sk, dk,
                _lib.strides3(qk), _lib.strides3(kk), _lib.strides3(vk), _lib.strides3(out),
                lens.data_ptr(), scale, stream_of(dev),
            )
    _lib.check(rc, "flash_decode")
    if dk != d:
        out = out[..., :d].contiguous()
    return out


def _table_operand(block_table, b: int, dev) -> torch.Tensor:
    if not isinstance(block_table, torch.Tensor):
        block_table = torch.as_tensor(block_table)
    if block_table.dim() != 2 or block_table.shape[0] != b:
        raise ValueError(f"block_table must have shape ({b}, max_pages), got "
                         f"{tuple(block_table.shape)}")
    if block_table.dtype.is_floating_point or block_table.dtype == torch.bool:
        raise ValueError(f"block_table must be an integer tensor, got {block_table.dtype}")
    return block_table.to(device=dev, dtype=torch.int32).contiguous()


def flash_decode_paged(q, k_pool, v_pool, block_table, cache_seqlens,
                       sm_scale: float | None = None, num_splits: int | None = None,
                       rope_cos=None, rope_sin=None, start_pos=0):
    """Decode over a paged KV cache.

    q (B, H_q, 1, D); k_pool, v_pool (num_pages, H_kv, page_size, D) with any
    page/head/row strides; block_table integer (B, max_pages): page of each
    page_size-key block of a row; cache_seqlens integer (B,): keys per row.
    Key j of row b is row ``j % page_size`` of page ``block_table[b, j // page_size]``.
    page_size must be a multiple of 32.  A page index outside the pool masks
    its keys; a row with no key gives zeros.  Returns (B, H_q, 1, D).  RoPE
    arguments as for ``flash_decode``."""
    if q.dim() != 4 or k_pool.dim() != 4 or v_pool.dim() != 4:
        raise ValueError("Expected 4D q (B, H, 1, D) and 4D page pools (pages, H_kv, page_size, D)")
    if k_pool.shape != v_pool.shape:
        raise ValueError(f"k_pool and v_pool shapes differ: {tuple(k_pool.shape)} vs "
                         f"{tuple(v_pool.shape)}")
    b, hq, sq, d = q.shape
    num_pages, hkv, page_size, dk_ = k_pool.shape
    assert sq == 1, f"flash_decode requires q_len == 1, got {sq}"
    if dk_ != d:
        raise ValueError(f"Head dimension mismatch: q has {d}, k has {dk_}")
    if hq % hkv != 0:
        raise ValueError(f"Query heads ({hq}) must be divisible by KV heads ({hkv}) for GQA/MQA")
    if page_size <= 0 or page_size % 32 != 0:
        raise ValueError(f"page_size (k_pool.shape[2]) must be a positive multiple of 32, "
                         f"got {page_size}")
    dev = check_device(q, k_pool, v_pool)
    table = _table_operand(block_table, b, dev)
    lens = _seqlens_operand(cache_seqlens, b, dev)
    rope = rope_args(rope_cos, rope_sin, start_pos, b, d, dev)
    max_pages = table.shape[1]
    scale = default_scale(d, sm_scale)
    dk = kernel_head_dim(d)
    qk, kk, vk = (kernel_operand(pad_head(t, dk)) for t in (q, k_pool, v_pool))
    lib = _lib.load()
    code = _lib.dtype_code(q.dtype)
    sk = max_pages * page_size
    ws, ns = decode_workspace(q.dtype, b, hq, hkv, sk, dk, dev, num_splits, per_row=True)
    out = torch.empty((b, hq, 1, dk), dtype=q.dtype, device=dev)
    paged_args = (code, qk.data_ptr(), kk.data_ptr(), vk.data_ptr(), out.data_ptr(),
                  ws.data_ptr(), ws.numel(), ns, b, hq, hkv, num_pages, page_size, max_pages, dk,
                  _lib.strides3(qk), _lib.strides3(kk), _lib.strides3(vk), _lib.strides3(out),
                  table.data_ptr(), lens.data_ptr())
    with torch.cuda.device(dev):
        if rope is None:
            rc = lib.sk_decode_paged(*paged_args, scale, stream_of(dev))
        else:
            rc = lib.sk_decode_paged_rope(*paged_args, *rope.args, scale, stream_of(dev))
    _lib.check(rc, "flash_decode")
    if dk != d:
        out = out[..., :d].contiguous()
    return out


__all__ = ["flash_decode", "flash_decode_paged", "plan"]
