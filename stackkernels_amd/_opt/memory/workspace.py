"""Scratch buffers of the attention path.

The reference's allocators (``src/stackkernels/_opt/memory/workspace.py:6-46``)
with the same shapes and dtypes, plus the byte-sized scratch the C ABI takes
(``sk_attn_bwd_workspace`` / ``sk_decode_plan``) for callers that bind the
library directly.  Everything comes from torch's caching allocator; the library
itself never allocates.
"""

from __future__ import annotations

import ctypes

import torch


def allocate_lse_buffer(batch_size: int, num_heads: int, seqlen: int,
                        device: torch.device) -> torch.Tensor:
    """Log-sum-exp buffer (B, H, S) in float32."""
    return torch.empty((batch_size, num_heads, seqlen), dtype=torch.float32, device=device)


def allocate_delta_buffer(batch_size: int, num_heads: int, seqlen: int,
                          device: torch.device) -> torch.Tensor:
    """Backward delta buffer D = sum(dO * O), (B, H, S) in float32."""
    return torch.empty((batch_size, num_heads, seqlen), dtype=torch.float32, device=device)


def allocate_split_kv_buffers(batch_size: int, num_heads: int, split_kv: int, head_dim: int,
                              device: torch.device, dtype: torch.dtype = torch.float32
                              ) -> tuple[torch.Tensor, torch.Tensor]:
    """Split-KV partials: (partial_out (B, H, split_kv, D), partial_lse (B, H, split_kv))."""
    partial_out = torch.empty((batch_size, num_heads, split_kv, head_dim), dtype=dtype,
                              device=device)
    partial_lse = torch.empty((batch_size, num_heads, split_kv), dtype=torch.float32,
                              device=device)
    return partial_out, partial_lse


def bwd_workspace(dtype: torch.dtype, B: int, Hq: int, Hkv: int, Sq: int, Sk: int, D: int,
                  is_causal: bool, device: torch.device) -> torch.Tensor:
    """The scratch ``sk_attn_bwd`` needs (uint8, at least 16 bytes)."""
    from stackkernels_amd._core.attention import _lib

    nb = ctypes.c_size_t(0)
    _lib.check(_lib.load().sk_attn_bwd_workspace(_lib.dtype_code(dtype), B, Hq, Hkv, Sq, Sk, D,
                                                 int(bool(is_causal)), ctypes.byref(nb)),
               "bwd_workspace")
    return torch.empty(max(nb.value, 16), dtype=torch.uint8, device=device)


def decode_workspace(dtype: torch.dtype, B: int, Hq: int, Hkv: int, Sk: int, D: int,
                     device: torch.device, num_splits: int = 0) -> tuple[torch.Tensor, int]:
    """(scratch, split count) for ``sk_decode*``: the gfx950 table's split count
    when ``num_splits`` is 0, else the given one."""
    from stackkernels_amd._core.attention import _lib

    lib = _lib.load()
    code = _lib.dtype_code(dtype)
    nb = ctypes.c_size_t(0)
    if num_splits == 0:
        ns = ctypes.c_int(0)
        _lib.check(lib.sk_decode_plan(code, B, Hq, Hkv, Sk, D, ctypes.byref(ns), ctypes.byref(nb)),
                   "decode_workspace")
        num_splits = ns.value
    else:
        _lib.check(lib.sk_decode_workspace(code, B, Hq, Hkv, Sk, D, int(num_splits),
                                           ctypes.byref(nb)), "decode_workspace")
    return torch.empty(max(nb.value, 16), dtype=torch.uint8, device=device), int(num_splits)


__all__ = [
    "allocate_lse_buffer",
    "allocate_delta_buffer",
    "allocate_split_kv_buffers",
    "bwd_workspace",
    "decode_workspace",
]
