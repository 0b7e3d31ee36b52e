"""Scratch buffers the C ABI takes, sized by the library and allocated by torch.

The reference allocates its scratch in the launchers
(``src/stackkernels/_opt/memory/workspace.py:6-46``: LSE, delta and the
split-KV partials as separate float32 tensors).  Here the library sizes one
byte buffer per call (``sk_attn_bwd_workspace``, ``sk_decode_plan`` /
``sk_decode_workspace``) and never allocates; these helpers take that buffer
from torch's caching allocator.  The launchers use them, and callers that bind
the library directly can too.
"""

from __future__ import annotations

import ctypes

import torch

from stackkernels_amd._core.attention import _lib


def bwd_workspace(dtype: torch.dtype, B: int, Hq: int, Hkv: int, Sq: int, Sk: int, D: int,
                  is_causal: bool, device) -> torch.Tensor:
    """uint8 scratch for ``sk_attn_bwd`` (D: the kernel head dim; at least 16 bytes).

    The library's preferred size (row statistics plus one chunk of the
    five-GEMM backward's dS tiles, at most ``SK_BWD_DS_CAP_BYTES`` of them);
    if torch cannot allocate that, the minimum (row statistics only), with
    which the call runs the seven-GEMM backward: the same results, slower.
    """
    lib = _lib.load()
    code = _lib.dtype_code(dtype)
    args = (code, B, Hq, Hkv, Sq, Sk, D, int(bool(is_causal)))
    nb = ctypes.c_size_t(0)
    _lib.check(lib.sk_attn_bwd_workspace(*args, ctypes.byref(nb)), "flash_attn_bwd")
    nmin = ctypes.c_size_t(0)
    _lib.check(lib.sk_attn_bwd_workspace_min(*args, ctypes.byref(nmin)), "flash_attn_bwd")
    try:
        return torch.empty(max(nb.value, 16), dtype=torch.uint8, device=device)
    except torch.OutOfMemoryError:
        if nb.value <= nmin.value:
            raise
    return torch.empty(max(nmin.value, 16), dtype=torch.uint8, device=device)


def decode_workspace(dtype: torch.dtype, B: int, Hq: int, Hkv: int, Sk: int, D: int, device,
                     num_splits: int | None = None,
                     per_row: bool = False) -> tuple[torch.Tensor, int]:
    """(uint8 scratch, split count) for ``sk_decode*`` (D: the kernel head dim):
    the gfx950 table's split count when ``num_splits`` is None (``per_row``:
    the plan for per-row cache lengths and paged pools), else the given one."""
    lib = _lib.load()
    code = _lib.dtype_code(dtype)
    nb = ctypes.c_size_t(0)
    if num_splits is None:
        ns = ctypes.c_int(0)
        fn = lib.sk_decode_plan_varlen if per_row else lib.sk_decode_plan
        _lib.check(fn(code, B, Hq, Hkv, Sk, D, ctypes.byref(ns), ctypes.byref(nb)),
                   "flash_decode plan")
        num_splits = ns.value
    else:
        _lib.check(lib.sk_decode_workspace(code, B, Hq, Hkv, Sk, D, int(num_splits),
                                           ctypes.byref(nb)), "flash_decode")
    return torch.empty(max(nb.value, 16), dtype=torch.uint8, device=device), int(num_splits)


__all__ = ["bwd_workspace", "decode_workspace"]
