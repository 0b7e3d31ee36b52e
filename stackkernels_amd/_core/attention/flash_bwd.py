"""Backward attention launcher over the gfx950 HIP kernels.

Same contract as the reference's ``flash_attn_bwd``
(``src/stackkernels/_core/attention/flash_bwd.py:362-528``): returns
``(dq, dk, dv)``; dk/dv are summed over each KV head's query group.
"""

from __future__ import annotations

import torch

from stackkernels_amd._core.attention import _lib
from stackkernels_amd._core.attention._common import (
    check_device,
    default_scale,
    kernel_head_dim,
    pad_head,
    stream_of,
)
from stackkernels_amd._core.attention.layout import validate_attention_layout
from stackkernels_amd._core.attention.workspace import bwd_workspace


def _contig(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def flash_attn_bwd(do, q, k, v, out, lse, is_causal: bool = False, sm_scale: float | None = None):
    """Launch the HIP backward; see module docstring."""
    b, hq, hkv, sq, sk, d = validate_attention_layout(q, k, v)
    dev = check_device(q, k, v, out, do)
    scale = default_scale(d, sm_scale)
    dk_ = kernel_head_dim(d)
    do_, q_, k_, v_, o_ = (_contig(pad_head(t, dk_)) for t in (do, q, k, v, out))
    lse_ = _contig(lse.float())
    dq = torch.empty((b, hq, sq, dk_), dtype=q.dtype, device=dev)
    dkk = torch.empty((b, hkv, sk, dk_), dtype=q.dtype, device=dev)
    dvv = torch.empty((b, hkv, sk, dk_), dtype=q.dtype, device=dev)
    lib = _lib.load()
    code = _lib.dtype_code(q.dtype)
    ws = bwd_workspace(q.dtype, b, hq, hkv, sq, sk, dk_, is_causal, dev)
    with torch.cuda.device(dev):
        rc = lib.sk_attn_bwd(
            code, do_.data_ptr(), q_.data_ptr(), k_.data_ptr(), v_.data_ptr(), o_.data_ptr(),
            lse_.data_ptr(), dq.data_ptr(), dkk.data_ptr(), dvv.data_ptr(), ws.data_ptr(),
            ws.numel(), b, hq, hkv, sq, sk, dk_, int(bool(is_causal)), scale, stream_of(dev),
        )
    _lib.check(rc, "flash_attn_bwd")
    if dk_ != d:
        dq, dkk, dvv = (t[..., :d].contiguous() for t in (dq, dkk, dvv))
    return dq, dkk, dvv


__all__ = ["flash_attn_bwd"]
