"""Forward attention launcher over the gfx950 HIP kernel.

Same contract as the reference's ``flash_attn_fwd``
(``src/stackkernels/_core/attention/flash_fwd.py:182-264``): returns
``(out, lse)`` with ``out`` (B, H_q, S_q, D) in the input dtype and ``lse``
(B, H_q, S_q) fp32; GQA/MQA by ``H_q % H_kv == 0``; bottom-right causal mask.
``rope_cos`` / ``rope_sin`` / ``start_pos`` rotate q in the kernel's prologue
(query row i at position ``start_pos + i``): the prefill step with the
reference's ``apply_rope`` on q fused in.  This launcher is forward only; the
torch-level ``flash_attention`` pairs it with a backward that rotates q again
(``sk_rope_rotate``) and carries dQ back through the rotation's adjoint.
"""

from __future__ import annotations

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


def flash_attn_fwd(q, k, v, is_causal: bool = False, sm_scale: float | None = None,
                   rope_cos=None, rope_sin=None, start_pos=0):
    """Launch the HIP forward kernel; see module docstring."""
    b, hq, hkv, sq, sk, d = validate_attention_layout(q, k, v)
    dev = check_device(q, k, v)
    rope = rope_args(rope_cos, rope_sin, start_pos, b, d, dev)
    scale = default_scale(d, sm_scale)
    dk = kernel_head_dim(d)
    qk, kk, vk = (kernel_operand(pad_head(t, dk)) for t in (q, k, v))
    out = torch.empty((b, hq, sq, dk), dtype=q.dtype, device=dev)
    lse = torch.empty((b, hq, sq), dtype=torch.float32, device=dev)
    lib = _lib.load()
    args = (_lib.dtype_code(q.dtype), qk.data_ptr(), kk.data_ptr(), vk.data_ptr(),
            out.data_ptr(), lse.data_ptr(), b, hq, hkv, sq, sk, dk,
            _lib.strides3(qk), _lib.strides3(kk), _lib.strides3(vk), _lib.strides3(out),
            int(bool(is_causal)))
    with torch.cuda.device(dev):
        if rope is None:
            rc = lib.sk_attn_fwd(*args, scale, stream_of(dev))
        else:
            rc = lib.sk_attn_fwd_rope(*args, *rope.args, scale, stream_of(dev))
    _lib.check(rc, "flash_attn_fwd")
    if dk != d:
        out = out[..., :d].contiguous()
    return out, lse


__all__ = ["flash_attn_fwd"]
