"""HIP attention launchers (forward, backward, split-KV decode) and the
bottom-right causal mask helpers, under the reference's names
(``src/stackkernels/_core/attention/__init__.py:3-14``)."""

from stackkernels_amd._core.attention._masks import build_causal_mask, causal_mask_check
from stackkernels_amd._core.attention.decode import flash_decode
from stackkernels_amd._core.attention.flash_bwd import flash_attn_bwd
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd

__all__ = [
    "flash_attn_fwd",
    "flash_attn_bwd",
    "flash_decode",
    "causal_mask_check",
    "build_causal_mask",
]
