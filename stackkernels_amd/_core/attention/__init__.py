"""HIP attention launchers: forward, backward, split-KV decode."""

from stackkernels_amd._core.attention.decode import flash_decode
from stackkernels_amd._core.attention.flash_bwd import flash_attn_bwd
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd

__all__ = ["flash_attn_fwd", "flash_attn_bwd", "flash_decode"]
