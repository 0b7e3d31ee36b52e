"""PyTorch frontend: the reference's ``stackkernels.torch`` attention API."""

from stackkernels_amd.torch.attention import (
    FlashAttention,
    FlashAttentionFunction,
    flash_attention,
    flash_decode,
)

from stackkernels_amd.torch.cache import kv_cache_update

__all__ = ["flash_attention", "flash_decode", "FlashAttention", "FlashAttentionFunction",
           "kv_cache_update"]
