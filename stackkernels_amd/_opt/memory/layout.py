"""Attention shape rules: the reference's ``_opt/memory/layout.py`` names.

``validate_attention_layout`` is the reference's check with its ``ValueError``
messages (``src/stackkernels/_opt/memory/layout.py:7-41``).
``get_padded_head_dim`` answers for this build's kernels: the head dim the
gfx950 kernels are compiled for and run at (64, 96, 128 or 256; the reference's
answer, ``:44-56``, is the Triton tile width, a power of two from 16).
"""

from __future__ import annotations

from stackkernels_amd._core.attention.layout import (
    MAX_HEAD_DIM,
    padded_head_dim,
    validate_attention_layout,
)


def get_padded_head_dim(D: int) -> int:
    """Head dim the kernels run ``D`` at; raises ValueError above 256."""
    p = padded_head_dim(int(D))
    if p == 0:
        raise ValueError(f"head dim {D} > {MAX_HEAD_DIM} has no kernel")
    return p


__all__ = ["validate_attention_layout", "get_padded_head_dim"]
