"""Bottom-right causal mask helper (torch), as ``_core/attention/_masks.py:22-35``.

The kernels apply the same rule inline: key j is visible to query i iff
j <= i + (S_k - S_q).
"""

from __future__ import annotations

import torch


def build_causal_mask(seqlen_q: int, seqlen_k: int, device=None, dtype=torch.bool) -> torch.Tensor:
    """(S_q, S_k) mask, True where the query may attend the key."""
    qi = torch.arange(seqlen_q, device=device)[:, None]
    kj = torch.arange(seqlen_k, device=device)[None, :]
    return (kj <= qi + (seqlen_k - seqlen_q)).to(dtype)


__all__ = ["build_causal_mask"]
