"""Bottom-right causal mask (reference ``_core/attention/_masks.py:9-35``).

Key j is visible to query i iff j <= i + (S_k - S_q): the last query row
sees every key, and when S_q > S_k the first S_q - S_k rows see none.  The
HIP kernels apply the same rule inline, per tile; these helpers give it to
Python callers (reference-path code, tests, masks for other libraries).
"""

from __future__ import annotations

import torch


def causal_mask_check(m_idx, n_idx, seqlen_q: int, seqlen_k: int):
    """True where query ``m_idx`` may attend key ``n_idx`` (ints or tensors,
    broadcast elementwise).  The reference's version (``_masks.py:9-19``) is a
    Triton device helper; here it is plain Python / torch arithmetic."""
    return n_idx <= m_idx + (seqlen_k - seqlen_q)


def build_causal_mask(seqlen_q: int, seqlen_k: int, device=None, dtype=torch.bool) -> torch.Tensor:
    """(S_q, S_k) mask in ``dtype``, True (1) where the query may attend the key."""
    qi = torch.arange(seqlen_q, device=device)[:, None]
    kj = torch.arange(seqlen_k, device=device)[None, :]
    return causal_mask_check(qi, kj, seqlen_q, seqlen_k).to(dtype)


__all__ = ["causal_mask_check", "build_causal_mask"]
