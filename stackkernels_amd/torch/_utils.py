"""Contiguity helper (reference ``src/stackkernels/torch/_utils.py:6-10``)."""

import torch


def ensure_contiguous(tensor: torch.Tensor) -> torch.Tensor:
    """Return ``tensor`` if contiguous, else a contiguous copy."""
    return tensor if tensor.is_contiguous() else tensor.contiguous()


__all__ = ["ensure_contiguous"]
