"""PyTorch reference RoPE: the rotation the fused decode and cache-append paths apply.

Same math as the reference's ``src/stackkernels/_reference/torch/rope.py``:
tables ``cos``/``sin`` of shape (max_seq_len, D) whose two halves repeat
(``precompute_freqs``, ``:6-29``), ``rotate_half(x) = (-x2, x1)`` (``:32-37``),
and ``out = x * cos + rotate_half(x) * sin`` in float32, cast back to x's dtype
(``apply_rope_single``, ``:40-58``).  Here the rotation takes one position per
(batch row, token), the form a decode step needs (the reference takes one
``start_pos`` for the whole batch), and tensors are BHSD.
"""

from __future__ import annotations

import torch


def precompute_freqs(dim: int, max_seq_len: int = 4096, base: float = 10000.0,
                     device: torch.device | str = "cpu",
                     dtype: torch.dtype = torch.float32) -> tuple[torch.Tensor, torch.Tensor]:
    """(cos, sin), each (max_seq_len, dim): angle t / base^(i / (dim/2)) for
    i < dim/2, repeated for the second half."""
    half = dim // 2
    inv_freq = 1.0 / (base ** (torch.arange(0, half, dtype=torch.float32, device=device) / half))
    t = torch.arange(max_seq_len, dtype=torch.float32, device=device)
    freqs = torch.outer(t, inv_freq)
    cos = torch.cat([torch.cos(freqs), torch.cos(freqs)], dim=-1).to(dtype)
    sin = torch.cat([torch.sin(freqs), torch.sin(freqs)], dim=-1).to(dtype)
    return cos, sin


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """(-x2, x1) over the two halves of the last dim."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def rope_positions(start_pos, b: int, tokens: int, rows: int) -> torch.Tensor:
    """(B, tokens) int64 positions: token t of row b at start_pos + t, or
    start_pos[b] + t for a per-row (B,) tensor.  With one int for the batch
    the positions must lie in the table, as the reference's table slice
    requires; per-row positions outside it are returned as they are (the
    rotation then leaves those tokens unrotated)."""
    t = torch.arange(tokens, dtype=torch.int64)
    if isinstance(start_pos, torch.Tensor):
        base = start_pos.to("cpu", torch.int64).reshape(b, 1)
        return base + t
    start = int(start_pos)
    if tokens > 0 and b > 0 and (start < 0 or start + tokens > rows):
        raise ValueError(f"positions [{start}, {start + tokens}) lie outside the rope table "
                         f"of {rows} rows")
    return (start + t).expand(b, tokens).clone()


def apply_rope_at(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                  positions: torch.Tensor) -> torch.Tensor:
    """Rotate x (B, H, S, D) with token (b, s) at position positions[b, s];
    a position outside [0, rows) leaves its token unrotated."""
    pos = positions.to("cpu", torch.int64)
    ok = (pos >= 0) & (pos < cos.shape[0])
    idx = torch.where(ok, pos, torch.zeros_like(pos))
    c = cos.to("cpu")[idx].float().unsqueeze(1).to(x.device)  # (B, 1, S, D)
    s = sin.to("cpu")[idx].float().unsqueeze(1).to(x.device)
    xf = x.float()
    out = ((xf * c) + (rotate_half(xf) * s)).to(x.dtype)
    return torch.where(ok[:, None, :, None].to(x.device), out, x)


__all__ = ["precompute_freqs", "rotate_half", "rope_positions", "apply_rope_at"]
