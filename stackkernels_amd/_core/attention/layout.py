"""Shape rules for the attention kernels.

``validate_attention_layout`` keeps the reference's checks and ``ValueError``
messages (``src/stackkernels/_opt/memory/layout.py:7-41``).
``get_padded_head_dim`` keeps the reference's helper and its values
(``layout.py:44-56``: the power-of-two tile width, 16 up to D = 16, 32 up to
32, then 64, 128, 256 and the next power of two beyond).  ``padded_head_dim``
is this build's own rule, what the launchers use: the gfx950 kernels are
compiled for head dims padded to 64, 96, 128 or 256 (0 above 256, where no
kernel exists).
"""

from __future__ import annotations


def validate_attention_layout(q, k, v) -> tuple[int, int, int, int, int, int]:
    """Check (B, H, S, D) shapes for MHA/GQA/MQA; return (B, H_q, H_kv, S_q, S_k, D)."""
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError(
            f"Expected 4D tensors (B, H, S, D), got q={q.ndim}D, k={k.ndim}D, v={v.ndim}D"
        )
    b, hq, sq, d = q.shape
    bk, hkv, sk, dk = k.shape
    bv, hv, sv, dv = v.shape
    if b != bk or b != bv:
        raise ValueError(f"Batch mismatch: q={b}, k={bk}, v={bv}")
    if hkv != hv:
        raise ValueError(f"K and V head count mismatch: {hkv} vs {hv}")
    if sk != sv:
        raise ValueError(f"K and V sequence length mismatch: {sk} vs {sv}")
    if d != dk or d != dv:
        raise ValueError(f"Head dimension mismatch: q={d}, k={dk}, v={dv}")
    if hkv == 0 or hq % hkv != 0:
        raise ValueError(f"Query heads ({hq}) must be divisible by KV heads ({hkv}) for GQA/MQA")
    return b, hq, hkv, sq, sk, d


def padded_head_dim(d: int) -> int:
    """Head dim the gfx950 kernels run at: 64, 96, 128 or 256 (0 if d > 256)."""
    for p in (64, 96, 128, 256):
        if d <= p:
            return p
    return 0


MAX_HEAD_DIM = 256


def get_padded_head_dim(D: int) -> int:
    """The reference's tile padding of ``D``: the smallest power of two >= D, at least
    16 (``src/stackkernels/_opt/memory/layout.py:44-56``).  The kernels here run at
    ``padded_head_dim(D)`` instead."""
    D = int(D)
    for p in (16, 32, 64, 128, 256):
        if D <= p:
            return p
    return 1 << (D - 1).bit_length()
