"""RoPE arguments of the fused ``*_rope`` library calls.

The rotation is the reference's ``apply_rope`` (``src/stackkernels/torch/embedding.py:67-100``;
math in ``src/stackkernels/_reference/torch/rope.py:32-58``), applied by the
kernels to q or to the new keys as they load them.  Tables are the
``(max_seq_len, D)`` ``cos`` / ``sin`` of ``precompute_freqs``
(``_reference/torch/rope.py:6-29``); ``start_pos`` is the reference's
``start_pos`` (an int for the whole batch) or, for a batch of sequences at
different lengths, an integer ``(B,)`` tensor of per-row positions.
"""

from __future__ import annotations

import torch

from stackkernels_amd._core.attention import _lib

_TABLE_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


class RopeArgs:
    """Validated tables and positions; ``args`` is the ctypes tail
    (cos, sin, dtype code, rows, row stride, positions or None, start)."""

    def __init__(self, cos, sin, start_pos, b: int, d: int, dev: torch.device):
        if cos is None or sin is None:
            raise ValueError("RoPE needs both cos and sin tables")
        for name, t in (("cos", cos), ("sin", sin)):
            if not isinstance(t, torch.Tensor) or t.dim() != 2:
                raise ValueError(f"{name} must be a 2-D (max_seq_len, D) tensor")
            if t.device != dev:
                raise ValueError(f"{name} is on {t.device}, the attention tensors on {dev}")
            if t.dtype not in _TABLE_DTYPES:
                raise NotImplementedError(f"{name} dtype {t.dtype} unsupported "
                                          f"(float32, float16, bfloat16)")
        if cos.shape != sin.shape or cos.dtype != sin.dtype:
            raise ValueError(f"cos {tuple(cos.shape)} {cos.dtype} and sin {tuple(sin.shape)} "
                             f"{sin.dtype} differ")
        if cos.shape[1] != d:
            raise ValueError(f"RoPE tables have {cos.shape[1]} columns, head dim is {d}")
        if d % 16 != 0:
            raise NotImplementedError(f"fused RoPE needs a head dim that is a multiple of 16, "
                                      f"got {d}")
        # The kernels read the tables with 16-byte vector loads.
        esz = cos.element_size()
        if (cos.stride(1) != 1 or sin.stride(1) != 1 or cos.stride(0) != sin.stride(0)
                or (cos.stride(0) * esz) % 16 or cos.data_ptr() % 16 or sin.data_ptr() % 16):
            cos, sin = cos.contiguous(), sin.contiguous()
            if cos.data_ptr() % 16:
                cos = cos.clone()
            if sin.data_ptr() % 16:
                sin = sin.clone()
        self.cos, self.sin = cos, sin
        self.pos = None
        start = 0
        if isinstance(start_pos, torch.Tensor):
            if start_pos.dim() != 1 or start_pos.shape[0] != b:
                raise ValueError(f"start_pos tensor must have shape ({b},), got "
                                 f"{tuple(start_pos.shape)}")
            if start_pos.dtype.is_floating_point or start_pos.dtype == torch.bool:
                raise ValueError(f"start_pos must be an integer tensor, got {start_pos.dtype}")
            self.pos = start_pos.to(device=dev, dtype=torch.int32).contiguous()
        else:
            start = int(start_pos)
        self.args = (cos.data_ptr(), sin.data_ptr(), _lib.dtype_code(cos.dtype), cos.shape[0],
                     cos.stride(0), None if self.pos is None else self.pos.data_ptr(), start)


def rope_args(cos, sin, start_pos, b: int, d: int, dev: torch.device) -> RopeArgs | None:
    """None when no table is given (no rotation), else the validated arguments."""
    if cos is None and sin is None:
        return None
    return RopeArgs(cos, sin, start_pos, b, d, dev)


def rope_rotate(x: torch.Tensor, rope: RopeArgs, inverse: bool = False,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """``sk_rope_rotate``: x (B, H, S, D) rotated by its RoPE angles, token t of
    row b at ``start_pos(+[b]) + t``, or by their negatives (``inverse``, the
    adjoint: the reference's ``rope_bwd``, ``src/stackkernels/_core/positional/
    rope.py:137-222``, ``torch/embedding.py:46-66``).  ``out`` may be ``x``."""
    b, h, s, d = x.shape
    if x.stride(-1) != 1 or x.data_ptr() % 16 or any(st % (16 // x.element_size())
                                                     for st in x.stride()[:3]):
        x = x.contiguous()
        if x.data_ptr() % 16:
            x = x.clone()
    if out is None:
        out = torch.empty_like(x, memory_format=torch.contiguous_format)
    lib = _lib.load()
    with torch.cuda.device(x.device):
        rc = lib.sk_rope_rotate(_lib.dtype_code(x.dtype), x.data_ptr(), out.data_ptr(), b, h, s,
                                d, _lib.strides3(x), _lib.strides3(out), *rope.args,
                                int(bool(inverse)), _lib.stream_ptr(x.device))
    _lib.check(rc, "rope_rotate")
    return out


__all__ = ["RopeArgs", "rope_args", "rope_rotate"]
