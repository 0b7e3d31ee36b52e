"""Argument preparation shared by the launchers."""

from __future__ import annotations

import math

import torch

from stackkernels_amd._core.attention import _lib
from stackkernels_amd._core.attention.layout import MAX_HEAD_DIM

_SUPPORTED = (torch.float32, torch.float16, torch.bfloat16)


def check_device(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device with one supported dtype; return the device."""
    dev = tensors[0].device
    dt = tensors[0].dtype
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                "the HIP attention kernels need ROCm device tensors; got a tensor on "
                f"{t.device} (use backend 'auto' or 'reference' for CPU tensors)"
            )
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} and {t.device}")
        if t.dtype != dt:
            raise ValueError(f"dtype mismatch: {dt} and {t.dtype}")
    if dt not in _SUPPORTED:
        raise NotImplementedError(f"dtype {dt} has no HIP kernel (supported: {_SUPPORTED})")
    return dev


def default_scale(d: int, sm_scale: float | None) -> float:
    """``1/sqrt(D)`` unless given (reference ``torch/attention.py:33-36``)."""
    return 1.0 / math.sqrt(d) if sm_scale is None else float(sm_scale)


def kernel_head_dim(d: int) -> int:
    """Head dim handed to the library: ``d`` rounded up to a multiple of 8."""
    if d > MAX_HEAD_DIM:
        raise NotImplementedError(f"head dim {d} > {MAX_HEAD_DIM} has no HIP kernel")
    return (d + 7) // 8 * 8


def pad_head(t: torch.Tensor, dk: int) -> torch.Tensor:
    """Zero-pad the last dim to ``dk`` (zeros leave q.k and the used O columns unchanged)."""
    d = t.shape[-1]
    if d == dk:
        return t
    return torch.nn.functional.pad(t, (0, dk - d))


def kernel_operand(t: torch.Tensor) -> torch.Tensor:
    """``t`` if the library can read it in place (unit D stride, 16-byte rows and base),
    else a contiguous copy."""
    unit = 4 if t.dtype == torch.float32 else 8
    ok = (
        t.stride(-1) == 1 or t.shape[-1] == 1
    ) and t.data_ptr() % 16 == 0 and all(s % unit == 0 for s in t.stride()[:3])
    if ok:
        return t
    c = t.contiguous()
    if c.data_ptr() % 16 != 0:
        c = c.clone()
    return c


def stream_of(device: torch.device) -> int:
    return _lib.stream_ptr(device)
