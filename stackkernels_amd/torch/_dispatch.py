"""Kernel-or-reference choice (reference ``src/stackkernels/torch/_dispatch.py:8-27``).

* ``reference``        -> the PyTorch reference path, always;
* ``triton`` / ``hip`` -> the HIP kernels, always (a CPU tensor then raises:
  there is no CPU kernel and no silent fallback);
* ``auto``             -> the HIP kernels for ROCm device tensors, the
  reference path for CPU tensors.
"""

import torch

from stackkernels_amd._options import KERNEL_BACKENDS, get_backend


def should_use_hip(tensor: torch.Tensor) -> bool:
    """True when the HIP kernels handle ``tensor``."""
    backend = get_backend()
    if backend == "reference":
        return False
    if backend in KERNEL_BACKENDS:
        return True
    return bool(tensor.is_cuda)


# The reference's name for the same decision; existing callers use it.
should_use_triton = should_use_hip

__all__ = ["should_use_hip", "should_use_triton"]
