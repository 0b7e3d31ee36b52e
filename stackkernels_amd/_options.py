"""Process-wide backend switch: ``auto`` | ``triton`` | ``hip`` | ``reference``.

Mirrors the reference's option object (``src/stackkernels/_options.py:10-55``):
the value comes from ``STACKKERNELS_BACKEND`` (default ``auto``), is
normalised to lower case, and an unknown name raises
``ValueError("Invalid backend ...")``.

Meaning on this build:

* ``auto``      -- ROCm device tensors run the gfx950 HIP kernels; CPU tensors
  run the PyTorch reference path (the reference's own CPU behaviour).
* ``triton``    -- kept so existing callers keep working; it forces the kernel
  path, which here is the HIP kernels (there is no Triton in this build).
* ``hip``       -- the same as ``triton``, under its real name.
* ``reference`` -- always the PyTorch reference path.

This module must never import torch.
"""

import os

VALID_BACKENDS: tuple[str, ...] = ("auto", "triton", "hip", "reference")
KERNEL_BACKENDS: frozenset[str] = frozenset({"triton", "hip"})


class Options:
    """Global configuration holder; ``backend`` is validated on every write."""

    def __init__(self, backend: str | None = None) -> None:
        self._backend = "auto"
        self.backend = os.environ.get("STACKKERNELS_BACKEND", "auto") if backend is None else backend

    @property
    def backend(self) -> str:
        return self._backend

    @backend.setter
    def backend(self, value: str) -> None:
        name = str(value).strip().lower()
        if name not in VALID_BACKENDS:
            raise ValueError(
                f"Invalid backend '{value}'. Must be one of: {', '.join(VALID_BACKENDS)}"
            )
        self._backend = name

    def __repr__(self) -> str:
        return f"Options(backend='{self._backend}')"


_GLOBAL = Options()


def get_backend() -> str:
    """Return the active backend name."""
    return _GLOBAL.backend


def set_backend(backend: str) -> None:
    """Select the backend; raises ``ValueError`` for an unknown name."""
    _GLOBAL.backend = backend


def options(backend: str | None = None) -> Options:
    """Return the global options object, setting the backend first if given."""
    if backend is not None:
        set_backend(backend)
    return _GLOBAL


__all__ = ["Options", "VALID_BACKENDS", "KERNEL_BACKENDS", "get_backend", "set_backend", "options"]
