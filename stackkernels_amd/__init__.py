"""MI355X-native StackKernels attention path.

The package root imports neither torch nor anything that loads the HIP
library, as the reference's root does (``src/stackkernels/__init__.py:1-36``):
``torch`` and the other subpackages resolve lazily on first attribute access.
"""

import importlib
from typing import Any

from stackkernels_amd._options import get_backend, options, set_backend

__version__ = "0.1.0"

_LAZY: dict[str, str] = {
    "torch": "stackkernels_amd.torch",
    "_core": "stackkernels_amd._core",
    "_reference": "stackkernels_amd._reference",
    "_opt": "stackkernels_amd._opt",
}

__all__ = ["__version__", "options", "get_backend", "set_backend", *_LAZY]


def __getattr__(name: str) -> Any:
    if name in _LAZY:
        return importlib.import_module(_LAZY[name])
    raise AttributeError(f"module '{__name__}' has no attribute '{name}'")


def __dir__() -> list[str]:
    return sorted(list(globals()) + list(_LAZY))
