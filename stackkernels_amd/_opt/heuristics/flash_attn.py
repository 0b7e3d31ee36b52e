"""Forward attention configuration: the reference's ``heuristic``
(``src/stackkernels/_opt/heuristics/flash_attn.py:9-12``) answered by the gfx950
table of the compiled forward kernel."""

from __future__ import annotations

from typing import Any

from stackkernels_amd._opt.hardware import DeviceProfile
from stackkernels_amd._opt.pick import pick


def heuristic(shape: Any = None, profile: DeviceProfile | None = None, dtype: str = "float16",
              **kwargs: Any) -> dict[str, Any]:
    """Tiles, wavefronts and ring depth of the forward at q's ``shape`` (B, H_q, S_q, D)."""
    return dict(pick("flash_attn", shape, dtype=dtype, profile=profile, **kwargs))


__all__ = ["heuristic"]
