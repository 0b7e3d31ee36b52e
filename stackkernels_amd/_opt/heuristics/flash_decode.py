"""Split-KV decode configuration: the reference's ``heuristic``
(``src/stackkernels/_opt/heuristics/flash_decode.py:9-12``) answered by the
gfx950 table.  ``kv_len`` is the key count (the reference's seed reads q's
length 1 from ``shape[2]`` instead and always returns one split)."""

from __future__ import annotations

from typing import Any

from stackkernels_amd._opt.hardware import DeviceProfile
from stackkernels_amd._opt.pick import pick


def heuristic(shape: Any = None, profile: DeviceProfile | None = None, dtype: str = "float16",
              **kwargs: Any) -> dict[str, Any]:
    """Split count, tile and kernel for ``flash_decode`` at q's ``shape`` (B, H_q, 1, D)."""
    return dict(pick("flash_decode", shape, dtype=dtype, profile=profile, **kwargs))


__all__ = ["heuristic"]
