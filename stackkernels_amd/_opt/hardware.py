"""Device profile of the GPU the attention kernels run on.

Interface kept from the reference (``src/stackkernels/_opt/hardware.py``):
the frozen ``DeviceProfile`` record with its field names (``:9-54``, which
``tests/test_opt/test_device_profile.py`` pins), its ``fingerprint()`` format
(``<name>_sm<major><minor>_<n>sm_<MiB>mb``, or ``cpu`` for the host) and
``get_device_profile(device=None)``.

Everything else is this build's.  The kernels are compiled for gfx950 only, so
the profile of a ROCm device comes from its architecture name
(``gcnArchName``), never from the (major, minor) pair torch reports, which on
ROCm is the gfx version ((9, 5) for gfx950) and means nothing to an NVIDIA
capability table.  A gfx950 device gets the tabulated MI355X figures, with the
CU count and memory the runtime reports (a partitioned GPU shows fewer CUs);
its fingerprint carries the architecture:
``amd-instinct-mi355x_gfx950_256cu_<MiB>mb``.  Any other GPU gets a profile
built from the runtime's properties alone, with no peak figures.
"""

from __future__ import annotations

import dataclasses
import os
from typing import Any


@dataclasses.dataclass(frozen=True)
class DeviceProfile:
    """What the configuration logic knows about a device.  Field names follow
    the reference's record: ``sm_count`` counts compute units, ``warp_size`` is
    the wavefront width and shared memory is LDS on AMD GPUs."""

    name: str
    compute_capability: tuple[int, int]
    sm_count: int
    warp_size: int
    max_regs_per_sm: int
    max_regs_per_thread: int
    max_threads_per_sm: int
    max_smem_per_block: int
    max_smem_per_sm: int
    l2_bytes: int
    total_memory_bytes: int
    peak_bandwidth_gbps: float | None = None
    peak_tflops: dict[str, float] | None = None
    has_cp_async: bool = False
    has_bf16: bool = False
    arch: str = ""  # ROCm architecture name, e.g. "gfx950"; "" otherwise

    @property
    def is_cuda(self) -> bool:
        """True for a GPU (torch's "cuda" device type, which ROCm devices use)."""
        return self.compute_capability != (0, 0)

    @property
    def is_rocm(self) -> bool:
        return self.arch != ""

    def fingerprint(self) -> str:
        """Cache-key string: ``cpu`` for the host; for a GPU its lower-cased
        name (spaces and slashes as dashes), its architecture and CU count
        (ROCm) or capability and SM count, and its memory in MiB."""
        if not self.is_cuda:
            return "cpu"
        slug = "".join("-" if c in " /" else c for c in self.name.lower())
        if self.arch:
            unit = f"{self.arch}_{self.sm_count}cu"
        else:
            major, minor = self.compute_capability
            unit = f"sm{major}{minor}_{self.sm_count}sm"
        return f"{slug}_{unit}_{self.total_memory_bytes >> 20}mb"


# MI355X (gfx950), published figures.  A CU has 4 SIMDs; each SIMD lane has
# 512 32-bit registers (architected + accumulation), and a CU runs at most
# 32 wavefronts of 64 lanes.  LDS is 160 KiB per CU, all of it available to
# one workgroup.  L2 is 4 MiB on each of the 8 XCDs (the 256 MiB Infinity
# Cache behind it is not counted).  Peaks are dense (no sparsity):
# 2.5 PFLOP/s bf16/fp16 MFMA, 8 TB/s HBM3E.  buffer_load ... lds moves global
# data to LDS without registers, the role of cp.async in the reference's record.
MI355X = DeviceProfile(
    name="AMD Instinct MI355X",
    compute_capability=(9, 5),
    sm_count=256,
    warp_size=64,
    max_regs_per_sm=4 * 64 * 512,
    max_regs_per_thread=512,
    max_threads_per_sm=32 * 64,
    max_smem_per_block=160 << 10,
    max_smem_per_sm=160 << 10,
    l2_bytes=8 * (4 << 20),
    total_memory_bytes=288 * 10**9,
    peak_bandwidth_gbps=8000.0,
    peak_tflops={"bf16": 2500.0, "fp16": 2500.0, "fp8": 5000.0, "fp32": 157.3, "fp64": 78.6},
    has_cp_async=True,
    has_bf16=True,
    arch="gfx950",
)

_BY_ARCH = {"gfx950": MI355X}

_PROFILES: dict[Any, DeviceProfile] = {}


def arch_profile(arch: str = "gfx950") -> DeviceProfile:
    """The tabulated profile of a ROCm architecture (KeyError if none is)."""
    return _BY_ARCH[arch]


def mi355x_profile() -> DeviceProfile:
    """The MI355X profile the gfx950 kernels are built for."""
    return MI355X


def host_profile() -> DeviceProfile:
    """Profile of the host CPU (fingerprint ``cpu``): compute units are cores."""
    return DeviceProfile(
        name="host cpu", compute_capability=(0, 0), sm_count=os.cpu_count() or 1, warp_size=1,
        max_regs_per_sm=0, max_regs_per_thread=0, max_threads_per_sm=1, max_smem_per_block=0,
        max_smem_per_sm=0, l2_bytes=0, total_memory_bytes=0)


def is_gpu_available() -> bool:
    """True when torch sees at least one GPU."""
    try:
        import torch
    except ImportError:
        return False
    try:
        return torch.cuda.is_available() and torch.cuda.device_count() > 0
    except RuntimeError:
        return False


def _forced_cpu() -> bool:
    return os.environ.get("STACKKERNELS_GPU_ARCH", "").strip().lower() == "cpu"


def get_gpu_arch(device_id: int = 0) -> str:
    """Architecture of GPU ``device_id`` (``gfx950`` on an MI355X), or ``cpu``.
    ``STACKKERNELS_GPU_ARCH`` overrides the answer."""
    forced = os.environ.get("STACKKERNELS_GPU_ARCH", "").strip().lower()
    if forced:
        return forced
    if not is_gpu_available():
        return "cpu"
    import torch

    props = torch.cuda.get_device_properties(device_id)
    arch = (getattr(props, "gcnArchName", "") or "").split(":")[0]
    return arch or "sm_{}{}".format(*torch.cuda.get_device_capability(device_id))


def profile_from_properties(props: Any, capability: tuple[int, int]) -> DeviceProfile:
    """Profile of a GPU from torch's device properties and reported capability.

    gfx950: the MI355X record, taking the runtime's CU count and memory size
    (the runtime's name is generic and its register and L2 figures cover one
    SIMD pair and one XCD, so those come from the record).  Anything else:
    the runtime's figures, with no peaks."""
    arch = (getattr(props, "gcnArchName", "") or "").split(":")[0]
    cus = int(getattr(props, "multi_processor_count", 0) or 0)
    mem = int(getattr(props, "total_memory", 0) or 0)
    known = _BY_ARCH.get(arch)
    if known is not None:
        return dataclasses.replace(known, sm_count=cus or known.sm_count,
                                   total_memory_bytes=mem or known.total_memory_bytes)
    wave = int(getattr(props, "warp_size", 0) or 0) or (64 if arch else 32)
    lds = int(getattr(props, "shared_memory_per_block", 0) or 0)
    return DeviceProfile(
        name=getattr(props, "name", "") or f"GPU {arch or 'sm_%d%d' % tuple(capability)}",
        compute_capability=tuple(capability),
        sm_count=cus,
        warp_size=wave,
        max_regs_per_sm=int(getattr(props, "regs_per_multiprocessor", 0) or 0),
        max_regs_per_thread=512 if arch else 255,
        max_threads_per_sm=int(getattr(props, "max_threads_per_multi_processor", 0) or 0),
        max_smem_per_block=lds,
        max_smem_per_sm=lds,
        l2_bytes=int(getattr(props, "L2_cache_size", 0) or 0),
        total_memory_bytes=mem,
        has_bf16=True,
        arch=arch,
    )


def get_device_profile(device: Any = None) -> DeviceProfile:
    """Profile of ``device`` (None: the current GPU; an index, ``"cuda:N"``,
    a ``torch.device``; ``"cpu"`` or a CPU device: the host).  Without a GPU,
    or with ``STACKKERNELS_GPU_ARCH=cpu``, every device is the host.
    Profiles are cached per device index."""
    if _forced_cpu() or not is_gpu_available():
        return _PROFILES.setdefault("cpu", host_profile())
    import torch

    if device is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    elif isinstance(device, int):
        dev = torch.device("cuda", device)
    else:
        dev = torch.device(device)
    if dev.type != "cuda":
        return _PROFILES.setdefault("cpu", host_profile())
    idx = torch.cuda.current_device() if dev.index is None else dev.index
    prof = _PROFILES.get(idx)
    if prof is None:
        prof = profile_from_properties(torch.cuda.get_device_properties(idx),
                                       torch.cuda.get_device_capability(idx))
        _PROFILES[idx] = prof
    return prof


__all__ = [
    "DeviceProfile",
    "MI355X",
    "arch_profile",
    "mi355x_profile",
    "host_profile",
    "profile_from_properties",
    "get_device_profile",
    "get_gpu_arch",
    "is_gpu_available",
]
