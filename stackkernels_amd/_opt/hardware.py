"""Device profiles, with AMD Instinct (gfx9) GPUs described correctly.

Same dataclass, fields, ``fingerprint()`` and resolution pipeline as the
reference's ``src/stackkernels/_opt/hardware.py:9-282``.  What changes:

* On ROCm, ``torch.cuda.get_device_capability`` reports the gfx major/minor
  (9, 5) for gfx950; the reference's fall-back table is keyed by NVIDIA
  compute capability and has no such entry (and (9, 0), gfx90a, collides with
  H100).  Here ROCm devices resolve through their architecture name
  (``gcnArchName``), in ``_ARCH_TABLE``.
* A ROCm profile carries ``arch`` (e.g. ``gfx950``), a 64-lane wavefront,
  CU counts as ``sm_count``, LDS as shared memory, and a fingerprint keyed by
  the architecture name: ``amd-instinct-mi355x_gfx950_256cu_<MiB>mb``.
* NVIDIA and CPU profiles behave as in the reference.
"""

from __future__ import annotations

import os
import platform
from dataclasses import dataclass
from typing import Any


@dataclass(frozen=True)
class DeviceProfile:
    """Device specifications used to guide optimization decisions."""

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
    arch: str = ""  # ROCm architecture name (gfx950 ...); "" on NVIDIA / CPU

    def fingerprint(self) -> str:
        """Return a stable normalized fingerprint string for cache keys."""
        if self.compute_capability == (0, 0):
            return "cpu"
        clean_name = self.name.lower().replace(" ", "-").replace("/", "-")
        mem_mb = self.total_memory_bytes // (1024 * 1024)
        if self.arch:
            return f"{clean_name}_{self.arch}_{self.sm_count}cu_{mem_mb}mb"
        maj, min_ = self.compute_capability
        return f"{clean_name}_sm{maj}{min_}_{self.sm_count}sm_{mem_mb}mb"

    @property
    def is_cuda(self) -> bool:
        """True for any GPU profile (torch's "cuda" device type, ROCm included)."""
        return self.compute_capability != (0, 0)

    @property
    def is_rocm(self) -> bool:
        return bool(self.arch)


@dataclass(frozen=True)
class HardwareInfo:
    """Legacy hardware info preserved for backwards compatibility."""

    name: str = "cpu"
    arch: str = "cpu"
    sm_count: int = 0
    shared_memory_per_sm: int = 0
    peak_bandwidth_gbps: float = 0.0
    peak_flops_fp16: float = 0.0
    has_gpu: bool = False


# AMD Instinct specifications by architecture name.  Per CU: 4 SIMDs, each with
# 512 32-bit registers per lane (architected + accumulation VGPRs) and up to 8
# wavefronts of 64 lanes; LDS is the shared memory.  Peaks are the published
# dense (non-sparse) figures.
_ARCH_TABLE: dict[str, dict[str, Any]] = {
    "gfx950": {
        "name": "AMD Instinct MI355X",
        "compute_capability": (9, 5),
        "sm_count": 256,
        "warp_size": 64,
        "max_regs_per_sm": 4 * 512 * 64,
        "max_regs_per_thread": 512,
        "max_threads_per_sm": 2048,
        "max_smem_per_block": 160 * 1024,
        "max_smem_per_sm": 160 * 1024,
        "l2_bytes": 8 * 4 * 1024 * 1024,  # 4 MiB per XCD, 8 XCDs (plus 256 MiB Infinity Cache)
        "total_memory_bytes": 288 * 1000**3,
        "peak_bandwidth_gbps": 8000.0,
        "peak_tflops": {"fp16": 2500.0, "bf16": 2500.0, "fp8": 5000.0, "fp32": 157.3,
                        "fp64": 78.6},
        "has_cp_async": True,  # buffer_load ... lds: global -> LDS without registers
        "has_bf16": True,
    },
    "gfx942": {
        "name": "AMD Instinct MI300X",
        "compute_capability": (9, 4),
        "sm_count": 304,
        "warp_size": 64,
        "max_regs_per_sm": 4 * 512 * 64,
        "max_regs_per_thread": 512,
        "max_threads_per_sm": 2048,
        "max_smem_per_block": 64 * 1024,
        "max_smem_per_sm": 64 * 1024,
        "l2_bytes": 8 * 4 * 1024 * 1024,
        "total_memory_bytes": 192 * 1000**3,
        "peak_bandwidth_gbps": 5300.0,
        "peak_tflops": {"fp16": 1307.4, "bf16": 1307.4, "fp8": 2614.9, "fp32": 163.4},
        "has_cp_async": True,
        "has_bf16": True,
    },
}

# The reference's table keyed by NVIDIA compute capability, kept for NVIDIA
# devices (src/stackkernels/_opt/hardware.py:57-109 lists the same three
# generations; figures are the published ones).
_FALLBACK_TABLE: dict[tuple[int, int], dict[str, Any]] = {
    (7, 5): {"name": "NVIDIA Turing GPU", "sm_count": 40, "warp_size": 32,
             "max_regs_per_sm": 65536, "max_regs_per_thread": 255, "max_threads_per_sm": 1024,
             "max_smem_per_block": 49152, "max_smem_per_sm": 65536, "l2_bytes": 4 * 1024**2,
             "total_memory_bytes": 16 * 1024**3, "peak_bandwidth_gbps": 320.0,
             "peak_tflops": {"fp16": 65.0, "fp32": 8.1}, "has_cp_async": False, "has_bf16": False},
    (8, 0): {"name": "NVIDIA A100-SXM4", "sm_count": 108, "warp_size": 32,
             "max_regs_per_sm": 65536, "max_regs_per_thread": 255, "max_threads_per_sm": 2048,
             "max_smem_per_block": 167936, "max_smem_per_sm": 167936, "l2_bytes": 40 * 1024**2,
             "total_memory_bytes": 40 * 1024**3, "peak_bandwidth_gbps": 1555.0,
             "peak_tflops": {"fp16": 312.0, "bf16": 312.0, "fp32": 19.5}, "has_cp_async": True,
             "has_bf16": True},
    (9, 0): {"name": "NVIDIA H100-SXM5", "sm_count": 132, "warp_size": 32,
             "max_regs_per_sm": 65536, "max_regs_per_thread": 255, "max_threads_per_sm": 2048,
             "max_smem_per_block": 232448, "max_smem_per_sm": 232448, "l2_bytes": 50 * 1024**2,
             "total_memory_bytes": 80 * 1024**3, "peak_bandwidth_gbps": 3350.0,
             "peak_tflops": {"fp16": 989.0, "bf16": 989.0, "fp32": 67.0}, "has_cp_async": True,
             "has_bf16": True},
}

_DEVICE_PROFILE_CACHE: dict[Any, DeviceProfile] = {}


def arch_profile(arch: str = "gfx950") -> DeviceProfile:
    """The tabulated profile of an AMD architecture (no device needed)."""
    spec = _ARCH_TABLE[arch]
    return DeviceProfile(arch=arch, **spec)


def mi355x_profile() -> DeviceProfile:
    """The MI355X (gfx950) profile the attention kernels are built for."""
    return arch_profile("gfx950")


def is_gpu_available() -> bool:
    """Check dynamically if a GPU device (ROCm or CUDA) is available."""
    try:
        import torch

        return bool(torch.cuda.is_available() and torch.cuda.device_count() > 0)
    except Exception:
        return False


def get_gpu_arch(device_id: int = 0) -> str:
    """Active GPU architecture: 'gfx950' etc. on ROCm, 'sm_80' etc. on NVIDIA, or 'cpu'."""
    env_arch = os.environ.get("STACKKERNELS_GPU_ARCH")
    if env_arch:
        return env_arch.lower().strip()
    if not is_gpu_available():
        return "cpu"
    try:
        import torch

        props = torch.cuda.get_device_properties(device_id)
        gcn = getattr(props, "gcnArchName", "")
        if gcn:
            return gcn.split(":")[0]
        major, minor = torch.cuda.get_device_capability(device_id)
        return f"sm_{major}{minor}"
    except Exception:
        return "cpu"


def _build_cpu_profile() -> DeviceProfile:
    """Build a clearly marked CPU profile."""
    cpu_cores = os.cpu_count() or 1
    cpu_name = platform.processor() or platform.machine() or "Host CPU"
    return DeviceProfile(
        name=f"CPU ({cpu_name})", compute_capability=(0, 0), sm_count=cpu_cores, warp_size=32,
        max_regs_per_sm=0, max_regs_per_thread=0, max_threads_per_sm=1, max_smem_per_block=0,
        max_smem_per_sm=0, l2_bytes=0, total_memory_bytes=0, peak_bandwidth_gbps=None,
        peak_tflops=None, has_cp_async=False, has_bf16=False,
    )


def profile_from_properties(props: Any, capability: tuple[int, int]) -> DeviceProfile:
    """DeviceProfile from torch device properties (and the reported capability):
    runtime values first, then the architecture (ROCm) or capability (NVIDIA)
    table, then conservative defaults."""
    major, minor = capability
    arch = (getattr(props, "gcnArchName", "") or "").split(":")[0]
    if arch:
        table = _ARCH_TABLE.get(arch, {})
        default_warp, default_regs_th = 64, 512
    else:
        table = _FALLBACK_TABLE.get((major, minor), {})
        default_warp, default_regs_th = 32, 255
    # A known AMD architecture takes its product name, register file and L2
    # from the table: the runtime reports a generic marketing name ("AMD Radeon
    # Graphics" on MI355X boxes), the registers of half a CU, and the L2 of one
    # of the eight XCDs.
    known = bool(arch) and bool(table)
    name = (table["name"] if known else "") or getattr(props, "name", "") or \
        table.get("name", f"GPU {arch or f'sm_{major}{minor}'}")
    smem_block = getattr(props, "shared_memory_per_block", 0)
    regs = table["max_regs_per_sm"] if known else getattr(props, "regs_per_multiprocessor", 0)
    l2 = table["l2_bytes"] if known else getattr(props, "L2_cache_size", 0)
    return DeviceProfile(
        name=name,
        compute_capability=(major, minor),
        sm_count=getattr(props, "multi_processor_count", 0) or table.get("sm_count", 32),
        warp_size=getattr(props, "warp_size", 0) or table.get("warp_size", default_warp),
        max_regs_per_sm=regs or table.get("max_regs_per_sm", 65536),
        max_regs_per_thread=table.get("max_regs_per_thread", default_regs_th),
        max_threads_per_sm=getattr(props, "max_threads_per_multi_processor", 0)
        or table.get("max_threads_per_sm", 1024),
        max_smem_per_block=smem_block or table.get("max_smem_per_block", 49152),
        max_smem_per_sm=table.get("max_smem_per_sm", smem_block or 65536),
        l2_bytes=l2 or table.get("l2_bytes", 4 * 1024**2),
        total_memory_bytes=getattr(props, "total_memory", 0)
        or table.get("total_memory_bytes", 8 * 1024**3),
        peak_bandwidth_gbps=table.get("peak_bandwidth_gbps"),
        peak_tflops=table.get("peak_tflops"),
        has_cp_async=table.get("has_cp_async", bool(arch) or major >= 8),
        has_bf16=table.get("has_bf16", bool(arch) or (major, minor) >= (8, 0)),
        arch=arch,
    )


def get_device_profile(device: Any = None) -> DeviceProfile:
    """DeviceProfile of a device (default: the current one); the CPU profile
    when there is no GPU or the device is the CPU."""
    cache_key = str(device) if device is not None else "default"
    if cache_key in _DEVICE_PROFILE_CACHE:
        return _DEVICE_PROFILE_CACHE[cache_key]
    env_arch = os.environ.get("STACKKERNELS_GPU_ARCH", "").lower().strip()
    if env_arch == "cpu" or not is_gpu_available():
        profile = _build_cpu_profile()
        _DEVICE_PROFILE_CACHE[cache_key] = profile
        return profile
    try:
        import torch

        if isinstance(device, int):
            idx = device
        elif isinstance(device, torch.device):
            if device.type != "cuda":
                profile = _build_cpu_profile()
                _DEVICE_PROFILE_CACHE[cache_key] = profile
                return profile
            idx = device.index or 0
        elif isinstance(device, str):
            if device == "cpu":
                profile = _build_cpu_profile()
                _DEVICE_PROFILE_CACHE[cache_key] = profile
                return profile
            idx = int(device.replace("cuda:", "").replace("cuda", "0") or 0)
        else:
            idx = torch.cuda.current_device()
        profile = profile_from_properties(torch.cuda.get_device_properties(idx),
                                          torch.cuda.get_device_capability(idx))
    except Exception:
        profile = _build_cpu_profile()
    _DEVICE_PROFILE_CACHE[cache_key] = profile
    return profile


def get_hardware_info(device_id: int = 0, arch: str | None = None) -> HardwareInfo:
    """Legacy HardwareInfo function for backwards compatibility."""
    profile = get_device_profile(device_id)
    if not profile.is_cuda:
        return HardwareInfo(name=profile.name, arch="cpu", sm_count=profile.sm_count,
                            has_gpu=False)
    maj, min_ = profile.compute_capability
    return HardwareInfo(
        name=profile.name,
        arch=profile.arch or f"sm_{maj}{min_}",
        sm_count=profile.sm_count,
        shared_memory_per_sm=profile.max_smem_per_sm,
        peak_bandwidth_gbps=profile.peak_bandwidth_gbps or 0.0,
        peak_flops_fp16=(profile.peak_tflops or {}).get("fp16", 0.0),
        has_gpu=True,
    )


__all__ = [
    "DeviceProfile",
    "HardwareInfo",
    "arch_profile",
    "mi355x_profile",
    "profile_from_properties",
    "get_device_profile",
    "get_hardware_info",
    "get_gpu_arch",
    "is_gpu_available",
]
