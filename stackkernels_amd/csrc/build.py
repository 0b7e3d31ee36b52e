"""Build libsk_attn.so for gfx950 with hipcc, in place.

Links against torch's own HIP runtime (``torch/lib/libamdhip64.so``, same
SONAME as ROCm's) with an rpath to it, so a process that has imported torch
maps exactly one HIP runtime and the library's launches run on torch's
streams.  Usage: ``python -m stackkernels_amd.csrc.build`` or ``build()``.
"""

from __future__ import annotations

import hashlib
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
INCLUDE = os.path.join(REPO, "include")
SOURCES = ["sk_abi.hip", "sk_fwd.hip", "sk_decode.hip", "sk_fp32.hip", "sk_bwd.hip", "sk_cache.hip",
           "sk_rotate.hip"]
LIB_NAME = "libsk_attn.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast",
    "-fvisibility=hidden",
    # packed fp32 arithmetic stays off: only scalar fp32 VALU ops are emitted.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def _torch_lib_dir() -> str:
    import importlib.util

    spec = importlib.util.find_spec("torch")
    if spec is None or spec.origin is None:
        raise RuntimeError("torch is not importable; it provides the HIP runtime to link against")
    return os.path.join(os.path.dirname(spec.origin), "lib")


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


# Kernels that stream tiles with buffer_load ... lds and count their own loads
# with s_waitcnt vmcnt.  A register spill would add scratch loads to that
# count, so the waits would no longer cover the tiles: such a build is refused.
RING_KERNELS = ("fwd_mfma_kernel", "bwd_dkv_kernel", "bwd_dq_kernel", "bwd_dq_ds_kernel")


def _check_no_scratch(src: str, remarks: str) -> None:
    name = None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name and int(m.group(1)) > 0 and any(k in name for k in RING_KERNELS):
            raise RuntimeError(f"{src}: kernel {name} spills {m.group(1)} bytes/lane to scratch; "
                               "its manual vmcnt waits require a spill-free build")


def lib_path() -> str:
    return os.path.join(HERE, LIB_NAME)


def build(verbose: bool = False, jobs: int = 5, defines: tuple = (), out: str | None = None) -> str:
    """Compile every HIP source for gfx950 and link ``libsk_attn.so`` next to them.

    ``defines`` (``NAME=VALUE`` strings) and ``out`` build a candidate library of
    a tile study elsewhere (e.g. ``SK_FWD_SYNC_TILES=1``, ``SK_FWD_D128_TILE=32,4,2``);
    load one with ``SK_ATTN_LIB=<path>``."""
    hipcc = _hipcc()
    tag = hashlib.sha1(" ".join(defines).encode()).hexdigest()[:10] if defines else ""
    out_dir = os.path.join(HERE, "_build" + (f"_{tag}" if tag else ""))
    os.makedirs(out_dir, exist_ok=True)
    objs = []

    def compile_one(src: str) -> str:
        obj = os.path.join(out_dir, src.replace(".hip", ".o"))
        cmd = [hipcc, *HIPCC_FLAGS, *(f"-D{d}" for d in defines), f"-I{INCLUDE}", f"-I{HERE}", "-c",
               os.path.join(HERE, src), "-o", obj, "-Rpass-analysis=kernel-resource-usage"]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{res.stderr}")
        _check_no_scratch(src, res.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tlib = _torch_lib_dir()
    target = out or lib_path()
    tmp = target + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
           f"-L{tlib}", "-lamdhip64", f"-Wl,-rpath,{tlib}", "-Wl,--no-undefined"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, target)
    return target


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="build libsk_attn.so for gfx950")
    ap.add_argument("-v", action="store_true", help="print the compile commands")
    ap.add_argument("-D", dest="defines", action="append", default=[],
                    help="NAME=VALUE macro for a tile-study candidate build (needs -o)")
    ap.add_argument("-o", dest="out", default=None, help="output path (default: in place)")
    a = ap.parse_args()
    if a.defines and not a.out:
        ap.error("a candidate build (-D) needs -o: the in-place library is the table's")
    print(build(verbose=a.v, defines=tuple(a.defines), out=a.out))
