"""Every tile-study build that the counter tables use still compiles.

The kernel sources read tile-study macros (``python -m stackkernels_amd.csrc.build
-D NAME=VALUE -o <path>``) that build the rejected candidates of the tile and
occupancy table; the table's own build never compiles those branches.  Each
case runs the device front end (``hipcc --cuda-device-only -fsyntax-only``:
template instantiation and static assertions included, no code generation) on
every source that reads the macro, so a change to a kernel cannot leave a
documented candidate unbuildable.  Candidates whose code has left the sources
(they build at the commit their counter rows name) are not listed.  Skipped
where hipcc is absent.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                    "stackkernels_amd", "csrc")
INCLUDE = os.path.join(os.path.dirname(CSRC), os.pardir, "include")

STUDY_BUILDS = [
    "SK_FWD_SYNC_TILES=1",
    "SK_FWD_D128_TILE=64,8,1,4",
    "SK_FWD_D128_TILE=64,4,2,2",
    "SK_FWD_D128_TILE=32,4,2,4",
    "SK_FWD_D128_TILE=32,8,1,4",
    "SK_FWD_D64_TILE=64,4,2,4",
    "SK_FWD_D64_TILE=64,8,1,4",
    "SK_FWD_LONG_KEYS=0",
    "SK_FWD_PAIR_ROUNDS=4",
    "SK_DEC_BN_W4=32",
    "SK_DEC_BN_W4=128",
    "SK_BWD_DKV_STAGES=4",
    "SK_BWD_DKV_STAGES_D64=4",
    "SK_BWD_DKV_DO_D256=256",
    "SK_BWD_DQ_TILE=32,2,0",
    "SK_BWD_DQ_TILE=64,2,0",
    "SK_BWD_DQ_TILE_D256=32,1,2",
    "SK_BWD_DQDS_TILE=2,6,1",
    "SK_BWD_DQDS_TILE=1,5,2",
    "SK_BWD_FIVE_GEMM=0",
    "SK_BWD_DS_NT=0",
    "SK_F32_MFMA=0",
]


def _hipcc():
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    return None


def _sources_reading(name: str) -> list[str]:
    """The .hip files that read macro `name`, directly or through a header."""
    files = sorted(os.listdir(CSRC))
    hips = [f for f in files if f.endswith(".hip")]
    out = set()
    for f in files:
        if not f.endswith((".hip", ".h")):
            continue
        with open(os.path.join(CSRC, f)) as fh:
            if name not in fh.read():
                continue
        if f.endswith(".hip"):
            out.add(f)
        else:
            for h in hips:
                with open(os.path.join(CSRC, h)) as fh:
                    if re.search(r'#include\s+"%s"' % re.escape(f), fh.read()):
                        out.add(h)
    return sorted(out)


def test_every_listed_macro_is_read_by_the_sources():
    for d in STUDY_BUILDS:
        name = d.split("=")[0]
        assert _sources_reading(name), f"no kernel source reads {name}"


@pytest.mark.parametrize("define", STUDY_BUILDS)
def test_study_build_compiles(define):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    for src in _sources_reading(define.split("=")[0]):
        cmd = [hipcc, "--offload-arch=gfx950", "-std=c++17", f"-I{INCLUDE}", f"-I{CSRC}",
               f"-D{define}", "--cuda-device-only", "-fsyntax-only", os.path.join(CSRC, src)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        errors = [ln for ln in res.stderr.splitlines() if " error" in ln]
        assert res.returncode == 0 and not errors, f"{src} with -D{define}:\n" + "\n".join(errors[:20])
