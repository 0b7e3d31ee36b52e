"""bench.py's host logic on the CPU: algorithmic work per step, the recorded
HBM-traffic figures and their source check, and the one-GPU contract."""

import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


@pytest.mark.parametrize("sq,sk", [(1, 1), (7, 7), (5, 13), (13, 5), (64, 256), (300, 300)])
def test_causal_pairs_matches_brute_force(sq, sk):
    # bottom-right mask: key j visible to query i iff j <= i + (sk - sq)
    brute = sum(1 for i in range(sq) for j in range(sk) if j <= i + sk - sq)
    assert bench.causal_pairs(sq, sk, True) == brute
    assert bench.causal_pairs(sq, sk, False) == sq * sk


def test_headline_work_units():
    c2 = bench.WORKLOADS["fwd"]
    flop, unit = bench.work_units(c2)
    assert unit == "TFLOP/s" and flop == 549_890_031_616  # 4*D*pairs*B*H at C2
    c3 = bench.WORKLOADS["fwdbwd"]
    pairs = 2048 * 6144 + 2048 * 2049 // 2
    assert bench.work_units(c3) == (float(14 * 128 * pairs * 2 * 32), "TFLOP/s")
    # decode: K and V once per KV head, q read and O written
    c5 = bench.WORKLOADS["decode_mqa"]
    assert bench.work_units(c5) == (float(2 * 8 * 1 * 131072 * 128 * 2 + 2 * 8 * 64 * 128 * 2),
                                    "GB/s")


def test_recorded_traffic_follows_the_kernel_sources(monkeypatch):
    monkeypatch.setattr(bench, "TRAFFIC_SOURCES_SHA256", bench.kernel_sources_digest())
    val, note = bench.recorded_traffic("fwd")
    assert val == bench.HBM_TRAFFIC_BYTES["fwd"] and "sha256" in note
    assert bench.recorded_traffic("no_such_workload")[0] is None
    # any other digest: the figures are stale and the line must not report them
    monkeypatch.setattr(bench, "TRAFFIC_SOURCES_SHA256", "0" * 64)
    val, note = bench.recorded_traffic("fwd")
    assert val is None and "re-run" in note


def test_kernel_sources_digest_covers_every_kernel_source(tmp_path, monkeypatch):
    d0 = bench.kernel_sources_digest()
    csrc = tmp_path / "stackkernels_amd" / "csrc"
    csrc.mkdir(parents=True)
    src = os.path.join(ROOT, "stackkernels_amd", "csrc")
    for name in os.listdir(src):
        if name.endswith((".hip", ".h")):
            (csrc / name).write_bytes(open(os.path.join(src, name), "rb").read())
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    assert bench.kernel_sources_digest() == d0
    # comments, blank lines and indentation do not count ...
    src = (csrc / "sk_bwd.hip").read_bytes()
    (csrc / "sk_bwd.hip").write_bytes(b"// a note\n/* and\n another */\n\n" + src.replace(b"\n", b"\n  "))
    assert bench.kernel_sources_digest() == d0
    # ... code does
    (csrc / "sk_bwd.hip").write_bytes(src + b"\nstatic int sk_digest_probe;\n")
    assert bench.kernel_sources_digest() != d0


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2 and "one GPU" in r.stderr
