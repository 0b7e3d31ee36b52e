"""Benchmark of the MI355X attention path (one JSON line on stdout).

Workloads (inputs synthetic, seeded, generated on the device):

* ``fwd``        -- C2, the headline line: flash_attention forward, bf16, causal
                    MHA, B=4, H=32, S=4096, D=128.  A step is one forward call
                    (``flash_attn_fwd``: the fwd kernel).  Metric TFLOP/s over the
                    exact unmasked pair count, 4*D*pairs*B*H.
* ``fwdbwd``     -- C3: forward + backward, bf16, causal GQA (bottom-right),
                    B=2, Hq=32, Hkv=8, Sq=2048, Sk=8192, D=128.  14*D*pairs*B*Hq.
* ``decode``     -- C4: flash_decode, bf16 GQA, B=64, Hq=32, Hkv=8, Sk=32768,
                    D=128.  GB/s over K+V read once + q read + O written.
* ``decode_mqa`` -- C5: flash_decode, fp16 MQA, B=8, Hq=64, Hkv=1, Sk=131072,
                    D=128 (two KV buffer sets alternate so the 256 MB
                    Infinity Cache cannot hold the working set).

* ``decode_varlen`` -- decode on the C4 cache with a seeded cache length per
                    batch row, uniform in [1, S_k] (``cache_seqlens``).  GB/s over
                    the keys each row sees + q read + O written.
* ``decode_paged`` -- ``decode_varlen`` over a paged pool: 64-key pages, each row's
                    pages drawn from one shuffled pool (``block_table``).  Same
                    bytes as ``decode_varlen``.
* ``kv_update``  -- in-place append of 128 new key/value tokens per row into the
                    C4 cache at seeded distinct slots (``kv_cache_update``).  GB/s
                    over the new K/V read + the cache rows written + the slots.
* ``decode_rope`` -- C4 decode with the RoPE rotation of q fused into the decode
                    kernel (fp32 (Sk, D) tables, every row's query at position
                    Sk - 1).  Bytes of ``decode`` + the table rows read.
* ``decode_step`` -- one serving decode step on the C4 cache, captured once as a HIP graph
                    and replayed: append one token per row at its cache length
                    (keys rotated) + decode over the grown cache (q rotated); per-row
                    lengths U[1, Sk - 1] (seed 3), fp32 tables.  Bytes of
                    ``decode_varlen`` over the grown rows + the append + table rows;
                    ``details`` also gives the eager (un-captured) step time.
* ``kv_update_rope`` -- the cache append with the new keys rotated on the way in:
                    128 tokens per row appended at seeded per-row positions
                    p_b .. p_b + 127 (slots = positions), fp32 tables.  Bytes of
                    ``kv_update`` + the distinct table rows read.

``python bench.py`` runs ``fwd`` as the headline (``value``) and, unless
``--no-extra``, the others as entries of ``extra``, followed by the
``gemm`` reference: a bf16 8192^3 ``torch.matmul`` (the vendor GEMM), the
dense MFMA rate this part sustains under its power limit.  Each line carries a
``roofline`` object for the dominant kernel (algorithmic work per launch over
the average launch time measured with HIP events on the launch stream) and a
``cpu_baseline`` measured on this host with the PyTorch reference path
(fp32, the reference's own CPU algorithm) on a bounded sample.

Before each workload's timed loops the GPU runs about 300 ms of bf16 matmuls
and about 150 ms of the workload's own steps, untimed (clocks settle after an
idle spell and after a change of kernel mix), then the W warm-up steps; then
exactly K steps are timed.

One GPU only: ``--gpus N`` with N > 1 exits with a message.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "attn fwd/bwd TFLOP/s (% bf16 MFMA peak); flash_decode KV GB/s (% HBM peak)"
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16/fp16 MFMA
PEAK_FP32_TFLOPS = 157.3  # MI355X dense fp32 MFMA (the fp32 study workloads)
PEAK_HBM_GBPS = 8000.0  # MI355X HBM3E
PEAK_NOTE = {
    "mfma": "MI355X published dense bf16/fp16 MFMA peak, 2500 TFLOP/s (256 CUs x 2.4 GHz x "
            "4096 FLOP/clk = 2516.6 would give a fraction 0.66% lower); the part is power-limited "
            "below it: the vendor's bf16 GEMM sustains about 1307 TFLOP/s at 70% MFMA busy and "
            "1.69 GHz (bench.py --workload gemm)",
    "hbm": "MI355X published HBM3E peak, 8000 GB/s",
    "mfma_f32": "MI355X published dense fp32 matrix peak, 157.3 TFLOP/s",
}

# HBM bytes per step of each workload's kernels, from two rocprofv3 --pmc runs
# (FETCH_SIZE, then WRITE_SIZE; profiles/hbm_traffic_counters.md), each scaled by
# what the same counter reads for a 1 GiB device copy (FETCH_SIZE x 2,
# WRITE_SIZE x 1).  Counter runs cannot share a process with the timed loops,
# so these are recorded figures.  TRAFFIC_SOURCES_SHA256 is the digest of the
# kernel sources (kernel_sources_digest) the counters were measured on; when
# the sources differ, the line reports traffic null rather than a stale figure.
TRAFFIC_SOURCES_SHA256 = "caabc7557ffd45bbbc639c87567a7368ad6532d52283fbb03d5e3d5445c1d131"
HBM_TRAFFIC_BYTES = {
    "fwd": 681_165_750,
    "fwd_long": 838_971_108,
    "fwdbwd": 4_535_370_302,
    "decode": 8_601_597_260,
    "decode_mqa": 573_053_237,
    "decode_varlen": 4_305_224_903,
    "kv_update": 67_240_127,
    "decode_paged": 4_305_376_554,
    "decode_rope": 8_601_618_835,
    "kv_update_rope": 75_523_377,
    "decode_step": 4_306_761_979,
}


def kernel_sources_digest() -> str:
    """SHA-256 over the HIP kernel sources and headers (sorted by name), with
    their comments, blank lines and indentation removed, so that an edit to a
    comment alone keeps the recorded counter figures."""
    import hashlib
    import re

    csrc = os.path.join(ROOT, "stackkernels_amd", "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h")):
            h.update(name.encode())
            with open(os.path.join(csrc, name), "rb") as f:
                text = f.read().decode()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            text = re.sub(r"//[^\n]*", "", text)
            lines = (" ".join(line.split()) for line in text.splitlines())
            h.update("\n".join(line for line in lines if line).encode())
    return h.hexdigest()


def recorded_traffic(key: str):
    """(HBM bytes per step, note) for workload key: the counter figure if it was
    measured on the current kernel sources, else (None, why)."""
    if kernel_sources_digest() != TRAFFIC_SOURCES_SHA256:
        return None, ("recorded counters predate the current kernel sources; re-run the "
                      "FETCH_SIZE / WRITE_SIZE passes")
    val = HBM_TRAFFIC_BYTES.get(key)
    return val, ("rocprofv3 FETCH_SIZE/WRITE_SIZE, copy-calibrated, measured on kernel sources "
                 f"sha256 {TRAFFIC_SOURCES_SHA256[:16]}" if val else "not measured")


def causal_pairs(sq: int, sk: int, causal: bool) -> int:
    """Unmasked (i, j) pairs per (batch, head) under the bottom-right mask."""
    if not causal:
        return sq * sk
    off = sk - sq
    return sum(max(0, min(sk, i + off + 1)) for i in range(sq))


WORKLOADS = {
    "fwd": dict(name="C2 flash_attention fwd bf16 causal MHA", B=4, Hq=32, Hkv=32, Sq=4096,
                Sk=4096, D=128, causal=True, dtype="bf16", kind="fwd"),
    # A long causal prefill on a full grid: the forward table's 8-wave entry.
    "fwd_long": dict(name="flash_attention fwd bf16 causal MHA, long sequence", B=1, Hq=32,
                     Hkv=32, Sq=16384, Sk=16384, D=128, causal=True, dtype="bf16", kind="fwd"),
    "fwdbwd": dict(name="C3 flash_attention fwd+bwd bf16 causal GQA bottom-right", B=2, Hq=32,
                   Hkv=8, Sq=2048, Sk=8192, D=128, causal=True, dtype="bf16", kind="fwdbwd"),
    "decode": dict(name="C4 flash_decode bf16 GQA", B=64, Hq=32, Hkv=8, Sq=1, Sk=32768, D=128,
                   causal=False, dtype="bf16", kind="decode"),
    "decode_mqa": dict(name="C5 flash_decode fp16 MQA start_pos=Sk-1", B=8, Hq=64, Hkv=1, Sq=1,
                       Sk=131072, D=128, causal=False, dtype="fp16", kind="decode"),
    # Next-row workloads (per-row cache lengths, in-place cache append) on the C4 cache.
    "decode_varlen": dict(name="flash_decode bf16 GQA, C4 cache, per-row lengths U[1, Sk]", B=64,
                          Hq=32, Hkv=8, Sq=1, Sk=32768, D=128, causal=False, dtype="bf16",
                          kind="decode_varlen"),
    "kv_update": dict(name="kv_cache_update bf16, C4 cache, 128 new tokens per row", B=64, Hq=32,
                      Hkv=8, Sq=128, Sk=32768, D=128, causal=False, dtype="bf16",
                      kind="kv_update"),
    "decode_paged": dict(name="flash_decode bf16 GQA over a paged pool: 64-key pages, shuffled "
                              "block table, C4 capacity, per-row lengths U[1, Sk]", B=64, Hq=32,
                         Hkv=8, Sq=1, Sk=32768, D=128, causal=False, dtype="bf16",
                         kind="decode_paged", page_size=64),
    # RoPE fused into the decode prologue and into the cache append.
    "decode_rope": dict(name="C4 flash_decode bf16 GQA, RoPE of q fused (fp32 tables, position "
                             "Sk-1)", B=64, Hq=32, Hkv=8, Sq=1, Sk=32768, D=128, causal=False,
                        dtype="bf16", kind="decode_rope"),
    "decode_step": dict(name="serving decode step, C4 cache, per-row lengths U[1, Sk-1]: append "
                             "(keys rotated) + decode (q rotated), replayed as a HIP graph", B=64,
                        Hq=32, Hkv=8, Sq=1, Sk=32768, D=128, causal=False, dtype="bf16",
                        kind="decode_step"),
    "kv_update_rope": dict(name="kv_cache_update bf16, RoPE of the new keys fused, C4 cache, 128 "
                                "new tokens per row at seeded per-row positions", B=64, Hq=32,
                           Hkv=8, Sq=128, Sk=32768, D=128, causal=False, dtype="bf16",
                           kind="kv_update_rope"),
}


# Tile-table study shapes: selectable with --workload, not part of the default
# run (the head dims and plans the headline configs do not exercise).
STUDY_WORKLOADS = {
    "fwd_d64": dict(name="tile study: flash_attention fwd bf16 causal MHA, D=64", B=4, Hq=32,
                    Hkv=32, Sq=4096, Sk=4096, D=64, causal=True, dtype="bf16", kind="fwd"),
    "fwd_d64_long": dict(name="tile study: flash_attention fwd bf16 causal MHA, D=64, long "
                              "sequence", B=1, Hq=32, Hkv=32, Sq=16384, Sk=16384, D=64,
                         causal=True, dtype="bf16", kind="fwd"),
    "fwd_d256": dict(name="tile study: flash_attention fwd bf16 causal MHA, D=256", B=2, Hq=16,
                     Hkv=16, Sq=4096, Sk=4096, D=256, causal=True, dtype="bf16", kind="fwd"),
    "fwdbwd_d64": dict(name="tile study: C3 shape fwd+bwd bf16 causal GQA bottom-right, D=64",
                       B=2, Hq=32, Hkv=8, Sq=2048, Sk=8192, D=64, causal=True, dtype="bf16",
                       kind="fwdbwd"),
    "fwdbwd_d256": dict(name="tile study: C3 shape fwd+bwd bf16 causal GQA bottom-right, D=256",
                        B=2, Hq=32, Hkv=8, Sq=2048, Sk=8192, D=256, causal=True, dtype="bf16",
                        kind="fwdbwd"),
}
# fp32 inputs (true fp32 products and accumulation on the fp32 MFMA), priced
# against the fp32 matrix peak; selectable with --workload.
STUDY_WORKLOADS.update({
    "fwd_f32": dict(name="fp32 study: flash_attention fwd fp32 causal MHA, C2 shape", B=4, Hq=32,
                    Hkv=32, Sq=4096, Sk=4096, D=128, causal=True, dtype="fp32", kind="fwd"),
    "fwdbwd_f32": dict(name="fp32 study: C3 shape fwd+bwd fp32 causal GQA bottom-right", B=2,
                       Hq=32, Hkv=8, Sq=2048, Sk=8192, D=128, causal=True, dtype="fp32",
                       kind="fwdbwd"),
})
ALL_WORKLOADS = {**WORKLOADS, **STUDY_WORKLOADS}


NUM_SPLITS = 0  # --num-splits: decode split count override (0: the gfx950 table's)


def varlen_lengths(w: dict):
    """Seeded per-row cache lengths of the decode_varlen workload, uniform in [1, Sk]."""
    import torch

    g = torch.Generator().manual_seed(3)
    return torch.randint(1, w["Sk"] + 1, (w["B"],), generator=g, dtype=torch.int32)


def paged_table(w: dict):
    """Seeded block table of the decode_paged workload: every row's pages drawn
    without repetition from one shuffled pool of B * Sk / page_size pages."""
    import torch

    per_row = w["Sk"] // w["page_size"]
    g = torch.Generator().manual_seed(5)
    return torch.randperm(w["B"] * per_row, generator=g).view(w["B"], per_row).to(torch.int32)


def update_slots(w: dict):
    """Seeded distinct cache slots of the kv_update workload: (B, T) int64."""
    import torch

    g = torch.Generator().manual_seed(4)
    return torch.stack([torch.randperm(w["Sk"], generator=g)[:w["Sq"]] for _ in range(w["B"])])


def rope_starts(w: dict):
    """Seeded per-row positions of the first appended token (kv_update_rope),
    uniform in [0, Sk - T]: int32 (B,)."""
    import torch

    g = torch.Generator().manual_seed(6)
    return torch.randint(0, w["Sk"] - w["Sq"] + 1, (w["B"],), generator=g, dtype=torch.int32)


def rope_tables(w: dict, dev):
    """fp32 (Sk, D) cos / sin tables (the reference's precompute_freqs)."""
    from stackkernels_amd._reference.torch.rope import precompute_freqs

    return precompute_freqs(w["D"], w["Sk"], device=dev)


def step_lengths(w: dict):
    """Cache lengths before the decode_step append: varlen_lengths capped at Sk - 1."""
    return varlen_lengths(w).clamp(max=w["Sk"] - 1)


def work_units(w: dict) -> tuple[float, str]:
    """Algorithmic work of one step: (FLOP or bytes, unit of the rate)."""
    if w["kind"] == "decode_step":
        lens = step_lengths(w).long()
        esz, D, Hkv = 2, w["D"], w["Hkv"]
        kv = 2 * int((lens + 1).sum()) * Hkv * D * esz    # keys each row sees after the append
        qo = 2 * w["B"] * w["Hq"] * D * esz
        app = 4 * w["B"] * Hkv * D * esz + w["B"] * 8      # new k, v read; cache rows written; slots
        tab = int(lens.unique().numel()) * 2 * D * 4       # (cos, sin) rows
        return float(kv + qo + app + tab), "GB/s"
    if w["kind"] == "decode_rope":
        base, unit = work_units(dict(w, kind="decode"))
        return base + 2 * w["D"] * 4, unit  # one (cos, sin) row pair: every query at Sk - 1
    if w["kind"] == "kv_update_rope":
        import torch

        base, unit = work_units(dict(w, kind="kv_update"))
        pos = rope_starts(w)[:, None].long() + torch.arange(w["Sq"])
        return base + int(pos.unique().numel()) * 2 * w["D"] * 4, unit
    if w["kind"] == "decode":
        esz = 2
        kv = 2 * w["B"] * w["Hkv"] * w["Sk"] * w["D"] * esz
        qo = 2 * w["B"] * w["Hq"] * w["D"] * esz
        return float(kv + qo), "GB/s"
    if w["kind"] in ("decode_varlen", "decode_paged"):
        esz = 2
        kv = 2 * int(varlen_lengths(w).sum()) * w["Hkv"] * w["D"] * esz  # the keys each row sees
        qo = 2 * w["B"] * w["Hq"] * w["D"] * esz
        return float(kv + qo), "GB/s"
    if w["kind"] == "kv_update":
        rows = w["B"] * w["Hkv"] * w["Sq"]
        return float(4 * rows * w["D"] * 2 + w["B"] * w["Sq"] * 8), "GB/s"  # K, V read + written
    pairs = causal_pairs(w["Sq"], w["Sk"], w["causal"])
    per = 4 if w["kind"] == "fwd" else 14
    return float(per * w["D"] * pairs * w["B"] * w["Hq"]), "TFLOP/s"


def _rate(units: float, unit: str, seconds: float) -> float:
    return units / seconds / (1e12 if unit == "TFLOP/s" else 1e9)


def _make_inputs(w: dict, torch, dev, sets: int = 1):
    dt = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}[w["dtype"]]
    g = torch.Generator(device=dev).manual_seed(0)
    out = []
    if w["kind"] == "decode_paged":  # (q, k_pool, v_pool)
        pages = w["B"] * w["Sk"] // w["page_size"]
        shp = (pages, w["Hkv"], w["page_size"], w["D"])
        return [(torch.randn(w["B"], w["Hq"], 1, w["D"], generator=g, device=dev, dtype=dt),
                 torch.randn(shp, generator=g, device=dev, dtype=dt),
                 torch.randn(shp, generator=g, device=dev, dtype=dt))]
    if w["kind"] in ("kv_update", "kv_update_rope"):  # (new k, new v, k_cache, v_cache)
        shp_new = (w["B"], w["Hkv"], w["Sq"], w["D"])
        shp_cache = (w["B"], w["Hkv"], w["Sk"], w["D"])
        return [(torch.randn(shp_new, generator=g, device=dev, dtype=dt),
                 torch.randn(shp_new, generator=g, device=dev, dtype=dt),
                 torch.randn(shp_cache, generator=g, device=dev, dtype=dt),
                 torch.randn(shp_cache, generator=g, device=dev, dtype=dt))]
    for _ in range(sets):
        q = torch.randn(w["B"], w["Hq"], w["Sq"], w["D"], generator=g, device=dev, dtype=dt)
        k = torch.randn(w["B"], w["Hkv"], w["Sk"], w["D"], generator=g, device=dev, dtype=dt)
        if w["name"].startswith("C5"):
            v = torch.rand(w["B"], w["Hkv"], w["Sk"], w["D"], generator=g, device=dev, dtype=dt)
            v.mul_(2).sub_(1)
        else:
            v = torch.randn(w["B"], w["Hkv"], w["Sk"], w["D"], generator=g, device=dev, dtype=dt)
        out.append((q, k, v))
    return out


def _abi_launcher(w: dict, inputs, do, torch, dev):
    """A closure that launches the dominant kernel(s) straight through the C ABI on
    preallocated buffers (no Python allocation), for per-launch timing."""
    import ctypes

    from stackkernels_amd._core.attention import _lib

    lib = _lib.load()
    code = _lib.dtype_code(inputs[0][0].dtype)
    stream = _lib.stream_ptr(dev)
    B, Hq, Hkv, Sq, Sk, D = (w[k_] for k_ in ("B", "Hq", "Hkv", "Sq", "Sk", "D"))
    scale = 1.0 / math.sqrt(D)
    q0 = inputs[0][0]
    if w["kind"] == "kv_update_rope":
        kn, vn, kc, vc = inputs[0]
        starts = rope_starts(w)
        slots = (starts[:, None].long() + torch.arange(Sq)).to(dev)
        cos, sin = rope_tables(w, dev)
        sts = [_lib.strides3(t) for t in (kn, vn, kc, vc)]
        starts_dev = starts.to(dev)

        def launch(i):
            rc = lib.sk_kv_cache_update_rope(code, kn.data_ptr(), vn.data_ptr(), kc.data_ptr(),
                                             vc.data_ptr(), slots.data_ptr(), B, Hkv, Sq, Sk, D,
                                             *sts, cos.data_ptr(), sin.data_ptr(), _lib.SK_F32,
                                             Sk, D, starts_dev.data_ptr(), 0, stream)
            _lib.check(rc, "sk_kv_cache_update_rope")
        return launch
    if w["kind"] == "decode_step":
        ns = ctypes.c_int(0)
        nb = ctypes.c_size_t(0)
        _lib.check(lib.sk_decode_plan_varlen(code, B, Hq, Hkv, Sk, D, ctypes.byref(ns),
                                             ctypes.byref(nb)), "plan")
        ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=dev)
        q, k, v = inputs[0]
        o = torch.empty_like(q)
        g = torch.Generator(device=dev).manual_seed(7)
        kn = torch.randn(B, Hkv, 1, D, generator=g, device=dev, dtype=q.dtype)
        vn = torch.randn(B, Hkv, 1, D, generator=g, device=dev, dtype=q.dtype)
        lens = step_lengths(w).to(dev)
        lens1 = (lens + 1).contiguous()
        slots = lens.to(torch.int64).contiguous()
        cos, sin = rope_tables(w, dev)
        rope = (cos.data_ptr(), sin.data_ptr(), _lib.SK_F32, Sk, D, lens.data_ptr(), 0)
        sts = [_lib.strides3(t) for t in (q, k, v, o)]
        sta = [_lib.strides3(t) for t in (kn, vn, k, v)]

        def launch(i):
            rc = lib.sk_kv_cache_update_rope(code, kn.data_ptr(), vn.data_ptr(), k.data_ptr(),
                                             v.data_ptr(), slots.data_ptr(), B, Hkv, 1, Sk, D,
                                             *sta, *rope, stream)
            _lib.check(rc, "sk_kv_cache_update_rope")
            rc = lib.sk_decode_rope(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                    ws.data_ptr(), ws.numel(), ns.value, B, Hq, Hkv, Sk, D, *sts,
                                    lens1.data_ptr(), *rope, scale, stream)
            _lib.check(rc, "sk_decode_rope")
        return launch
    if w["kind"] == "decode_rope":
        ns = ctypes.c_int(0)
        nb = ctypes.c_size_t(0)
        _lib.check(lib.sk_decode_plan(code, B, Hq, Hkv, Sk, D, ctypes.byref(ns), ctypes.byref(nb)),
                   "plan")
        ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=dev)
        q, k, v = inputs[0]
        o = torch.empty_like(q)
        cos, sin = rope_tables(w, dev)
        sts = [_lib.strides3(t) for t in (q, k, v, o)]

        def launch(i):
            rc = lib.sk_decode_rope(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                    ws.data_ptr(), ws.numel(), ns.value, B, Hq, Hkv, Sk, D, *sts,
                                    None, cos.data_ptr(), sin.data_ptr(), _lib.SK_F32, Sk, D,
                                    None, Sk - 1, scale, stream)
            _lib.check(rc, "sk_decode_rope")
        return launch
    if w["kind"] == "kv_update":
        kn, vn, kc, vc = inputs[0]
        slots = update_slots(w).to(dev)
        sts = [_lib.strides3(t) for t in (kn, vn, kc, vc)]

        def launch(i):
            rc = lib.sk_kv_cache_update(code, kn.data_ptr(), vn.data_ptr(), kc.data_ptr(),
                                        vc.data_ptr(), slots.data_ptr(), B, Hkv, Sq, Sk, D,
                                        *sts, stream)
            _lib.check(rc, "sk_kv_cache_update")
        return launch
    if w["kind"] == "decode_paged":
        ns = ctypes.c_int(0)
        nb = ctypes.c_size_t(0)
        _lib.check(lib.sk_decode_plan_varlen(code, B, Hq, Hkv, Sk, D, ctypes.byref(ns),
                                             ctypes.byref(nb)), "plan")
        if NUM_SPLITS:
            ns.value = NUM_SPLITS
            _lib.check(lib.sk_decode_workspace(code, B, Hq, Hkv, Sk, D, NUM_SPLITS,
                                               ctypes.byref(nb)), "workspace")
        ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=dev)
        q, kp, vp = inputs[0]
        o = torch.empty_like(q)
        lens = varlen_lengths(w).to(dev)
        table = paged_table(w).to(dev)
        sts = [_lib.strides3(t) for t in (q, kp, vp, o)]
        ps = w["page_size"]

        def launch(i):
            rc = lib.sk_decode_paged(code, q.data_ptr(), kp.data_ptr(), vp.data_ptr(), o.data_ptr(),
                                     ws.data_ptr(), ws.numel(), ns.value, B, Hq, Hkv, kp.shape[0],
                                     ps, table.shape[1], D, *sts, table.data_ptr(),
                                     lens.data_ptr(), scale, stream)
            _lib.check(rc, "sk_decode_paged")
        return launch
    if w["kind"] == "decode_varlen":
        ns = ctypes.c_int(0)
        nb = ctypes.c_size_t(0)
        _lib.check(lib.sk_decode_plan_varlen(code, B, Hq, Hkv, Sk, D, ctypes.byref(ns),
                                             ctypes.byref(nb)), "plan")
        if NUM_SPLITS:
            ns.value = NUM_SPLITS
            _lib.check(lib.sk_decode_workspace(code, B, Hq, Hkv, Sk, D, NUM_SPLITS,
                                               ctypes.byref(nb)), "workspace")
        ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=dev)
        q, k, v = inputs[0]
        o = torch.empty_like(q)
        lens = varlen_lengths(w).to(dev)
        sts = [_lib.strides3(t) for t in (q, k, v, o)]

        def launch(i):
            rc = lib.sk_decode_varlen(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                      ws.data_ptr(), ws.numel(), ns.value, B, Hq, Hkv, Sk, D,
                                      *sts, lens.data_ptr(), scale, stream)
            _lib.check(rc, "sk_decode_varlen")
        return launch
    if w["kind"] == "decode":
        ns = ctypes.c_int(0)
        nb = ctypes.c_size_t(0)
        _lib.check(lib.sk_decode_plan(code, B, Hq, Hkv, Sk, D, ctypes.byref(ns), ctypes.byref(nb)),
                   "plan")
        if NUM_SPLITS:
            ns.value = NUM_SPLITS
            _lib.check(lib.sk_decode_workspace(code, B, Hq, Hkv, Sk, D, NUM_SPLITS,
                                               ctypes.byref(nb)), "workspace")
        ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=dev)
        o = torch.empty_like(q0)
        st = [(_lib.strides3(q), _lib.strides3(k), _lib.strides3(v)) for q, k, v in inputs]
        so = _lib.strides3(o)

        def launch(i):
            q, k, v = inputs[i % len(inputs)]
            sq_, sk_, sv_ = st[i % len(inputs)]
            rc = lib.sk_decode(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                               ws.data_ptr(), ws.numel(), ns.value, B, Hq, Hkv, Sk, D,
                               sq_, sk_, sv_, so, scale, stream)
            _lib.check(rc, "sk_decode")
        return launch
    q, k, v = inputs[0]
    o = torch.empty_like(q)
    lse = torch.empty(B, Hq, Sq, dtype=torch.float32, device=dev)
    sq_, sk_, sv_, so = (_lib.strides3(t) for t in (q, k, v, o))

    def fwd():
        rc = lib.sk_attn_fwd(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                             lse.data_ptr(), B, Hq, Hkv, Sq, Sk, D, sq_, sk_, sv_, so,
                             int(w["causal"]), scale, stream)
        _lib.check(rc, "sk_attn_fwd")
    if w["kind"] == "fwd":
        return lambda i: fwd()
    nb = ctypes.c_size_t(0)
    _lib.check(lib.sk_attn_bwd_workspace(code, B, Hq, Hkv, Sq, Sk, D, int(w["causal"]),
                                         ctypes.byref(nb)), "bwd workspace")
    ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)

    def fwdbwd(i):
        fwd()
        rc = lib.sk_attn_bwd(code, do.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                             o.data_ptr(), lse.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                             dv.data_ptr(), ws.data_ptr(), ws.numel(), B, Hq, Hkv, Sq, Sk, D,
                             int(w["causal"]), scale, stream)
        _lib.check(rc, "sk_attn_bwd")
    return fwdbwd


def _time_loop(fn, steps: int, warmup: int, torch, stream, per_step: bool = False):
    """Run ``fn(i)`` warmup + steps times; return (total ms / steps, sorted per-step ms).

    The total is one event pair around the ``steps`` back-to-back steps.  With
    ``per_step`` each step is also bracketed by its own event pair on the launch
    stream, which measures exactly that step's kernels while the host keeps the
    queue full; the extra event packets add a few microseconds between steps,
    so the total of such a loop is not used as the step time."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps if per_step else 0)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for i in range(steps):
        if per_step:
            evs[i][0].record(stream)
        fn(i)
        if per_step:
            evs[i][1].record(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps, sorted(a.elapsed_time(b) for a, b in evs)


def _warm_device(torch, dev, ms: float = 300.0):
    """Bring the GPU out of its idle clocks right before a timed loop: about
    ``ms`` of plain bf16 matmuls (not a step of any workload).  After an idle
    spell the first ~20 ms of attention kernels otherwise run up to 15% slow
    while the power controller settles."""
    a = torch.randn(4096, 4096, device=dev, dtype=torch.bfloat16)
    a = (a @ a) * 1e-3  # the first product may load the BLAS library: not part of the budget
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(10):
            a = (a @ a) * 1e-3
        torch.cuda.synchronize()
    for _ in range(20):  # left in the queue: no idle gap before the caller's first launch
        a = (a @ a) * 1e-3


def _settle(fn, torch, ms: float = 150.0, max_calls: int = 400):
    """Run the workload's own step untimed for about ``ms`` (at most
    ``max_calls`` calls) so the clocks have settled on this kernel mix before
    the timed loops: straight after the matmul warm-up the first loop of
    attention kernels runs about 6% slow."""
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    n = 0
    while (time.perf_counter() - t0) * 1e3 < ms and n < max_calls:
        for _ in range(4):
            fn(n)
            n += 1
        torch.cuda.synchronize()


def run_gpu(w: dict, steps: int, warmup: int):
    """Time ``steps`` steps of the public API and of the bare C-ABI launches;
    return (ms per API step, mean ms per C-ABI launch, details)."""
    import torch

    from stackkernels_amd._core.attention import _lib
    from stackkernels_amd._core.attention.decode import flash_decode, plan
    from stackkernels_amd._core.attention.flash_bwd import flash_attn_bwd
    from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd

    dev = torch.device("cuda:0")
    sets = 2 if w["name"].startswith("C5") else 1
    inputs = _make_inputs(w, torch, dev, sets)
    details: dict = {}
    eager_fn = None
    do = None
    if w["kind"] == "fwdbwd":
        g = torch.Generator(device=dev).manual_seed(1)
        do = torch.randn(inputs[0][0].shape, generator=g, device=dev, dtype=inputs[0][0].dtype)

    if w["kind"] == "decode":
        q0 = inputs[0][0]
        details["num_splits"] = (NUM_SPLITS or
                                 plan(q0.dtype, w["B"], w["Hq"], w["Hkv"], w["Sk"], w["D"])[0])

        def step(i):
            q, k, v = inputs[i % sets]
            flash_decode(q, k, v, num_splits=NUM_SPLITS or None)
    elif w["kind"] == "decode_varlen":
        q0 = inputs[0][0]
        details["num_splits"] = (NUM_SPLITS or plan(q0.dtype, w["B"], w["Hq"], w["Hkv"], w["Sk"],
                                                    w["D"], per_row=True)[0])
        lens_dev = varlen_lengths(w).to(dev)
        details["mean_length"] = round(float(lens_dev.float().mean()), 1)

        def step(i):
            q, k, v = inputs[0]
            flash_decode(q, k, v, cache_seqlens=lens_dev, num_splits=NUM_SPLITS or None)
    elif w["kind"] == "decode_paged":
        from stackkernels_amd._core.attention.decode import flash_decode_paged

        q0 = inputs[0][0]
        details["num_splits"] = (NUM_SPLITS or plan(q0.dtype, w["B"], w["Hq"], w["Hkv"], w["Sk"],
                                                    w["D"], per_row=True)[0])
        lens_dev = varlen_lengths(w).to(dev)
        table_dev = paged_table(w).to(dev)
        details["mean_length"] = round(float(lens_dev.float().mean()), 1)
        details["page_size"] = w["page_size"]

        def step(i):
            q, kp, vp = inputs[0]
            flash_decode_paged(q, kp, vp, table_dev, lens_dev, num_splits=NUM_SPLITS or None)
    elif w["kind"] == "decode_rope":
        q0 = inputs[0][0]
        details["num_splits"] = plan(q0.dtype, w["B"], w["Hq"], w["Hkv"], w["Sk"], w["D"])[0]
        cos, sin = rope_tables(w, dev)

        def step(i):
            q, k, v = inputs[0]
            flash_decode(q, k, v, rope_cos=cos, rope_sin=sin, start_pos=w["Sk"] - 1)
    elif w["kind"] == "decode_step":
        from stackkernels_amd.torch.attention import flash_decode as api_decode
        from stackkernels_amd.torch.cache import kv_cache_update

        q, kc, vc = inputs[0]
        g = torch.Generator(device=dev).manual_seed(7)
        kn = torch.randn(w["B"], w["Hkv"], 1, w["D"], generator=g, device=dev, dtype=q.dtype)
        vn = torch.randn(w["B"], w["Hkv"], 1, w["D"], generator=g, device=dev, dtype=q.dtype)
        lens = step_lengths(w).to(dev)
        cos, sin = rope_tables(w, dev)
        details["num_splits"] = plan(q.dtype, w["B"], w["Hq"], w["Hkv"], w["Sk"], w["D"],
                                     per_row=True)[0]
        details["mean_length"] = round(float(lens.float().mean()) + 1, 1)

        def eager(i):
            kv_cache_update(kn, vn, kc, vc, lens.to(torch.int64).view(-1, 1), rope_cos=cos,
                            rope_sin=sin, start_pos=lens)
            return api_decode(q, kc, vc, cache_seqlens=lens + 1, rope_cos=cos, rope_sin=sin,
                              start_pos=lens)

        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            eager(0)
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            eager(0)
        eager_fn = eager

        def step(i):
            graph.replay()
    elif w["kind"] == "kv_update_rope":
        from stackkernels_amd.torch.cache import kv_cache_update

        starts = rope_starts(w)
        slots_dev = (starts[:, None].long() + torch.arange(w["Sq"])).to(dev)
        starts_dev = starts.to(dev)
        cos, sin = rope_tables(w, dev)

        def step(i):
            kn, vn, kc, vc = inputs[0]
            kv_cache_update(kn, vn, kc, vc, slots_dev, rope_cos=cos, rope_sin=sin,
                            start_pos=starts_dev)
    elif w["kind"] == "kv_update":
        from stackkernels_amd.torch.cache import kv_cache_update

        slots_dev = update_slots(w).to(dev)

        def step(i):
            kn, vn, kc, vc = inputs[0]
            kv_cache_update(kn, vn, kc, vc, slots_dev)
    elif w["kind"] == "fwd":
        def step(i):
            q, k, v = inputs[0]
            flash_attn_fwd(q, k, v, is_causal=w["causal"])
    else:
        def step(i):
            q, k, v = inputs[0]
            o, lse = flash_attn_fwd(q, k, v, is_causal=w["causal"])
            flash_attn_bwd(do, q, k, v, o, lse, is_causal=w["causal"])

    stream = torch.cuda.current_stream(dev)
    launch = _abi_launcher(w, inputs, do, torch, dev)
    _warm_device(torch, dev)
    _settle(step, torch)
    ms_step, _ = _time_loop(step, steps, warmup, torch, stream)
    _, per = _time_loop(launch, steps, warmup, torch, stream, per_step=True)
    if eager_fn is not None:  # the same step without the graph (public API calls)
        details["eager_ms_per_step"] = round(_time_loop(eager_fn, steps, warmup, torch, stream)[0], 5)
    details["launch_ms_median"] = round(per[len(per) // 2], 5)
    details["launch_ms_min"] = round(per[0], 5)
    mean = sum(per) / len(per)
    details["launch_ms_mean"] = round(mean, 5)
    assert _lib._lib is not None, "native library was not loaded"
    return ms_step, mean, details


def _cpu_baseline_next_rows(w: dict, budget_s: float):
    """CPU baseline of the next-row workloads: this build's own CPU path on one batch
    row (decode over row 0's cache length; the cache append of row 0's tokens)."""
    import torch

    from stackkernels_amd.torch.attention import flash_decode
    from stackkernels_amd.torch.cache import kv_cache_update

    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)
    D, Hq, Hkv = w["D"], w["Hq"], w["Hkv"]
    if w["kind"] == "decode_paged":
        n = int(varlen_lengths(w)[0])
        ps = w["page_size"]
        n_pages = (n + ps - 1) // ps
        q = torch.randn(1, Hq, 1, D, generator=g).bfloat16()
        kp = torch.randn(n_pages, Hkv, ps, D, generator=g).bfloat16()
        vp = torch.randn(n_pages, Hkv, ps, D, generator=g).bfloat16()
        table = torch.randperm(n_pages, generator=g).view(1, n_pages)
        units_one = 2 * n * Hkv * D * 2 + 2 * Hq * D * 2
        fn = lambda: flash_decode(q, kp, vp, cache_seqlens=torch.tensor([n]),  # noqa: E731
                                  block_table=table)
        what = (f"paged flash_decode reference path on batch row 0 (length {n}, {n_pages} "
                f"pages of {ps} keys, {Hq} query heads)")
    elif w["kind"] == "decode_varlen":
        n = int(varlen_lengths(w)[0])
        q = torch.randn(1, Hq, 1, D, generator=g).bfloat16()
        k = torch.randn(1, Hkv, n, D, generator=g).bfloat16()
        v = torch.randn(1, Hkv, n, D, generator=g).bfloat16()
        units_one = 2 * n * Hkv * D * 2 + 2 * Hq * D * 2
        fn = lambda: flash_decode(q, k, v, cache_seqlens=torch.tensor([n]))  # noqa: E731
        what = f"flash_decode reference path on batch row 0 (length {n}, {Hq} query heads)"
    elif w["kind"] == "decode_rope":
        n = w["Sk"]
        q = torch.randn(1, Hq, 1, D, generator=g).bfloat16()
        k = torch.randn(1, Hkv, n, D, generator=g).bfloat16()
        v = torch.randn(1, Hkv, n, D, generator=g).bfloat16()
        cos, sin = rope_tables(w, "cpu")
        units_one = 2 * n * Hkv * D * 2 + 2 * Hq * D * 2 + 2 * D * 4
        fn = lambda: flash_decode(q, k, v, rope_cos=cos, rope_sin=sin,  # noqa: E731
                                  start_pos=n - 1)
        what = f"flash_decode reference path with RoPE of q on batch row 0 ({n} keys)"
    elif w["kind"] == "decode_step":
        n = int(step_lengths(w)[0])
        q = torch.randn(1, Hq, 1, D, generator=g).bfloat16()
        kc = torch.randn(1, Hkv, n + 1, D, generator=g).bfloat16()
        vc = torch.randn(1, Hkv, n + 1, D, generator=g).bfloat16()
        kn = torch.randn(1, Hkv, 1, D, generator=g).bfloat16()
        vn = torch.randn(1, Hkv, 1, D, generator=g).bfloat16()
        cos, sin = rope_tables(w, "cpu")
        units_one = 2 * (n + 1) * Hkv * D * 2 + 2 * Hq * D * 2 + 4 * Hkv * D * 2 + 8 + 2 * D * 4

        def fn():
            kv_cache_update(kn, vn, kc, vc, torch.tensor([[n]]), rope_cos=cos, rope_sin=sin,
                            start_pos=n)
            flash_decode(q, kc, vc, rope_cos=cos, rope_sin=sin, start_pos=n)
        what = f"append + decode reference path with RoPE on batch row 0 (length {n} + 1)"
    elif w["kind"] == "kv_update_rope":
        T = w["Sq"]
        kn = torch.randn(1, Hkv, T, D, generator=g).bfloat16()
        vn = torch.randn(1, Hkv, T, D, generator=g).bfloat16()
        kc = torch.zeros(1, Hkv, w["Sk"], D, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        st = rope_starts(w)[:1]
        sl = st[:, None].long() + torch.arange(T)
        cos, sin = rope_tables(w, "cpu")
        units_one = 4 * Hkv * T * D * 2 + T * 8 + T * 2 * D * 4
        fn = lambda: kv_cache_update(kn, vn, kc, vc, sl, rope_cos=cos, rope_sin=sin,  # noqa: E731
                                     start_pos=st)
        what = f"kv_cache_update reference path with RoPE of k on batch row 0 ({T} tokens)"
    else:
        T = w["Sq"]
        kn = torch.randn(1, Hkv, T, D, generator=g).bfloat16()
        vn = torch.randn(1, Hkv, T, D, generator=g).bfloat16()
        kc = torch.zeros(1, Hkv, w["Sk"], D, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        sl = update_slots(w)[:1]
        units_one = 4 * Hkv * T * D * 2 + T * 8
        fn = lambda: kv_cache_update(kn, vn, kc, vc, sl)  # noqa: E731
        what = f"kv_cache_update reference path (torch indexing) on batch row 0 ({T} tokens)"
    done = 0
    t0 = time.perf_counter()
    while True:
        fn()
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return {
        "value": round(_rate(units_one * done, "GB/s", el), 6),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{what} of {w['name']}, {done} repetition(s) in {el:.1f} s; "
                   f"host {os.cpu_count()} CPUs ({host_cpu_model()}), torch threads {threads}"),
        "host_cpu": host_cpu_model(),
    }


def host_cpu_model() -> str:
    """The host CPU's model line, as ``lscpu`` prints it ("Model name"), read from
    /proc/cpuinfo; ``lscpu`` itself where that file has none."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.lower().startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return "unknown"


def run_cpu_baseline(w: dict, budget_s: float):
    """The reference's CPU algorithm (fp32 torch, ``attention_reference``) on a bounded
    sample of the workload: one batch row, KV-head groups in turn, repeated until
    ``budget_s`` of CPU time has passed.  Returns the cpu_baseline object."""
    import torch

    from stackkernels_amd._reference.torch.attention import attention_reference

    if w["kind"] in ("decode_varlen", "kv_update", "decode_paged", "decode_rope",
                     "kv_update_rope", "decode_step"):
        return _cpu_baseline_next_rows(w, budget_s)
    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)
    grp = w["Hq"] // w["Hkv"]
    if w["kind"] == "decode":
        hkv_chunk = 1
    else:
        # 4 query heads per chunk bounds the score tensor, one for long sequences
        # (16,384^2 fp32 scores are 1 GiB per head)
        hkv_chunk = max(1, 4 // grp) if w["Sq"] * w["Sk"] <= (1 << 26) else 1
    hq_chunk = hkv_chunk * grp
    def rnd(*shape):  # 16-bit workloads: values representable in the input type
        x = torch.randn(*shape, generator=g)
        return x if w["dtype"] == "fp32" else x.bfloat16().float()

    q = rnd(1, hq_chunk, w["Sq"], w["D"])
    k = rnd(1, hkv_chunk, w["Sk"], w["D"])
    v = rnd(1, hkv_chunk, w["Sk"], w["D"])
    do = torch.randn_like(q) if w["kind"] == "fwdbwd" else None
    done = 0
    t0 = time.perf_counter()
    while True:
        if w["kind"] == "fwdbwd":
            qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
            out, _ = attention_reference(qr, kr, vr, is_causal=w["causal"])
            out.backward(do)
        else:
            attention_reference(q, k, v, is_causal=w["causal"])
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    units_total, unit = work_units(w)
    frac = hq_chunk / (w["B"] * w["Hq"])
    units = units_total * frac * done
    return {
        "value": round(_rate(units, unit, el), 6),
        "unit": unit,
        "cores": threads,
        "kind": "port",
        "sample": (f"attention_reference (fp32 torch restatement of the reference CPU path) on "
                   f"batch row 0, {hq_chunk} query head(s) / {hkv_chunk} KV head(s) of {w['name']}, "
                   f"{done} repetition(s) in {el:.1f} s; host {os.cpu_count()} CPUs "
                   f"({host_cpu_model()}), "
                   f"torch threads {threads}"),
        "host_cpu": host_cpu_model(),
    }


def measure(key: str, steps: int, warmup: int, cpu_s: float) -> dict:
    w = ALL_WORKLOADS[key]
    units, unit = work_units(w)
    ms_step, ms_kernel, details = run_gpu(w, steps, warmup)
    value = _rate(units, unit, ms_step / 1e3)
    achieved = _rate(units, unit, ms_kernel / 1e3)
    bound = "hbm" if unit == "GB/s" else "mfma"
    f32 = w["dtype"] == "fp32"
    peak = PEAK_HBM_GBPS if bound == "hbm" else PEAK_FP32_TFLOPS if f32 else PEAK_BF16_TFLOPS
    kernel = {"fwd": "fwd_f32_mfma_kernel" if f32 else "fwd_mfma_kernel", "fwdbwd": "fwd + bwd kernels",
              "decode": "decode_split_kernel + decode_combine_kernel",
              "decode_varlen": "decode_split_kernel + decode_combine_kernel",
              "decode_paged": "decode_split_kernel (paged) + decode_combine_kernel",
              "kv_update": "kv_cache_update_kernel",
              "decode_rope": "decode_split_kernel (q rotated on load) + decode_combine_kernel",
              "kv_update_rope": "kv_cache_update_rope_kernel",
              "decode_step": "kv_cache_update_rope_kernel + decode_split_kernel (q rotated) + "
                             "decode_combine_kernel"}[w["kind"]]
    traffic, traffic_note = recorded_traffic(key)
    res = {
        "workload": key,
        "config": {k_: w[k_] for k_ in ("name", "B", "Hq", "Hkv", "Sq", "Sk", "D", "causal", "dtype")},
        "value": round(value, 3),
        "unit": unit,
        "ms_per_step": round(ms_step, 5),
        "roofline": {
            "bound": bound,
            "kernel": kernel,
            "achieved": round(achieved, 3),
            "peak": peak,
            "unit": unit,
            "frac": round(achieved / peak, 4),
            "peak_basis": PEAK_NOTE["mfma_f32" if f32 and bound == "mfma" else bound],
            "traffic": traffic,
            "traffic_unit": "HBM bytes per step",
            "traffic_note": traffic_note,
            "work_per_launch": units,
        },
        "details": details,
    }
    if cpu_s > 0:
        res["cpu_baseline"] = run_cpu_baseline(w, cpu_s)
    return res


def copy_calibration(steps: int, warmup: int) -> dict:
    """Time ``y.copy_(x)`` on a 1 GiB buffer: 1 GiB read + 1 GiB written per launch.

    Its FETCH_SIZE / WRITE_SIZE counters give the factor that turns those
    counters into HBM bytes for the attention kernels."""
    import torch

    dev = torch.device("cuda:0")
    n = 1 << 30
    x = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    y = torch.empty_like(x)
    stream = torch.cuda.current_stream(dev)
    _, per = _time_loop(lambda i: y.copy_(x), steps, warmup, torch, stream, per_step=True)
    mean = sum(per) / len(per)
    return {"workload": "copy", "bytes_read": n, "bytes_written": n, "ms_mean": round(mean, 5),
            "GB/s": round(2 * n / mean / 1e6, 1)}


def gemm_calibration(steps: int, warmup: int, n: int = 8192) -> dict:
    """Time a plain bf16 ``torch.matmul`` of two n x n matrices (the vendor GEMM).

    Its rate, with the clock and MFMA busy fraction its counters give, is the
    MFMA throughput this part sustains under its power limit, the reference
    point beside the published peak for the attention kernels' fractions."""
    import torch

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn(n, n, generator=g, device=dev, dtype=torch.bfloat16)
    b = torch.randn(n, n, generator=g, device=dev, dtype=torch.bfloat16)
    c = torch.empty(n, n, device=dev, dtype=torch.bfloat16)
    stream = torch.cuda.current_stream(dev)
    _, per = _time_loop(lambda i: torch.matmul(a, b, out=c), steps, warmup, torch, stream,
                        per_step=True)
    mean = sum(per) / len(per)
    flop = 2 * n ** 3
    return {"workload": "gemm", "n": n, "flop": flop, "ms_mean": round(mean, 5),
            "TFLOP/s": round(flop / mean / 1e9, 1),
            "frac_of_published_peak": round(flop / mean / 1e9 / PEAK_BF16_TFLOPS, 4)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    # defaults: 10 untimed and 50 timed steps per loop, so every launch median
    # is taken over 50 launches
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", choices=sorted(ALL_WORKLOADS) + ["copy", "gemm"], default="fwd",
                    help="headline workload (default fwd = C2); 'copy' times a plain 1 GiB "
                         "device copy, the calibration kernel for the HBM-traffic counters; "
                         "'gemm' times a bf16 8192^3 torch.matmul, the sustained-MFMA reference; "
                         "fwd_d64, fwd_d64_long, fwd_d256, fwdbwd_d64, fwdbwd_d256 are tile-study "
                         "shapes and fwd_f32, fwdbwd_f32 fp32 shapes, outside the default run")
    ap.add_argument("--no-extra", action="store_true", help="skip the other workloads")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="CPU-baseline budget per workload (0 disables)")
    ap.add_argument("--num-splits", type=int, default=0,
                    help="decode, decode_mqa, decode_varlen, decode_paged: run this split count "
                         "instead of the table's (tile-table study; 0 = the table)")
    args = ap.parse_args()
    global NUM_SPLITS
    NUM_SPLITS = args.num_splits
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the attention path is "
              "built and measured on a single MI355X in this build.", file=sys.stderr)
        return 2
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if args.workload == "copy":
        print(json.dumps(copy_calibration(args.steps, args.warmup)), flush=True)
        return 0
    if args.workload == "gemm":
        print(json.dumps(gemm_calibration(args.steps, args.warmup)), flush=True)
        return 0
    head = measure(args.workload, args.steps, args.warmup, args.cpu_seconds)
    extra = []
    if not args.no_extra:
        for key in WORKLOADS:
            if key == args.workload:
                continue
            try:
                extra.append(measure(key, args.steps, args.warmup, args.cpu_seconds))
                print(f"# {key}: {extra[-1]['value']} {extra[-1]['unit']}", file=sys.stderr,
                      flush=True)
            except (RuntimeError, NotImplementedError) as e:
                extra.append({"workload": key, "error": str(e)[:300]})
                print(f"# {key}: failed: {e}", file=sys.stderr, flush=True)
        # the sustained-MFMA reference of this part, beside the attention rates
        extra.append(gemm_calibration(args.steps, args.warmup))
        print(f"# gemm: {extra[-1]['TFLOP/s']} TFLOP/s", file=sys.stderr, flush=True)
    w = ALL_WORKLOADS[args.workload]
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w["dtype"],
        "data": "synthetic (seeded N(0,1) on device; C5 V ~ U(-1,1))",
        "config": {"workload": w["name"], "B": w["B"], "Hq": w["Hq"], "Hkv": w["Hkv"],
                   "Sq": w["Sq"], "Sk": w["Sk"], "D": w["D"], "causal": w["causal"]},
        "roofline": head["roofline"],
        "cpu_baseline": head.get("cpu_baseline"),
        "details": head["details"],
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
