"""GPU test of concurrent calls from several host threads, each on its own stream.

The library keeps per-process state that concurrent callers share: the table
of side streams (one per caller stream, made on first use under a mutex) that
the seven-GEMM backward forks its dQ kernel onto, and the thread-local error
text; every call takes its scratch from the caller's workspace.  Four jobs run
at once, on four host threads and four streams, three times each:
* a D = 64 causal backward large enough to fork (512 dK/dV workgroups);
* a D = 128 five-GEMM backward (its dS tiles in the call's own workspace);
* a per-row-length decode;
* a paged decode.

Every result must equal, bit for bit, that of the same job run alone first:
each kernel's result is fixed by its inputs (no atomics, fixed split plans),
so any difference means two calls shared a buffer or an ordering they must
not.
"""

import threading

import pytest
import torch

from stackkernels_amd._core.attention.flash_bwd import flash_attn_bwd
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd
from stackkernels_amd.torch import flash_decode

from _gpu_util import native_loaded

pytestmark = pytest.mark.gpu
ROUNDS = 3


def _rand(shape, dtype, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(dtype).cuda()


def _train_job(b, hq, hkv, s, d, dtype, causal, seed):
    q, k, v, do = (_rand((b, h, s, d), dtype, seed + i)
                   for i, h in enumerate((hq, hkv, hkv, hq)))

    def run():
        # the launchers, not autograd: autograd would run every thread's
        # backward on its one device thread
        out, lse = flash_attn_fwd(q, k, v, is_causal=causal)
        return (out, lse, *flash_attn_bwd(do, q, k, v, out, lse, is_causal=causal))

    return run


def _decode_job(paged, seed):
    dtype = torch.float16 if paged else torch.bfloat16
    b, hq, hkv, d = 8, 32, 8, 128
    q = _rand((b, hq, 1, d), dtype, seed)
    lens = torch.randint(0, 4096, (b,), generator=torch.Generator().manual_seed(seed)).int().cuda()
    if not paged:
        k, v = _rand((b, hkv, 4096, d), dtype, seed + 1), _rand((b, hkv, 4096, d), dtype, seed + 2)
        return lambda: (flash_decode(q, k, v, cache_seqlens=lens),)
    ps, per_row = 64, 64
    kp = _rand((b * per_row, hkv, ps, d), dtype, seed + 1)
    vp = _rand((b * per_row, hkv, ps, d), dtype, seed + 2)
    table = torch.randperm(b * per_row, generator=torch.Generator().manual_seed(seed))
    table = table.view(b, per_row).int().cuda()
    return lambda: (flash_decode(q, kp, vp, cache_seqlens=lens, block_table=table),)


def test_concurrent_threads_and_streams_match_serial_results(device):
    jobs = {
        "bwd_d64_forked": _train_job(2, 8, 8, 4096, 64, torch.bfloat16, True, 10),
        "bwd_d128_five_gemm": _train_job(1, 8, 2, 1024, 128, torch.float16, False, 20),
        "decode_varlen": _decode_job(False, 30),
        "decode_paged": _decode_job(True, 40),
    }
    expect = {name: job() for name, job in jobs.items()}
    torch.cuda.synchronize()
    assert native_loaded()

    got = {name: [] for name in jobs}
    errors = []
    start = threading.Barrier(len(jobs))

    def worker(name):
        try:
            stream = torch.cuda.Stream()
            start.wait()
            with torch.cuda.stream(stream):
                for _ in range(ROUNDS):
                    got[name].append(jobs[name]())
            stream.synchronize()
        except Exception as e:  # noqa: BLE001 -- reported by the main thread
            errors.append(f"{name}: {e!r}")

    threads = [threading.Thread(target=worker, args=(n,)) for n in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    torch.cuda.synchronize()
    assert not errors, errors
    for name, runs in got.items():
        assert len(runs) == ROUNDS, name
        for r, outs in enumerate(runs):
            for i, (a, b) in enumerate(zip(outs, expect[name])):
                assert torch.equal(a, b), f"{name}, round {r}, output {i} differs from the serial run"
