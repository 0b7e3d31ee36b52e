"""The backward's two launch shapes, eagerly and under HIP graph capture.

Seven GEMMs (head dims other than 65-128): when the dK/dV grid runs more than
one round of workgroups, ``sk_attn_bwd`` forks the dQ kernel onto the side
stream the library keeps for the caller's stream, after the preprocess pass,
and joins it back with events.  Five GEMMs (D = 128): the dK/dV kernel stores
dS in the workspace and the dQ kernel reads it after it, on the caller's
stream.  The kernels use no atomics, so the result does not depend on how
they overlap: every replay of a captured backward (fork and join become graph
edges) must equal, bit for bit, the eager call on the same inputs, and the
eager call must match the oracle-checked fp32 reference within the bf16
tolerance.
"""

import pytest
import torch

from stackkernels_amd._core.attention.flash_bwd import flash_attn_bwd
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd
from stackkernels_amd._reference.torch.attention import attention_reference

from _gpu_util import TOL, assert_close_maxabs, native_loaded

pytestmark = pytest.mark.gpu

# B=2, H_kv=8, S_k=4096: 32 key blocks x 16 = 512 dK/dV workgroups, two rounds.
SHAPE = dict(b=2, hq=16, hkv=8, sq=512, sk=4096)
DIMS = {"seven_gemm_fork": 64, "five_gemm": 128}


@pytest.fixture(params=sorted(DIMS), autouse=True)
def _head_dim(request):
    SHAPE["d"] = DIMS[request.param]
    yield


def _inputs(dtype, seed):
    s = SHAPE
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(s["b"], s["hq"], s["sq"], s["d"], generator=g, device="cuda").to(dtype)
    k = torch.randn(s["b"], s["hkv"], s["sk"], s["d"], generator=g, device="cuda").to(dtype)
    v = torch.randn(s["b"], s["hkv"], s["sk"], s["d"], generator=g, device="cuda").to(dtype)
    do = torch.randn(s["b"], s["hq"], s["sq"], s["d"], generator=g, device="cuda").to(dtype)
    return q, k, v, do


def test_forked_backward_matches_reference():
    dtype = torch.bfloat16
    q, k, v, do = _inputs(dtype, 0)
    out, lse = flash_attn_fwd(q, k, v, True)
    dq, dk, dv = flash_attn_bwd(do, q, k, v, out, lse, True)
    torch.cuda.synchronize()
    assert native_loaded()
    qr, kr, vr = (t.float().requires_grad_() for t in (q, k, v))
    ref, _ = attention_reference(qr, kr, vr, True)
    ref.backward(do.float())
    for name, got, want in (("dQ", dq, qr.grad), ("dK", dk, kr.grad), ("dV", dv, vr.grad)):
        assert_close_maxabs(got, want.double().cpu().numpy(), TOL[dtype], f"forked backward {name}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_backward_graph_replays_match_eager(dtype):
    q, k, v, do = _inputs(dtype, 1)
    out, lse = flash_attn_fwd(q, k, v, True)

    # eager call first, on the stream the capture will use: loads the library
    # and creates that stream's side stream, so the capture records the fork
    # and the join as graph edges
    cap = torch.cuda.Stream()
    cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cap):
        flash_attn_bwd(do, q, k, v, out, lse, True)
    torch.cuda.current_stream().wait_stream(cap)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        grads = flash_attn_bwd(do, q, k, v, out, lse, True)

    for step in range(3):
        q2, k2, v2, do2 = _inputs(dtype, 10 + step)
        o2, lse2 = flash_attn_fwd(q2, k2, v2, True)
        for dst, src in ((q, q2), (k, k2), (v, v2), (do, do2), (out, o2), (lse, lse2)):
            dst.copy_(src)
        want = flash_attn_bwd(do2, q2, k2, v2, o2, lse2, True)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(("dQ", "dK", "dV"), grads, want):
            assert torch.equal(got, ref), f"replay {step}: {name} differs from the eager call"


def test_capture_beside_eager_thread():
    """One thread captures a forked backward while another runs forked
    backwards eagerly on its own stream: neither picks up the other's work
    (each caller stream has its own side stream).  The captured graph's
    replays and every eager result equal a plain eager call bit for bit."""
    import threading

    dtype = torch.bfloat16
    q, k, v, do = _inputs(dtype, 2)
    out, lse = flash_attn_fwd(q, k, v, True)
    want = flash_attn_bwd(do, q, k, v, out, lse, True)
    torch.cuda.synchronize()

    cap = torch.cuda.Stream()
    eag = torch.cuda.Stream()
    for st in (cap, eag):  # make both streams' side streams before the capture
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            flash_attn_bwd(do, q, k, v, out, lse, True)
        torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    captured = {}
    eager_results = []
    errors = []
    started = threading.Event()

    def capture():
        try:
            with torch.cuda.graph(graph, stream=cap, capture_error_mode="thread_local"):
                started.set()
                captured["grads"] = flash_attn_bwd(do, q, k, v, out, lse, True)
        except Exception as e:  # noqa: BLE001 -- reported by the main thread
            errors.append(e)
            started.set()

    def eager():
        try:
            started.wait(timeout=30)
            with torch.cuda.stream(eag):
                for _ in range(4):
                    eager_results.append(flash_attn_bwd(do, q, k, v, out, lse, True))
            eag.synchronize()
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    threads = [threading.Thread(target=capture), threading.Thread(target=eager)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors, errors
    assert len(eager_results) == 4
    torch.cuda.synchronize()
    for i, res in enumerate(eager_results):
        for name, got, ref in zip(("dQ", "dK", "dV"), res, want):
            assert torch.equal(got, ref), f"eager call {i} beside the capture: {name} differs"
    for step in range(2):
        graph.replay()
        torch.cuda.synchronize()
        for name, got, ref in zip(("dQ", "dK", "dV"), captured["grads"], want):
            assert torch.equal(got, ref), f"replay {step}: {name} differs from the eager call"
