"""A decode step captured in a HIP graph (torch.cuda.CUDAGraph) and replayed.

The library allocates nothing, synchronises nothing and launches on the
caller's stream, so a serving loop can capture "append the new k, v (keys
rotated) + decode (q rotated)" once and replay it.  Each replay here gets new
q, k, v and advanced cache lengths copied into the captured buffers, with
eager work and synchronisations between the replays, and must match the same
step run eagerly bit for bit (the same kernels on the same inputs).
"""

import pytest
import torch

import stackkernels_amd
from stackkernels_amd._reference.torch.rope import precompute_freqs
from stackkernels_amd.torch import flash_attention, flash_decode, kv_cache_update

from _gpu_util import native_loaded

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _auto_backend():
    original = stackkernels_amd.get_backend()
    stackkernels_amd.set_backend("auto")
    yield
    stackkernels_amd.set_backend(original)


def _step(q, k_new, v_new, kc, vc, lens, cos, sin):
    slots = lens.to(torch.int64).view(-1, 1)
    kv_cache_update(k_new, v_new, kc, vc, slots, rope_cos=cos, rope_sin=sin, start_pos=lens)
    return flash_decode(q, kc, vc, cache_seqlens=lens + 1, rope_cos=cos, rope_sin=sin,
                        start_pos=lens)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_decode_step_graph_replays_match_eager(dtype):
    dev = "cuda"
    b, hq, hkv, s_cap, d = 4, 32, 8, 2048, 128
    g = torch.Generator(device=dev).manual_seed(0)
    kc = torch.randn(b, hkv, s_cap, d, generator=g, device=dev).to(dtype)
    vc = torch.randn(b, hkv, s_cap, d, generator=g, device=dev).to(dtype)
    cos, sin = (t.to(dev) for t in precompute_freqs(d, s_cap))
    q = torch.zeros(b, hq, 1, d, device=dev, dtype=dtype)
    k_new = torch.zeros(b, hkv, 1, d, device=dev, dtype=dtype)
    v_new = torch.zeros(b, hkv, 1, d, device=dev, dtype=dtype)
    lens = torch.tensor([100, 1500, 7, 2000], dtype=torch.int32, device=dev)

    # warm up on a side stream (allocator, library load), then capture
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _step(q, k_new, v_new, kc.clone(), vc.clone(), lens, cos, sin)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = _step(q, k_new, v_new, kc, vc, lens, cos, sin)

    kc_ref, vc_ref = kc.clone(), vc.clone()  # the capture itself ran nothing
    for r in range(3):
        q.copy_(torch.randn(q.shape, generator=g, device=dev).to(dtype))
        k_new.copy_(torch.randn(k_new.shape, generator=g, device=dev).to(dtype))
        v_new.copy_(torch.randn(v_new.shape, generator=g, device=dev).to(dtype))
        want = _step(q, k_new, v_new, kc_ref, vc_ref, lens, cos, sin)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r}: output differs from eager"
        assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), f"replay {r}: caches differ"
        lens.add_(1)  # next position, read by the captured kernels on the next replay
        flash_attention(q, kc_ref[:, :, :16], vc_ref[:, :, :16])  # unrelated eager work
    assert native_loaded()
