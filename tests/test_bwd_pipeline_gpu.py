"""GPU parity of the backward's software pipelines at every short trip count.

The dK/dV kernel at D = 64 and 128 runs a 6-deep ring with S computed one query tile
ahead and a step's first operands read before its barrier; the dQ kernel at
D <= 128 computes S^T one key tile ahead with the last tile peeled out of a
loop unrolled by the ring depth.  Their prologues, wait counts and tails
depend on how many tiles a workgroup walks, so this walks 1 to 9 query tiles
(32 queries each, times the GQA group) and 1 to 9 key tiles (32 keys each),
with and without the causal mask, against the float64 oracle at the stated
2e-2 max-abs bound.
"""

import pytest
import torch

import stackkernels_amd
from stackkernels_amd.torch import flash_attention

from _gpu_util import TOL, assert_close_maxabs, make_qkv, native_loaded, np64

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _auto_backend():
    original = stackkernels_amd.get_backend()
    stackkernels_amd.set_backend("auto")
    yield
    stackkernels_amd.set_backend(original)


def _check(b, hq, hkv, sq, sk, d, dtype, causal, seed):
    from oracle import attention_oracle as orc

    q, k, v = make_qkv(b, hq, hkv, sq, sk, d, dtype, seed=seed)
    for t in (q, k, v):
        t.requires_grad_(True)
    out = flash_attention(q, k, v, is_causal=causal)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed + 1)).to(dtype)
    out.backward(g.to(out.device))
    assert native_loaded()
    dq, dk, dv = orc.attention_backward(np64(q), np64(k), np64(v), np64(g), causal, None)
    what = f"(sq={sq}, sk={sk}, hq={hq}, hkv={hkv}, causal={causal})"
    assert_close_maxabs(q.grad, dq, TOL[dtype], "dQ " + what)
    assert_close_maxabs(k.grad, dk, TOL[dtype], "dK " + what)
    assert_close_maxabs(v.grad, dv, TOL[dtype], "dV " + what)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", list(range(1, 10)))
def test_dkv_query_tile_counts(n, causal):
    # one KV head with a group of 1: the dK/dV workgroup walks n query tiles
    _check(1, 2, 2, 32 * n, 128, 128, torch.bfloat16, causal, seed=100 + n)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", list(range(1, 10)))
def test_dkv_query_tile_counts_d64(n, causal):
    # the same 6-deep schedule at D = 64
    _check(1, 2, 2, 32 * n, 128, 64, torch.float16, causal, seed=150 + n)


@pytest.mark.parametrize("n", [1, 2, 3, 5])
def test_dkv_query_tiles_across_group_heads(n):
    # a group of 4: the walk continues over the group's query heads
    _check(1, 8, 2, 32 * n, 160, 128, torch.float16, True, seed=200 + n)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("n", list(range(1, 10)))
def test_dq_key_tile_counts(n, causal):
    # the dQ workgroup walks n key tiles (the last one peeled)
    _check(1, 2, 1, 96, 32 * n, 128, torch.bfloat16, causal, seed=300 + n)


@pytest.mark.parametrize("n", [1, 2, 4, 7])
def test_dq_key_tile_counts_d64(n):
    _check(2, 4, 2, 64, 32 * n + 17, 64, torch.float16, False, seed=400 + n)
