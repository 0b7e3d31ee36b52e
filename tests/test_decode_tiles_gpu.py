"""GPU tests of the decode split kernel's tile boundaries in its 64-key form.

The four-wave split kernel (groups of 33 to 64 query heads, head dim up to
128, contiguous caches) reads K/V in 64-key tiles, while a split's keys are a
multiple of 32: a split's last tile may be half empty, a split may hold fewer
keys than one tile, and with more splits than 32-key blocks some splits hold
none.  Cache lengths on both sides of the 32- and 64-key boundaries, split
counts that produce each of these cases, every head dim of that path (80 runs
on the 96 kernel with zero-padded columns) and per-row lengths including 0,
against the float64 oracle.
"""

import pytest
import torch

from stackkernels_amd._core.attention.decode import flash_decode as core_decode
from stackkernels_amd._opt.pick import pick
from stackkernels_amd.torch import flash_decode

from _gpu_util import TOL, assert_close_maxabs, make_qkv, native_loaded, np64, oracle_fwd
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

LENGTHS = (1, 31, 33, 63, 64, 65, 127, 129, 200)
SPLITS = (1, 2, 3, 7)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("group", [33, 48, 64])
@pytest.mark.parametrize("head_dim", [64, 80, 96, 128])
def test_tile_boundaries(device, dtype, group, head_dim):
    cfg = pick("flash_decode", (2, group, 1, head_dim), kv_len=200, num_kv_heads=1)
    assert cfg["num_warps"] == 4 and cfg["BLOCK_N"] == 64
    for sk in LENGTHS:
        q, k, v = make_qkv(2, group, 1, 1, sk, head_dim, dtype, seed=sk + group + head_dim)
        ref = oracle_fwd(q, k, v, False)[0]
        for ns in SPLITS:
            print(f"tile case {dtype} group={group} D={head_dim} S_k={sk} splits={ns}", flush=True)
            out = core_decode(q, k, v, num_splits=ns)
            assert_close_maxabs(out, ref, TOL[dtype], f"O (S_k={sk}, splits={ns})")
    assert native_loaded()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("head_dim", [64, 128])
def test_tile_boundaries_per_row_lengths(device, dtype, head_dim):
    lens = torch.tensor([0, 1, 31, 33, 63, 64, 65, 127, 300, 1000])
    q, k, v = make_qkv(len(lens), 64, 1, 1, 1000, head_dim, dtype, seed=head_dim)
    ref = orc.decode_varlen(np64(q), np64(k), np64(v), lens.numpy())
    out = flash_decode(q, k, v, cache_seqlens=lens)
    assert_close_maxabs(out, ref, TOL[dtype], "O")
    for ns in SPLITS:
        out = core_decode(q, k, v, num_splits=ns, cache_seqlens=lens)
        assert_close_maxabs(out, ref, TOL[dtype], f"O (splits={ns})")
    assert native_loaded()
