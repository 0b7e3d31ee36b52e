"""GPU parity of the HIP split-KV decode against the oracle.

Grid follows the reference's tests/ops/test_flash_decode.py (heads x kv_len x
head dim) in fp32/fp16/bf16, plus: GQA groups up to 64 (MQA), strided caches
(no copy), explicit split counts (split-count invariance of the combine), a
tail that is not a multiple of the 32-key tile, and the two full-size
BASELINE decode configs checked against the fp32 reference path.
"""

import pytest
import torch

import stackkernels_amd
from stackkernels_amd._core.attention.decode import flash_decode as core_decode
from stackkernels_amd._core.attention.decode import plan
from stackkernels_amd._reference.torch.attention import attention_reference
from stackkernels_amd.torch import flash_decode

from _gpu_util import TOL, assert_close_maxabs, make_qkv, native_loaded, oracle_fwd

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.fixture(autouse=True)
def _auto_backend():
    original = stackkernels_amd.get_backend()
    stackkernels_amd.set_backend("auto")
    yield
    stackkernels_amd.set_backend(original)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("heads", [(8, 8), (8, 2), (8, 1)])
@pytest.mark.parametrize("kv_len", [32, 128, 512, 1024])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_decode_grid(device, dtype, heads, kv_len, head_dim):
    hq, hkv = heads
    q, k, v = make_qkv(2, hq, hkv, 1, kv_len, head_dim, dtype)
    out = flash_decode(q, k, v)
    assert native_loaded()
    ref, _ = oracle_fwd(q, k, v, False)
    assert out.dtype == dtype and out.shape == q.shape
    assert_close_maxabs(out, ref, TOL[dtype], "O")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("group", [1, 3, 4, 8, 16, 32, 64])
@pytest.mark.parametrize("head_dim", [64, 80, 96, 128, 256])
def test_decode_groups_and_head_dims(device, dtype, group, head_dim):
    q, k, v = make_qkv(2, 2 * group, 2, 1, 1000, head_dim, dtype, seed=group)
    out = flash_decode(q, k, v)
    assert_close_maxabs(out, oracle_fwd(q, k, v, False)[0], TOL[dtype], "O")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("splits", [1, 2, 3, 7, 64, 100])
def test_split_count_invariance(device, dtype, splits):
    q, k, v = make_qkv(3, 8, 2, 1, 3001, 128, dtype, seed=splits)
    out = core_decode(q, k, v, num_splits=splits)
    assert_close_maxabs(out, oracle_fwd(q, k, v, False)[0], TOL[dtype], "O")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_strided_cache_no_copy(device, dtype):
    # a cache allocated for 4096 positions, of which the first 1500 are live
    g = torch.Generator().manual_seed(5)
    kc = torch.randn(2, 4, 4096, 128, generator=g).to(dtype).to(device)
    vc = torch.randn(2, 4, 4096, 128, generator=g).to(dtype).to(device)
    q = torch.randn(2, 16, 1, 128, generator=g).to(dtype).to(device)
    k, v = kc[:, :, :1500], vc[:, :, :1500]
    out = flash_decode(q, k, v)
    assert_close_maxabs(out, oracle_fwd(q, k, v, False)[0], TOL[dtype], "O")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
def test_decode_scale_and_tail(device, dtype):
    q, k, v = make_qkv(1, 4, 1, 1, 33, 64, dtype)
    for scale in (0.3, -0.2):
        out = flash_decode(q, k, v, sm_scale=scale)
        assert_close_maxabs(out, oracle_fwd(q, k, v, False, scale)[0], TOL[dtype], "O")


def test_decode_requires_single_query(device):
    q, k, v = make_qkv(1, 4, 1, 2, 33, 64, torch.bfloat16)
    with pytest.raises(AssertionError, match="q_len == 1"):
        flash_decode(q, k, v)


def test_decode_deterministic(device):
    q, k, v = make_qkv(4, 32, 8, 1, 5000, 128, torch.bfloat16)
    assert torch.equal(flash_decode(q, k, v), flash_decode(q, k, v))


def _ref_decode_fp32(q, k, v, chunk):
    outs = []
    for b0 in range(0, q.shape[0], chunk):
        o, _ = attention_reference(q[b0:b0 + chunk].float(), k[b0:b0 + chunk].float(),
                                   v[b0:b0 + chunk].float())
        outs.append(o)
    return torch.cat(outs)


def test_config4_full_size_decode(device):
    """bf16 GQA decode B=64 Hq=32 Hkv=8 Sk=32768 D=128."""
    q, k, v = make_qkv(64, 32, 8, 1, 32768, 128, torch.bfloat16, seed=0)
    ns, _ = plan(torch.bfloat16, 64, 32, 8, 32768, 128)
    assert ns > 1
    out = flash_decode(q, k, v)
    assert_close_maxabs(out.float(), _ref_decode_fp32(q, k, v, 4), 2e-2, "O")


def test_config5_full_size_mqa_decode(device):
    """fp16 MQA B=8 Hq=64 Hkv=1 Sk=131072 D=128, V ~ U(-1, 1)."""
    g = torch.Generator().manual_seed(0)
    q = torch.randn(8, 64, 1, 128, generator=g).half().to(device)
    k = torch.randn(8, 1, 131072, 128, generator=g).half().to(device)
    v = (torch.rand(8, 1, 131072, 128, generator=g) * 2 - 1).half().to(device)
    out = flash_decode(q, k, v)
    assert_close_maxabs(out.float(), _ref_decode_fp32(q, k, v, 1), 2e-2, "O")


def test_flash_decode_op_compiled_matches_eager():
    """The decode custom op (``stackkernels::flash_decode_op``) in a compiled
    graph runs the same kernels as eager ``flash_decode``: identical bits."""
    q, k, v = make_qkv(4, 32, 8, 1, 4096, 128, torch.bfloat16, seed=3)
    lens = torch.tensor([4096, 100, 1, 2500], dtype=torch.int32, device="cuda")
    fn = torch.compile(lambda a, b, c, n: torch.ops.stackkernels.flash_decode_op(a, b, c, None, n),
                       backend="aot_eager", fullgraph=True)
    out = fn(q, k, v, lens)
    ref = flash_decode(q, k, v, cache_seqlens=lens)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert native_loaded()
