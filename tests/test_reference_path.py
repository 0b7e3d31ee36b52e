"""The CPU / reference-backend path against the oracle.

Mirrors the reference's own attention tests (tests/ops/test_flash_attn.py,
tests/ops/test_flash_decode.py): same grids, seed 42, but checked against the
float64 oracle instead of against the path itself.
"""

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd
from stackkernels_amd._reference.torch.attention import attention_reference, repeat_kv
from stackkernels_amd.torch import FlashAttention, flash_attention, flash_decode


def _np(t):
    return t.detach().double().numpy()


@pytest.mark.parametrize("heads", [(8, 8), (8, 2), (8, 1)])
@pytest.mark.parametrize("seq_lens", [(32, 32), (16, 64), (64, 32)])
@pytest.mark.parametrize("head_dim", [64, 80, 96, 128, 256])
@pytest.mark.parametrize("is_causal", [False, True])
def test_forward_grid(heads, seq_lens, head_dim, is_causal):
    torch.manual_seed(42)
    hq, hkv = heads
    sq, sk = seq_lens
    q = torch.randn(2, hq, sq, head_dim)
    k = torch.randn(2, hkv, sk, head_dim)
    v = torch.randn(2, hkv, sk, head_dim)
    out = flash_attention(q, k, v, is_causal=is_causal)
    ref, ref_lse = orc.attention_forward(_np(q), _np(k), _np(v), is_causal)
    np.testing.assert_allclose(_np(out), ref, atol=1e-5, rtol=0)
    _, lse = attention_reference(q, k, v, is_causal=is_causal)
    fin = np.isfinite(ref_lse)
    np.testing.assert_array_equal(np.isneginf(_np(lse)), ~fin)
    np.testing.assert_allclose(_np(lse)[fin], ref_lse[fin], atol=1e-5)


@pytest.mark.parametrize("heads", [(4, 4), (4, 2), (4, 1)])
@pytest.mark.parametrize("is_causal", [False, True])
def test_backward_grid(heads, is_causal):
    torch.manual_seed(42)
    hq, hkv = heads
    q = torch.randn(2, hq, 16, 64, requires_grad=True)
    k = torch.randn(2, hkv, 16, 64, requires_grad=True)
    v = torch.randn(2, hkv, 16, 64, requires_grad=True)
    out = flash_attention(q, k, v, is_causal=is_causal)
    g = torch.randn_like(out)
    out.backward(g)
    dq, dk, dv = orc.attention_backward(_np(q), _np(k), _np(v), _np(g), is_causal)
    np.testing.assert_allclose(_np(q.grad), dq, atol=1e-5)
    np.testing.assert_allclose(_np(k.grad), dk, atol=1e-5)
    np.testing.assert_allclose(_np(v.grad), dv, atol=1e-5)


@pytest.mark.parametrize("heads", [(8, 8), (8, 2), (8, 1)])
@pytest.mark.parametrize("kv_len", [32, 128, 512, 1024])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_decode_grid(heads, kv_len, head_dim):
    torch.manual_seed(42)
    hq, hkv = heads
    q = torch.randn(2, hq, 1, head_dim)
    k = torch.randn(2, hkv, kv_len, head_dim)
    v = torch.randn(2, hkv, kv_len, head_dim)
    out = flash_decode(q, k, v)
    np.testing.assert_allclose(_np(out), orc.decode(_np(q), _np(k), _np(v)), atol=1e-5)


def test_module_and_custom_op():
    torch.manual_seed(42)
    q, k, v = torch.randn(1, 4, 16, 64), torch.randn(1, 2, 16, 64), torch.randn(1, 2, 16, 64)
    out = FlashAttention(is_causal=True)(q, k, v)
    assert out.shape == q.shape and not torch.isnan(out).any()
    op = torch.ops.stackkernels.flash_attn_op(q, k, v, True, None)
    torch.testing.assert_close(op, out)


def test_fully_masked_rows_reference_path():
    q, k, v = torch.randn(1, 2, 6, 8), torch.randn(1, 1, 2, 8), torch.randn(1, 1, 2, 8)
    out, lse = attention_reference(q, k, v, is_causal=True)
    assert torch.all(out[:, :, :4] == 0) and torch.all(torch.isneginf(lse[:, :, :4]))


def test_repeat_kv():
    x = torch.arange(6.0).reshape(1, 2, 3, 1)
    r = repeat_kv(x, 2)
    assert r.shape == (1, 4, 3, 1)
    assert torch.equal(r[:, 0], x[:, 0]) and torch.equal(r[:, 1], x[:, 0]) and torch.equal(r[:, 2], x[:, 1])


@pytest.mark.parametrize("shapes,msg", [
    (((2, 4, 8, 64), (2, 3, 8, 64), (2, 3, 8, 64)), "divisible"),
    (((2, 4, 8, 64), (1, 4, 8, 64), (1, 4, 8, 64)), "Batch mismatch"),
    (((2, 4, 8, 64), (2, 4, 8, 32), (2, 4, 8, 32)), "Head dimension mismatch"),
    (((2, 4, 8, 64), (2, 4, 8, 64), (2, 2, 8, 64)), "K and V head count mismatch"),
    (((2, 4, 8, 64), (2, 4, 8, 64), (2, 4, 9, 64)), "K and V sequence length mismatch"),
    (((4, 8, 64), (2, 4, 8, 64), (2, 4, 8, 64)), "Expected 4D"),
])
def test_launcher_rejects_bad_layouts(shapes, msg):
    q, k, v = (torch.zeros(s) for s in shapes)
    with pytest.raises(ValueError, match=msg):
        flash_attn_fwd(q, k, v)


def test_decode_varlen_reference_path():
    torch.manual_seed(3)
    q, k, v = torch.randn(4, 8, 1, 32), torch.randn(4, 2, 40, 32), torch.randn(4, 2, 40, 32)
    lens = torch.tensor([0, 1, 17, 99])
    out = flash_decode(q, k, v, cache_seqlens=lens)
    np.testing.assert_allclose(_np(out), orc.decode_varlen(_np(q), _np(k), _np(v), lens.numpy()),
                               atol=1e-5)
    with pytest.raises(ValueError, match="cache_seqlens"):
        flash_decode(q, k, v, cache_seqlens=torch.tensor([1, 2]))


def test_kv_cache_update_reference_path():
    from stackkernels_amd.torch import kv_cache_update

    torch.manual_seed(4)
    k, v = torch.randn(2, 3, 4, 16), torch.randn(2, 3, 4, 16)
    kc, vc = torch.randn(2, 3, 10, 16), torch.randn(2, 3, 10, 16)
    slots = torch.tensor([[2, -1, 9, 0], [5, 6, 30, 1]])
    ek, ev = orc.kv_cache_update(_np(k), _np(v), _np(kc), _np(vc), slots.numpy())
    kv_cache_update(k, v, kc, vc, slots)
    assert np.array_equal(_np(kc), ek) and np.array_equal(_np(vc), ev)
    with pytest.raises(ValueError, match="slot_indices"):
        kv_cache_update(k, v, kc, vc, slots[:1])


def test_decode_paged_and_cache_update_paged_reference_path():
    from stackkernels_amd.torch import kv_cache_update

    torch.manual_seed(5)
    q = torch.randn(2, 4, 1, 16)
    kp, vp = torch.randn(6, 2, 32, 16), torch.randn(6, 2, 32, 16)
    table = torch.tensor([[5, 0, 2], [1, -1, 4]])
    lens = torch.tensor([70, 96])
    out = flash_decode(q, kp, vp, cache_seqlens=lens, block_table=table)
    ref = orc.decode_paged(_np(q), _np(kp), _np(vp), table.numpy(), lens.numpy())
    np.testing.assert_allclose(_np(out), ref, atol=1e-5)
    k, v = torch.randn(2, 2, 3, 16), torch.randn(2, 2, 3, 16)
    slots = torch.tensor([[0, 33, -1], [191, 64, 500]])
    ek, ev = orc.kv_cache_update_paged(_np(k), _np(v), _np(kp), _np(vp), slots.numpy())
    kv_cache_update(k, v, kp, vp, slots, paged=True)
    assert np.array_equal(_np(kp), ek) and np.array_equal(_np(vp), ev)
