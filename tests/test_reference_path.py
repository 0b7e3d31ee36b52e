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


# ------------------------------------------------------- fused RoPE (CPU path)

_NP_DT = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def _tables(d, rows, dtype=torch.float32):
    from stackkernels_amd._reference.torch.rope import precompute_freqs

    return precompute_freqs(d, rows, dtype=dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("start_pos", [0, 15, 64])
def test_rope_reference_matches_oracle_bitwise(dtype, start_pos):
    from stackkernels_amd._reference.torch.rope import apply_rope_at, rope_positions

    g = torch.Generator().manual_seed(start_pos)
    x = torch.randn(2, 4, 8, 64, generator=g).to(dtype)
    cos, sin = _tables(64, start_pos + 8 + 64)
    pos = rope_positions(start_pos, 2, 8, cos.shape[0])
    got = apply_rope_at(x, cos, sin, pos).float().numpy()
    want = orc.round_to(orc.rope_rotate(x.float().numpy(), cos.numpy(), sin.numpy(),
                                        pos.numpy()), _NP_DT[dtype])
    np.testing.assert_array_equal(got, want)


def test_flash_decode_rope_reference_path():
    from stackkernels_amd.torch import kv_cache_update

    g = torch.Generator().manual_seed(7)
    b, hq, hkv, sk, d = 3, 8, 2, 40, 64
    q = torch.randn(b, hq, 1, d, generator=g)
    k = torch.randn(b, hkv, sk, d, generator=g)
    v = torch.randn(b, hkv, sk, d, generator=g)
    cos, sin = _tables(d, 128)
    lens = torch.tensor([40, 17, 1])
    pos = lens - 1
    out = flash_decode(q, k, v, cache_seqlens=lens, rope_cos=cos, rope_sin=sin, start_pos=pos)
    qr = orc.rope_rotate(q.numpy(), cos.numpy(), sin.numpy(), pos.numpy()[:, None])
    want = orc.decode_varlen(qr, k.numpy(), v.numpy(), lens.numpy())
    np.testing.assert_allclose(out.numpy(), want, rtol=0, atol=1e-5)
    # scalar start_pos, full cache
    out = flash_decode(q, k, v, rope_cos=cos, rope_sin=sin, start_pos=39)
    qr = orc.rope_rotate(q.numpy(), cos.numpy(), sin.numpy(), orc.rope_positions(39, b, 1))
    np.testing.assert_allclose(out.numpy(), orc.decode(qr, k.numpy(), v.numpy()), rtol=0, atol=1e-5)
    with pytest.raises(ValueError, match="outside the rope table"):
        flash_decode(q, k, v, rope_cos=cos, rope_sin=sin, start_pos=128)
    # paged
    page = 32
    pool_k = torch.randn(6, hkv, page, d, generator=g)
    pool_v = torch.randn(6, hkv, page, d, generator=g)
    table = torch.tensor([[0, 1], [5, 2], [3, 4]])
    out = flash_decode(q, pool_k, pool_v, cache_seqlens=lens, block_table=table, rope_cos=cos,
                       rope_sin=sin, start_pos=pos)
    qr = orc.rope_rotate(q.numpy(), cos.numpy(), sin.numpy(), pos.numpy()[:, None])
    want = orc.decode_paged(qr, pool_k.numpy(), pool_v.numpy(), table.numpy(), lens.numpy())
    np.testing.assert_allclose(out.numpy(), want, rtol=0, atol=1e-5)
    # rotated append: keys rotated at start_pos + t, values as they are
    kc = torch.zeros(b, hkv, 16, d)
    vc = torch.zeros(b, hkv, 16, d)
    kn = torch.randn(b, hkv, 3, d, generator=g)
    vn = torch.randn(b, hkv, 3, d, generator=g)
    slots = torch.tensor([[0, 1, 2], [5, 6, -1], [13, 14, 15]])
    starts = torch.tensor([0, 5, 13])
    kv_cache_update(kn, vn, kc, vc, slots, rope_cos=cos, rope_sin=sin, start_pos=starts)
    kr = orc.rope_rotate(kn.numpy(), cos.numpy(), sin.numpy(),
                         orc.rope_positions(starts.numpy(), b, 3))
    wk, wv = orc.kv_cache_update(kr, vn.numpy(), np.zeros(kc.shape, np.float32),
                                 np.zeros(vc.shape, np.float32), slots.numpy())
    np.testing.assert_array_equal(kc.numpy(), wk)
    np.testing.assert_array_equal(vc.numpy(), wv)


def test_flash_attention_rope_reference_path():
    g = torch.Generator().manual_seed(8)
    b, hq, hkv, sq, sk, d = 2, 4, 2, 6, 10, 32
    q = torch.randn(b, hq, sq, d, generator=g)
    k = torch.randn(b, hkv, sk, d, generator=g)
    v = torch.randn(b, hkv, sk, d, generator=g)
    cos, sin = _tables(d, 64)
    out = flash_attention(q, k, v, True, rope_cos=cos, rope_sin=sin, start_pos=4)
    qr = orc.rope_rotate(q.numpy(), cos.numpy(), sin.numpy(), orc.rope_positions(4, b, sq))
    want, _ = orc.attention_forward(qr, k.numpy(), v.numpy(), is_causal=True)
    np.testing.assert_allclose(out.numpy(), want, rtol=0, atol=1e-5)
    with pytest.raises(ValueError, match="RoPE tables"):
        flash_attention(q.detach(), k, v, rope_cos=cos[:, :16], rope_sin=sin[:, :16])


def test_flash_attention_rope_reference_path_backward():
    """The CPU path with fused-RoPE arguments is the unfused pipeline under autograd:
    dq = R^T (dq at the rotated q), dk and dv those of attention at the rotated q."""
    g = torch.Generator().manual_seed(9)
    b, hq, hkv, sq, sk, d = 2, 4, 2, 6, 10, 32
    q = torch.randn(b, hq, sq, d, generator=g, dtype=torch.float64).float()
    k = torch.randn(b, hkv, sk, d, generator=g).requires_grad_(True)
    v = torch.randn(b, hkv, sk, d, generator=g).requires_grad_(True)
    do = torch.randn(b, hq, sq, d, generator=g)
    cos, sin = _tables(d, 64)
    qg = q.clone().requires_grad_(True)
    flash_attention(qg, k, v, True, rope_cos=cos, rope_sin=sin, start_pos=4).backward(do)
    pos = orc.rope_positions(4, b, sq)
    qr = orc.rope_rotate(q.numpy(), cos.numpy(), sin.numpy(), pos)
    dqr, dk, dv = orc.attention_backward(qr, k.detach().numpy(), v.detach().numpy(), do.numpy(),
                                         True)
    dq = orc.rope_rotate_adjoint(dqr, cos.numpy(), sin.numpy(), pos, dtype=np.float64)
    np.testing.assert_allclose(qg.grad.numpy(), dq, rtol=0, atol=1e-4)
    np.testing.assert_allclose(k.grad.numpy(), dk, rtol=0, atol=1e-4)
    np.testing.assert_allclose(v.grad.numpy(), dv, rtol=0, atol=1e-4)
