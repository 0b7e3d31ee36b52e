"""GPU tests that no kernel reads memory its call does not cover.

Every element a call must not see is NaN: cache slots at or past a row's
``cache_seqlens``, rows past S_k / S_q and head-dim columns past D of views
into larger buffers, the tail of a row's last page, and every pool page its
block table does not reach.  A kernel that loads such an element, even for a
key it then masks, turns the output into NaN (0 * NaN in the output product)
or moves it off the oracle's value, so each result must be finite and equal
to the float64 oracle over the visible keys only, within the usual bounds.
The reference's kernels mask these loads the same way
(src/stackkernels/_core/attention/decode.py:15-121,
src/stackkernels/_core/attention/flash_fwd.py:101-153).
"""

import numpy as np
import pytest
import torch

from stackkernels_amd._core.attention.decode import flash_decode as core_decode
from stackkernels_amd.torch import flash_attention, flash_decode

from _bwd_bound import check_backward, rounding_mass
from _gpu_util import TOL, assert_close_maxabs, assert_lse_close, native_loaded, np64
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu
NAN = float("nan")


def _randn(shape, dtype, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


def _poisoned_cache(b, hkv, s_alloc, d, lens, dtype, seed):
    """(b, hkv, s_alloc, d) caches: random values in the first lens[r] slots of
    row r, NaN in every other slot."""
    k, v = _randn((b, hkv, s_alloc, d), dtype, seed), _randn((b, hkv, s_alloc, d), dtype, seed + 1)
    for r, n in enumerate(lens):
        k[r, :, n:] = NAN
        v[r, :, n:] = NAN
    return k.cuda(), v.cuda()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("group", [1, 4, 16, 64])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_decode_varlen_ignores_slots_past_length(device, dtype, group, d):
    """Per-row lengths on both sides of the 32- and 64-key tile edges, 0 and the full
    cache; the slots at and past each length are NaN."""
    lens = [0, 1, 31, 33, 64, 65, 127, 300, 511, 512]
    b, hkv, s_alloc = len(lens), 2, 512
    k, v = _poisoned_cache(b, hkv, s_alloc, d, lens, dtype, seed=group + d)
    q = _randn((b, hkv * group, 1, d), dtype, seed=d).cuda()
    lt = torch.tensor(lens, dtype=torch.int32)
    ref = orc.decode_varlen(np64(q), np64(k), np64(v), lt.numpy())
    out = flash_decode(q, k, v, cache_seqlens=lt.cuda())
    torch.cuda.synchronize()
    assert native_loaded()
    assert_close_maxabs(out, ref, TOL[dtype], "O")
    assert torch.all(out[0] == 0)
    for ns in (1, 3, 16):
        out = core_decode(q, k, v, num_splits=ns, cache_seqlens=lt.cuda())
        assert_close_maxabs(out, ref, TOL[dtype], f"O (splits={ns})")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("group", [1, 8, 48])
@pytest.mark.parametrize("sk,d", [(200, 128), (1000, 64), (333, 80)])
def test_decode_view_ignores_rows_and_columns_past_the_view(device, dtype, group, sk, d):
    """K/V are [..., :sk, :d] views of NaN-padded buffers (64 more rows, 16 or 32 more
    columns), so the view's rows are not contiguous and the padding sits right after
    each row and after the last row."""
    b, hkv = 3, 2
    dpad = d + (16 if d % 32 else 32)
    kb = torch.full((b, hkv, sk + 64, dpad), NAN, dtype=dtype)
    vb = torch.full((b, hkv, sk + 64, dpad), NAN, dtype=dtype)
    kb[:, :, :sk, :d] = _randn((b, hkv, sk, d), dtype, seed=sk)
    vb[:, :, :sk, :d] = _randn((b, hkv, sk, d), dtype, seed=sk + 1)
    kb, vb = kb.cuda(), vb.cuda()
    k, v = kb[:, :, :sk, :d], vb[:, :, :sk, :d]
    q = _randn((b, hkv * group, 1, d), dtype, seed=group).cuda()
    ref = orc.decode(np64(q), np64(k), np64(v))
    out = flash_decode(q, k, v)
    torch.cuda.synchronize()
    assert_close_maxabs(out, ref, TOL[dtype], "O")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("group", [1, 4, 64])
@pytest.mark.parametrize("ps", [32, 64, 128])
def test_decode_paged_ignores_unreferenced_pages_and_page_tails(device, dtype, group, ps):
    """A pool that is NaN everywhere except the slots the rows' tables and lengths
    reach.  Each table is full length (its unused entries name NaN pages), one entry
    inside a row's length is -1 (those keys are masked, the kernel reads nothing)."""
    b, hkv, d, max_pages = 6, 2, 128, 5
    pages = b * max_pages + 4
    lens = [0, 1, ps - 1, ps + 1, 3 * ps + 7, max_pages * ps]
    table = torch.randperm(pages, generator=torch.Generator().manual_seed(ps))[: b * max_pages]
    table = table.view(b, max_pages).to(torch.int32)
    table[4, 1] = -1
    kp = torch.full((pages, hkv, ps, d), NAN, dtype=dtype)
    vp = torch.full((pages, hkv, ps, d), NAN, dtype=dtype)
    vals_k = _randn((b, hkv, max_pages * ps, d), dtype, seed=group)
    vals_v = _randn((b, hkv, max_pages * ps, d), dtype, seed=group + 1)
    for r, n in enumerate(lens):
        for j in range(max_pages):
            pg, lo = int(table[r, j]), j * ps
            if pg < 0 or lo >= n:
                continue
            m = min(ps, n - lo)
            kp[pg, :, :m] = vals_k[r, :, lo:lo + m]
            vp[pg, :, :m] = vals_v[r, :, lo:lo + m]
    kp, vp = kp.cuda(), vp.cuda()
    q = _randn((b, hkv * group, 1, d), dtype, seed=ps).cuda()
    lt = torch.tensor(lens, dtype=torch.int32)
    ref = orc.decode_paged(np64(q), np64(kp), np64(vp), table.numpy(), lt.numpy())
    out = flash_decode(q, kp, vp, cache_seqlens=lt.cuda(), block_table=table.cuda())
    torch.cuda.synchronize()
    assert native_loaded()
    assert_close_maxabs(out, ref, TOL[dtype], "O")
    assert torch.all(out[0] == 0)


def _padded_views(b, h, s, d, dtype, seed, extra_rows, extra_cols):
    """A (b, h, s, d) view of a NaN-filled (b, h, s + extra_rows, d + extra_cols) buffer."""
    buf = torch.full((b, h, s + extra_rows, d + extra_cols), NAN, dtype=dtype)
    buf[:, :, :s, :d] = _randn((b, h, s, d), dtype, seed)
    buf = buf.cuda()
    return buf[:, :, :s, :d]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk,d", [(100, 130, 128), (257, 191, 64), (70, 300, 80), (129, 65, 256)])
def test_forward_ignores_rows_and_columns_past_views(device, dtype, causal, sq, sk, d):
    """Q, K and V as views whose rows and columns past S_q / S_k and D are NaN (ragged
    lengths that end inside a 64-key tile and a 128-row block)."""
    b, hq, hkv = 2, 4, 2
    q = _padded_views(b, hq, sq, d, dtype, 1, 40, 16)
    k = _padded_views(b, hkv, sk, d, dtype, 2, 70, 16)
    v = _padded_views(b, hkv, sk, d, dtype, 3, 70, 16)
    out = flash_attention(q, k, v, is_causal=causal)
    torch.cuda.synchronize()
    assert native_loaded()
    ro, _ = orc.attention_forward(np64(q), np64(k), np64(v), causal)
    assert_close_maxabs(out, ro, TOL[dtype], "O")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sq,sk,d", [(100, 130, 128), (257, 191, 64), (70, 300, 96)])
def test_backward_ignores_rows_and_columns_past_views(device, dtype, causal, sq, sk, d):
    """The same views through autograd: O and every gradient finite and within the
    rounding bound of the oracle's (NaN in dO's padding too)."""
    b, hq, hkv = 2, 4, 2
    q = _padded_views(b, hq, sq, d, dtype, 1, 40, 16).requires_grad_(True)
    k = _padded_views(b, hkv, sk, d, dtype, 2, 70, 16).requires_grad_(True)
    v = _padded_views(b, hkv, sk, d, dtype, 3, 70, 16).requires_grad_(True)
    do = _padded_views(b, hq, sq, d, dtype, 4, 40, 16)
    out = flash_attention(q, k, v, is_causal=causal)
    out.backward(do)
    torch.cuda.synchronize()
    exact = orc.attention_backward(np64(q), np64(k), np64(v), np64(do), causal)
    ro, _ = orc.attention_forward(np64(q), np64(k), np64(v), causal)
    assert_close_maxabs(out, ro, TOL[dtype], "O")
    dt = "bf16" if dtype == torch.bfloat16 else "f16"
    mass = rounding_mass(np64(q), np64(k), np64(v), np64(do), causal, None, dt)
    from stackkernels_amd._reference.torch.attention import attention_reference

    qr, kr, vr = (t.detach().cpu().float().requires_grad_(True) for t in (q, k, v))
    ref, _ = attention_reference(qr, kr, vr, is_causal=causal)
    ref.backward(do.cpu().float())
    path = [np64(t.grad.to(dtype)) for t in (qr, kr, vr)]
    for i, (name, t) in enumerate((("dQ", q), ("dK", k), ("dV", v))):
        got = np64(t.grad)
        assert np.isfinite(got).all(), f"{name}: non-finite values"
        check_backward(got, path[i], exact[i], mass[i], dt, name)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
def test_forward_lse_with_poisoned_tail(device, dtype):
    """The launcher's LSE as well, on a causal shape whose last key tile and query block
    are both partial."""
    from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd

    q = _padded_views(1, 2, 150, 128, dtype, 5, 30, 16)
    k = _padded_views(1, 2, 170, 128, dtype, 6, 30, 16)
    v = _padded_views(1, 2, 170, 128, dtype, 7, 30, 16)
    out, lse = flash_attn_fwd(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    ro, rl = orc.attention_forward(np64(q), np64(k), np64(v), True)
    assert_close_maxabs(out, ro, TOL[dtype], "O")
    assert_lse_close(lse, rl)
