"""GPU parity of decode with per-row cache lengths (``flash_decode(...,
cache_seqlens=...)``, C ABI ``sk_decode_varlen``) against the oracle's
``decode_varlen``, and of the KV-cache append (``kv_cache_update``, C ABI
``sk_kv_cache_update``) against the oracle's ``kv_cache_update``.

Decode: every dtype, GQA groups 1-64 (both split kernels), head dims 64-256,
lengths 0, 1, ragged, full and over-long (clamped), explicit split counts,
strided caches; the C4 cache shape with random lengths.  Tolerances as for
decode: max-abs 1e-4 (fp32), 2e-2 (fp16/bf16).  Cache update: bit-exact
(it copies bytes), for unaligned head dims too, with padded (-1) and
out-of-range slots, strided caches, and the C4 cache appending one token per
row.
"""

import numpy as np
import pytest
import torch

import stackkernels_amd
from stackkernels_amd._core.attention.decode import flash_decode as core_decode
from stackkernels_amd.torch import flash_decode, kv_cache_update

from _gpu_util import TOL, assert_close_maxabs, make_qkv, native_loaded, np64
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


@pytest.fixture(autouse=True)
def _auto_backend():
    original = stackkernels_amd.get_backend()
    stackkernels_amd.set_backend("auto")
    yield
    stackkernels_amd.set_backend(original)


def _device_qkv(b, hq, hkv, sk, d, dtype, seed, device):
    """Full-size inputs generated on the device (seeded): N(0,1) cast to dtype."""
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(b, hq, 1, d, generator=g, device=device).to(dtype)
    k = torch.randn(b, hkv, sk, d, generator=g, device=device).to(dtype)
    v = torch.randn(b, hkv, sk, d, generator=g, device=device).to(dtype)
    return q, k, v


def _lens(b, sk, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(0, sk + 1, (b,), generator=g)
    lens[0] = 0
    if b > 1:
        lens[1] = sk
    if b > 2:
        lens[2] = 1
    if b > 3:
        lens[3] = sk + 77  # clamped to the capacity
    return lens


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("group", [1, 4, 8, 16, 32, 64])
@pytest.mark.parametrize("sk", [1, 300, 2049])
def test_decode_varlen_groups(device, dtype, group, sk):
    b = 6
    q, k, v = make_qkv(b, 2 * group, 2, 1, sk, 128, dtype, seed=group * 10 + sk)
    lens = _lens(b, sk, seed=sk)
    out = flash_decode(q, k, v, cache_seqlens=lens.to(q.device))
    assert native_loaded()
    ref = orc.decode_varlen(np64(q), np64(k), np64(v), lens.numpy())
    assert out.dtype == dtype and out.shape == q.shape
    assert_close_maxabs(out, ref, TOL[dtype], "O")
    assert torch.all(out[0] == 0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("head_dim", [64, 80, 96, 256])
@pytest.mark.parametrize("group", [4, 64])
def test_decode_varlen_head_dims(device, dtype, head_dim, group):
    q, k, v = make_qkv(5, group, 1, 1, 1500, head_dim, dtype, seed=head_dim)
    lens = _lens(5, 1500, seed=head_dim)
    out = flash_decode(q, k, v, cache_seqlens=lens)  # host tensor, int64: converted
    ref = orc.decode_varlen(np64(q), np64(k), np64(v), lens.numpy())
    assert_close_maxabs(out, ref, TOL[dtype], "O")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=str)
@pytest.mark.parametrize("splits", [1, 2, 7, 64])
def test_decode_varlen_split_counts(device, dtype, splits):
    q, k, v = make_qkv(4, 8, 2, 1, 3001, 128, dtype, seed=splits)
    lens = torch.tensor([3001, 17, 0, 2500], dtype=torch.int32)
    out = core_decode(q, k, v, num_splits=splits, cache_seqlens=lens.to(q.device))
    ref = orc.decode_varlen(np64(q), np64(k), np64(v), lens.numpy())
    assert_close_maxabs(out, ref, TOL[dtype], "O")


@pytest.mark.parametrize("b", [65, 130, 256, 300])
@pytest.mark.parametrize("group", [4, 64])
def test_decode_varlen_many_rows(device, b, group):
    """Many batch rows with repeated lengths: rows are handed to workgroups
    longest first (ranked in the kernel, ties by row) up to B = 256, in grid
    order above; every row must land in its own output slot either way."""
    sk = 320
    q, k, v = make_qkv(b, group, 1, 1, sk, 64, torch.bfloat16, seed=b + group)
    g = torch.Generator().manual_seed(b)
    lens = torch.randint(0, sk + 40, (b,), generator=g, dtype=torch.int32)
    lens[::7] = 100  # ties
    out = flash_decode(q, k, v, cache_seqlens=lens.to(q.device))
    ref = orc.decode_varlen(np64(q), np64(k), np64(v), lens.numpy())
    assert_close_maxabs(out, ref, TOL[torch.bfloat16], "O")


def test_decode_varlen_full_lengths_equal_decode(device):
    q, k, v = make_qkv(3, 16, 4, 1, 1234, 128, torch.bfloat16, seed=3)
    full = torch.full((3,), 1234, dtype=torch.int32, device=q.device)
    torch.testing.assert_close(flash_decode(q, k, v, cache_seqlens=full), flash_decode(q, k, v),
                               rtol=0, atol=0)


def test_decode_varlen_strided_cache(device):
    dt = torch.bfloat16
    g = torch.Generator().manual_seed(11)
    kb = torch.randn(3, 900, 2, 128, generator=g).to(dt).to(device)  # BSHD cache, read in place
    vb = torch.randn(3, 900, 2, 128, generator=g).to(dt).to(device)
    k, v = kb.transpose(1, 2), vb.transpose(1, 2)
    q = torch.randn(3, 8, 1, 128, generator=g).to(dt).to(device)
    lens = torch.tensor([900, 450, 3], dtype=torch.int32, device=device)
    out = flash_decode(q, k, v, cache_seqlens=lens)
    ref = orc.decode_varlen(np64(q), np64(k), np64(v), lens.cpu().numpy())
    assert_close_maxabs(out, ref, TOL[dt], "O")


def test_decode_varlen_bad_lengths_shape(device):
    q, k, v = make_qkv(2, 4, 2, 1, 64, 64, torch.bfloat16)
    with pytest.raises(ValueError, match="cache_seqlens"):
        flash_decode(q, k, v, cache_seqlens=torch.tensor([1, 2, 3], device=q.device))


def test_config4_cache_shape_varlen(device):
    """The C4 cache (B=64, Hq=32, Hkv=8, S_k=32768, D=128, bf16) with random lengths;
    four rows checked against the oracle in float64."""
    dt = torch.bfloat16
    q, k, v = _device_qkv(64, 32, 8, 32768, 128, dt, 0, device)
    lens = _lens(64, 32768, seed=4)
    out = flash_decode(q, k, v, cache_seqlens=lens.to(q.device))
    torch.cuda.synchronize()
    assert torch.all(out[0] == 0)
    for b in (1, 2, 3, 40):
        ref = orc.decode_varlen(np64(q[b:b + 1]), np64(k[b:b + 1]), np64(v[b:b + 1]),
                                lens[b:b + 1].numpy())
        assert_close_maxabs(out[b:b + 1], ref, TOL[dt], f"O row {b}")


# ---- KV-cache append ----------------------------------------------------------

def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16 if t.element_size() == 2 else torch.int32)


def _slots(b, t, s, seed):
    rng = np.random.default_rng(seed)
    sl = np.stack([rng.permutation(s)[:t] for _ in range(b)]).astype(np.int64)
    if t > 1:
        sl[0, 0] = -1        # padding
        sl[-1, -1] = s + 5   # out of range: skipped
    return torch.from_numpy(sl)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("d", [3, 4, 12, 64, 80, 128, 256])
def test_kv_cache_update_exact(device, dtype, d):
    b, h, t, s = 3, 4, 7, 50
    g = torch.Generator().manual_seed(d)
    k = torch.randn(b, h, t, d, generator=g).to(dtype)
    v = torch.randn(b, h, t, d, generator=g).to(dtype)
    kc = torch.randn(b, h, s, d, generator=g).to(dtype)
    vc = torch.randn(b, h, s, d, generator=g).to(dtype)
    sl = _slots(b, t, s, seed=d)
    ek, ev = orc.kv_cache_update(_bits(k).numpy(), _bits(v).numpy(), _bits(kc).numpy(),
                                 _bits(vc).numpy(), sl.numpy())
    kd, vd, kcd, vcd = (x.to(device) for x in (k, v, kc, vc))
    kv_cache_update(kd, vd, kcd, vcd, sl.to(device))
    assert native_loaded()
    assert np.array_equal(_bits(kcd).numpy(), ek) and np.array_equal(_bits(vcd).numpy(), ev)


def test_kv_cache_update_strided(device):
    """Caches allocated (B, S, H, D) and viewed as (B, H, S, D); new tokens as a
    transposed view; int32 slots on the host."""
    dt = torch.bfloat16
    b, h, t, s, d = 2, 8, 5, 64, 128
    g = torch.Generator().manual_seed(5)
    kc = torch.randn(b, s, h, d, generator=g).to(dt).to(device).transpose(1, 2)
    vc = torch.randn(b, s, h, d, generator=g).to(dt).to(device).transpose(1, 2)
    k = torch.randn(b, t, h, d, generator=g).to(dt).to(device).transpose(1, 2)
    v = torch.randn(b, t, h, d, generator=g).to(dt).to(device).transpose(1, 2)
    sl = _slots(b, t, s, seed=6).to(torch.int32)
    ek, ev = orc.kv_cache_update(_bits(k).numpy(), _bits(v).numpy(), _bits(kc).numpy(),
                                 _bits(vc).numpy(), sl.numpy())
    kv_cache_update(k, v, kc, vc, sl)
    assert np.array_equal(_bits(kc).numpy(), ek) and np.array_equal(_bits(vc).numpy(), ev)


def test_kv_cache_update_empty_and_errors(device):
    dt = torch.float16
    kc = torch.zeros(2, 2, 8, 64, dtype=dt, device=device)
    vc = torch.zeros_like(kc)
    k0 = torch.zeros(2, 2, 0, 64, dtype=dt, device=device)
    kv_cache_update(k0, k0, kc, vc, torch.zeros(2, 0, dtype=torch.int64, device=device))
    assert torch.all(kc == 0)
    k = torch.ones(2, 2, 1, 64, dtype=dt, device=device)
    with pytest.raises(ValueError, match="slot_indices"):
        kv_cache_update(k, k, kc, vc, torch.zeros(3, 1, dtype=torch.int64, device=device))
    with pytest.raises(ValueError, match="does not match"):
        kv_cache_update(torch.ones(2, 3, 1, 64, dtype=dt, device=device),
                        torch.ones(2, 3, 1, 64, dtype=dt, device=device), kc, vc,
                        torch.zeros(2, 1, dtype=torch.int64, device=device))


def test_config4_cache_append_one_token(device):
    """Append one token per row into the C4 cache (B=64, Hkv=8, S=32768, D=128, bf16)
    at each row's length, then decode with lengths + 1: the appended key/value
    rows are exactly the inputs and the decode sees them."""
    dt = torch.bfloat16
    b, hkv, s, d = 64, 8, 32768, 128
    q, kc, vc = _device_qkv(b, 32, hkv, s, d, dt, 1, device)
    g = torch.Generator().manual_seed(2)
    k = torch.randn(b, hkv, 1, d, generator=g).to(dt).to(device)
    v = torch.randn(b, hkv, 1, d, generator=g).to(dt).to(device)
    lens = torch.randint(0, s, (b,), generator=g)
    before = kc[5, :, 100].clone()
    kv_cache_update(k, v, kc, vc, lens.view(b, 1).to(device))
    rows = torch.arange(b, device=device)
    assert torch.equal(kc[rows, :, lens.to(device)], k[:, :, 0])
    assert torch.equal(vc[rows, :, lens.to(device)], v[:, :, 0])
    if int(lens[5]) != 100:
        assert torch.equal(kc[5, :, 100], before)
    out = flash_decode(q, kc, vc, cache_seqlens=(lens + 1).to(device))
    for r in (0, 9):
        ref = orc.decode_varlen(np64(q[r:r + 1]), np64(kc[r:r + 1]), np64(vc[r:r + 1]),
                                (lens[r:r + 1] + 1).numpy())
        assert_close_maxabs(out[r:r + 1], ref, TOL[dt], f"O row {r}")


# ---- paged pools ----------------------------------------------------------------

def _pool(pages, hkv, ps, d, dtype, seed, device):
    g = torch.Generator().manual_seed(seed)
    kp = torch.randn(pages, hkv, ps, d, generator=g).to(dtype).to(device)
    vp = torch.randn(pages, hkv, ps, d, generator=g).to(dtype).to(device)
    return kp, vp


def _table(b, pages, max_pages, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.stack([torch.randperm(pages, generator=g)[:max_pages] for _ in range(b)]).to(torch.int32)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("group", [1, 4, 16, 32, 64])
@pytest.mark.parametrize("ps", [32, 64, 256])
def test_decode_paged(device, dtype, group, ps):
    b, hkv, d, max_pages = 5, 2, 128, 6
    pages = b * max_pages + 3
    kp, vp = _pool(pages, hkv, ps, d, dtype, seed=ps + group, device=device)
    q = torch.randn(b, hkv * group, 1, d, generator=torch.Generator().manual_seed(group)).to(dtype).to(device)
    table = _table(b, pages, max_pages, seed=ps)
    table[2, 1] = -1          # outside the pool: those keys are masked
    table[3, 0] = pages + 4
    lens = torch.tensor([0, max_pages * ps, max_pages * ps - 5, 3 * ps + 7, max_pages * ps + 50])
    out = flash_decode(q, kp, vp, cache_seqlens=lens.to(device), block_table=table.to(device))
    assert native_loaded()
    ref = orc.decode_paged(np64(q), np64(kp), np64(vp), table.numpy(), lens.numpy())
    assert out.shape == q.shape and out.dtype == dtype
    assert_close_maxabs(out, ref, TOL[dtype], "O")
    assert torch.all(out[0] == 0)


def test_decode_paged_bshd_pool_and_split_counts(device):
    """A pool allocated (pages, page_size, H_kv, D) and viewed as (pages, H_kv, page_size, D)."""
    dt = torch.bfloat16
    b, hkv, ps, d, max_pages = 4, 4, 64, 128, 8
    pages = 40
    g = torch.Generator().manual_seed(9)
    kp = torch.randn(pages, ps, hkv, d, generator=g).to(dt).to(device).transpose(1, 2)
    vp = torch.randn(pages, ps, hkv, d, generator=g).to(dt).to(device).transpose(1, 2)
    q = torch.randn(b, 16, 1, d, generator=g).to(dt).to(device)
    table = _table(b, pages, max_pages, seed=10)
    lens = torch.tensor([512, 100, 1, 300], dtype=torch.int32)
    ref = orc.decode_paged(np64(q), np64(kp), np64(vp), table.numpy(), lens.numpy())
    from stackkernels_amd._core.attention.decode import flash_decode_paged

    for ns in (None, 1, 3, 16):
        out = flash_decode_paged(q, kp, vp, table.to(device), lens.to(device), num_splits=ns)
        assert_close_maxabs(out, ref, TOL[dt], f"O splits={ns}")


def test_decode_paged_errors(device):
    dt = torch.float16
    kp, vp = _pool(4, 2, 48, 64, dt, seed=1, device=device)  # page_size 48: not a multiple of 32
    q = torch.zeros(1, 2, 1, 64, dtype=dt, device=device)
    with pytest.raises(ValueError, match="multiple of 32"):
        flash_decode(q, kp, vp, cache_seqlens=torch.tensor([10]), block_table=torch.tensor([[0]]))
    kp, vp = _pool(4, 2, 64, 64, dt, seed=1, device=device)
    with pytest.raises(ValueError, match="cache_seqlens"):
        flash_decode(q, kp, vp, block_table=torch.tensor([[0]], device=device))


def test_config4_paged_pool(device):
    """The C4 decode shape (B=64, Hq=32, Hkv=8, D=128, bf16) over a paged pool of 64-key
    pages (512 pages per row, shuffled), random lengths; four rows against the oracle."""
    dt = torch.bfloat16
    b, hkv, ps, d, max_pages = 64, 8, 64, 128, 512
    pages = b * max_pages
    gd = torch.Generator(device=device).manual_seed(3)
    kp = torch.randn(pages, hkv, ps, d, generator=gd, device=device).to(dt)
    vp = torch.randn(pages, hkv, ps, d, generator=gd, device=device).to(dt)
    q = torch.randn(b, 32, 1, d, generator=gd, device=device).to(dt)
    table = torch.randperm(pages, generator=torch.Generator().manual_seed(4)).view(b, max_pages).to(torch.int32)
    lens = _lens(b, max_pages * ps, seed=5)
    out = flash_decode(q, kp, vp, cache_seqlens=lens.to(device), block_table=table.to(device))
    torch.cuda.synchronize()
    for r in (0, 1, 2, 33):
        pages_r = table[r].long().to(device)
        ref = orc.decode_paged(np64(q[r:r + 1]), np64(kp[pages_r]), np64(vp[pages_r]),
                               np.arange(max_pages)[None], lens[r:r + 1].numpy())
        assert_close_maxabs(out[r:r + 1], ref, TOL[dt], f"O row {r}")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("d", [4, 64, 128])
def test_kv_cache_update_paged_exact(device, dtype, d):
    b, h, t, pages, ps = 3, 2, 5, 7, 32
    g = torch.Generator().manual_seed(d + 1)
    k = torch.randn(b, h, t, d, generator=g).to(dtype)
    v = torch.randn(b, h, t, d, generator=g).to(dtype)
    kp = torch.randn(pages, h, ps, d, generator=g).to(dtype)
    vp = torch.randn(pages, h, ps, d, generator=g).to(dtype)
    sl = torch.randperm(pages * ps, generator=g)[:b * t].view(b, t)
    sl[0, 0] = -1
    sl[2, 4] = pages * ps + 3
    ek, ev = orc.kv_cache_update_paged(_bits(k).numpy(), _bits(v).numpy(), _bits(kp).numpy(),
                                       _bits(vp).numpy(), sl.numpy())
    kd, vd, kpd, vpd = (x.to(device) for x in (k, v, kp, vp))
    kv_cache_update(kd, vd, kpd, vpd, sl.to(device), paged=True)
    assert np.array_equal(_bits(kpd).numpy(), ek) and np.array_equal(_bits(vpd).numpy(), ev)
