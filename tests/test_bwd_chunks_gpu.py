"""GPU tests of the five-GEMM backward's dS workspace: chunking, the causal
tile layout and keys past S_k.

``sk_attn_bwd`` runs the five-GEMM backward when the workspace past the row
statistics holds at least one (batch, KV head) pair's dS tiles, in the fewest
even chunks of pairs whose tiles fit (at most 2 GiB of them), and the
seven-GEMM backward when it holds only the row statistics.  Every chunking
must give the same bits, equal to the seven-GEMM backward's (the same dS
values summed into dQ in the same key order), and the oracle's gradients
within the stated bounds.  Shapes cover causal offsets S_k - S_q that are
not multiples of 32 or 128, S_q > S_k (fully masked rows), GQA groups and
ragged lengths, so every branch of the tile layout is read back.
"""

import ctypes

import numpy as np
import pytest
import torch

from stackkernels_amd._core.attention import _lib
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd
from stackkernels_amd._opt.pick import pick
from stackkernels_amd._reference.torch.attention import attention_reference

from _bwd_bound import check_backward, rounding_mass
from _gpu_util import TOL, assert_close_maxabs, make_qkv, native_loaded, np64

pytestmark = pytest.mark.gpu


def _sizes(dtype, b, hq, hkv, sq, sk, d, causal):
    lib = _lib.load()
    code = _lib.dtype_code(dtype)
    pref, mn = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.sk_attn_bwd_workspace(code, b, hq, hkv, sq, sk, d, int(causal),
                                     ctypes.byref(pref)) == 0
    assert lib.sk_attn_bwd_workspace_min(code, b, hq, hkv, sq, sk, d, int(causal),
                                         ctypes.byref(mn)) == 0
    one = ctypes.c_size_t()  # one pair: the same query group, B = 1, H_kv = 1
    assert lib.sk_attn_bwd_workspace(code, 1, hq // hkv, 1, sq, sk, d, int(causal),
                                     ctypes.byref(one)) == 0
    one_min = ctypes.c_size_t()
    assert lib.sk_attn_bwd_workspace_min(code, 1, hq // hkv, 1, sq, sk, d, int(causal),
                                         ctypes.byref(one_min)) == 0
    return pref.value, mn.value, one.value - one_min.value


def _bwd(do, q, k, v, o, lse, causal, ws_bytes):
    """sk_attn_bwd through the C ABI with a workspace of exactly ws_bytes."""
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    lib = _lib.load()
    rc = lib.sk_attn_bwd(_lib.dtype_code(q.dtype), do.data_ptr(), q.data_ptr(), k.data_ptr(),
                         v.data_ptr(), o.data_ptr(), lse.data_ptr(), dq.data_ptr(),
                         dk.data_ptr(), dv.data_ptr(), ws.data_ptr(), ws_bytes, b, hq, hkv, sq,
                         sk, d, int(causal), 1.0 / d ** 0.5,
                         torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "sk_attn_bwd")
    return dq, dk, dv


def _check_bound(q, k, v, do, causal, grads):
    """Gradients against the float64 oracle, elementwise within the repo's PyTorch
    reference path's own error plus the rounding allowance of the kernels' 16-bit
    operands (``tests/_bwd_bound.py``): the group sums of dK/dV here reach 5-10, where
    one bf16 step is 0.03-0.06, so an absolute 2e-2 is not a bound for them."""
    from oracle import attention_oracle as orc

    exact = orc.attention_backward(np64(q), np64(k), np64(v), np64(do), causal)
    dt = "bf16" if q.dtype == torch.bfloat16 else "f16"
    mass = rounding_mass(np64(q), np64(k), np64(v), np64(do), causal, None, dt)
    qr, kr, vr = (t.detach().cpu().requires_grad_(True) for t in (q, k, v))
    ref, _ = attention_reference(qr, kr, vr, is_causal=causal)
    ref.backward(do.cpu())
    for i, (name, path) in enumerate((("dQ", qr.grad), ("dK", kr.grad), ("dV", vr.grad))):
        check_backward(np64(grads[i]), np64(path), exact[i], mass[i], dt, name)


SHAPES = [
    # b, hq, hkv, sq, sk, causal
    (2, 4, 2, 200, 333, True),    # S_k - S_q = 133: not a multiple of 32
    (1, 4, 1, 300, 100, True),    # S_q > S_k: 200 rows see no key
    (3, 2, 2, 64, 1000, True),    # long keys, short queries
    (2, 6, 3, 257, 257, False),   # ragged, no mask
    (2, 8, 2, 513, 640, True),    # S_k - S_q = 127
    (1, 2, 1, 1024, 1024, True),  # square causal: about half of the rectangle allocated
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("d", [96, 128])
def test_chunkings_bit_identical(device, dtype, shape, d):
    b, hq, hkv, sq, sk, causal = shape
    print(f"chunking case {dtype} {shape} D={d}", flush=True)
    q, k, v = make_qkv(b, hq, hkv, sq, sk, d, dtype, seed=sq + sk)
    g = torch.Generator().manual_seed(3)
    do = torch.randn(q.shape, generator=g).to(dtype).to(q.device)
    o, lse = flash_attn_fwd(q, k, v, is_causal=causal)
    pref, mn, pair = _sizes(dtype, b, hq, hkv, sq, sk, d, causal)
    pairs = b * hkv
    assert pref == mn + pairs * pair  # small shapes: one chunk
    full = _bwd(do, q, k, v, o, lse, causal, pref)
    runs = {"seven": _bwd(do, q, k, v, o, lse, causal, mn),
            "one_pair": _bwd(do, q, k, v, o, lse, causal, mn + pair),
            # one byte short of two pairs: still chunks of one
            "short": _bwd(do, q, k, v, o, lse, causal, mn + 2 * pair - 1)}
    if pairs >= 3:
        runs["uneven"] = _bwd(do, q, k, v, o, lse, causal, mn + (pairs - 1) * pair)
    torch.cuda.synchronize()
    assert native_loaded()
    for name, r in runs.items():
        for x, y, what in zip(full, r, ("dQ", "dK", "dV")):
            assert torch.equal(x, y), f"{what} of the {name} workspace differs"
    _check_bound(q, k, v, do, causal, full)


def test_workspace_below_minimum_is_rejected(device):
    q, k, v = make_qkv(1, 2, 2, 64, 64, 128, torch.bfloat16)
    o, lse = flash_attn_fwd(q, k, v)
    pref, mn, pair = _sizes(torch.bfloat16, 1, 2, 2, 64, 64, 128, False)
    with pytest.raises(RuntimeError, match="workspace"):
        _bwd(torch.ones_like(q), q, k, v, o, lse, False, mn - 1)


@pytest.mark.parametrize("dtype,amp", [(torch.float16, 1.5), (torch.bfloat16, 3.0)], ids=str)
def test_keys_past_sk_with_very_negative_lse(device, dtype, amp):
    """No mask, S_k % 32 != 0, every query anti-aligned with every key, so lse << 0 and
    exp2(-lse log2 e) * delta -- the dS a key slot past S_k would carry -- overflows the
    16-bit type (fp16) or fp32 (bf16).  The five-GEMM backward stores those slots as
    zeros; dQ must be finite, within the rounding bound of the oracle and equal to the
    seven-GEMM backward's, which masks the keys."""
    b, hq, hkv, sq, sk, d = 1, 4, 2, 96, 100, 128
    g = torch.Generator().manual_seed(17)
    q = (-amp + 0.1 * torch.randn(b, hq, sq, d, generator=g)).to(dtype)
    k = (amp + 0.1 * torch.randn(b, hkv, sk, d, generator=g)).to(dtype)
    v = torch.randn(b, hkv, sk, d, generator=g).to(dtype)
    do = (8.0 * torch.randn(b, hq, sq, d, generator=g)).to(dtype)
    q, k, v, do = (t.to(device) for t in (q, k, v, do))
    o, lse = flash_attn_fwd(q, k, v)
    # fp16: exp(15) = 3.3e6 > 65504; bf16: exp(88) > 2^127
    assert float(lse.max()) < (-15.0 if dtype == torch.float16 else -88.0)
    pref, mn, pair = _sizes(dtype, b, hq, hkv, sq, sk, d, False)
    five = _bwd(do, q, k, v, o, lse, False, pref)
    seven = _bwd(do, q, k, v, o, lse, False, mn)
    torch.cuda.synchronize()
    for x, y, what in zip(five, seven, ("dQ", "dK", "dV")):
        assert torch.isfinite(x).all(), f"{what}: non-finite values"
        assert torch.equal(x, y), what
    _check_bound(q, k, v, do, False, five)


def test_many_chunks_full_size(device):
    """B = 4, H = 32, S = 8192 causal bf16: 8.7 GB of dS tiles in all, so the same five-GEMM
    kernels run in 5 chunks of 26, 26, 26, 26 and 24 pairs (about 1.8 GB of tiles each,
    byte offsets up to that within a chunk).  Heads on both sides of the first chunk seam
    and the last head are checked against the float64 oracle; the whole result equals the seven-GEMM
    backward's bit for bit."""
    B, H, S, D = 4, 32, 8192, 128
    dt = torch.bfloat16
    cfg = pick("flash_bwd", (B, H, S, D), dtype="bfloat16", is_causal=True)
    assert cfg["kernel_variant"] == "bwd_dkv_kernel+bwd_dq_ds_kernel" and cfg["chunks"] == 5
    gen = torch.Generator(device=device).manual_seed(5)
    q, k, v, do = (torch.randn(B, H, S, D, generator=gen, device=device, dtype=dt)
                   for _ in range(4))
    o, lse = flash_attn_fwd(q, k, v, is_causal=True)
    pref, mn, pair = _sizes(dt, B, H, H, S, S, D, True)
    assert pref == mn + 26 * pair and pref - mn <= 2 << 30
    five = _bwd(do, q, k, v, o, lse, True, pref)
    seven = _bwd(do, q, k, v, o, lse, True, mn)
    torch.cuda.synchronize()
    assert native_loaded()
    for x, y, what in zip(five, seven, ("dQ", "dK", "dV")):
        assert torch.equal(x, y), what
    del seven
    torch.cuda.empty_cache()
    from oracle import attention_oracle as orc

    # pair index b * H + h; chunks start at pairs 0, 26, 52, 78, 104
    for b, h in ((0, 25), (0, 26), (3, 31)):
        sl = lambda t: np64(t[b:b + 1, h:h + 1])  # noqa: E731
        exact = orc.attention_backward(sl(q), sl(k), sl(v), sl(do), True)
        for x, e, what in zip(five, exact, ("dQ", "dK", "dV")):
            assert_close_maxabs(x[b:b + 1, h:h + 1], e, TOL[dt], f"{what} (b={b}, h={h})")
        assert np.isfinite(exact[0]).all()


def _random_shapes(n, seed):
    g = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hkv = int(g.integers(1, 5))
        out.append((int(g.integers(1, 4)), hkv * int(g.choice([1, 2, 4])), hkv,
                    int(g.integers(1, 700)), int(g.integers(1, 900)), int(g.choice([80, 96, 128])),
                    i % 2 == 0,
                    torch.bfloat16 if g.integers(0, 2) else torch.float16))
    return out


@pytest.mark.parametrize("shape", _random_shapes(12, 2024),
                         ids=lambda s: "x".join(map(str, s[:6])) + ("c" if s[6] else "n"))
def test_random_shapes_every_chunking_bit_identical(device, shape):
    """Seeded random shapes (ragged S_q and S_k in either order, GQA, head dims 80 (run
    zero-padded to 96), 96 and 128, every other one causal, fp16 or bf16): the one-chunk five-GEMM backward, chunks of
    one pair and the seven-GEMM backward give the same bits, and the oracle's gradients
    within the rounding bound."""
    b, hq, hkv, sq, sk, d, causal, dtype = shape
    print(f"random chunking case {shape}", flush=True)
    q, k, v = make_qkv(b, hq, hkv, sq, sk, d, dtype, seed=sq * 7 + sk)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(sk)).to(dtype).to(q.device)
    o, lse = flash_attn_fwd(q, k, v, is_causal=causal)
    pref, mn, pair = _sizes(dtype, b, hq, hkv, sq, sk, d, causal)
    full = _bwd(do, q, k, v, o, lse, causal, pref)
    ones = _bwd(do, q, k, v, o, lse, causal, mn + pair)
    seven = _bwd(do, q, k, v, o, lse, causal, mn)
    torch.cuda.synchronize()
    for x, y, z, what in zip(full, ones, seven, ("dQ", "dK", "dV")):
        assert torch.equal(x, y), f"{what}: chunks of one pair differ"
        assert torch.equal(x, z), f"{what}: seven-GEMM backward differs"
    _check_bound(q, k, v, do, causal, full)
