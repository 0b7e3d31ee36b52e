"""GPU parity of RoPE fused into the attention prologue (C ABI
``sk_attn_fwd_rope``, ``sk_decode_rope``, ``sk_decode_paged_rope``,
``sk_kv_cache_update_rope``, ``sk_kv_cache_update_paged_rope``).

The rotation inside a kernel is bit-exact against the oracle's ``rope_rotate``
rounded to the tensor type, so:

* the rotating cache append must write exactly the oracle's rotated keys and
  the unrotated values (bit-exact, every dtype and table dtype, contiguous and
  paged caches, per-row and shared positions, out-of-table positions);
* a fused decode / forward must equal, bit for bit, the same call without
  RoPE on the oracle-rotated q (same kernels, same split plan), at small
  shapes and at the C4 decode shape; and it must be within the decode /
  forward tolerance (max-abs 1e-4 fp32, 2e-2 fp16/bf16) of the oracle's
  float64 attention on the rotated q.
"""

import numpy as np
import pytest
import torch

import stackkernels_amd
from stackkernels_amd._reference.torch.rope import precompute_freqs
from stackkernels_amd.torch import flash_attention, flash_decode, kv_cache_update

from _gpu_util import TOL, assert_close_maxabs, make_qkv, native_loaded, np64
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
NP_DT = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}


@pytest.fixture(autouse=True)
def _auto_backend():
    original = stackkernels_amd.get_backend()
    stackkernels_amd.set_backend("auto")
    yield
    stackkernels_amd.set_backend(original)


def _tables(d, rows, table_dtype=torch.float32, device="cuda"):
    cos, sin = precompute_freqs(d, rows, dtype=table_dtype)
    return cos.to(device), sin.to(device)


def _rotated(x, cos, sin, positions):
    """Oracle rotation of device tensor x (B, H, S, D) at positions (B, S), as
    a device tensor of x's dtype."""
    r = orc.rope_rotate(x.float().cpu().numpy(), cos.float().cpu().numpy(),
                        sin.float().cpu().numpy(), positions)
    r = orc.round_to(r, NP_DT[x.dtype])
    return torch.from_numpy(r).to(x.dtype).to(x.device)


# ------------------------------------------------------------ cache append

@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("table_dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [64, 128, 256])
def test_kv_cache_update_rope_bitexact(dtype, table_dtype, d):
    b, h, t, s = 3, 2, 5, 24
    g = torch.Generator().manual_seed(d)
    k = torch.randn(b, h, t, d, generator=g).to(dtype).cuda()
    v = torch.randn(b, h, t, d, generator=g).to(dtype).cuda()
    kc0 = torch.randn(b, h, s, d, generator=g).to(dtype)
    vc0 = torch.randn(b, h, s, d, generator=g).to(dtype)
    kc, vc = kc0.cuda(), vc0.cuda()
    cos, sin = _tables(d, 40, table_dtype)
    slots = torch.tensor([[0, 1, 2, 3, 4], [7, -1, 9, 30, 8], [23, 22, 21, 20, 19]])
    # per-row positions; row 2 runs past the 40-row table (tokens left unrotated)
    starts = torch.tensor([0, 17, 37], dtype=torch.int32)
    kv_cache_update(k, v, kc, vc, slots.cuda(), rope_cos=cos, rope_sin=sin,
                    start_pos=starts.cuda())
    torch.cuda.synchronize()
    pos = orc.rope_positions(starts.numpy(), b, t)
    kr = orc.round_to(orc.rope_rotate(np64(k).astype(np.float32), np64(cos), np64(sin), pos),
                      NP_DT[dtype])
    wk, wv = orc.kv_cache_update(kr, np64(v), np64(kc0), np64(vc0), slots.numpy())
    np.testing.assert_array_equal(np64(kc), wk)
    np.testing.assert_array_equal(np64(vc), wv)
    assert native_loaded()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_kv_cache_update_paged_rope_bitexact(dtype):
    b, h, t, d, page, pages = 2, 4, 3, 128, 32, 5
    g = torch.Generator().manual_seed(3)
    k = torch.randn(b, h, t, d, generator=g).to(dtype).cuda()
    v = torch.randn(b, h, t, d, generator=g).to(dtype).cuda()
    kp0 = torch.randn(pages, h, page, d, generator=g).to(dtype)
    vp0 = torch.randn(pages, h, page, d, generator=g).to(dtype)
    kp, vp = kp0.cuda(), vp0.cuda()
    cos, sin = _tables(d, 64)
    slots = torch.tensor([[33, 34, 35], [159, -1, 3]])
    kv_cache_update(k, v, kp, vp, slots.cuda(), paged=True, rope_cos=cos, rope_sin=sin,
                    start_pos=9)
    torch.cuda.synchronize()
    kr = orc.round_to(orc.rope_rotate(np64(k).astype(np.float32), np64(cos), np64(sin),
                                      orc.rope_positions(9, b, t)), NP_DT[dtype])
    wk, wv = orc.kv_cache_update_paged(kr, np64(v), np64(kp0), np64(vp0), slots.numpy())
    np.testing.assert_array_equal(np64(kp), wk)
    np.testing.assert_array_equal(np64(vp), wv)


# ------------------------------------------------------------------ decode

@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("hq,hkv", [(8, 2), (32, 1), (64, 2)])
@pytest.mark.parametrize("d", [64, 96, 128, 256])
def test_decode_rope_equals_decode_on_rotated_q(dtype, hq, hkv, d):
    b, sk = 3, 700
    q, k, v = make_qkv(b, hq, hkv, 1, sk, d, dtype, seed=hq + d)
    cos, sin = _tables(d, 2048)
    lens = torch.tensor([700, 333, 1], dtype=torch.int32)
    pos = (lens - 1).cuda()
    out = flash_decode(q, k, v, cache_seqlens=lens.cuda(), rope_cos=cos, rope_sin=sin,
                       start_pos=pos)
    qr = _rotated(q, cos, sin, (lens - 1).numpy()[:, None])
    base = flash_decode(qr, k, v, cache_seqlens=lens.cuda())
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    want = orc.decode_varlen(np64(qr), np64(k), np64(v), lens.numpy())
    assert_close_maxabs(out, want, TOL[dtype], f"decode rope {dtype} {hq}/{hkv} d={d}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_decode_rope_shared_start_negative_scale_and_half_tables(dtype):
    b, hq, hkv, sk, d = 2, 16, 4, 512, 128
    q, k, v = make_qkv(b, hq, hkv, 1, sk, d, dtype, seed=5)
    cos, sin = _tables(d, 1024, dtype)
    out = flash_decode(q, k, v, sm_scale=-0.05, rope_cos=cos, rope_sin=sin, start_pos=511)
    qr = _rotated(q, cos, sin, orc.rope_positions(511, b, 1))
    base = flash_decode(qr, k, v, sm_scale=-0.05)
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    assert_close_maxabs(out, orc.decode(np64(qr), np64(k), np64(v), -0.05), TOL[dtype],
                        "decode rope negative scale")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=str)
def test_decode_paged_rope_equals_paged_on_rotated_q(dtype):
    b, hq, hkv, d, page, pages, max_pages = 3, 32, 2, 128, 64, 12, 4
    g = torch.Generator().manual_seed(11)
    q = torch.randn(b, hq, 1, d, generator=g).to(dtype).cuda()
    kp = torch.randn(pages, hkv, page, d, generator=g).to(dtype).cuda()
    vp = torch.randn(pages, hkv, page, d, generator=g).to(dtype).cuda()
    table = torch.tensor([[0, 3, 5, 7], [11, 10, 9, 8], [1, 2, 4, 6]], dtype=torch.int32).cuda()
    lens = torch.tensor([256, 130, 7], dtype=torch.int32)
    cos, sin = _tables(d, 300)
    out = flash_decode(q, kp, vp, cache_seqlens=lens.cuda(), block_table=table, rope_cos=cos,
                       rope_sin=sin, start_pos=(lens - 1).cuda())
    qr = _rotated(q, cos, sin, (lens - 1).numpy()[:, None])
    base = flash_decode(qr, kp, vp, cache_seqlens=lens.cuda(), block_table=table)
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    want = orc.decode_paged(np64(qr), np64(kp), np64(vp), table.cpu().numpy(), lens.numpy())
    assert_close_maxabs(out, want, TOL[dtype], "paged decode rope")


def test_decode_rope_c4_shape_equals_decode_on_rotated_q():
    """C4 (bf16, B=64, Hq=32, Hkv=8, S_k=32768, D=128): fused rotation of q
    gives the bits of the plain decode on the oracle-rotated q."""
    b, hq, hkv, sk, d = 64, 32, 8, 32768, 128
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(21)
    q = torch.randn(b, hq, 1, d, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(b, hkv, sk, d, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(b, hkv, sk, d, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = _tables(d, sk)
    pos = torch.randint(0, sk, (b,), generator=torch.Generator().manual_seed(2), dtype=torch.int32)
    out = flash_decode(q, k, v, rope_cos=cos, rope_sin=sin, start_pos=pos.cuda())
    qr = _rotated(q, cos, sin, pos.numpy()[:, None])
    base = flash_decode(qr, k, v)
    torch.cuda.synchronize()
    assert torch.equal(out, base)


# ----------------------------------------------------------------- forward

@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_forward_rope_equals_forward_on_rotated_q(dtype, causal, d):
    b, hq, hkv, sq, sk = 2, 4, 2, 300, 420
    q, k, v = make_qkv(b, hq, hkv, sq, sk, d, dtype, seed=d + causal)
    cos, sin = _tables(d, 1024)
    starts = torch.tensor([0, 500], dtype=torch.int32)
    with torch.no_grad():
        out = flash_attention(q, k, v, causal, rope_cos=cos, rope_sin=sin,
                              start_pos=starts.cuda())
        qr = _rotated(q, cos, sin, orc.rope_positions(starts.numpy(), b, sq))
        base = flash_attention(qr, k, v, causal)
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    want, _ = orc.attention_forward(np64(qr), np64(k), np64(v), causal)
    assert_close_maxabs(out, want, TOL[dtype], f"forward rope {dtype} causal={causal} d={d}")


def test_forward_rope_paired_causal_blocks():
    """Enough causal work for the kernel to pair query blocks per workgroup."""
    b, hq, hkv, s, d = 2, 32, 8, 2048, 128
    q, k, v = make_qkv(b, hq, hkv, s, s, d, torch.bfloat16, seed=9)
    cos, sin = _tables(d, 4096)
    with torch.no_grad():
        out = flash_attention(q, k, v, True, rope_cos=cos, rope_sin=sin, start_pos=1000)
        qr = _rotated(q, cos, sin, orc.rope_positions(1000, b, s))
        base = flash_attention(qr, k, v, True)
    torch.cuda.synchronize()
    assert torch.equal(out, base)


def test_forward_rope_c2_shape_equals_forward_on_rotated_q():
    """C2 (bf16 causal MHA, B=4, H=32, S=4096, D=128): the fused rotation of q
    in the forward gives the bits of the plain forward on the oracle-rotated q,
    at per-row start positions."""
    b, h, s, d = 4, 32, 4096, 128
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(31)
    q = torch.randn(b, h, s, d, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(b, h, s, d, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(b, h, s, d, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = _tables(d, 3 * s)
    starts = torch.tensor([0, 1, 4096, 8191 - s + 1], dtype=torch.int32)
    with torch.no_grad():
        out = flash_attention(q, k, v, True, rope_cos=cos, rope_sin=sin, start_pos=starts.cuda())
        qr = _rotated(q, cos, sin, orc.rope_positions(starts.numpy(), b, s))
        base = flash_attention(qr, k, v, True)
    torch.cuda.synchronize()
    assert torch.equal(out, base)


def test_forward_rope_long_work_entry_equals_forward_on_rotated_q():
    """A shape past the short-work limits of the D = 128 forward table (causal,
    S_q = 4352, 2,176 blocks of 256 rows: the 8-wave entry): the fused rotation
    still gives the bits of the plain forward on the oracle-rotated q."""
    from stackkernels_amd._opt.pick import pick

    b, h, s, d = 4, 32, 4352, 128
    assert pick("flash_attn", (b, h, s, d), dtype="bfloat16", is_causal=True)["BLOCK_M"] == 256
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(37)
    q = torch.randn(b, h, s, d, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(b, h, s, d, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(b, h, s, d, generator=g, device=dev).to(torch.bfloat16)
    cos, sin = _tables(d, 2 * s)
    starts = torch.tensor([0, 7, 1000, s - 1], dtype=torch.int32)
    with torch.no_grad():
        out = flash_attention(q, k, v, True, rope_cos=cos, rope_sin=sin, start_pos=starts.cuda())
        qr = _rotated(q, cos, sin, orc.rope_positions(starts.numpy(), b, s))
        base = flash_attention(qr, k, v, True)
    torch.cuda.synchronize()
    assert torch.equal(out, base)


# ------------------------------------------------------------ standalone rotation

@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("table_dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("inverse", [False, True])
@pytest.mark.parametrize("in_place", [False, True])
def test_rope_rotate_kernel_bitexact(dtype, table_dtype, inverse, in_place):
    """sk_rope_rotate against the oracle's float32 rotation / adjoint rounded to the
    tensor type, bit for bit.  Tables with unequal halves, so a sine taken from the
    wrong half shows; per-row positions, one running past the table; a BSHD view."""
    from stackkernels_amd._core.attention._rope import rope_args, rope_rotate

    b, h, s, d = 3, 4, 37, 128
    g = torch.Generator().manual_seed(21 + inverse)
    x = torch.randn(b, s, h, d, generator=g).to(dtype).cuda().transpose(1, 2)  # strided view
    cos = torch.randn(50, d, generator=g).to(table_dtype).cuda()
    sin = torch.randn(50, d, generator=g).to(table_dtype).cuda()
    starts = torch.tensor([0, 9, 30], dtype=torch.int32)
    ra = rope_args(cos, sin, starts.cuda(), b, d, x.device)
    src = x.contiguous() if in_place else x
    keep = src.clone()
    y = rope_rotate(src, ra, inverse=inverse, out=src if in_place else None)
    torch.cuda.synchronize()
    assert native_loaded()
    if in_place:
        assert y.data_ptr() == src.data_ptr()
    pos = orc.rope_positions(starts.numpy(), b, s)
    fn = orc.rope_rotate_adjoint if inverse else orc.rope_rotate
    want = orc.round_to(fn(np64(keep).astype(np.float32), np64(cos), np64(sin), pos), NP_DT[dtype])
    np.testing.assert_array_equal(np64(y), want)


def test_rope_rotate_argument_errors():
    from stackkernels_amd._core.attention._rope import rope_args, rope_rotate

    x = torch.zeros(1, 2, 8, 128, dtype=torch.bfloat16, device="cuda")
    cos, sin = _tables(128, 4)
    with pytest.raises(ValueError, match="outside the rope table"):
        rope_rotate(x, rope_args(cos, sin, 0, 1, 128, x.device))
    cos, sin = _tables(128, 64)
    big = torch.zeros(1, 2, 16, 128, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="overlaps"):
        rope_rotate(big[:, :, :8], rope_args(cos, sin, 0, 1, 128, x.device), out=big[:, :, 4:12])


# ------------------------------------------------------------ fused-RoPE backward

@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("per_row", [False, True])
def test_forward_rope_backward_matches_oracle(dtype, causal, d, per_row):
    """flash_attention(..., rope_cos=, rope_sin=) under autograd: dQ, dK, dV against the
    float64 oracle of the unfused pipeline -- attention_backward at the rotated q (q
    rotated as the forward kernel rotates it, rounded to the type), then the adjoint of
    the rotation on dQ -- within the stated tolerance (1e-4 fp32, 2e-2 fp16/bf16); O as
    the forward on the rotated q."""
    b, hq, hkv, sq, sk = 2, 4, 2, 150, 230
    q, k, v = make_qkv(b, hq, hkv, sq, sk, d, dtype, seed=d + 2 * causal + per_row)
    cos, sin = _tables(d, 1024)
    starts = torch.tensor([3, 700], dtype=torch.int32) if per_row else None
    sp = starts.cuda() if per_row else 77
    for t in (q, k, v):
        t.requires_grad_(True)
    out = flash_attention(q, k, v, causal, rope_cos=cos, rope_sin=sin, start_pos=sp)
    do = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(dtype).cuda()
    out.backward(do)
    torch.cuda.synchronize()
    assert native_loaded()
    pos = orc.rope_positions(starts.numpy() if per_row else 77, b, sq)
    qr = orc.round_to(orc.rope_rotate(np64(q).astype(np.float32), np64(cos), np64(sin), pos),
                      NP_DT[dtype]).astype(np.float64)
    o_ref, _ = orc.attention_forward(qr, np64(k), np64(v), causal)
    assert_close_maxabs(out, o_ref, TOL[dtype], "O")
    dqr, dk, dv = orc.attention_backward(qr, np64(k), np64(v), np64(do), causal)
    dq = orc.rope_rotate_adjoint(dqr, np64(cos), np64(sin), pos, dtype=np.float64)
    assert_close_maxabs(q.grad, dq, TOL[dtype], "dQ")
    assert_close_maxabs(k.grad, dk, TOL[dtype], "dK")
    assert_close_maxabs(v.grad, dv, TOL[dtype], "dV")


def test_forward_rope_backward_c3_shape():
    """C3 shape (bf16 causal GQA, bottom-right mask, B=2 Hq=32 Hkv=8 Sq=2048 Sk=8192): the
    fused-RoPE training step gives dK/dV equal to the plain backward at the oracle-rotated
    q, and dQ equal to the kernel's adjoint rotation of that backward's dQ, bit for bit;
    one batch row's dQ against the float64 oracle of the composite."""
    from stackkernels_amd._core.attention._rope import rope_args, rope_rotate

    b, hq, hkv, sq, sk, d = 2, 32, 8, 2048, 8192, 128
    q, k, v = make_qkv(b, hq, hkv, sq, sk, d, torch.bfloat16, seed=41)
    cos, sin = _tables(d, 8192)
    for t in (q, k, v):
        t.requires_grad_(True)
    out = flash_attention(q, k, v, True, rope_cos=cos, rope_sin=sin, start_pos=sk - sq)
    do = torch.randn(out.shape, generator=torch.Generator(device="cuda").manual_seed(6),
                     device="cuda").to(torch.bfloat16)
    out.backward(do)
    pos = orc.rope_positions(sk - sq, b, sq)
    qr = _rotated(q.detach(), cos, sin, pos).requires_grad_(True)
    kp, vp = k.detach().clone().requires_grad_(True), v.detach().clone().requires_grad_(True)
    base = flash_attention(qr, kp, vp, True)
    base.backward(do)
    dq = rope_rotate(qr.grad, rope_args(cos, sin, sk - sq, b, d, q.device), inverse=True)
    torch.cuda.synchronize()
    assert torch.equal(out, base)
    assert torch.equal(k.grad, kp.grad) and torch.equal(v.grad, vp.grad)
    assert torch.equal(q.grad, dq)
    dqr, _, _ = orc.attention_backward(np64(qr[1:2, :4]), np64(k[1:2, :1]), np64(v[1:2, :1]),
                                       np64(do[1:2, :4]), True)
    want = orc.rope_rotate_adjoint(dqr, np64(cos), np64(sin), pos[1:2], dtype=np.float64)
    assert_close_maxabs(q.grad[1:2, :4], want, TOL[torch.bfloat16], "dQ (batch 1, heads 0-3)")
