"""GPU test of the reference-side ctypes binding that ships with this package.

The integration guide at the repository root gives the code a maintainer of
the reference would add as ``src/stackkernels/_core/attention/_hip.py`` (plus
the bindings of the per-row-length, paged, cache-append, RoPE and
introspection entry points).  This test takes that code verbatim from the
guide, loads it against the built library, and checks every function it
defines against this package's own launcher for the same call, bit for bit:
the two drive the same kernels with the same plans, so any difference is a
mistake in the published binding (an argument order, a stride, a workspace
size).
"""

import os
import pathlib
import re
import textwrap

import pytest
import torch

from stackkernels_amd._core.attention.decode import flash_decode as pkg_decode
from stackkernels_amd._core.attention.decode import flash_decode_paged as pkg_decode_paged
from stackkernels_amd._core.attention.flash_bwd import flash_attn_bwd as pkg_bwd
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd as pkg_fwd
from stackkernels_amd.csrc.build import lib_path
from stackkernels_amd.torch import flash_attention as pkg_attention
from stackkernels_amd.torch.cache import kv_cache_update as pkg_update

from _gpu_util import make_qkv, native_loaded

pytestmark = pytest.mark.gpu

GUIDE = pathlib.Path(__file__).resolve().parents[1] / "INTEGRATION.md"


@pytest.fixture(scope="module")
def stub():
    blocks = re.findall(r"```python\n(.*?)```", GUIDE.read_text(), re.S)
    binding = [b for b in blocks if "_lib" in b]
    assert len(binding) >= 5, "the guide's binding blocks were not found"
    old = os.environ.get("SK_ATTN_LIB")
    os.environ["SK_ATTN_LIB"] = lib_path()
    ns: dict = {}
    try:
        for b in binding:
            exec(compile(textwrap.dedent(b), str(GUIDE), "exec"), ns)  # noqa: S102
    finally:
        if old is None:
            os.environ.pop("SK_ATTN_LIB")
        else:
            os.environ["SK_ATTN_LIB"] = old
    return ns


def _tables(d, rows, dtype=torch.float32):
    g = torch.Generator().manual_seed(d + rows)
    ang = torch.rand(rows, d // 2, generator=g, dtype=torch.float64) * 6.0
    ang = torch.cat([ang, ang], dim=1)
    return ang.cos().to(dtype).cuda(), ang.sin().to(dtype).cuda()


@pytest.mark.parametrize("causal", [False, True])
def test_forward_and_backward(device, stub, causal):
    q, k, v = make_qkv(2, 8, 2, 300, 500, 128, torch.bfloat16, seed=3)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(4)).to(q.dtype).cuda()
    o, lse = stub["flash_attn_fwd"](q, k, v, causal)
    o2, lse2 = pkg_fwd(q, k, v, is_causal=causal)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    grads = stub["flash_attn_bwd"](do, q, k, v, o, lse, causal)
    grads2 = pkg_bwd(do, q, k, v, o2, lse2, is_causal=causal)
    torch.cuda.synchronize()
    assert native_loaded()
    for a, b, what in zip(grads, grads2, ("dQ", "dK", "dV")):
        assert torch.equal(a, b), what


def test_decode_forms(device, stub):
    q, k, v = make_qkv(4, 32, 8, 1, 3000, 128, torch.float16, seed=5)
    assert torch.equal(stub["flash_decode"](q, k, v), pkg_decode(q, k, v))
    lens = torch.tensor([0, 1, 1777, 3000], dtype=torch.int32)
    assert torch.equal(stub["flash_decode_varlen"](q, k, v, lens.cuda()),
                       pkg_decode(q, k, v, cache_seqlens=lens.cuda()))
    # a shuffled pool of 64-key pages holding the same cache
    page, pages_per_row = 64, (3000 + 63) // 64
    n_pages = 4 * pages_per_row
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(6))
    table = perm.view(4, pages_per_row).to(torch.int32)
    kp = torch.zeros(n_pages, 8, page, 128, dtype=q.dtype, device=q.device)
    vp = torch.zeros_like(kp)
    for b in range(4):
        for j in range(pages_per_row):
            n = min(page, 3000 - j * page)
            kp[table[b, j], :, :n] = k[b, :, j * page:j * page + n]
            vp[table[b, j], :, :n] = v[b, :, j * page:j * page + n]
    out = stub["flash_decode_paged"](q, kp, vp, table.cuda(), lens.cuda())
    ref = pkg_decode_paged(q, kp, vp, table.cuda(), lens.cuda())
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_cache_append_and_rope_step(device, stub):
    q, kc, vc = make_qkv(3, 16, 4, 1, 1024, 128, torch.bfloat16, seed=7)
    g = torch.Generator().manual_seed(8)
    kn = torch.randn(3, 4, 5, 128, generator=g).to(q.dtype).cuda()
    vn = torch.randn(3, 4, 5, 128, generator=g).to(q.dtype).cuda()
    slots = torch.tensor([[0, 1, 2, 3, 4], [100, 101, 102, -1, 104], [1019, 1020, 1021, 1022, 1023]])
    a_k, a_v, b_k, b_v = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    stub["kv_cache_update"](kn, vn, a_k, a_v, slots.cuda())
    pkg_update(kn, vn, b_k, b_v, slots.cuda())
    assert torch.equal(a_k, b_k) and torch.equal(a_v, b_v)
    # one serving step: append the new token (keys rotated), decode with q rotated
    cos, sin = _tables(128, 2048)
    lens = torch.tensor([5, 900, 1023], dtype=torch.int32).cuda()
    k1, v1 = kn[:, :, :1].contiguous(), vn[:, :, :1].contiguous()
    a_k, a_v, b_k, b_v = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    out = stub["decode_step"](q, k1, v1, a_k, a_v, lens, cos, sin)
    pkg_update(k1, v1, b_k, b_v, lens.to(torch.int64).view(-1, 1), rope_cos=cos, rope_sin=sin,
               start_pos=lens)
    from stackkernels_amd.torch import flash_decode as api_decode

    ref = api_decode(q, b_k, b_v, cache_seqlens=lens + 1, rope_cos=cos, rope_sin=sin,
                     start_pos=lens)
    torch.cuda.synchronize()
    assert torch.equal(a_k, b_k) and torch.equal(a_v, b_v)
    assert torch.equal(out, ref)


def test_trainable_fused_rope(device, stub):
    q, k, v = make_qkv(2, 8, 4, 256, 384, 128, torch.bfloat16, seed=9)
    cos, sin = _tables(128, 1024)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(10)).to(q.dtype).cuda()
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    qb, kb, vb = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = stub["FlashAttentionRoPE"].apply(qa, ka, va, True, cos, sin, 128)
    ref = pkg_attention(qb, kb, vb, True, rope_cos=cos, rope_sin=sin, start_pos=128)
    out.backward(do)
    ref.backward(do)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    for a, b, what in zip((qa, ka, va), (qb, kb, vb), ("dQ", "dK", "dV")):
        assert torch.equal(a.grad, b.grad), what


def test_rotation_and_kernel_config(device, stub):
    x = torch.randn(2, 4, 50, 128, generator=torch.Generator().manual_seed(11)).to(
        torch.bfloat16).cuda()
    cos, sin = _tables(128, 256)
    from stackkernels_amd._core.attention._rope import rope_args, rope_rotate

    ra = rope_args(cos, sin, 7, 2, 128, x.device)
    for inverse in (False, True):
        assert torch.equal(stub["rope_rotate"](x, cos, sin, 7, inverse=inverse),
                           rope_rotate(x, ra, inverse=inverse))
    # the introspection example ran at load: C4's plan
    assert stub["split_kv"] >= 1 and stub["grid"] == 64 * 8 * stub["split_kv"]
