"""GPU parity of the HIP backward (bf16 / fp16 and fp32 MFMA kernels, the fp32
vector kernels at D = 256) against the oracle.

The grid follows the reference's tests/ops/test_flash_attn.py::test_flash_attn_backward
(heads {(4,4),(4,2),(4,1)} x causal, random upstream gradient) widened to every
head dim the reference supports and to ragged / fully-masked shapes; the
full-size BASELINE config 3 (bf16 causal GQA, bottom-right mask) is checked
against the repo's PyTorch reference path run in fp32 on the device, whose
gradients come from autograd exactly as the reference's backward does.
Tolerance: max-abs <= 2e-2 on dQ / dK / dV (bf16 / fp16) and 1e-4 (fp32), stated by
the target.
"""

import pytest
import torch

import stackkernels_amd
from stackkernels_amd._core.attention.flash_bwd import flash_attn_bwd
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd
from stackkernels_amd._reference.torch.attention import attention_reference
from stackkernels_amd.torch import flash_attention

from _bwd_bound import check_backward, rounding_mass
from _gpu_util import (TOL, assert_close_maxabs, assert_lse_close, make_qkv, native_loaded, np64,
                       oracle_fwd)

pytestmark = pytest.mark.gpu

HALF = [torch.float16, torch.bfloat16]
ALL = [torch.float32, *HALF]


@pytest.fixture(autouse=True)
def _auto_backend():
    original = stackkernels_amd.get_backend()
    stackkernels_amd.set_backend("auto")
    yield
    stackkernels_amd.set_backend(original)


def _grads(q, k, v, g, causal, scale=None):
    from oracle import attention_oracle as orc

    return orc.attention_backward(np64(q), np64(k), np64(v), np64(g), causal, scale)


def _run(b, hq, hkv, sq, sk, d, dtype, causal, seed=42, scale=None):
    q, k, v = make_qkv(b, hq, hkv, sq, sk, d, dtype, seed=seed)
    for t in (q, k, v):
        t.requires_grad_(True)
    out = flash_attention(q, k, v, is_causal=causal, sm_scale=scale)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(seed + 1)).to(dtype)
    out.backward(g.to(out.device))
    assert native_loaded()
    return q, k, v, g


def _check(q, k, v, g, causal, dtype, scale=None):
    dq, dk, dv = _grads(q, k, v, g, causal, scale)
    assert q.grad.dtype == dtype and k.grad.shape == k.shape and v.grad.shape == v.shape
    assert_close_maxabs(q.grad, dq, TOL[dtype], "dQ")
    assert_close_maxabs(k.grad, dk, TOL[dtype], "dK")
    assert_close_maxabs(v.grad, dv, TOL[dtype], "dV")


@pytest.mark.parametrize("dtype", ALL, ids=str)
@pytest.mark.parametrize("heads", [(4, 4), (4, 2), (4, 1)])
@pytest.mark.parametrize("is_causal", [False, True])
def test_backward_reference_grid(device, dtype, heads, is_causal):
    """The reference's own backward grid: S = 16, D = 64, B = 2."""
    q, k, v, g = _run(2, heads[0], heads[1], 16, 16, 64, dtype, is_causal)
    _check(q, k, v, g, is_causal, dtype)


@pytest.mark.parametrize("dtype", ALL, ids=str)
@pytest.mark.parametrize("head_dim", [64, 80, 96, 128, 256])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("heads", [(8, 8), (8, 2), (8, 1)])
def test_backward_head_dims(device, dtype, head_dim, is_causal, heads):
    q, k, v, g = _run(1, heads[0], heads[1], 96, 160, head_dim, dtype, is_causal)
    _check(q, k, v, g, is_causal, dtype)


@pytest.mark.parametrize("dtype", ALL, ids=str)
@pytest.mark.parametrize("sq,sk", [(1, 1), (1, 300), (3, 5), (65, 65), (127, 129), (200, 77),
                                   (129, 1000), (300, 300), (513, 257)])
@pytest.mark.parametrize("is_causal", [False, True])
def test_backward_ragged_shapes(device, dtype, sq, sk, is_causal):
    q, k, v, g = _run(1, 4, 2, sq, sk, 128, dtype, is_causal, seed=sq * 1000 + sk)
    _check(q, k, v, g, is_causal, dtype)


@pytest.mark.parametrize("dtype", ALL, ids=str)
def test_backward_fully_masked_rows(device, dtype):
    # causal, S_q > S_k: rows i < S_q - S_k see no key; their dQ is 0 and they add nothing to dK/dV
    q, k, v, g = _run(2, 4, 2, 200, 70, 64, dtype, True)
    assert torch.all(q.grad[:, :, :130] == 0)
    assert torch.isfinite(k.grad).all() and torch.isfinite(v.grad).all()
    _check(q, k, v, g, True, dtype)


@pytest.mark.parametrize("dtype", HALF, ids=str)
@pytest.mark.parametrize("scale", [0.05, 1.0, -0.09])
def test_backward_custom_and_negative_scale(device, dtype, scale):
    """Non-default scales.  At scale 1.0 (D = 64) the softmax is sharp and |dQ|, |dK| reach
    ~28, where one bf16 step is 0.125: the repo's PyTorch reference path itself (fp32 autograd,
    gradients returned in bf16) is off the fp64 oracle by ~0.06 there, so an absolute 2e-2
    cannot hold in bf16.  Each element is held to the reference path's own error plus the
    rounding allowance of the kernel's 16-bit operands (``tests/_bwd_bound.py``); at the
    default scale every test holds the absolute 2e-2."""
    q, k, v, g = _run(1, 4, 4, 70, 90, 64, dtype, True, scale=scale)
    exact = _grads(q, k, v, g, True, scale)
    dt = "bf16" if dtype == torch.bfloat16 else "f16"
    mass = rounding_mass(np64(q), np64(k), np64(v), np64(g), True, scale, dt)
    qr, kr, vr = (t.detach().cpu().requires_grad_(True) for t in (q, k, v))
    ref, _ = attention_reference(qr, kr, vr, is_causal=True, sm_scale=scale)
    ref.backward(g.cpu())
    for i, (name, ours, path) in enumerate((("dQ", q.grad, qr.grad), ("dK", k.grad, kr.grad),
                                            ("dV", v.grad, vr.grad))):
        check_backward(np64(ours), np64(path), exact[i], mass[i], dt, name)


@pytest.mark.parametrize("scale", [0.05, 1.0, -0.09])
def test_backward_fp32_custom_and_negative_scale(device, scale):
    """fp32 at non-default scales: every gradient within 1e-4 of the oracle (at scale 1.0
    |dQ| and |dK| reach ~28, where fp32 still resolves 2e-6)."""
    q, k, v, g = _run(1, 4, 4, 70, 90, 64, torch.float32, True, scale=scale)
    _check(q, k, v, g, True, torch.float32, scale)


@pytest.mark.parametrize("head_dim,kernels", [
    (64, "bwd_dkv_f32_mfma_kernel+bwd_dq_f32_mfma_kernel"),
    (96, "bwd_dkv_f32_mfma_kernel+bwd_dq_f32_mfma_kernel"),
    (256, "bwd_dkv_f32_kernel+bwd_dq_f32_kernel"),
])
def test_backward_fp32_kernels_and_long_sequence(device, head_dim, kernels):
    """The fp32 backward runs on the matrix cores up to a padded head dim of 128 (the
    vector kernels at 256); a causal GQA shape over several 128-key and 128-query blocks
    with ragged ends, against the oracle at 1e-4."""
    from stackkernels_amd._opt.pick import pick

    cfg = pick("flash_bwd", (1, 8, 700, head_dim), dtype="float32", kv_len=900, num_kv_heads=2,
               is_causal=True)
    assert cfg["kernel_variant"] == kernels
    q, k, v, g = _run(1, 8, 2, 700, 900, head_dim, torch.float32, True, seed=head_dim)
    _check(q, k, v, g, True, torch.float32)


@pytest.mark.parametrize("dtype", ALL, ids=str)
def test_backward_empty_sequences(device, dtype):
    # no keys: O = 0, every gradient 0; no queries: dK = dV = 0
    for sq, sk in ((10, 0), (0, 10)):
        q, k, v = make_qkv(1, 2, 2, sq, sk, 64, dtype)
        o, lse = flash_attn_fwd(q, k, v)
        do = torch.randn_like(o)
        dq, dk, dv = flash_attn_bwd(do, q, k, v, o, lse)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
        assert torch.all(dq == 0) and torch.all(dk == 0) and torch.all(dv == 0)


@pytest.mark.parametrize("dtype", ALL, ids=str)
def test_backward_deterministic(device, dtype):
    q, k, v = make_qkv(2, 8, 2, 300, 333, 128, dtype)
    o, lse = flash_attn_fwd(q, k, v, is_causal=True)
    do = torch.randn_like(o)
    a = flash_attn_bwd(do, q, k, v, o, lse, is_causal=True)
    b = flash_attn_bwd(do, q, k, v, o, lse, is_causal=True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_backward_gqa_equals_mha_on_repeated_kv(device):
    """dK/dV of a GQA head = sum over its query group of the MHA grads on repeated K/V."""
    dt = torch.bfloat16
    q, k, v = make_qkv(1, 8, 2, 128, 192, 64, dt)
    o, lse = flash_attn_fwd(q, k, v, is_causal=True)
    do = torch.randn(o.shape, generator=torch.Generator().manual_seed(5)).to(dt).to(o.device)
    dq, dk, dv = flash_attn_bwd(do, q, k, v, o, lse, is_causal=True)
    kr, vr = k.repeat_interleave(4, dim=1), v.repeat_interleave(4, dim=1)
    o2, lse2 = flash_attn_fwd(q, kr, vr, is_causal=True)
    dq2, dk2, dv2 = flash_attn_bwd(do, q, kr, vr, o2, lse2, is_causal=True)
    assert torch.equal(dq, dq2)
    assert_close_maxabs(dk, dk2.float().view(1, 2, 4, 192, 64).sum(2), 2e-2, "dK")
    assert_close_maxabs(dv, dv2.float().view(1, 2, 4, 192, 64).sum(2), 2e-2, "dV")


@pytest.mark.parametrize("compiled", [False, True])
def test_custom_op_backward(device, compiled):
    """torch.ops.stackkernels.flash_attn_op forward + backward on the device (the HIP
    kernels through stackkernels_amd::attn_fwd / attn_bwd), eager and compiled."""
    dt = torch.bfloat16
    q, k, v = make_qkv(2, 8, 2, 96, 160, 128, dt, seed=7)
    for t in (q, k, v):
        t.requires_grad_(True)
    fn = lambda a, b, c: torch.ops.stackkernels.flash_attn_op(a, b, c, True, None)  # noqa: E731
    if compiled:
        fn = torch.compile(fn, backend="aot_eager", fullgraph=True)
    out = fn(q, k, v)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(8)).to(dt)
    out.backward(g.to(out.device))
    assert native_loaded()
    o_ref = oracle_fwd(q, k, v, True)[0]
    assert_close_maxabs(out, o_ref, TOL[dt], "O")
    _check(q, k, v, g, True, dt)


def test_config3_full_size_backward(device):
    """bf16 causal GQA bottom-right, B=2 Hq=32 Hkv=8 Sq=2048 Sk=8192 D=128,
    against autograd through the repo's PyTorch reference path in fp32 (one batch at a time):
    O, dQ, dK, dV within 2e-2 and the forward's LSE (which the backward consumes) within 1e-3."""
    dt = torch.bfloat16
    q, k, v = make_qkv(2, 32, 8, 2048, 8192, 128, dt, seed=0)
    g = torch.Generator(device=q.device).manual_seed(1)
    do = torch.randn(q.shape, generator=g, device=q.device).to(dt)
    o, lse = flash_attn_fwd(q, k, v, is_causal=True)
    dq, dk, dv = flash_attn_bwd(do, q, k, v, o, lse, is_causal=True)
    torch.cuda.synchronize()
    for b in range(2):
        qr, kr, vr = (t[b:b + 1].float().requires_grad_(True) for t in (q, k, v))
        ref, ref_lse = attention_reference(qr, kr, vr, is_causal=True)
        ref.backward(do[b:b + 1].float())
        assert_close_maxabs(o[b:b + 1].float(), ref.detach(), 2e-2, f"O batch {b}")
        assert_lse_close(lse[b:b + 1], ref_lse.detach(), f"LSE batch {b}")
        assert_close_maxabs(dq[b:b + 1].float(), qr.grad, 2e-2, f"dQ batch {b}")
        assert_close_maxabs(dk[b:b + 1].float(), kr.grad, 2e-2, f"dK batch {b}")
        assert_close_maxabs(dv[b:b + 1].float(), vr.grad, 2e-2, f"dV batch {b}")
        del qr, kr, vr, ref
        torch.cuda.empty_cache()
