"""torch.library ops: ``stackkernels::flash_attn_op`` (the reference's name and
schema, src/stackkernels/torch/attention.py:200-223) made differentiable
through ``stackkernels_amd::attn_fwd`` / ``attn_bwd`` with register_autograd
and fake implementations, so torch.compile graphs keep the backward.

CPU: the ops' reference-path implementations against autograd through
``attention_reference``; torch.library.opcheck on both ops; a compiled
(aot_eager) forward + backward.  The closed-form reference backward is
checked against autograd on MHA/GQA/MQA, causal, fully masked and ragged
shapes.  The GPU variant lives in tests/test_flash_bwd_gpu.py.
"""

import pytest
import torch

import stackkernels_amd.torch  # noqa: F401  (registers the ops)
from stackkernels_amd._reference.torch.attention import (
    attention_reference,
    attention_reference_backward,
)


def _autograd_ref(q, k, v, do, is_causal, scale):
    qr, kr, vr = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    out, _ = attention_reference(qr, kr, vr, is_causal=is_causal, sm_scale=scale)
    out.backward(do)
    return out.detach(), qr.grad, kr.grad, vr.grad


SHAPES = [
    ((2, 4, 16, 32), (2, 4, 16, 32)),   # MHA
    ((2, 4, 16, 32), (2, 2, 24, 32)),   # GQA, S_k > S_q
    ((1, 8, 12, 16), (1, 1, 12, 16)),   # MQA
    ((1, 2, 9, 16), (1, 1, 4, 16)),     # S_q > S_k: causal rows with no visible key
]


@pytest.mark.parametrize("qs,ks", SHAPES)
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("scale", [None, 0.3, -0.5])
def test_closed_form_backward_matches_autograd(qs, ks, is_causal, scale):
    torch.manual_seed(0)
    q, k, v = torch.randn(qs), torch.randn(ks), torch.randn(ks)
    do = torch.randn(qs)
    _, dq, dk, dv = _autograd_ref(q, k, v, do, is_causal, scale)
    cq, ck, cv = attention_reference_backward(do, q, k, v, is_causal=is_causal, sm_scale=scale)
    for a, b in ((cq, dq), (ck, dk), (cv, dv)):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("qs,ks", SHAPES)
@pytest.mark.parametrize("is_causal", [False, True])
def test_flash_attn_op_backward(qs, ks, is_causal):
    torch.manual_seed(1)
    q, k, v = (torch.randn(s, requires_grad=True) for s in (qs, ks, ks))
    do = torch.randn(qs)
    out = torch.ops.stackkernels.flash_attn_op(q, k, v, is_causal, None)
    out.backward(do)
    ro, dq, dk, dv = _autograd_ref(q, k, v, do, is_causal, None)
    torch.testing.assert_close(out.detach(), ro)
    for a, b in ((q.grad, dq), (k.grad, dk), (v.grad, dv)):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_flash_attn_op_compiled_forward_backward():
    torch.manual_seed(2)
    q, k, v = (torch.randn(s, requires_grad=True) for s in ((2, 4, 16, 32), (2, 2, 16, 32), (2, 2, 16, 32)))
    do = torch.randn(2, 4, 16, 32)
    fn = torch.compile(lambda a, b, c: torch.ops.stackkernels.flash_attn_op(a, b, c, True, None),
                       backend="aot_eager", fullgraph=True)
    out = fn(q, k, v)
    out.backward(do)
    ro, dq, dk, dv = _autograd_ref(q, k, v, do, True, None)
    torch.testing.assert_close(out.detach(), ro)
    for a, b in ((q.grad, dq), (k.grad, dk), (v.grad, dv)):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)


def test_opcheck_attn_ops():
    torch.manual_seed(3)
    q, k, v = torch.randn(1, 4, 8, 16), torch.randn(1, 2, 8, 16), torch.randn(1, 2, 8, 16)
    torch.library.opcheck(torch.ops.stackkernels_amd.attn_fwd.default, (q, k, v, True, 0.25))
    out, lse = torch.ops.stackkernels_amd.attn_fwd(q, k, v, True, 0.25)
    do = torch.randn_like(out)
    torch.library.opcheck(torch.ops.stackkernels_amd.attn_bwd.default,
                          (do, q, k, v, out, lse, True, 0.25))


def test_fake_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 8, 5, 64, dtype=torch.bfloat16)
        k = torch.empty(2, 2, 7, 64, dtype=torch.bfloat16)
        out, lse = torch.ops.stackkernels_amd.attn_fwd(q, k, k, False, 0.125)
        assert out.shape == q.shape and out.dtype == q.dtype
        assert lse.shape == (2, 8, 5) and lse.dtype == torch.float32
        dq, dk, dv = torch.ops.stackkernels_amd.attn_bwd(out, q, k, k, out, lse, False, 0.125)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape
        o2 = torch.ops.stackkernels.flash_attn_op(q, k, k, True, None)
        assert o2.shape == q.shape


# ------------------------------------------------------------ decode custom op

def _decode_inputs(seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(2, 8, 1, 64, generator=g)
    k = torch.randn(2, 2, 40, 64, generator=g)
    v = torch.randn(2, 2, 40, 64, generator=g)
    return q, k, v


def test_flash_decode_op_matches_flash_decode():
    from stackkernels_amd.torch import flash_decode

    q, k, v = _decode_inputs()
    lens = torch.tensor([40, 7])
    torch.testing.assert_close(torch.ops.stackkernels.flash_decode_op(q, k, v, None),
                               flash_decode(q, k, v), rtol=0, atol=0)
    torch.testing.assert_close(torch.ops.stackkernels.flash_decode_op(q, k, v, 0.2, lens),
                               flash_decode(q, k, v, sm_scale=0.2, cache_seqlens=lens),
                               rtol=0, atol=0)


def test_flash_decode_op_compiled_fullgraph():
    from stackkernels_amd.torch import flash_decode

    q, k, v = _decode_inputs(1)
    lens = torch.tensor([33, 40])
    fn = torch.compile(lambda a, b, c, n: torch.ops.stackkernels.flash_decode_op(a, b, c, 0.1, n),
                       backend="aot_eager", fullgraph=True)
    torch.testing.assert_close(fn(q, k, v, lens),
                               flash_decode(q, k, v, sm_scale=0.1, cache_seqlens=lens),
                               rtol=0, atol=0)


def test_opcheck_decode_op():
    from stackkernels_amd._reference.torch.rope import precompute_freqs

    op = torch.ops.stackkernels_amd.decode.default
    q, k, v = _decode_inputs(2)
    lens = torch.tensor([40, 12])
    cos, sin = precompute_freqs(64, 64)
    torch.library.opcheck(op, (q, k, v, 0.125, lens, None, cos, sin, None, 5))
    torch.library.opcheck(op, (q, k, v, 0.125, None, None, None, None, None, 0))
    pool_k = torch.randn(4, 2, 32, 64)
    pool_v = torch.randn(4, 2, 32, 64)
    table = torch.tensor([[0, 1], [3, 2]])
    torch.library.opcheck(op, (q, pool_k, pool_v, 0.125, lens, table, cos, sin, lens - 1, 0))


def test_fakes_are_contiguous_for_strided_inputs():
    """The implementations return contiguous tensors whatever the inputs'
    strides, so the fakes must too (a stride mismatch breaks inductor)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(2, 7, 4, 32).transpose(1, 2)   # BSHD view of (2, 4, 7, 32)
        k = torch.empty(2, 9, 2, 32).transpose(1, 2)
        out, lse = torch.ops.stackkernels_amd.attn_fwd(q, k, k, True, 0.2)
        assert out.is_contiguous() and lse.is_contiguous()
        dq, dk, dv = torch.ops.stackkernels_amd.attn_bwd(q, q, k, k, out, lse, True, 0.2)
        assert dq.is_contiguous() and dk.is_contiguous() and dv.is_contiguous()
        qd = torch.empty(2, 1, 4, 32).transpose(1, 2)
        od = torch.ops.stackkernels_amd.decode(qd, k, k, 0.2, None, None, None, None, None, 0)
        assert od.is_contiguous()


def test_flash_attn_op_inductor_transposed_inputs():
    """torch.compile(backend='inductor', fullgraph=True), forward and backward,
    on BSHD inputs viewed as BHSD (transposed strides)."""
    torch.manual_seed(5)
    qb = torch.randn(2, 16, 4, 32)   # (B, S, H, D)
    kb = torch.randn(2, 24, 2, 32)
    vb = torch.randn(2, 24, 2, 32)
    do = torch.randn(2, 4, 16, 32)

    def run(fn):
        q, k, v = (t.clone().requires_grad_(True) for t in (qb, kb, vb))
        out = fn(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
        out.backward(do)
        return out.detach(), q.grad, k.grad, v.grad

    op = lambda a, b, c: torch.ops.stackkernels.flash_attn_op(a, b, c, True, None)  # noqa: E731
    got = run(torch.compile(op, backend="inductor", fullgraph=True))
    want = run(op)
    for a, b in zip(got, want):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
