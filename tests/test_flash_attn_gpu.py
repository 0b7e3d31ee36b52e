"""GPU parity of the HIP forward (and fp32 backward) against the oracle.

Grids follow the reference's tests/ops/test_flash_attn.py (heads x seq lens x
head dims x causal), here in fp32, fp16 and bf16 on the device, plus the edge
cases the kernels have to get right: ragged tiles, fully masked rows, empty
keys, strided inputs, custom and negative scales, and the full-size BASELINE
forward config checked against the repo's PyTorch reference path run in fp32.
"""

import numpy as np
import pytest
import torch

import stackkernels_amd
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd
from stackkernels_amd._reference.torch.attention import attention_reference
from stackkernels_amd.torch import FlashAttention, flash_attention

from _gpu_util import (TOL, assert_close_maxabs, assert_lse_close, make_qkv, native_loaded,
                       np64, oracle_fwd)

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
@pytest.mark.parametrize("seq_lens", [(32, 32), (16, 64), (64, 32)])
@pytest.mark.parametrize("head_dim", [64, 80, 96, 128, 256])
@pytest.mark.parametrize("is_causal", [False, True])
def test_forward_grid(device, dtype, heads, seq_lens, head_dim, is_causal):
    hq, hkv = heads
    sq, sk = seq_lens
    q, k, v = make_qkv(2, hq, hkv, sq, sk, head_dim, dtype)
    out, lse = flash_attn_fwd(q, k, v, is_causal=is_causal)
    assert native_loaded()
    ref, ref_lse = oracle_fwd(q, k, v, is_causal)
    assert out.dtype == dtype and out.shape == q.shape
    assert_close_maxabs(out, ref, TOL[dtype], "O")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("sq,sk", [(1, 1), (1, 300), (3, 5), (65, 65), (127, 129), (200, 77),
                                   (129, 1000), (300, 300), (513, 257)])
@pytest.mark.parametrize("is_causal", [False, True])
def test_forward_ragged_shapes(device, dtype, sq, sk, is_causal):
    q, k, v = make_qkv(1, 4, 2, sq, sk, 128, dtype, seed=sq * 1000 + sk)
    out, lse = flash_attn_fwd(q, k, v, is_causal=is_causal)
    ref, ref_lse = oracle_fwd(q, k, v, is_causal)
    assert_close_maxabs(out, ref, TOL[dtype], "O")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_fully_masked_rows_are_zero(device, dtype):
    # causal with S_q > S_k: rows i < S_q - S_k see no key -> O = 0, LSE = -inf
    q, k, v = make_qkv(2, 4, 2, 200, 70, 64, dtype)
    out, lse = flash_attn_fwd(q, k, v, is_causal=True)
    assert torch.all(out[:, :, :130] == 0)
    assert torch.all(torch.isneginf(lse[:, :, :130]))
    ref, ref_lse = oracle_fwd(q, k, v, True)
    assert_close_maxabs(out, ref, TOL[dtype], "O")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_empty_keys(device, dtype):
    q, k, v = make_qkv(1, 2, 2, 10, 0, 64, dtype)
    out, lse = flash_attn_fwd(q, k, v)
    assert torch.all(out == 0) and torch.all(torch.isneginf(lse))


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("scale", [0.05, 1.0, -0.09])
def test_custom_and_negative_scale(device, dtype, scale):
    q, k, v = make_qkv(1, 4, 4, 70, 90, 64, dtype)
    out, lse = flash_attn_fwd(q, k, v, is_causal=True, sm_scale=scale)
    ref, ref_lse = oracle_fwd(q, k, v, True, scale)
    assert_close_maxabs(out, ref, TOL[dtype], "O")
    assert_lse_close(lse, ref_lse)


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
def test_strided_bshd_inputs(device, dtype):
    # (B, S, H, D) storage viewed as BHSD, the layout of examples/stackformer_integration.py
    g = torch.Generator().manual_seed(3)
    base = [torch.randn(2, 100, 8, 64, generator=g).to(dtype).to(device) for _ in range(3)]
    q, k, v = (t.transpose(1, 2) for t in base)
    out = flash_attention(q, k, v, is_causal=True)
    ref, _ = oracle_fwd(q, k, v, True)
    assert_close_maxabs(out, ref, TOL[dtype], "O")


def test_module_and_custom_op_on_device(device):
    q, k, v = make_qkv(1, 4, 2, 64, 64, 64, torch.bfloat16)
    out = FlashAttention(is_causal=True)(q, k, v)
    op = torch.ops.stackkernels.flash_attn_op(q, k, v, True, None)
    assert torch.equal(out, op)
    assert_close_maxabs(out, oracle_fwd(q, k, v, True)[0], TOL[torch.bfloat16], "O")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
def test_forward_deterministic(device, dtype):
    q, k, v = make_qkv(2, 8, 2, 300, 300, 128, dtype)
    a, la = flash_attn_fwd(q, k, v, is_causal=True)
    b, lb = flash_attn_fwd(q, k, v, is_causal=True)
    assert torch.equal(a, b) and torch.equal(la, lb)


def test_config1_fp32_plumbing_anchor(device):
    """fp32 non-causal MHA B=2 H=4 S=128 D=64 -- fp32 tolerance 1e-4."""
    q, k, v = make_qkv(2, 4, 4, 128, 128, 64, torch.float32, seed=0)
    out, lse = flash_attn_fwd(q, k, v)
    ref, ref_lse = oracle_fwd(q, k, v, False)
    assert_close_maxabs(out, ref, 1e-4, "O")
    assert_lse_close(lse, ref_lse)
    cpu_out, _ = attention_reference(q.cpu(), k.cpu(), v.cpu())
    assert_close_maxabs(out, cpu_out, 1e-4, "O vs CPU reference path")


def _reference_fp32_chunked(q, k, v, causal):
    """The repo's PyTorch reference path in fp32 on the device, one batch at a time."""
    outs, lses = [], []
    for b in range(q.shape[0]):
        o, l = attention_reference(q[b:b + 1].float(), k[b:b + 1].float(), v[b:b + 1].float(),
                                   is_causal=causal)
        outs.append(o)
        lses.append(l)
    return torch.cat(outs), torch.cat(lses)


def test_config2_full_size_forward(device):
    """bf16 causal MHA B=4 H=32 S=4096 D=128 vs the fp32 reference path."""
    q, k, v = make_qkv(4, 32, 32, 4096, 4096, 128, torch.bfloat16, seed=0)
    out, lse = flash_attn_fwd(q, k, v, is_causal=True)
    torch.cuda.synchronize()
    for b in range(4):
        ref, ref_lse = attention_reference(q[b:b + 1].float(), k[b:b + 1].float(), v[b:b + 1].float(),
                                           is_causal=True)
        assert_close_maxabs(out[b:b + 1].float(), ref, 2e-2, f"O batch {b}")
        assert_lse_close(lse[b:b + 1], ref_lse, f"lse batch {b}")


@pytest.mark.parametrize("heads", [(4, 4), (4, 2), (4, 1)])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("sq,sk", [(16, 16), (70, 130), (130, 70)])
def test_backward_fp32(device, heads, is_causal, sq, sk):
    from oracle import attention_oracle as orc

    hq, hkv = heads
    q, k, v = make_qkv(2, hq, hkv, sq, sk, 64, torch.float32)
    q.requires_grad_(True), k.requires_grad_(True), v.requires_grad_(True)
    out = flash_attention(q, k, v, is_causal=is_causal)
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(7)).to(device)
    out.backward(g)
    dq, dk, dv = orc.attention_backward(np64(q), np64(k), np64(v), np64(g), is_causal)
    assert_close_maxabs(q.grad, dq, 1e-4, "dQ")
    assert_close_maxabs(k.grad, dk, 1e-4, "dK")
    assert_close_maxabs(v.grad, dv, 1e-4, "dV")
