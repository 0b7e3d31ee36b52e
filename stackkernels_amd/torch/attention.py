"""PyTorch attention API over the gfx950 HIP kernels.

Drop-in for ``stackkernels.torch.attention``
(``src/stackkernels/torch/attention.py:17-231``): the same functions,
autograd Function, module, custom op and ``__all__``.  What changes is what
runs behind them: ROCm device tensors go to ``libsk_attn.so`` (forward,
backward and split-KV decode kernels written for gfx950); CPU tensors and
``backend='reference'`` run the PyTorch reference path, exactly where the
reference did.
"""

from __future__ import annotations

import math
from typing import Any

import torch
import torch.nn as nn

from stackkernels_amd._core.attention.decode import flash_decode as core_flash_decode
from stackkernels_amd._core.attention.decode import flash_decode_paged as core_flash_decode_paged
from stackkernels_amd._core.attention.flash_bwd import flash_attn_bwd
from stackkernels_amd._core.attention._rope import rope_args, rope_rotate
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd
from stackkernels_amd._reference.torch.attention import (
    attention_reference,
    attention_reference_backward,
)
from stackkernels_amd._reference.torch.rope import apply_rope_at, rope_positions
from stackkernels_amd.torch._dispatch import should_use_hip
from stackkernels_amd.torch._utils import ensure_contiguous


class FlashAttentionFunction(torch.autograd.Function):
    """FlashAttention-2 forward/backward with MHA, GQA and MQA support.

    ``forward(ctx, q, k, v, is_causal=False, sm_scale=None)`` returns the
    output; ``backward`` returns ``(dq, dk, dv, None, None)``.  Reference:
    ``src/stackkernels/torch/attention.py:17-102``.
    """

    @staticmethod
    def forward(
        ctx: Any,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        is_causal: bool = False,
        sm_scale: float | None = None,
    ) -> torch.Tensor:
        use_hip = should_use_hip(q)
        scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else sm_scale
        ctx.use_hip = use_hip
        ctx.is_causal = is_causal
        ctx.sm_scale = scale
        qc, kc, vc = ensure_contiguous(q), ensure_contiguous(k), ensure_contiguous(v)
        if use_hip:
            out, lse = flash_attn_fwd(qc, kc, vc, is_causal=is_causal, sm_scale=scale)
        else:
            out, lse = attention_reference(qc, kc, vc, is_causal=is_causal, sm_scale=scale)
        ctx.save_for_backward(qc, kc, vc, out, lse)
        return out

    @staticmethod
    def backward(ctx: Any, do: torch.Tensor):
        q, k, v, out, lse = ctx.saved_tensors
        do = ensure_contiguous(do)
        if ctx.use_hip:
            dq, dk, dv = flash_attn_bwd(do, q, k, v, out, lse, is_causal=ctx.is_causal,
                                        sm_scale=ctx.sm_scale)
            return dq, dk, dv, None, None
        # Reference path: autograd through the reference forward
        # (src/stackkernels/torch/attention.py:82-102).
        qr, kr, vr = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        with torch.enable_grad():
            out_ref, _ = attention_reference(qr, kr, vr, is_causal=ctx.is_causal,
                                             sm_scale=ctx.sm_scale)
            out_ref.backward(do)
        return qr.grad, kr.grad, vr.grad, None, None


def flash_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    is_causal: bool = False,
    sm_scale: float | None = None,
    *,
    rope_cos: torch.Tensor | None = None,
    rope_sin: torch.Tensor | None = None,
    start_pos: int | torch.Tensor = 0,
) -> torch.Tensor:
    """Flash Attention forward (differentiable).

    Supports MHA (H_q == H_kv), GQA (H_q > H_kv > 1), MQA (H_kv == 1), the
    bottom-right causal mask ``k <= q + (S_k - S_q)`` and head dims up to 256
    (64, 80, 96, 128, 256 as in the reference, and any other up to 256).

    Args:
        q: (B, H_q, S_q, D).  k, v: (B, H_kv, S_k, D).
        is_causal: apply the bottom-right causal mask.
        sm_scale: score scale, default 1/sqrt(D).
        rope_cos, rope_sin: optional (max_seq_len, D) RoPE tables
            (``precompute_freqs``).  q is then rotated as the reference's
            ``apply_rope(q, cos=..., sin=..., start_pos=...)`` would, inside the
            kernel's prologue: query row i at position ``start_pos + i``.  k is
            taken as already rotated (as ``kv_cache_update`` with the same tables
            stores it).  Differentiable: the backward rotates dq back by the
            adjoint, as the reference's ``RoPEFunction.backward`` does.  Not in
            the reference, which rotates in a separate pass.
        start_pos: int, or integer (B,) tensor of per-row positions.

    Returns:
        (B, H_q, S_q, D) in q's dtype.
    """
    if rope_cos is None and rope_sin is None:
        return FlashAttentionFunction.apply(q, k, v, is_causal, sm_scale)
    if should_use_hip(q):
        return _FlashAttentionRoPEFunction.apply(q, k, v, is_causal, sm_scale, rope_cos, rope_sin,
                                                 start_pos)
    # CPU / reference path: the unfused pipeline, differentiable through autograd.
    qr = _rope_reference(q, rope_cos, rope_sin, start_pos)
    out, _ = attention_reference(qr, k, v, is_causal=is_causal, sm_scale=sm_scale)
    return out


class _FlashAttentionRoPEFunction(torch.autograd.Function):
    """``flash_attention`` with q rotated in the forward kernel's prologue.

    Forward: ``sk_attn_fwd_rope`` (the rotated q is never written out).
    Backward: the unfused pipeline's gradient, with the rotated q rebuilt by
    ``sk_rope_rotate`` bit for bit as the forward formed it:
    ``dq = R^T dq_rot`` where ``(dq_rot, dk, dv)`` is the attention backward at
    the rotated q, i.e. the reference's ``RoPEFunction.backward``
    (``src/stackkernels/torch/embedding.py:46-66``) after its attention
    backward (``torch/attention.py:63-102``).  k is taken as already rotated,
    so its gradient is the attention's.  The tables get no gradient.
    """

    @staticmethod
    def forward(ctx: Any, q, k, v, is_causal, sm_scale, rope_cos, rope_sin, start_pos):
        scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else sm_scale
        qc, kc, vc = ensure_contiguous(q), ensure_contiguous(k), ensure_contiguous(v)
        out, lse = flash_attn_fwd(qc, kc, vc, is_causal=is_causal, sm_scale=scale,
                                  rope_cos=rope_cos, rope_sin=rope_sin, start_pos=start_pos)
        ctx.is_causal = is_causal
        ctx.sm_scale = scale
        ctx.rope = rope_args(rope_cos, rope_sin, start_pos, q.shape[0], q.shape[-1], q.device)
        ctx.save_for_backward(qc, kc, vc, out, lse)
        return out

    @staticmethod
    def backward(ctx: Any, do: torch.Tensor):
        q, k, v, out, lse = ctx.saved_tensors
        q_rot = rope_rotate(q, ctx.rope)
        dq, dk, dv = flash_attn_bwd(ensure_contiguous(do), q_rot, k, v, out, lse,
                                    is_causal=ctx.is_causal, sm_scale=ctx.sm_scale)
        del q_rot
        dq = rope_rotate(dq, ctx.rope, inverse=True, out=dq)
        return dq, dk, dv, None, None, None, None, None


def _rope_reference(x, cos, sin, start_pos):
    """CPU path of the fused rotation: token t of row b at start_pos(+[b]) + t."""
    if cos is None or sin is None:
        raise ValueError("RoPE needs both cos and sin tables")
    if cos.dim() != 2 or cos.shape != sin.shape or cos.shape[1] != x.shape[-1]:
        raise ValueError(f"RoPE tables must be (max_seq_len, {x.shape[-1]}), got "
                         f"{tuple(cos.shape)} and {tuple(sin.shape)}")
    pos = rope_positions(start_pos, x.shape[0], x.shape[2], cos.shape[0])
    return apply_rope_at(x, cos, sin, pos)


def flash_decode(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    sm_scale: float | None = None,
    cache_seqlens: torch.Tensor | None = None,
    block_table: torch.Tensor | None = None,
    *,
    rope_cos: torch.Tensor | None = None,
    rope_sin: torch.Tensor | None = None,
    start_pos: int | torch.Tensor = 0,
) -> torch.Tensor:
    """Split-KV decode for one query token (S_q = 1) over the whole cache.

    Args:
        q: (B, H_q, 1, D).  k, v: (B, H_kv, S_k, D); any b/h/s strides.
        sm_scale: score scale, default 1/sqrt(D).
        cache_seqlens: optional integer (B,): row b attends to the first
            ``min(cache_seqlens[b], S_k)`` keys of its cache; a row with no
            key gives zeros.  Not in the reference, which decodes every row
            over all S_k keys (``None``, the default, does the same).
        block_table: optional integer (B, max_pages) for a paged cache: then
            k, v are page pools (num_pages, H_kv, page_size, D), page_size a
            multiple of 32, key j of row b is row ``j % page_size`` of page
            ``block_table[b, j // page_size]``, and cache_seqlens is required.
        rope_cos, rope_sin: optional (max_seq_len, D) RoPE tables; q is then
            rotated to position ``start_pos`` inside the decode kernel (the
            reference's ``apply_rope`` on q, fused).  The cache holds rotated
            keys (``kv_cache_update`` with the same tables writes them so).
        start_pos: int, or integer (B,) tensor: each row's query position
            (typically ``cache_seqlens - 1``).

    Returns:
        (B, H_q, 1, D) in q's dtype.
    """
    rope = {}
    if rope_cos is not None or rope_sin is not None:
        rope = dict(rope_cos=rope_cos, rope_sin=rope_sin, start_pos=start_pos)
    if block_table is not None:
        if cache_seqlens is None:
            raise ValueError("a paged decode (block_table) needs cache_seqlens")
        if should_use_hip(q):
            return core_flash_decode_paged(q, k, v, block_table, cache_seqlens, sm_scale=sm_scale,
                                           **rope)
        if rope:
            q = _rope_reference(q, rope_cos, rope_sin, start_pos)
        return _decode_paged_reference(q, k, v, sm_scale, cache_seqlens, block_table)
    elif should_use_hip(q):
        return core_flash_decode(q, k, v, sm_scale=sm_scale, cache_seqlens=cache_seqlens, **rope)
    if rope:
        q = _rope_reference(q, rope_cos, rope_sin, start_pos)
    if cache_seqlens is None:
        out, _ = attention_reference(q, k, v, is_causal=False, sm_scale=sm_scale)
        return out
    return _decode_varlen_reference(q, k, v, sm_scale, cache_seqlens)


def _decode_paged_reference(q, k_pool, v_pool, sm_scale, cache_seqlens, block_table):
    """CPU path of the paged decode: each row's visible keys gathered from its
    pages (keys past the row's length, or in a page outside the pool, are
    left out), then the reference attention; zeros for a row with no key."""
    table = torch.as_tensor(block_table).to("cpu", torch.int64)
    lens = torch.as_tensor(cache_seqlens).to("cpu", torch.int64)
    num_pages, _, page_size, _ = k_pool.shape
    b, max_pages = table.shape
    if lens.dim() != 1 or lens.shape[0] != b or q.shape[0] != b:
        raise ValueError(f"cache_seqlens must have shape ({b},), got {tuple(lens.shape)}")
    out = torch.zeros_like(q)
    for i in range(b):
        n = int(min(max(int(lens[i]), 0), max_pages * page_size))
        keys = [j for j in range(n) if 0 <= int(table[i, j // page_size]) < num_pages]
        if not keys:
            continue
        idx = torch.tensor(keys)
        pg = table[i, idx // page_size].to(k_pool.device)
        off = (idx % page_size).to(k_pool.device)
        k = k_pool[pg, :, off].permute(1, 0, 2).unsqueeze(0)  # (1, H_kv, n_keys, D)
        v = v_pool[pg, :, off].permute(1, 0, 2).unsqueeze(0)
        out[i:i + 1], _ = attention_reference(q[i:i + 1], k, v, is_causal=False, sm_scale=sm_scale)
    return out


def _decode_varlen_reference(q, k, v, sm_scale, cache_seqlens):
    """CPU path of flash_decode with per-row cache lengths: the reference
    attention of each row over its first keys (zeros for an empty row)."""
    b, _, sq, _ = q.shape
    assert sq == 1, f"flash_decode requires q_len == 1, got {sq}"
    lens = torch.as_tensor(cache_seqlens).to("cpu", torch.int64)
    if lens.dim() != 1 or lens.shape[0] != b:
        raise ValueError(f"cache_seqlens must have shape ({b},), got {tuple(lens.shape)}")
    out = torch.zeros_like(q)
    sk = k.shape[2]
    for i in range(b):
        n = int(min(max(int(lens[i]), 0), sk))
        if n > 0:
            out[i:i + 1], _ = attention_reference(q[i:i + 1], k[i:i + 1, :, :n], v[i:i + 1, :, :n],
                                                  is_causal=False, sm_scale=sm_scale)
    return out


class FlashAttention(nn.Module):
    """FlashAttention module with MHA, GQA and MQA support.

    Args:
        is_causal: apply the bottom-right aligned causal mask. Default: False.
        sm_scale: softmax scale. Default: 1/sqrt(D).

    Examples:
        >>> attn = FlashAttention(is_causal=True)
        >>> q = torch.randn(2, 8, 1024, 64)
        >>> out = attn(q, q, q)
    """

    def __init__(self, is_causal: bool = False, sm_scale: float | None = None) -> None:
        super().__init__()
        self.is_causal = is_causal
        self.sm_scale = sm_scale

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        return flash_attention(q, k, v, is_causal=self.is_causal, sm_scale=self.sm_scale)


# torch.library ops.  ``torch.ops.stackkernels.flash_attn_op`` keeps the
# reference's name and schema (src/stackkernels/torch/attention.py:200-223)
# and becomes differentiable: it is a composite of two ops of this package,
# ``stackkernels_amd::attn_fwd`` (output and LSE) and ``attn_bwd``, each with
# a fake (meta) implementation, and attn_fwd carries register_autograd, so
# torch.compile graphs run both the forward and the backward without a graph
# break.  If flash_attn_op is already registered in this process (the
# original package imported alongside), that registration is kept.
def _attn_fwd_impl(q, k, v, is_causal, sm_scale):
    qc, kc, vc = ensure_contiguous(q), ensure_contiguous(k), ensure_contiguous(v)
    if should_use_hip(qc):
        return flash_attn_fwd(qc, kc, vc, is_causal=is_causal, sm_scale=sm_scale)
    return attention_reference(qc, kc, vc, is_causal=is_causal, sm_scale=sm_scale)


def _attn_bwd_impl(do, q, k, v, out, lse, is_causal, sm_scale):
    do = ensure_contiguous(do)
    if should_use_hip(q):
        return flash_attn_bwd(do, q, k, v, out, lse, is_causal=is_causal, sm_scale=sm_scale)
    return attention_reference_backward(do, q, k, v, is_causal=is_causal, sm_scale=sm_scale)


def _register_ops() -> bool:
    @torch.library.custom_op("stackkernels_amd::attn_fwd", mutates_args=())
    def _attn_fwd_op(
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        is_causal: bool,
        sm_scale: float,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        out, lse = _attn_fwd_impl(q, k, v, is_causal, sm_scale)
        return out, lse

    # The fakes return contiguous tensors, as the implementations do (both
    # paths make their inputs contiguous first), whatever the inputs' strides.
    @_attn_fwd_op.register_fake
    def _attn_fwd_fake(q, k, v, is_causal, sm_scale):
        B, Hq, Sq, _ = q.shape
        return q.new_empty(q.shape), q.new_empty((B, Hq, Sq), dtype=torch.float32)

    @torch.library.custom_op("stackkernels_amd::attn_bwd", mutates_args=())
    def _attn_bwd_op(
        do: torch.Tensor,
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        out: torch.Tensor,
        lse: torch.Tensor,
        is_causal: bool,
        sm_scale: float,
    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        dq, dk, dv = _attn_bwd_impl(do, q, k, v, out, lse, is_causal, sm_scale)
        return dq, dk, dv

    @_attn_bwd_op.register_fake
    def _attn_bwd_fake(do, q, k, v, out, lse, is_causal, sm_scale):
        return q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape)

    def _setup_context(ctx, inputs, output):
        q, k, v, is_causal, sm_scale = inputs
        out, lse = output
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.is_causal = is_causal
        ctx.sm_scale = sm_scale

    def _backward(ctx, dout, dlse):
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = torch.ops.stackkernels_amd.attn_bwd(
            dout, q, k, v, out, lse, ctx.is_causal, ctx.sm_scale)
        return dq, dk, dv, None, None

    _attn_fwd_op.register_autograd(_backward, setup_context=_setup_context)

    try:
        torch.ops.stackkernels.flash_attn_op  # noqa: B018
        return False
    except (AttributeError, RuntimeError):
        pass
    lib = torch.library.Library("stackkernels", "FRAGMENT")
    lib.define("flash_attn_op(Tensor q, Tensor k, Tensor v, bool is_causal, float? sm_scale) -> Tensor")

    def _flash_attn_op(q, k, v, is_causal, sm_scale):
        scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else sm_scale
        return torch.ops.stackkernels_amd.attn_fwd(q, k, v, is_causal, scale)[0]

    lib.impl("flash_attn_op", _flash_attn_op, "CompositeImplicitAutograd")
    _LIBS.append(lib)  # a Library's registrations last as long as the object
    return True


def _register_decode_ops() -> None:
    """``torch.ops.stackkernels_amd.decode`` (every flash_decode argument, fake
    implementation for tracing) and ``torch.ops.stackkernels.flash_decode_op``
    (the decode counterpart of ``flash_attn_op``), so compiled graphs keep the
    decode kernel instead of breaking at the library call.  Eager
    ``flash_decode`` calls the launchers directly."""

    @torch.library.custom_op("stackkernels_amd::decode", mutates_args=())
    def _decode_op(
        q: torch.Tensor,
        k: torch.Tensor,
        v: torch.Tensor,
        sm_scale: float,
        cache_seqlens: torch.Tensor | None,
        block_table: torch.Tensor | None,
        rope_cos: torch.Tensor | None,
        rope_sin: torch.Tensor | None,
        rope_positions: torch.Tensor | None,
        start_pos: int,
    ) -> torch.Tensor:
        pos = rope_positions if rope_positions is not None else start_pos
        out = flash_decode(q, k, v, sm_scale=sm_scale, cache_seqlens=cache_seqlens,
                           block_table=block_table, rope_cos=rope_cos, rope_sin=rope_sin,
                           start_pos=pos)
        # (a custom op may not return an input or a view of one)
        return out.clone() if out.data_ptr() == q.data_ptr() else out

    @_decode_op.register_fake
    def _decode_fake(q, k, v, sm_scale, cache_seqlens, block_table, rope_cos, rope_sin,
                     rope_positions, start_pos):
        return q.new_empty(q.shape)

    try:
        torch.ops.stackkernels.flash_decode_op  # noqa: B018
        return
    except (AttributeError, RuntimeError):
        pass
    lib = torch.library.Library("stackkernels", "FRAGMENT")
    lib.define("flash_decode_op(Tensor q, Tensor k, Tensor v, float? sm_scale, "
               "Tensor? cache_seqlens=None) -> Tensor")

    def _flash_decode_op(q, k, v, sm_scale, cache_seqlens=None):
        scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else sm_scale
        return torch.ops.stackkernels_amd.decode(q, k, v, scale, cache_seqlens, None, None, None,
                                                 None, 0)

    lib.impl("flash_decode_op", _flash_decode_op, "CompositeImplicitAutograd")
    _LIBS.append(lib)


_LIBS: list = []
_CUSTOM_OP_REGISTERED = _register_ops()
_register_decode_ops()


__all__ = [
    "flash_attention",
    "flash_decode",
    "FlashAttention",
    "FlashAttentionFunction",
]
