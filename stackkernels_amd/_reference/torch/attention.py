"""PyTorch reference attention: the path CPU tensors and ``backend='reference'`` take.

Same function, arguments and results as the reference's
``attention_reference`` / ``repeat_kv``
(``src/stackkernels/_reference/torch/attention.py:10-76``), which this
build must keep so existing callers and tests behave identically:

* inputs upcast to float32; KV heads repeated in place for GQA/MQA;
* scores = q k^T * sm_scale (default 1/sqrt(D));
* bottom-right causal mask: key j visible to query i iff j <= i + (S_k - S_q);
* LSE = logsumexp over keys (``-inf`` on a row with no visible key);
* P = softmax with NaN (fully masked rows) replaced by 0;
* out = (P v) cast back to q's dtype.

The backward of this path is autograd through this function, as the
reference's ``FlashAttentionFunction.backward`` does.  Where autograd is not
available (inside a torch.library op implementation, which runs below the
autograd dispatch key), ``attention_reference_backward`` gives the same
gradients in closed form.
"""

from __future__ import annotations

import math

import torch


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    """(B, H_kv, S, D) -> (B, H_kv * n_rep, S, D); query head h reads KV head h // n_rep."""
    return x if n_rep == 1 else torch.repeat_interleave(x, repeats=n_rep, dim=1)


def attention_reference(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    is_causal: bool = False,
    sm_scale: float | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Scaled dot-product attention with MHA/GQA/MQA; returns (out, lse)."""
    _, h_q, s_q, d = q.shape
    _, h_kv, s_k, d_k = k.shape
    assert d == d_k, f"Head dimensions must match: {d} != {d_k}"
    assert h_q % h_kv == 0, f"Query heads {h_q} must be divisible by KV heads {h_kv}"
    scale = 1.0 / math.sqrt(d) if sm_scale is None else sm_scale

    # The reference's op sequence, op for op (same torch calls on the same
    # operands), so a CPU caller gets the reference's results bit for bit.
    # On a GPU the transposed key operand is made contiguous first: the
    # platform notes for these MI355X machines list torch's batched bf16
    # products with a transposed right operand among the forms that have
    # faulted the GPU (this build has not run that form there), and a device
    # result is compared within tolerance only.
    group = h_q // h_kv
    qf = q.float()
    kf = repeat_kv(k, group).float()
    vf = repeat_kv(v, group).float()
    kt = kf.transpose(-2, -1)
    if kt.device.type != "cpu":
        kt = kt.contiguous()
    scores = torch.matmul(qf, kt) * scale
    if is_causal:
        rows = torch.arange(s_q, device=q.device).unsqueeze(1)
        cols = torch.arange(s_k, device=k.device).unsqueeze(0)
        hidden = cols > (rows + (s_k - s_q))
        scores = scores.masked_fill(hidden.unsqueeze(0).unsqueeze(0), float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    probs = torch.nan_to_num(torch.softmax(scores, dim=-1), nan=0.0)
    out = torch.matmul(probs, vf).to(q.dtype)
    return out, lse


def attention_reference_backward(
    do: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    is_causal: bool = False,
    sm_scale: float | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gradients (dq, dk, dv) of ``attention_reference``'s output for upstream dO.

    The closed form of that function's autograd graph: P = softmax(S) with
    fully masked rows 0, dV = P^T dO, dP = dO V^T, dS = P * (dP - rowsum(dP * P)),
    dQ = scale dS K, dK = scale dS^T Q, with the GQA group summed for dK, dV.
    Computed in float32; results take the inputs' dtypes.
    """
    b, h_q, s_q, d = q.shape
    _, h_kv, s_k, _ = k.shape
    scale = 1.0 / math.sqrt(d) if sm_scale is None else sm_scale
    group = h_q // h_kv
    qf = q.float()
    kf = repeat_kv(k, group).float()
    vf = repeat_kv(v, group).float()
    dof = do.float()
    scores = (qf @ kf.transpose(-2, -1).contiguous()) * scale
    if is_causal:
        rows = torch.arange(s_q, device=q.device)[:, None]
        cols = torch.arange(s_k, device=q.device)[None, :]
        scores = scores.masked_fill(cols > rows + (s_k - s_q), float("-inf"))
    probs = torch.nan_to_num(torch.softmax(scores, dim=-1), nan=0.0)
    dvf = probs.transpose(-2, -1).contiguous() @ dof
    dp = dof @ vf.transpose(-2, -1).contiguous()
    ds = probs * (dp - (dp * probs).sum(dim=-1, keepdim=True))
    dqf = (ds @ kf) * scale
    dkf = (ds.transpose(-2, -1).contiguous() @ qf) * scale
    if group > 1:
        dkf = dkf.view(b, h_kv, group, s_k, d).sum(dim=2)
        dvf = dvf.view(b, h_kv, group, s_k, d).sum(dim=2)
    return dqf.to(q.dtype), dkf.to(k.dtype), dvf.to(v.dtype)


__all__ = ["attention_reference", "attention_reference_backward", "repeat_kv"]
