"""Write the golden attention vectors in this directory (``golden_attention.npz``).

Expected values come from torch's own ``scaled_dot_product_attention`` in
float64 on the CPU, with an explicit bottom-right boolean mask, ``enable_gqa``
for grouped heads, and torch autograd for the gradients -- a library routine
independent of ``oracle/attention_oracle.py``, which these vectors pin.  LSE
comes from ``scipy.special.logsumexp`` over float64 scores.

Rows that see no key (causal with S_q > S_k) are not passed to SDPA (it
returns NaN there); their expected values are the reference's rule for such
rows (``src/stackkernels/_reference/torch/attention.py:70-73``): O = 0,
LSE = -inf, dQ = 0, and no contribution to dK/dV.  Attention rows are
independent, so SDPA on the remaining rows gives their exact values.

Run: ``python tests/golden/make_golden.py`` (CPU, a few seconds).
"""

import os

import numpy as np
import scipy.special
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))

# name: (B, Hq, Hkv, Sq, Sk, D, causal, sm_scale)
CASES = {
    "mha_noncausal": (1, 4, 4, 16, 16, 32, False, None),
    "gqa_causal_prefix": (1, 4, 2, 8, 24, 32, True, None),
    "mqa_causal_square": (1, 2, 1, 12, 12, 16, True, None),
    "gqa_causal_chunked": (1, 4, 2, 10, 6, 32, True, None),
    "decode_mqa": (1, 4, 1, 1, 40, 32, False, None),
    "custom_scale": (1, 2, 2, 5, 7, 8, False, -0.3),
}


def sdpa_case(b, hq, hkv, sq, sk, d, causal, sm_scale, rng):
    q = rng.standard_normal((b, hq, sq, d))
    k = rng.standard_normal((b, hkv, sk, d))
    v = rng.standard_normal((b, hkv, sk, d))
    do = rng.standard_normal((b, hq, sq, d))
    scale = 1.0 / np.sqrt(d) if sm_scale is None else sm_scale
    i = np.arange(sq)[:, None]
    j = np.arange(sk)[None, :]
    allowed = (j <= i + (sk - sq)) if causal else np.ones((sq, sk), bool)
    live = allowed.any(axis=1)  # rows that see at least one key

    tq = torch.tensor(q[:, :, live], requires_grad=True)
    tk = torch.tensor(k, requires_grad=True)
    tv = torch.tensor(v, requires_grad=True)
    mask = torch.tensor(allowed[live])
    out_live = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=scale,
                                              enable_gqa=(hq != hkv))
    out_live.backward(torch.tensor(do[:, :, live]))

    out = np.zeros((b, hq, sq, d))
    out[:, :, live] = out_live.detach().numpy()
    dq = np.zeros((b, hq, sq, d))
    dq[:, :, live] = tq.grad.numpy()
    dk = tk.grad.numpy()
    dv = tv.grad.numpy()

    kk = np.repeat(k, hq // hkv, axis=1)
    scores = np.einsum("bhid,bhjd->bhij", q, kk) * scale
    scores = np.where(allowed[None, None], scores, -np.inf)
    with np.errstate(divide="ignore"):
        lse = scipy.special.logsumexp(scores, axis=-1)
    lse = np.where(live[None, None], lse, -np.inf)
    return dict(q=q, k=k, v=v, do=do, out=out, lse=lse, dq=dq, dk=dk, dv=dv,
                meta=np.array([b, hq, hkv, sq, sk, d, int(causal)]),
                scale=np.array(scale))


def main():
    rng = np.random.default_rng(20261201)
    arrays = {}
    for name, spec in CASES.items():
        for key, val in sdpa_case(*spec, rng).items():
            arrays[f"{name}/{key}"] = val
    path = os.path.join(HERE, "golden_attention.npz")
    np.savez_compressed(path, **arrays)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
