"""Elementwise error bound for a 16-bit FlashAttention-2 backward (test helper).

The 16-bit kernels compute the backward in fp32 but round some operands to the
input type (bf16 / fp16, unit roundoff u = 2^-8 / 2^-11) on the way, as
FlashAttention-2 does:

* O is stored in the input type by the forward (whose P was rounded before
  P V), so delta = rowsum(dO * O) is off by at most 2u * sum_d (P|V|)_d |dO_d|;
* P is rounded before dV = P^T dO;
* dS = P (dP - delta) is rounded before dQ = scale dS K and dK = scale dS^T Q;
* above 128 head-dim columns (padded head dim 256) the dK/dV kernel hands P
  from one of its wave roles to the other in the input type (its LDS
  budget), so dS is formed from a rounded P as well;
* each gradient is rounded to the input type at the end.

Running the error of each rounding through the products gives, per element,
the sum of magnitudes the rounding can move (float64, from the exact P, dP,
delta of the oracle):

    A_dV = P^T |dO|                       (summed over a KV head's query group)
    A_dQ = |scale| (|dS| + 2 P e) |K|,    e_i = sum_d (P|V|)_id |dO_id|
    A_dK = |scale| (|dS| + 2 P e)^T |Q|   (summed over the group)

Each rounding can also be off by half the type's subnormal spacing (eta =
2^-25 in fp16, where P and dS values below 2^-14 lose relative precision;
negligible in bf16), so every visible (i, j) adds eta / u to the weights of
P and dS above.  Where dS is formed from a rounded P (head dim above 128),
that rounding adds |dS| and (eta / u) |dP - delta| to the weight of dS.  The
bound is

    |ours - exact| <= |path - exact| + K u (|exact| + A),   K = 2,

where ``path`` is the repo's PyTorch reference path (fp32 autograd, gradients
returned in the input type) and ``exact`` the float64 oracle.  K = 2 leaves
room for fp32 accumulation and for first-order terms counted once; the fp32
exponentials and the saved LSE add errors near 2^-23, far below u.  A
kernel that drops or misplaces a term misses the bound by orders of
magnitude, since A is a sum of magnitudes scaled by u, while the kernel's
rounding stays within it whatever the gradient's size.
"""

import numpy as np

from oracle import attention_oracle as orc

K_ROUNDING = 2.0
UNIT_ROUNDOFF = {"bf16": 2.0 ** -8, "f16": 2.0 ** -11}
SUBNORMAL_HALF_STEP = {"bf16": 2.0 ** -134, "f16": 2.0 ** -25}


def rounding_mass(q, k, v, do, causal, scale, dtype):
    """(A_dQ, A_dK, A_dV), float64, shaped like dQ, dK, dV, for element type
    ``dtype`` ("bf16" / "f16")."""
    q, k, v, do = (np.asarray(t, dtype=np.float64) for t in (q, k, v, do))
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    g = hq // hkv
    sc = 1.0 / np.sqrt(d) if scale is None else float(scale)
    kk = orc.repeat_kv(k, g)
    vv = orc.repeat_kv(v, g)
    p = orc.softmax_probs(q, k, causal, scale)
    out = p @ vv
    dp = do @ np.swapaxes(vv, -1, -2)
    delta = (do * out).sum(-1, keepdims=True)
    ds = p * (dp - delta)
    e = ((p @ np.abs(vv)) * np.abs(do)).sum(-1, keepdims=True)
    floor = (SUBNORMAL_HALF_STEP[dtype] / UNIT_ROUNDOFF[dtype]) * (p > 0)
    w = np.abs(ds) + 2.0 * p * e + floor
    if d > 128:  # dS formed from P rounded to the input type
        w = w + np.abs(ds) + floor * np.abs(dp - delta)
    a_dq = abs(sc) * (w @ np.abs(kk))
    a_dk = abs(sc) * (np.swapaxes(w, -1, -2) @ np.abs(q))
    a_dv = np.swapaxes(p + floor, -1, -2) @ np.abs(do)
    a_dk = a_dk.reshape(b, hkv, g, sk, d).sum(2)
    a_dv = a_dv.reshape(b, hkv, g, sk, d).sum(2)
    return a_dq, a_dk, a_dv


def check_backward(ours, path, exact, mass, dtype: str, what: str):
    """Assert |ours - exact| <= |path - exact| + K u (|exact| + mass) elementwise.
    Returns the largest fraction of the rounding allowance used."""
    ours, path, exact, mass = (np.asarray(t, dtype=np.float64) for t in (ours, path, exact, mass))
    assert ours.shape == exact.shape, (what, ours.shape, exact.shape)
    assert np.isfinite(ours).all(), f"{what}: non-finite values"
    allow = K_ROUNDING * UNIT_ROUNDOFF[dtype] * (np.abs(exact) + mass) + 1e-7
    excess = np.abs(ours - exact) - np.abs(path - exact)
    used = float((excess / allow).max()) if ours.size else 0.0
    if used > 1.0:
        i = np.unravel_index(int(np.argmax(excess / allow)), ours.shape)
        raise AssertionError(
            f"{what}: error {abs(ours[i] - exact[i]):.3e} at {i} exceeds the path's "
            f"{abs(path[i] - exact[i]):.3e} + rounding allowance {allow[i]:.3e} "
            f"(|exact| {abs(exact[i]):.3e}, mass {mass[i]:.3e})")
    return used
