"""The 16-bit backward's error bound (``tests/_bwd_bound.py``) is neither too
tight nor too loose: a numpy model of a bf16 / fp16 FlashAttention-2 backward
with the GPU kernels' rounding points stays within it on the shapes whose
gradients reach 10-30 (where a fixed 2e-2 cannot hold), and plausible kernel
mistakes, planted in the model, break it."""

import numpy as np
import pytest

from oracle import attention_oracle as orc

from _bwd_bound import check_backward, rounding_mass


def _model_backward(q, k, v, do, causal, scale, dt, mistake=None):
    """fp32 FlashAttention-2 backward with the kernels' rounding: O stored in
    dt by a forward that rounds P before P V; delta from the stored O; P and
    dS rounded to dt before their products (above 128 head-dim columns dS is
    formed from the rounded P, which the dK/dV kernel hands between its wave
    roles in dt); gradients rounded to dt."""
    r = lambda x: orc.round_to(np.asarray(x, dtype=np.float32), dt)  # noqa: E731
    b, hq, sq, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    g = hq // hkv
    sc = np.float32(1.0 / np.sqrt(d) if scale is None else scale)
    q32, k32, v32, do32 = (np.asarray(t, dtype=np.float32) for t in (q, k, v, do))
    kk, vv = orc.repeat_kv(k32, g), orc.repeat_kv(v32, g)
    s = (q32 @ np.swapaxes(kk, -1, -2)) * sc
    if causal:
        s = np.where(orc.allowed_mask(sq, sk)[None, None], s, -np.inf)
    m = np.max(s, -1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0)
    l = np.exp(s - m).sum(-1, keepdims=True)
    lse = np.where(l > 0, m + np.log(np.where(l > 0, l, 1)), np.inf)
    p = np.where(np.isfinite(lse), np.exp(s - lse), 0).astype(np.float32)
    o = r(r(p) @ vv)
    do_eff = do32
    delta = (do_eff * o).sum(-1, keepdims=True)
    if mistake == "delta_from_next_row":
        delta = np.roll(delta, 1, axis=2)
    dp = do_eff @ np.swapaxes(vv, -1, -2)
    ds = (r(p) if d > 128 else p) * (dp - delta)
    if mistake == "ds_without_p":
        ds = dp - delta
    dv = np.swapaxes(r(p), -1, -2) @ do_eff
    dq = (r(ds) @ kk) * sc
    dk = (np.swapaxes(r(ds), -1, -2) @ q32) * sc
    if mistake == "dk_unscaled":
        dk = dk / sc
    dk = dk.reshape(b, hkv, g, sk, d).sum(2)
    dv = dv.reshape(b, hkv, g, sk, d).sum(2)
    if mistake == "dv_one_head":
        dv = (np.swapaxes(r(p), -1, -2) @ do_eff).reshape(b, hkv, g, sk, d)[:, :, 0]
    return r(dq), r(dk), r(dv)


def _path(q, k, v, do, causal, scale, dt):
    """The fp32 reference path's gradients returned in dt (closed form)."""
    import torch

    from stackkernels_amd._reference.torch.attention import attention_reference_backward

    t = [torch.from_numpy(np.asarray(x, dtype=np.float32)) for x in (q, k, v, do)]
    gq, gk, gv = attention_reference_backward(t[3], t[0], t[1], t[2], is_causal=causal,
                                              sm_scale=scale)
    return [orc.round_to(x.numpy(), dt) for x in (gq, gk, gv)]


# (b, hq, hkv, sq, sk, d, causal, scale): the shape classes of the random-shape
# GPU test that exceed a fixed 2e-2 (sharp softmax, wide heads, group 8)
CASES = [
    (1, 8, 1, 40, 60, 160, False, None),
    (1, 8, 1, 40, 50, 240, True, 0.3),
    (1, 4, 4, 30, 40, 64, True, 1.0),
    (2, 4, 2, 33, 17, 96, True, -0.5),
    # head dim above 128 with fp16 P values down in the subnormal range
    # (two random-shape seeds that the bound without that rounding missed)
    (3, 6, 3, 121, 160, 144, True, 0.3),
    (3, 6, 3, 160, 160, 216, True, 0.3),
]


def _inputs(case, dt, seed):
    b, hq, hkv, sq, sk, d, causal, scale = case
    rng = np.random.default_rng(seed)
    q, k, v, do = (orc.round_to(rng.standard_normal(s).astype(np.float32), dt)
                   for s in ((b, hq, sq, d), (b, hkv, sk, d), (b, hkv, sk, d), (b, hq, sq, d)))
    return q, k, v, do, causal, scale


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_model_backward_within_bound(case, dt):
    q, k, v, do, causal, scale = _inputs(case, dt, 1)
    exact = orc.attention_backward(q, k, v, do, causal, scale)
    mass = rounding_mass(q, k, v, do, causal, scale, dt)
    path = _path(q, k, v, do, causal, scale, dt)
    model = _model_backward(q, k, v, do, causal, scale, dt)
    for name, i in (("dQ", 0), ("dK", 1), ("dV", 2)):
        used = check_backward(model[i], path[i], exact[i], mass[i], dt, name)
        assert used <= 1.0


def test_bound_is_beyond_a_fixed_tolerance():
    # the magnitudes that made a fixed 2e-2 fail: the bound, not the tolerance, applies
    q, k, v, do, causal, scale = _inputs(CASES[1], "bf16", 1)
    exact = orc.attention_backward(q, k, v, do, causal, scale)
    model = _model_backward(q, k, v, do, causal, scale, "bf16")
    assert max(float(np.abs(m - e).max()) for m, e in zip(model, exact)) > 2e-2


@pytest.mark.parametrize("mistake", ["delta_from_next_row", "ds_without_p", "dk_unscaled",
                                     "dv_one_head"])
def test_planted_mistakes_break_the_bound(mistake):
    q, k, v, do, causal, scale = _inputs(CASES[3], "bf16", 2)
    exact = orc.attention_backward(q, k, v, do, causal, scale)
    mass = rounding_mass(q, k, v, do, causal, scale, "bf16")
    path = _path(q, k, v, do, causal, scale, "bf16")
    model = _model_backward(q, k, v, do, causal, scale, "bf16", mistake)
    failed = 0
    for i, name in enumerate(("dQ", "dK", "dV")):
        try:
            check_backward(model[i], path[i], exact[i], mass[i], "bf16", name)
        except AssertionError:
            failed += 1
    assert failed >= 1, f"planted mistake {mistake} passed the bound"
