"""Helpers for the GPU parity tests (imported by tests only)."""

import numpy as np
import torch

from oracle import attention_oracle as orc

# Tolerances stated by the target: max-abs on O / dQ / dK / dV, and on LSE.
TOL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2}
LSE_TOL = 1e-3


def make_qkv(b, hq, hkv, sq, sk, d, dtype, seed=42, device="cuda"):
    """Seeded N(0,1) inputs generated on the CPU, cast to dtype, moved to the device."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, sq, d, generator=g).to(dtype)
    k = torch.randn(b, hkv, sk, d, generator=g).to(dtype)
    v = torch.randn(b, hkv, sk, d, generator=g).to(dtype)
    return q.to(device), k.to(device), v.to(device)


def np64(t):
    return t.detach().to("cpu", torch.float64).numpy()


def assert_close_maxabs(actual, expected, tol, what):
    a = np64(actual) if isinstance(actual, torch.Tensor) else actual
    e = np64(expected) if isinstance(expected, torch.Tensor) else expected
    assert a.shape == e.shape, (what, a.shape, e.shape)
    assert np.isfinite(a).all(), f"{what}: non-finite values"
    err = float(np.abs(a - e).max()) if a.size else 0.0
    assert err <= tol, f"{what}: max-abs error {err:.3e} > {tol:.1e}"
    return err


def assert_lse_close(lse, ref_lse, what="lse"):
    a = np64(lse) if isinstance(lse, torch.Tensor) else lse
    e = np64(ref_lse) if isinstance(ref_lse, torch.Tensor) else ref_lse
    dead = np.isneginf(e)
    assert np.array_equal(np.isneginf(a), dead), f"{what}: -inf rows differ"
    if (~dead).any():
        err = float(np.abs(a[~dead] - e[~dead]).max())
        assert err <= LSE_TOL, f"{what}: max-abs error {err:.3e} > {LSE_TOL:.0e}"


def oracle_fwd(q, k, v, causal, scale=None):
    return orc.attention_forward(np64(q), np64(k), np64(v), causal, scale)


def native_loaded():
    from stackkernels_amd._core.attention import _lib

    return _lib._lib is not None
