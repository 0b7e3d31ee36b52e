"""``build_causal_mask`` / ``causal_mask_check`` against the oracle's mask, bit for bit.

The grid is the reference's (S_q, S_k) test grid (tests/ops/test_flash_attn.py)
plus the edges of the bottom-right rule: empty sides, one row, S_q > S_k
(leading rows that see no key) and S_q < S_k.
"""

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc
from stackkernels_amd._core.attention import build_causal_mask, causal_mask_check

SHAPES = [(32, 32), (16, 64), (64, 32), (0, 5), (5, 0), (1, 1), (1, 7), (7, 1), (9, 4), (3, 130),
          (128, 128), (2048, 8192)]


@pytest.mark.parametrize("sq,sk", SHAPES)
def test_build_causal_mask_matches_oracle(sq, sk):
    got = build_causal_mask(sq, sk)
    assert got.dtype == torch.bool and tuple(got.shape) == (sq, sk)
    np.testing.assert_array_equal(got.numpy(), orc.allowed_mask(sq, sk))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int32, torch.uint8])
def test_build_causal_mask_dtype(dtype):
    got = build_causal_mask(16, 64, dtype=dtype)
    assert got.dtype == dtype
    np.testing.assert_array_equal(got.float().numpy(), orc.allowed_mask(16, 64).astype(np.float32))


def test_mask_rows_and_counts():
    # Row i sees exactly clamp(i + S_k - S_q + 1, 0, S_k) keys, the count the
    # forward kernel's tile bound and the oracle's pair count use.
    for sq, sk in [(64, 32), (16, 64), (9, 4)]:
        m = build_causal_mask(sq, sk)
        want = np.clip(np.arange(sq) + sk - sq + 1, 0, sk)
        np.testing.assert_array_equal(m.sum(1).numpy(), want)


def test_causal_mask_check_scalars_and_tensors():
    assert causal_mask_check(0, 0, 4, 4)
    assert not causal_mask_check(0, 1, 4, 4)
    assert causal_mask_check(0, 4, 4, 8)
    assert not causal_mask_check(0, 5, 4, 8)
    assert not causal_mask_check(0, 0, 5, 4)  # S_q > S_k: row 0 sees no key
    m = torch.arange(9)[:, None]
    n = torch.arange(4)[None, :]
    np.testing.assert_array_equal(causal_mask_check(m, n, 9, 4).numpy(), orc.allowed_mask(9, 4))


def test_exported_like_the_reference():
    import stackkernels_amd._core.attention as core

    for name in ("flash_attn_fwd", "flash_attn_bwd", "flash_decode", "causal_mask_check",
                 "build_causal_mask"):
        assert name in core.__all__ and hasattr(core, name)
