"""BASELINE config 1 on the CPU reference path, bit for bit against the
reference's own outputs (``tests/golden/c1_reference.npz``, written by
``tests/golden/make_c1_golden.py`` from the reference's ``attention_reference``).

Config 1 is the fp32 non-causal MHA forward B=2, H=4, S=128, D=64 with
q/k/v ~ N(0, 1) from a fixed seed: the plumbing anchor whose CPU result must
be the reference's exactly.  A causal GQA case with S_q < S_k covers the mask
and the head repetition.  Both run single-threaded, as the fixture was made.
"""

import os
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

from make_c1_golden import CASES, c1_inputs, input_digest  # noqa: E402

from stackkernels_amd._reference.torch.attention import attention_reference  # noqa: E402
from stackkernels_amd.torch import flash_attention  # noqa: E402

GOLDEN = np.load(os.path.join(HERE, "golden", "c1_reference.npz"))


@pytest.fixture
def one_thread():
    n = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(n)


@pytest.mark.parametrize("name", sorted(CASES))
def test_cpu_path_is_bit_identical_to_the_reference(name, one_thread):
    b, hq, hkv, sq, sk, d, causal = CASES[name]
    q, k, v = c1_inputs(b, hq, hkv, sq, sk, d)
    assert input_digest(q, k, v) == str(GOLDEN[f"{name}_inputs_sha256"]), \
        "torch's CPU random stream changed: regenerate the fixture"
    out, lse = attention_reference(q, k, v, is_causal=causal)
    np.testing.assert_array_equal(out.numpy(), GOLDEN[f"{name}_out"])
    np.testing.assert_array_equal(lse.numpy(), GOLDEN[f"{name}_lse"])
    # the public API on CPU tensors takes the same path
    api = flash_attention(q, k, v, is_causal=causal)
    np.testing.assert_array_equal(api.numpy(), GOLDEN[f"{name}_out"])
