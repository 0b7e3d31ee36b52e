"""Write ``c1_reference.npz``: the reference's own CPU outputs for BASELINE
config 1, the bit-for-bit anchor of the CPU reference path.

BASELINE config 1 is the fp32 non-causal MHA forward B=2, H=4, S=128, D=64
with q/k/v ~ N(0, 1) from a fixed seed, run on the reference's PyTorch
reference path, whose result this repo's CPU path must reproduce bit for bit.
Nothing else pins bit identity (the oracle and the SDPA vectors pin values
within tolerance), so the expected outputs come from running the reference's
``attention_reference`` (``src/stackkernels/_reference/torch/attention.py``)
itself, in the build container, where the reference checkout is present.  A
causal GQA case with ragged lengths exercises the mask and head repetition too.

The fixture holds, per case, the output and LSE (float32) and the SHA-256 of
the float32 bytes of q, k and v, so a test regenerating the inputs from the
seed can tell a changed random stream from a changed result.

Run: ``python tests/golden/make_c1_golden.py [reference src dir]`` (CPU, seconds).
"""

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

# name: (B, Hq, Hkv, Sq, Sk, D, causal)
CASES = {
    "c1": (2, 4, 4, 128, 128, 64, False),
    "causal_gqa": (2, 8, 2, 64, 96, 64, True),
}
SEED = 0


def c1_inputs(b, hq, hkv, sq, sk, d):
    """q, k, v ~ N(0, 1) float32 from ``torch.Generator().manual_seed(SEED)``, in that order."""
    g = torch.Generator().manual_seed(SEED)
    q = torch.randn(b, hq, sq, d, generator=g)
    k = torch.randn(b, hkv, sk, d, generator=g)
    v = torch.randn(b, hkv, sk, d, generator=g)
    return q, k, v


def input_digest(q, k, v) -> str:
    h = hashlib.sha256()
    for t in (q, k, v):
        h.update(t.contiguous().numpy().tobytes())
    return h.hexdigest()


def main() -> None:
    src = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src"
    sys.path.insert(0, src)
    from stackkernels._reference.torch.attention import attention_reference

    torch.set_num_threads(1)
    out = {}
    for name, (b, hq, hkv, sq, sk, d, causal) in CASES.items():
        q, k, v = c1_inputs(b, hq, hkv, sq, sk, d)
        o, lse = attention_reference(q, k, v, is_causal=causal)
        out[f"{name}_out"] = o.numpy()
        out[f"{name}_lse"] = lse.numpy()
        out[f"{name}_inputs_sha256"] = np.array(input_digest(q, k, v))
    np.savez_compressed(os.path.join(HERE, "c1_reference.npz"), **out)
    print("wrote", os.path.join(HERE, "c1_reference.npz"), sorted(out))


if __name__ == "__main__":
    main()
