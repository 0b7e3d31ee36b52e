"""Forward and backward on tensors of more than 2^31 elements (bf16, causal MHA).

Every pointer the kernels form is a 64-bit offset; an int32 product anywhere
(row x head dim, head x rows, ...) would wrap for the heads past element 2^31.
Q, K, V, O, dO and the three gradients here hold 4,100 x 32 x 128 x 128 =
2,149,580,800 elements each (4.3 GB; 35 GB on the device in all).  Each
(batch, head) is independent in MHA, so heads at the start, the middle and the
end of the tensors are checked against the float64 oracle at the stated
bounds (2e-2 max-abs on O, dQ, dK, dV; 1e-3 on the LSE).
"""

import pytest
import torch

from stackkernels_amd._core.attention.flash_bwd import flash_attn_bwd
from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd

from _gpu_util import TOL, assert_close_maxabs, assert_lse_close, native_loaded, np64

pytestmark = pytest.mark.gpu


def test_offsets_beyond_2_31_elements():
    from oracle import attention_oracle as orc

    B, H, S, D = 4100, 32, 128, 128
    dev = torch.device("cuda:0")
    dt = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(11)
    t = {}
    try:
        q, k, v, do = t["q"], t["k"], t["v"], t["do"] = tuple(
            torch.randn(B, H, S, D, generator=g, device=dev, dtype=dt) for _ in range(4))
        assert q.numel() > 2 ** 31
        out, lse = t["out"], t["lse"] = flash_attn_fwd(q, k, v, is_causal=True)
        dq, dk, dv = t["dq"], t["dk"], t["dv"] = flash_attn_bwd(do, q, k, v, out, lse,
                                                                 is_causal=True)
        torch.cuda.synchronize()
        assert native_loaded()
        for b, h in ((0, 0), (B // 2, 17), (B - 1, H - 1)):
            def sl(t):
                return t[b:b + 1, h:h + 1]

            o_ref, lse_ref = orc.attention_forward(np64(sl(q)), np64(sl(k)), np64(sl(v)), True)
            assert_close_maxabs(sl(out), o_ref, TOL[dt], f"O (b={b}, h={h})")
            assert_lse_close(sl(lse), lse_ref, f"LSE (b={b}, h={h})")
            dq_ref, dk_ref, dv_ref = orc.attention_backward(np64(sl(q)), np64(sl(k)), np64(sl(v)),
                                                            np64(sl(do)), True)
            assert_close_maxabs(sl(dq), dq_ref, TOL[dt], f"dQ (b={b}, h={h})")
            assert_close_maxabs(sl(dk), dk_ref, TOL[dt], f"dK (b={b}, h={h})")
            assert_close_maxabs(sl(dv), dv_ref, TOL[dt], f"dV (b={b}, h={h})")
    finally:
        # 35 GB: hand it back before the next test
        t.clear()
        q = k = v = do = out = lse = dq = dk = dv = None
        torch.cuda.empty_cache()
