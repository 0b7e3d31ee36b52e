"""GPU parity of both entries of the forward tile table at D = 128 and D = 64, and of
the fp32 forward's matrix-core kernel at its block and tile edges.

The table picks by shape: short work (S_q <= 2048, causal S_q <= 4096, or
fewer than 2048 blocks of 256 rows in the grid) runs 4 waves with two
workgroups per CU (a 2-deep K/V ring at D = 128, 4-deep at D = 64); long
work runs 8 waves with one workgroup per CU on a 4-deep ring, and so do
query blocks that see 4,096 keys or more on average where the long entry's
workgroups fill whole rounds of the 256 CUs.  The BASELINE-size tests exercise the short entry, so these
shapes sit just past its limits (and one long sequence on a small grid stays
in it), or pair short query sequences with long key sequences.  Each case first asserts which entry ``pick``
reports, then checks heads at the start, middle and end of the batch against
the float64 oracle: O within the stated 2e-2 max-abs, LSE within 1e-3.
Inputs are generated on the device (seeded) so the large cases stay quick.
"""

import pytest
import torch

from stackkernels_amd._core.attention.flash_fwd import flash_attn_fwd
from stackkernels_amd._opt.pick import pick

from _gpu_util import TOL, assert_close_maxabs, assert_lse_close, native_loaded, np64

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("b,h,s,sk,d,causal,dt,rows", [
    (8, 32, 2304, 2304, 128, False, torch.bfloat16, 256),  # non-causal past S_q = 2048, 2,304 blocks
    (4, 32, 4352, 4352, 128, True, torch.bfloat16, 256),   # causal past S_q = 4096, 2,176 blocks
    (8, 32, 2112, 2112, 128, False, torch.float16, 256),   # fp16, ragged last block
    (1, 8, 5000, 5000, 128, True, torch.bfloat16, 128),    # long but a small grid: the short entry
    (2, 16, 4096, 4096, 128, True, torch.float16, 128),    # causal S_q = 4096: the short entry
    (4, 32, 4352, 4352, 64, True, torch.bfloat16, 256),    # D = 64, both entries
    (2, 16, 2112, 2112, 64, False, torch.float16, 128),
    (4, 32, 2048, 8192, 128, True, torch.bfloat16, 256),   # long key rows, paired blocks
    (2, 32, 2048, 8192, 128, True, torch.bfloat16, 256),   # the same rows, 256 paired workgroups
    (1, 32, 2048, 4608, 128, True, torch.float16, 128),    # 3,584 keys per row on average: short
    (2, 32, 2000, 8192, 128, False, torch.float16, 256),   # long key rows, no mask, ragged
    (1, 32, 2048, 16384, 64, True, torch.bfloat16, 256),   # D = 64, 256 blocks in one round
    (1, 16, 4096, 4096, 256, True, torch.bfloat16, 128),   # D = 256, 256 paired workgroups
])
def test_forward_table_entry_matches_oracle(b, h, s, sk, d, causal, dt, rows):
    from oracle import attention_oracle as orc

    name = {torch.bfloat16: "bfloat16", torch.float16: "float16"}[dt]
    cfg = pick("flash_attn", (b, h, s, d), dtype=name, kv_len=sk, is_causal=causal)
    assert cfg["BLOCK_M"] == rows and cfg["num_warps"] == rows // 32
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(s + sk)
    q = torch.randn(b, h, s, d, generator=g, device=dev, dtype=dt)
    k, v = (torch.randn(b, h, sk, d, generator=g, device=dev, dtype=dt) for _ in range(2))
    out, lse = flash_attn_fwd(q, k, v, is_causal=causal)
    torch.cuda.synchronize()
    assert native_loaded()
    for bi, hi in ((0, 0), (b // 2, h // 2 + 1), (b - 1, h - 1)):
        def sl(t):
            return t[bi:bi + 1, hi:hi + 1]

        o_ref, lse_ref = orc.attention_forward(np64(sl(q)), np64(sl(k)), np64(sl(v)), causal)
        what = f"(b={bi}, h={hi}, S_q={s}, S_k={sk}, D={d}, causal={causal}, {name})"
        assert_close_maxabs(sl(out), o_ref, TOL[dt], "O " + what)
        assert_lse_close(sl(lse), lse_ref, "LSE " + what)


@pytest.mark.parametrize("b,h,hkv,s,sk,d,causal,scale,kernel", [
    (2, 4, 2, 256, 256, 128, True, None, "fwd_f32_mfma_kernel"),   # one whole block
    (2, 4, 2, 257, 300, 128, True, None, "fwd_f32_mfma_kernel"),   # one row into a second block
    (1, 8, 1, 513, 130, 96, True, None, "fwd_f32_mfma_kernel"),    # S_q > S_k: rows see no key
    (1, 4, 4, 700, 1000, 80, False, -0.2, "fwd_f32_mfma_kernel"),  # D = 80 on the 128 kernel
    (2, 6, 3, 300, 65, 64, False, 0.5, "fwd_f32_mfma_kernel"),     # keys end 1 past a tile
    (2, 4, 2, 32, 2000, 40, True, None, "fwd_f32_mfma_kernel"),    # the shortest query run
    (2, 4, 2, 31, 500, 128, True, None, "fwd_f32_kernel"),         # one row short of it
])
def test_fp32_forward_matches_oracle(b, h, hkv, s, sk, d, causal, scale, kernel):
    """The fp32 forward on the matrix cores (256-row blocks, 64-key tiles, padded head
    dims 64 and 128) at block and tile edges, and the vector kernel just below its
    query-length threshold: O within 1e-4, LSE within 1e-3 of the float64 oracle."""
    from oracle import attention_oracle as orc

    from _gpu_util import make_qkv

    cfg = pick("flash_attn", (b, h, s, d), dtype="float32", kv_len=sk, is_causal=causal)
    assert cfg["kernel_variant"] == kernel
    q, k, v = make_qkv(b, h, hkv, s, sk, d, torch.float32, seed=s + sk + d)
    out, lse = flash_attn_fwd(q, k, v, is_causal=causal, sm_scale=scale)
    torch.cuda.synchronize()
    assert native_loaded()
    o_ref, lse_ref = orc.attention_forward(np64(q), np64(k), np64(v), causal, scale)
    what = f"(S_q={s}, S_k={sk}, D={d}, causal={causal}, scale={scale})"
    assert_close_maxabs(out, o_ref, TOL[torch.float32], f"O {what}")
    assert_lse_close(lse, lse_ref, f"LSE {what}")
