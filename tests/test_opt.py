"""Device profiles and ``pick`` (the reference's ``_opt`` API for the attention
path): a correct MI355X / gfx950 profile and fingerprint, and ``pick``
answers that are the library's own launch plans.  No GPU needed:
``sk_kernel_config`` without a device query makes no HIP call."""

import ctypes
from types import SimpleNamespace

import pytest

from stackkernels_amd._opt import hardware as hw
from stackkernels_amd._opt.pick import pick


def _rocm_props(**kw):
    base = dict(name="AMD Instinct MI355X", gcnArchName="gfx950:sramecc+:xnack-",
                multi_processor_count=256, warp_size=64, total_memory=288 * 10**9,
                max_threads_per_multi_processor=2048, regs_per_multiprocessor=131072,
                shared_memory_per_block=160 * 1024, L2_cache_size=4 * 1024 * 1024)
    base.update(kw)
    return SimpleNamespace(**base)


def test_mi355x_profile_and_fingerprint():
    p = hw.mi355x_profile()
    assert p.arch == "gfx950" and p.is_rocm and p.is_cuda
    assert (p.sm_count, p.warp_size, p.max_smem_per_sm) == (256, 64, 160 * 1024)
    assert p.peak_bandwidth_gbps == 8000.0 and p.peak_tflops["bf16"] == 2500.0
    assert p.fingerprint() == f"amd-instinct-mi355x_gfx950_256cu_{288 * 10**9 // 2**20}mb"


def test_profile_from_rocm_properties_uses_the_arch_not_the_capability():
    # torch on ROCm reports (9, 5) for gfx950; gfx90a reports (9, 0), which the
    # NVIDIA table would read as an H100.
    # the runtime's generic name and half-CU register count give way to the table
    p = hw.profile_from_properties(_rocm_props(name="AMD Radeon Graphics",
                                               regs_per_multiprocessor=65536), (9, 5))
    assert p.arch == "gfx950" and p.warp_size == 64 and p.sm_count == 256
    assert p.name == "AMD Instinct MI355X" and p.max_regs_per_sm == 4 * 512 * 64
    assert p.l2_bytes == 32 * 1024 * 1024
    assert p.peak_bandwidth_gbps == 8000.0 and p.has_bf16
    assert "_gfx950_256cu_" in p.fingerprint()
    q = hw.profile_from_properties(_rocm_props(gcnArchName="gfx90a:xnack-", name="AMD MI250X",
                                               multi_processor_count=110, warp_size=0), (9, 0))
    assert q.arch == "gfx90a" and q.warp_size == 64 and q.peak_bandwidth_gbps is None
    assert "H100" not in q.name


def test_profile_from_other_gpu_properties():
    # not a gfx950: the runtime's figures only, no peaks; the reference's
    # fingerprint format with capability and SM count
    props = SimpleNamespace(name="NVIDIA H100 80GB HBM3", multi_processor_count=132,
                            total_memory=80 * 2**30, max_threads_per_multi_processor=2048)
    p = hw.profile_from_properties(props, (9, 0))
    assert p.arch == "" and p.warp_size == 32 and p.peak_bandwidth_gbps is None
    assert p.fingerprint() == "nvidia-h100-80gb-hbm3_sm90_132sm_81920mb"


def test_partitioned_gfx950_keeps_runtime_cus():
    p = hw.profile_from_properties(_rocm_props(multi_processor_count=32, total_memory=36 * 10**9),
                                   (9, 5))
    assert p.name == "AMD Instinct MI355X" and p.sm_count == 32
    assert p.fingerprint() == f"amd-instinct-mi355x_gfx950_32cu_{36 * 10**9 // 2**20}mb"


def test_fingerprint_format_of_reference_profiles():
    # the reference's fixture shapes (tests/fixtures/profiles.py): sm format, and "cpu"
    t4 = hw.DeviceProfile(name="Tesla T4", compute_capability=(7, 5), sm_count=40, warp_size=32,
                          max_regs_per_sm=65536, max_regs_per_thread=255, max_threads_per_sm=1024,
                          max_smem_per_block=49152, max_smem_per_sm=65536, l2_bytes=4 << 20,
                          total_memory_bytes=16 * 2**30)
    fp = t4.fingerprint()
    assert "tesla-t4" in fp and "sm75" in fp and "40sm" in fp
    assert hw.host_profile().fingerprint() == "cpu"


def test_get_device_profile_cpu_arguments():
    import torch

    for dev in ("cpu", torch.device("cpu")):
        p = hw.get_device_profile(dev)
        assert p.compute_capability == (0, 0) and not p.is_cuda and p.fingerprint() == "cpu"


def test_pick_decode_matches_the_launch_plan():
    from stackkernels_amd._core.attention.decode import plan

    cfg = pick("flash_decode", (64, 32, 1, 128), dtype="bfloat16", kv_len=32768, num_kv_heads=8)
    ns, nbytes = plan(__import__("torch").bfloat16, 64, 32, 8, 32768, 128)
    assert cfg["SPLIT_KV"] == ns > 1  # kv_len is honoured (one split in the reference)
    assert cfg["workspace_bytes"] == nbytes
    assert cfg["kernel_variant"] == "decode_split_kernel" and cfg["num_warps"] == 1
    assert cfg["grid"] == ns * 64 * 8
    assert cfg["combine"]["grid"] == 64 * 32
    # per-row lengths (and paged pools): the varlen plan
    vl = pick("flash_decode", (64, 32, 1, 128), dtype="bfloat16", kv_len=32768, num_kv_heads=8,
              varlen=True)
    assert vl["SPLIT_KV"] == plan(__import__("torch").bfloat16, 64, 32, 8, 32768, 128,
                                  per_row=True)[0] == 2 * cfg["SPLIT_KV"]
    pg = pick("flash_decode", (64, 32, 1, 128), dtype="bfloat16", kv_len=32768, num_kv_heads=8,
              paged=True)
    assert pg["SPLIT_KV"] == vl["SPLIT_KV"]
    # MQA C5: four waves per workgroup share each tile; one round of 64 splits
    c5 = pick("flash_decode", (8, 64, 1, 128), dtype="float16", kv_len=131072, num_kv_heads=1)
    assert c5["kernel_variant"] == "decode_split_kernel" and c5["num_warps"] == 4
    assert c5["SPLIT_KV"] == 64 and c5["grid"] == 64 * 8
    # 64-key tiles for the multi-wave kernel, 32 for one-wave workgroups and paged pools
    assert c5["BLOCK_N"] == 64 and cfg["BLOCK_N"] == 32
    c5p = pick("flash_decode", (8, 64, 1, 128), dtype="float16", kv_len=131072, num_kv_heads=1,
               paged=True)
    assert c5p["BLOCK_N"] == 32 and c5p["num_warps"] == 4
    # short cache: one split, no combine pass
    one = pick("flash_decode", (2, 8, 1, 64), kv_len=100, num_kv_heads=2)
    assert one["SPLIT_KV"] == 1 and "combine" not in one and one["workspace_bytes"] == 0
    # variants show in the kernel name
    pg = pick("flash_decode", (2, 8, 1, 64), kv_len=4096, num_kv_heads=2, paged=True, rope=True)
    assert "paged=1" in pg["kernel"] and "rope=1" in pg["kernel"]


def test_pick_forward_and_backward():
    # D = 128, causal S <= 4096: the short-work entry, 4 waves and two workgroups per CU
    f = pick("flash_attn", (4, 32, 4096, 128), dtype="bfloat16", is_causal=True)
    assert (f["BLOCK_M"], f["BLOCK_N"], f["num_warps"], f["num_stages"]) == (128, 64, 4, 2)
    assert f["paired_causal_blocks"] and f["grid"] == 16 * 4 * 32
    # non-causal S = 4096 on a full grid (2,048 blocks of 256 rows): the 8-wave entry
    nc = pick("flash_attention", {"batch": 4, "heads": 32, "seq_q": 4096, "head_dim": 128},
              dtype="bfloat16")
    assert (nc["BLOCK_M"], nc["num_warps"], nc["num_stages"]) == (256, 8, 4)
    assert not nc["paired_causal_blocks"] and nc["grid"] == 16 * 4 * 32
    nc2 = pick("flash_attn", (8, 32, 2048, 128), dtype="bfloat16")
    assert (nc2["BLOCK_M"], nc2["num_warps"], nc2["num_stages"]) == (128, 4, 2)
    # long work on a full grid (2,048 blocks of 256 rows): 8 waves, one workgroup per CU
    lg = pick("flash_attn", (1, 32, 16384, 128), dtype="bfloat16", is_causal=True)
    assert (lg["BLOCK_M"], lg["BLOCK_N"], lg["num_warps"], lg["num_stages"]) == (256, 64, 8, 4)
    assert lg["grid"] == 32 * 32
    # long but a small grid: the short-work entry again where the 8-wave grid would leave
    # part of a round idle (384 paired workgroups on 256 CUs), the 8-wave one where it
    # fills one round (256 paired workgroups)
    sm = pick("flash_attn", (1, 24, 8192, 128), dtype="bfloat16", is_causal=True)
    assert (sm["BLOCK_M"], sm["num_warps"], sm["num_stages"]) == (128, 4, 2)
    sm8 = pick("flash_attn", (1, 8, 16384, 128), dtype="bfloat16", is_causal=True)
    assert (sm8["BLOCK_M"], sm8["num_warps"], sm8["num_stages"]) == (256, 8, 4)
    assert sm8["paired_causal_blocks"] and sm8["grid"] == 256
    # short query sequences against long key sequences: the 8-wave entry where its grid
    # fills whole rounds of 256 workgroups, the short one elsewhere
    def rows(b, sq, sk, causal):
        return pick("flash_attn", (b, 32, sq, 128), dtype="bfloat16", kv_len=sk,
                    num_kv_heads=8, is_causal=causal)["BLOCK_M"]
    assert rows(2, 2048, 8192, True) == 256    # 256 paired workgroups (one per CU)
    assert rows(2, 1024, 8192, True) == 256    # 256 blocks, one round, unpaired
    assert rows(1, 2048, 4608, True) == 128    # 3,584 keys per row on average
    assert rows(4, 2048, 8192, True) == 256    # 512 paired workgroups
    assert rows(2, 2048, 8192, False) == 256   # no mask
    assert rows(1, 2048, 16384, True) == 256   # 256 blocks, one round
    assert rows(4, 2048, 4096, True) == 128    # 3,072 keys per row on average
    assert rows(4, 4096, 4096, False) == 256   # full grid (unchanged)
    assert rows(3, 2048, 8192, False) == 256   # 768 blocks of 256 rows: 3 whole rounds
    assert rows(6, 2048, 8192, True) == 256    # 768 paired workgroups: 3 whole rounds
    for b, h, causal in ((1, 40, False), (3, 40, True)):  # 320 blocks; 480 paired workgroups
        assert pick("flash_attn", (b, h, 2048, 128), dtype="bfloat16", kv_len=8192,
                    is_causal=causal)["BLOCK_M"] == 128
    d256 = pick("flash_fwd", (1, 8, 512, 256), dtype="float16")
    assert (d256["BLOCK_M"], d256["BLOCK_N"], d256["num_warps"]) == (128, 32, 4)
    # causal blocks are paired while the paired grid fills one round: 256 workgroups at one
    # per CU (D = 256, the 8-wave entry), 512 at two per CU (the short-work entry)
    p256 = pick("flash_fwd", (1, 16, 4096, 256), dtype="bfloat16", is_causal=True)
    assert p256["paired_causal_blocks"] and p256["grid"] == 256
    u256 = pick("flash_fwd", (1, 8, 4096, 256), dtype="bfloat16", is_causal=True)
    assert not u256["paired_causal_blocks"] and u256["grid"] == 256
    s128 = pick("flash_fwd", (1, 16, 4096, 128), dtype="bfloat16", is_causal=True)
    assert s128["BLOCK_M"] == 128 and not s128["paired_causal_blocks"] and s128["grid"] == 512
    # fp32: the matrix-core forward (8 waves x 32 rows) for head dims up to 128 and at
    # least 32 query rows, the vector-ALU kernel (64 rows) for D = 256 and short queries
    f32 = pick("flash_attn", (1, 8, 512, 64), dtype="float32")
    assert f32["kernel_variant"] == "fwd_f32_mfma_kernel"
    assert (f32["BLOCK_M"], f32["BLOCK_N"], f32["grid"]) == (256, 64, 2 * 8)
    assert pick("flash_attn", (1, 8, 512, 96), dtype="float32")["head_dim_padded"] == 128
    for shape in ((1, 8, 16, 64), (1, 8, 512, 256)):
        v = pick("flash_attn", shape, dtype="float32")
        assert v["kernel_variant"] == "fwd_f32_kernel" and v["BLOCK_M"] == 64
    b = pick("flash_bwd", (2, 32, 2048, 128), dtype="bfloat16", kv_len=8192, num_kv_heads=8,
             is_causal=True)
    # D = 128: the five-GEMM backward (dQ from the dS tiles dK/dV stores)
    assert b["kernel_variant"] == "bwd_dkv_kernel+bwd_dq_ds_kernel"
    assert b["grid"] == (8192 // 128) * 2 * 8 and b["dq"]["grid"] == (2048 // 256) * 2 * 32
    # dK/dV: the 6-deep pipelined ring at D = 128 (and 64), the 4-deep one at D = 256;
    # 8 waves (two roles x four 32-key groups) in both
    assert (b["num_stages"], b["num_warps"]) == (6, 8)
    # the same 6-deep ring at D = 64, the 4-deep one at D = 256; both seven GEMMs
    for d, stages in ((64, 6), (256, 4)):
        o = pick("flash_bwd", (2, 8, 512, d), dtype="bfloat16", kv_len=1024, num_kv_heads=2)
        assert (o["num_stages"], o["num_warps"]) == (stages, 8)
        assert o["kernel_variant"] == "bwd_dkv_kernel+bwd_dq_kernel"  # seven GEMMs
    # dQ from the stored dS: 4 waves x 64 queries, 32-key tiles, 3-deep ring
    assert (b["dq"]["num_stages"], b["dq"]["num_warps"], b["dq"]["BLOCK_N"],
            b["dq"]["BLOCK_M"]) == (3, 4, 32, 256)
    # row statistics + the dS tiles visible key blocks write (0.875 of the rectangle), one chunk
    assert b["workspace_bytes"] == 2 * 2 * 32 * 2048 * 4 + 2 * 32 * 4 * 2048 * sum(
        64 - max(0, 4 * kb - 192) for kb in range(64))
    assert b["chunks"] == 1
    # B = 4, H = 32, S = 8192 causal: the same five-GEMM kernels, in 5 chunks under the cap
    big = pick("flash_bwd", (4, 32, 8192, 128), dtype="bfloat16", is_causal=True)
    assert big["kernel_variant"] == "bwd_dkv_kernel+bwd_dq_ds_kernel" and big["chunks"] == 5
    assert big["grid"] == (8192 // 128) * 26 and big["dq"]["grid"] == (8192 // 256) * 26
    assert big["workspace_bytes"] <= 4 * 32 * 8192 * 8 + (2 << 30)
    for d in (64, 256):
        o = pick("flash_bwd", (2, 8, 512, d), dtype="bfloat16", kv_len=1024, num_kv_heads=2)
        assert (o["dq"]["num_stages"], o["dq"]["num_warps"]) == (4, 4)


def test_pick_explain_override_and_errors():
    cfg, text = pick("flash_decode", (64, 32, 1, 128), dtype="bfloat16", kv_len=32768,
                     num_kv_heads=8, explain=True)
    assert "gfx950 table" in text and "decode_split_kernel<BF16, D=128" in text
    assert f"{cfg['SPLIT_KV']} splits of {cfg['keys_per_split']} keys" in text
    ov, text = pick("flash_decode", (8, 64, 1, 128), kv_len=131072, num_kv_heads=1,
                    override={"SPLIT_KV": 16}, explain=True)
    assert ov == {"SPLIT_KV": 16} and "user_override" in text and "16 splits" in text
    assert "applied through num_splits" in text
    _, text = pick("flash_attn", (1, 8, 128, 64), override={"BLOCK_M": 64}, explain=True)
    assert "returned as given" in text and "Rejected Candidates: None" in text
    _, text = pick("flash_attn", (4, 32, 4096, 128), is_causal=True, explain=True)
    assert "BM=128" in text and "the other D = 128 forward entry" in text
    with pytest.raises(NotImplementedError, match="attention path"):
        pick("rms_norm", (4, 1024))
    with pytest.raises(ValueError, match="dtype"):
        pick("flash_attn", (1, 8, 128, 64), dtype="int8")
    with pytest.raises(NotImplementedError, match="head dim"):
        pick("flash_attn", (1, 8, 128, 3000))  # head dim > 256 has no kernel
    with pytest.raises(NotImplementedError):
        pick("flash_decode", (1, 128, 1, 64), kv_len=64, num_kv_heads=1)  # group of 128


def test_kernel_config_abi_errors():
    from stackkernels_amd._core.attention import _lib

    lib = _lib.load()
    cfg = (ctypes.c_int64 * 16)()
    assert lib.sk_kernel_config(9, 2, 1, 8, 8, 64, 64, 64, 0, 0, 0, 0, cfg, None, 0) == _lib.SK_EINVAL
    assert "unknown op" in _lib.last_error()
    assert lib.sk_kernel_config(0, 2, 1, 8, 3, 64, 64, 64, 0, 0, 0, 0, cfg, None, 0) == _lib.SK_EINVAL
    assert lib.sk_kernel_config(0, 2, 1, 8, 8, 64, 64, 64, 0, 0, 0, 0, None, None, 0) == _lib.SK_EINVAL
    assert lib.sk_kernel_config(3, 2, 1, 8, 8, 1, 64, 64, 0, 2000, 0, 0, cfg, None, 0) == _lib.SK_EINVAL
    # no device query: device slots are -1
    assert lib.sk_kernel_config(0, 2, 1, 8, 8, 64, 64, 64, 0, 0, 0, 0, cfg, None, 0) == _lib.SK_OK
    assert cfg[10] == cfg[11] == cfg[12] == -1


def test_layout_and_workspace():
    import torch

    from stackkernels_amd._core.attention import layout, workspace

    q = torch.zeros(2, 8, 16, 80)
    k = torch.zeros(2, 2, 32, 80)
    assert layout.validate_attention_layout(q, k, k) == (2, 8, 2, 16, 32, 80)
    with pytest.raises(ValueError, match="divisible"):
        layout.validate_attention_layout(torch.zeros(2, 3, 16, 80), k, k)
    # the reference's helper and values (power-of-two tile width, at least 16) ...
    assert [layout.get_padded_head_dim(d) for d in (1, 16, 17, 32, 64, 80, 96, 128, 200, 256,
                                                    300, 513)] == \
        [16, 16, 32, 32, 64, 128, 128, 128, 256, 256, 512, 1024]
    # ... and the head dims the gfx950 kernels run at
    assert [layout.padded_head_dim(d) for d in (16, 64, 80, 96, 128, 200, 256, 300)] == \
        [64, 64, 96, 96, 128, 256, 256, 0]
    ws, ns = workspace.decode_workspace(torch.bfloat16, 64, 32, 8, 32768, 128, "cpu")
    assert ns == 4 and ws.numel() == 64 * 32 * 4 * (128 + 1) * 4
    ws, ns = workspace.decode_workspace(torch.bfloat16, 64, 32, 8, 32768, 128, "cpu", per_row=True)
    assert ns == 8 and ws.numel() == 64 * 32 * 8 * (128 + 1) * 4
    ws, ns = workspace.decode_workspace(torch.bfloat16, 64, 32, 8, 32768, 128, "cpu", num_splits=4)
    assert ns == 4 and ws.numel() == 64 * 32 * 4 * (128 + 1) * 4
    bw = workspace.bwd_workspace(torch.bfloat16, 2, 32, 8, 2048, 8192, 128, True, "cpu")
    assert bw.numel() >= 2 * 2 * 32 * 2048 * 4
