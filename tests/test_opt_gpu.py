"""On the MI355X: the device profile reads gfx950 correctly, and the
occupancy the HIP runtime reports for the kernels ``pick`` names equals what
the gfx950 table was sized for (one 8-wave forward workgroup per CU, or two
4-wave ones for short work at D <= 128; one dK/dV workgroup per CU, two dQ
workgroups per CU at D <= 128, eight one-wave decode workgroups, three 4-wave
MQA decode workgroups)."""

import pytest

from stackkernels_amd._opt import hardware as hw
from stackkernels_amd._opt.pick import pick

pytestmark = pytest.mark.gpu


def test_device_profile_is_mi355x():
    hw._PROFILES.clear()
    p = hw.get_device_profile()
    print(p)
    assert p.arch == "gfx950" and p.warp_size == 64 and p.sm_count == 256
    assert p.compute_capability == (9, 5)
    assert p.name == "AMD Instinct MI355X"
    assert p.fingerprint().startswith("amd-instinct-mi355x_gfx950_256cu_")
    assert hw.get_gpu_arch() == "gfx950"


@pytest.mark.parametrize("op,shape,kw,lds,per_cu", [
    ("flash_attn", (4, 32, 4096, 128), dict(dtype="bfloat16", is_causal=True), 65536, 2),
    ("flash_attn", (1, 32, 16384, 128), dict(dtype="bfloat16", is_causal=True), 131072, 1),
    ("flash_attn", (2, 16, 1024, 64), dict(dtype="float16"), 65536, 2),
    ("flash_attn", (1, 32, 16384, 64), dict(dtype="float16", is_causal=True), 65536, 1),
    ("flash_decode", (64, 32, 1, 128), dict(dtype="bfloat16", kv_len=32768, num_kv_heads=8),
     None, 8),
    # C5: 64-key K and V tiles (2 x 18 KiB); the 512 workgroups run two per CU
    ("flash_decode", (8, 64, 1, 128), dict(dtype="float16", kv_len=131072, num_kv_heads=1),
     36864, 2),
])
def test_reported_occupancy_matches_the_table(op, shape, kw, lds, per_cu):
    cfg, text = pick(op, shape, explain=True, **kw)
    print(text)
    assert cfg["wg_per_cu"] == per_cu
    if lds is not None:
        assert cfg["lds_bytes"] == lds
    assert 0 < cfg["vgprs"] <= 512


def test_backward_occupancy():
    cfg = pick("flash_bwd", (2, 32, 2048, 128), dtype="bfloat16", kv_len=8192, num_kv_heads=8,
               is_causal=True)
    print(cfg)
    assert cfg["wg_per_cu"] == 1
    assert cfg["dq"]["wg_per_cu"] == 2
