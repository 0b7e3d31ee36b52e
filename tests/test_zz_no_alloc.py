"""sk_decode_noalloc (decode with the library's static per-GPU scratch, no
workspace argument) against sk_decode with a caller workspace: the same
kernels at the same split count, so the outputs must be equal bit for bit.
Two calls in a row on different shapes, the second smaller, then a shape
whose table split count is lowered to fit the scratch, fp32, and a repeat of
the first call (the scratch keeps the previous call's contents)."""

import ctypes
import math

import pytest
import torch

from stackkernels_amd._core.attention import _lib

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20


def _inputs(b, hq, hkv, sk, d, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(b, hq, 1, d, generator=g, device="cuda").to(dtype)
    k = torch.randn(b, hkv, sk, d, generator=g, device="cuda").to(dtype)
    v = torch.randn(b, hkv, sk, d, generator=g, device="cuda").to(dtype)
    return q, k, v


def _plan(lib, code, b, hq, hkv, sk, d):
    ns, nb = ctypes.c_int(0), ctypes.c_size_t(0)
    _lib.check(lib.sk_decode_plan(code, b, hq, hkv, sk, d, ctypes.byref(ns), ctypes.byref(nb)),
               "plan")
    return ns.value


def _both(lib, q, k, v, num_splits):
    """(noalloc output, sk_decode output at the split count noalloc used)."""
    b, hq, _, d = q.shape
    hkv, sk = k.shape[1], k.shape[2]
    code = _lib.dtype_code(q.dtype)
    stream = torch.cuda.current_stream().cuda_stream
    sts = [_lib.strides3(t) for t in (q, k, v)]
    scale = 1.0 / math.sqrt(d)
    o1 = torch.full_like(q, float("nan"))
    rc = lib.sk_decode_noalloc(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), o1.data_ptr(),
                               num_splits, b, hq, hkv, sk, d, *sts, _lib.strides3(o1), scale,
                               stream)
    _lib.check(rc, "sk_decode_noalloc")
    used = num_splits
    if used == 0 and code != _lib.SK_F32:
        per_split = b * hq * (d + 1) * 4  # d is a padded head dim in these cases
        used = min(_plan(lib, code, b, hq, hkv, sk, d), max(1, SCRATCH // per_split))
    nb = ctypes.c_size_t(0)
    _lib.check(lib.sk_decode_workspace(code, b, hq, hkv, sk, d, max(used, 1), ctypes.byref(nb)),
               "ws")
    ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device="cuda")
    o2 = torch.full_like(q, float("nan"))
    rc = lib.sk_decode(code, q.data_ptr(), k.data_ptr(), v.data_ptr(), o2.data_ptr(),
                       ws.data_ptr(), ws.numel(), used, b, hq, hkv, sk, d, *sts,
                       _lib.strides3(o2), scale, stream)
    _lib.check(rc, "sk_decode")
    torch.cuda.synchronize()
    return o1, o2, used


def test_noalloc_decode_matches_workspace_decode():
    lib = _lib.load()
    # 1: C4-like GQA, the table's split count
    q, k, v = _inputs(16, 32, 8, 8192, 128, torch.bfloat16, 0)
    o1, o2, used = _both(lib, q, k, v, 0)
    assert used > 1
    assert torch.equal(o1, o2), "call 1 (bf16 GQA, table splits)"
    # 2: a smaller MQA input, explicit split count
    q, k, v = _inputs(4, 64, 1, 3000, 64, torch.float16, 1)
    o1, o2, _ = _both(lib, q, k, v, 7)
    assert torch.equal(o1, o2), "call 2 (fp16 MQA, 7 splits)"
    # 3: the table's count lowered to fit the scratch
    q, k, v = _inputs(8, 128, 8, 16384, 256, torch.bfloat16, 2)
    o1, o2, used = _both(lib, q, k, v, 0)
    per_split = 8 * 128 * 257 * 4
    table = _plan(lib, _lib.SK_BF16, 8, 128, 8, 16384, 256)
    assert table * per_split > SCRATCH and used == SCRATCH // per_split < table
    assert torch.equal(o1, o2), "call 3 (split count lowered to fit)"
    # 4: fp32 (unsplit; LSE in the scratch)
    q, k, v = _inputs(2, 8, 2, 500, 64, torch.float32, 3)
    o1, o2, _ = _both(lib, q, k, v, 0)
    assert torch.equal(o1, o2), "call 4 (fp32)"
    # 5: the first shape again, after the scratch held other calls' data
    q, k, v = _inputs(16, 32, 8, 8192, 128, torch.bfloat16, 0)
    o1, o2, _ = _both(lib, q, k, v, 0)
    assert torch.equal(o1, o2), "call 5 (repeat of call 1)"
    assert torch.isfinite(o1.float()).all()
