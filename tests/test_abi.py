"""The C-ABI library: it loads, exports what include/sk_attn.h declares, binds
torch's HIP runtime, and rejects bad arguments before launching anything.
No test here launches a kernel, so all of it runs without a GPU."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sk_attn.h")


@pytest.fixture(scope="module")
def lib():
    from stackkernels_amd._core.attention import _lib
    from stackkernels_amd.csrc import build

    if not os.path.exists(_lib.LIB_PATH):
        build.build()
    return _lib.load()


def header_functions():
    text = open(HEADER).read()
    return re.findall(r"SK_API\s+[\w\s\*]+?\b(sk_\w+)\s*\(", text)


def test_header_declares_expected_api():
    names = set(header_functions())
    assert {"sk_abi_version", "sk_last_error", "sk_attn_fwd", "sk_attn_bwd",
            "sk_attn_bwd_workspace", "sk_attn_bwd_workspace_min", "sk_decode_plan",
            "sk_decode_plan_varlen", "sk_rope_rotate", "sk_decode",
            "sk_decode_workspace",
            "sk_decode_varlen", "sk_kv_cache_update", "sk_decode_paged",
            "sk_kv_cache_update_paged", "sk_attn_fwd_rope", "sk_decode_rope",
            "sk_decode_paged_rope", "sk_kv_cache_update_rope",
            "sk_kv_cache_update_paged_rope", "sk_kernel_config"} <= names


def test_every_declared_symbol_is_exported(lib):
    for name in header_functions():
        assert hasattr(lib, name), f"{name} declared in sk_attn.h but not exported"


def test_abi_version(lib):
    from stackkernels_amd._core.attention import _lib

    assert lib.sk_abi_version() == _lib.ABI_VERSION


def test_single_hip_runtime(lib):
    from stackkernels_amd._core.attention import _lib

    runtimes = _lib.loaded_hip_runtimes()
    assert len(runtimes) == 1, runtimes
    assert "torch" in runtimes[0]


def _st(*x):
    return (ctypes.c_int64 * 3)(*x)


def _fwd(lib, **kw):
    a = dict(dtype=2, q=16, k=16, v=16, o=16, lse=16, B=1, Hq=4, Hkv=2, Sq=8, Sk=8, D=64,
             qs=_st(2048, 512, 64), ks=_st(1024, 512, 64), vs=_st(1024, 512, 64), os_=_st(2048, 512, 64),
             causal=0, scale=0.125)
    a.update(kw)
    return lib.sk_attn_fwd(a["dtype"], a["q"], a["k"], a["v"], a["o"], a["lse"], a["B"], a["Hq"],
                           a["Hkv"], a["Sq"], a["Sk"], a["D"], a["qs"], a["ks"], a["vs"], a["os_"],
                           a["causal"], a["scale"], None)


def test_fwd_argument_errors(lib):
    from stackkernels_amd._core.attention import _lib

    assert _fwd(lib, Hq=3) == _lib.SK_EINVAL
    assert "divisible" in _lib.last_error()
    assert _fwd(lib, D=12) == _lib.SK_EUNSUPPORTED
    assert _fwd(lib, D=264) == _lib.SK_EUNSUPPORTED
    assert _fwd(lib, dtype=7) == _lib.SK_EUNSUPPORTED
    assert _fwd(lib, q=17) == _lib.SK_EINVAL and "aligned" in _lib.last_error()
    assert _fwd(lib, q=None) == _lib.SK_EINVAL
    assert _fwd(lib, qs=_st(2048, 512, 60)) == _lib.SK_EINVAL and "stride" in _lib.last_error()
    assert _fwd(lib, B=0) == _lib.SK_OK  # empty: nothing to launch


def test_decode_plan_table(lib):
    ns, nb = ctypes.c_int(), ctypes.c_size_t()
    # C4: bf16 GQA B=64 Hq=32 Hkv=8 Sk=32768 D=128
    assert lib.sk_decode_plan(2, 64, 32, 8, 32768, 128, ctypes.byref(ns), ctypes.byref(nb)) == 0
    assert 1 < ns.value <= 1024
    assert nb.value == 64 * 32 * ns.value * (128 + 1) * 4
    # uniform length: one round of one-wave workgroups (256 CUs x 8 / 512 (b, h_kv) units = 4);
    # per-row lengths / paged pools: about two rounds (8)
    assert ns.value == 4
    assert lib.sk_decode_plan_varlen(2, 64, 32, 8, 32768, 128, ctypes.byref(ns),
                                     ctypes.byref(nb)) == 0
    assert ns.value == 8 and nb.value == 64 * 32 * 8 * (128 + 1) * 4
    # small cache: one split, no scratch
    assert lib.sk_decode_plan(2, 2, 8, 2, 32, 64, ctypes.byref(ns), ctypes.byref(nb)) == 0
    assert ns.value == 1 and nb.value == 0
    # C5: fp16 MQA B=8 Hq=64 Hkv=1 Sk=131072
    assert lib.sk_decode_plan(1, 8, 64, 1, 131072, 128, ctypes.byref(ns), ctypes.byref(nb)) == 0
    assert ns.value >= 64
    # groups above 16 heads: one round in both plans
    c5 = ns.value
    assert lib.sk_decode_plan_varlen(1, 8, 64, 1, 131072, 128, ctypes.byref(ns),
                                     ctypes.byref(nb)) == 0
    assert ns.value == c5


def test_decode_argument_errors(lib):
    from stackkernels_amd._core.attention import _lib

    st = _st(1024, 128, 128)
    rc = lib.sk_decode(2, 16, 16, 16, 16, None, 0, 4, 1, 8, 2, 100, 128, st, st, st, st, 0.1, None)
    assert rc == _lib.SK_EWORKSPACE
    rc = lib.sk_decode(2, 16, 16, 16, 16, None, 0, 2000, 1, 8, 2, 100, 128, st, st, st, st, 0.1, None)
    assert rc == _lib.SK_EINVAL


def _ds_pair_bytes(hq, hkv, sq, sk, causal):
    """dS bytes per (batch, KV head) pair, from the mask: key block kb (keys
    128 kb ..) writes a 2 KiB tile for each of its four 32-key tiles and every
    query tile from the first one holding a row that sees key 128 kb."""
    nqt = -(-sq // 32)
    tiles = 0
    for kb in range(-(-sk // 128)):
        first = 0
        if causal:  # first query row i with 128 kb <= i + (sk - sq)
            first = max(0, 128 * kb - (sk - sq))
        if first < sq:
            tiles += 4 * (nqt - first // 32)
    return (hq // hkv) * tiles * 2048


def test_bwd_workspace(lib):
    nb, nmin = ctypes.c_size_t(), ctypes.c_size_t()
    rows = 2 * 2 * 32 * 2048 * 4  # delta and lse * log2(e), fp32 per query row
    # C3 (bf16, D = 128): plus the five-GEMM backward's dS tiles, only those a
    # visible key block writes (0.875 of the rectangle here), all 16 pairs in one chunk
    assert lib.sk_attn_bwd_workspace(2, 2, 32, 8, 2048, 8192, 128, 1, ctypes.byref(nb)) == 0
    pair = _ds_pair_bytes(32, 8, 2048, 8192, True)
    assert pair == 4 * 4 * sum(64 - max(0, 4 * kb - 192) for kb in range(64)) * 2048
    assert nb.value == rows + 16 * pair and 16 * pair < 0.9 * 2 * 32 * 256 * 64 * 2048
    assert lib.sk_attn_bwd_workspace_min(2, 2, 32, 8, 2048, 8192, 128, 1, ctypes.byref(nmin)) == 0
    assert nmin.value == rows
    # without the mask: the whole rectangle
    assert lib.sk_attn_bwd_workspace(2, 2, 32, 8, 2048, 8192, 128, 0, ctypes.byref(nb)) == 0
    assert nb.value == rows + 2 * 32 * (8192 // 32) * (2048 // 32) * 2048
    # square causal: about half of it
    assert lib.sk_attn_bwd_workspace(2, 1, 4, 4, 4096, 4096, 128, 1, ctypes.byref(nb)) == 0
    assert nb.value == 2 * 4 * 4096 * 4 + 4 * _ds_pair_bytes(4, 4, 4096, 4096, True)
    # ragged lengths round up to whole tiles; S_q > S_k and S_q < S_k under the mask
    assert lib.sk_attn_bwd_workspace(1, 1, 2, 1, 33, 65, 96, 0, ctypes.byref(nb)) == 0
    assert nb.value == 2 * 512 + 2 * 4 * 2 * 2048  # 66 fp32 rows -> 264 bytes -> 512 (256-aligned)
    for sq, sk in ((33, 65), (200, 70), (1000, 300), (70, 1000), (2048, 2048 + 40), (129, 4000)):
        for causal in (0, 1):
            assert lib.sk_attn_bwd_workspace(2, 3, 4, 2, sq, sk, 128, causal, ctypes.byref(nb)) == 0
            row_b = 2 * (-(-3 * 4 * sq * 4 // 256) * 256)
            assert nb.value == row_b + 6 * _ds_pair_bytes(4, 2, sq, sk, causal), (sq, sk, causal)
    # above the 2 GiB cap: the fewest even chunks (B = 4, H = 32, S = 8192 causal: 68 MB
    # per pair, 31 fit, so 5 chunks of 26 pairs)
    pair = _ds_pair_bytes(32, 32, 8192, 8192, True)
    assert (2 << 30) // pair == 31
    assert lib.sk_attn_bwd_workspace(2, 4, 32, 32, 8192, 8192, 128, 1, ctypes.byref(nb)) == 0
    assert nb.value == 4 * 32 * 8192 * 4 * 2 + 26 * pair
    assert nb.value - 4 * 32 * 8192 * 8 <= 2 << 30
    # the seven-GEMM backward (no dS tiles): D = 64, D = 256, fp32, and one pair's tiles
    # beyond the cap (S = 65536 causal, 4 query heads per KV head)
    for dtype, d, sq, sk in ((2, 64, 2048, 8192), (2, 256, 2048, 8192), (0, 128, 2048, 8192),
                             (2, 128, 65536, 65536)):
        assert lib.sk_attn_bwd_workspace(dtype, 2, 32, 8, sq, sk, d, 1, ctypes.byref(nb)) == 0
        assert nb.value == 2 * 2 * 32 * sq * 4, (dtype, d)


def test_varlen_and_cache_argument_errors(lib):
    from stackkernels_amd._core.attention import _lib

    st = _st(1024, 512, 64)
    # sk_decode_varlen without the lengths array
    rc = lib.sk_decode_varlen(2, 16, 16, 16, 16, 16, 1 << 20, 1, 1, 4, 2, 8, 64,
                              st, st, st, st, None, 0.125, None)
    assert rc == _lib.SK_EINVAL and "cache_seqlens" in _lib.last_error()

    def upd(dtype=2, k=16, v=16, kc=16, vc=16, slots=16, B=1, H=2, T=3, S=8, D=64, sts=None):
        s4 = sts or [st, st, st, st]
        return lib.sk_kv_cache_update(dtype, k, v, kc, vc, slots, B, H, T, S, D, *s4, None)

    assert upd(dtype=9) == _lib.SK_EUNSUPPORTED
    assert upd(H=0) == _lib.SK_EINVAL and "invalid sizes" in _lib.last_error()
    assert upd(D=0) == _lib.SK_EINVAL
    assert upd(sts=[st, None, st, st]) == _lib.SK_EINVAL and "strides" in _lib.last_error()
    assert upd(sts=[st, st, _st(-1, 0, 0), st]) == _lib.SK_EINVAL
    assert upd(slots=None) == _lib.SK_EINVAL and "slot_indices" in _lib.last_error()
    assert upd(T=0) == _lib.SK_OK  # nothing to write: no launch
    assert upd(B=0, k=None) == _lib.SK_OK


def test_paged_argument_errors(lib):
    from stackkernels_amd._core.attention import _lib

    st = _st(1024, 512, 64)

    def dec(page_size=64, num_pages=4, max_pages=2, table=16, lens=16, B=1):
        return lib.sk_decode_paged(2, 16, 16, 16, 16, 16, 1 << 20, 1, B, 4, 2, num_pages,
                                   page_size, max_pages, 64, st, st, st, st, table, lens,
                                   0.125, None)

    assert dec(page_size=48) == _lib.SK_EINVAL and "multiple of 32" in _lib.last_error()
    assert dec(page_size=0) == _lib.SK_EINVAL
    assert dec(max_pages=-1) == _lib.SK_EINVAL
    assert dec(table=None) == _lib.SK_EINVAL and "block_table" in _lib.last_error()
    assert dec(lens=None) == _lib.SK_EINVAL
    assert dec(num_pages=0) == _lib.SK_EINVAL and "pool" in _lib.last_error()
    assert dec(B=0) == _lib.SK_OK

    def upd(page_size=32, num_pages=4, T=3):
        return lib.sk_kv_cache_update_paged(2, 16, 16, 16, 16, 16, 1, 2, T, num_pages, page_size,
                                            64, st, st, st, st, None)

    assert upd(page_size=0) == _lib.SK_EINVAL
    assert upd(num_pages=-1) == _lib.SK_EINVAL
    assert upd(T=0) == _lib.SK_OK


def test_rope_argument_errors(lib):
    """The RoPE arguments are checked before anything else is launched."""
    from stackkernels_amd._core.attention import _lib

    st = _st(1024, 512, 64)

    def rope(cos=16, sin=16, dt=0, rows=128, stride=64, pos=None, start=0):
        return (cos, sin, dt, rows, stride, pos, start)

    def dec(D=64, B=1, **kw):
        return lib.sk_decode_rope(2, 16, 16, 16, 16, 16, 1 << 20, 1, B, 4, 2, 8, D,
                                  st, st, st, st, None, *rope(**kw), 0.125, None)

    assert dec(cos=None) == _lib.SK_EINVAL and "cos/sin" in _lib.last_error()
    assert dec(dt=5) == _lib.SK_EUNSUPPORTED and "table dtype" in _lib.last_error()
    assert dec(D=72) == _lib.SK_EUNSUPPORTED and "multiple of 16" in _lib.last_error()
    assert dec(rows=0) == _lib.SK_EINVAL
    assert dec(stride=32) == _lib.SK_EINVAL and "row stride" in _lib.last_error()
    assert dec(cos=24) == _lib.SK_EINVAL and "16-byte aligned" in _lib.last_error()
    assert dec(stride=66) == _lib.SK_EINVAL and "16-byte aligned" in _lib.last_error()
    assert dec(start=128) == _lib.SK_EINVAL and "outside the rope table" in _lib.last_error()
    assert dec(start=-1) == _lib.SK_EINVAL
    assert dec(B=0) == _lib.SK_OK

    def fwd(Sq=8, **kw):
        return lib.sk_attn_fwd_rope(2, 16, 16, 16, 16, 16, 1, 4, 2, Sq, 8, 64, st, st, st, st, 1,
                                    *rope(**kw), 0.125, None)

    # one base for the batch: all of [start, start + S_q) must be in the table
    assert fwd(start=121) == _lib.SK_EINVAL and "[121, 129)" in _lib.last_error()
    assert fwd(Sq=0, start=121) == _lib.SK_OK

    def upd(T=3, **kw):
        return lib.sk_kv_cache_update_rope(2, 16, 16, 16, 16, 16, 1, 2, T, 8, 64, st, st, st, st,
                                           *rope(**kw), None)

    assert upd(start=126) == _lib.SK_EINVAL and "outside the rope table" in _lib.last_error()
    assert upd(T=0) == _lib.SK_OK

    def pupd(page_size=32, **kw):
        return lib.sk_kv_cache_update_paged_rope(2, 16, 16, 16, 16, 16, 1, 2, 3, 4, page_size, 64,
                                                 st, st, st, st, *rope(**kw), None)

    assert pupd(page_size=0) == _lib.SK_EINVAL
    assert pupd(sin=None) == _lib.SK_EINVAL

    def pdec(**kw):
        return lib.sk_decode_paged_rope(2, 16, 16, 16, 16, 16, 1 << 20, 1, 1, 4, 2, 4, 48, 2, 64,
                                        st, st, st, st, 16, 16, *rope(**kw), 0.125, None)

    assert pdec() == _lib.SK_EINVAL and "multiple of 32" in _lib.last_error()


def test_rope_rotate_argument_errors(lib):
    """sk_rope_rotate checks its layout before launching: out's rows must not
    overlap, in place needs equal strides, a partial overlap of x and out is
    rejected.  (Every case here fails before the launch: the pointers are
    not device memory.)"""
    from stackkernels_amd._core.attention import _lib

    def rot(x=4096, out=1 << 20, xs=(4096, 1024, 64), os_=(4096, 1024, 64), B=2, H=4, S=16, D=64):
        return lib.sk_rope_rotate(2, x, out, B, H, S, D, _st(*xs), _st(*os_), 16, 16, 0, 64, 64,
                                  None, 0, 0, None)

    assert rot(os_=(4096, 1024, 0)) == _lib.SK_EINVAL and "overlap" in _lib.last_error()
    assert rot(os_=(4096, 32, 64)) == _lib.SK_EINVAL and "overlap" in _lib.last_error()
    assert rot(os_=(64, 1024, 64)) == _lib.SK_EINVAL and "overlap" in _lib.last_error()
    assert rot(out=4096, os_=(8192, 1024, 64)) == _lib.SK_EINVAL and "in place" in _lib.last_error()
    assert rot(out=4096 + 256) == _lib.SK_EINVAL and "overlaps x" in _lib.last_error()


def test_decode_noalloc_rejects_oversized_splits(lib):
    """An explicit split count whose partials exceed the static scratch is
    rejected before anything runs (no device call on this path)."""
    from stackkernels_amd._core.attention import _lib

    st = _st(1024, 128, 128)
    # 64 x 64 heads x 64 splits x (128 + 1) x 4 bytes = 135 MB > 32 MiB
    rc = lib.sk_decode_noalloc(2, 16, 16, 16, 16, 64, 64, 64, 8, 32768, 128, st, st, st, st, 0.1,
                               None)
    assert rc == _lib.SK_EWORKSPACE
    assert "static scratch" in _lib.last_error()
    rc = lib.sk_decode_noalloc(2, 16, 16, 16, 16, 2000, 1, 8, 2, 100, 128, st, st, st, st, 0.1,
                               None)
    assert rc == _lib.SK_EINVAL
    rc = lib.sk_decode_noalloc(2, 16, 16, 16, 16, 0, 1, 6, 4, 100, 128, st, st, st, st, 0.1, None)
    assert rc == _lib.SK_EINVAL and "divisible" in _lib.last_error()
