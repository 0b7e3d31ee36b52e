"""Pin the CPU oracle (oracle/attention_oracle.py) before it is used as the checker.

Each function is checked against something other than its own formula:
torch SDPA golden vectors (tests/golden), a brute-force loop, finite
differences, and invariants chosen so that a dropped term, wrong sign, wrong
mask alignment or wrong GQA mapping fails at least one of them.
"""

import math
import os

import numpy as np
import pytest

from oracle import attention_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden_attention.npz")
CASES = ["mha_noncausal", "gqa_causal_prefix", "mqa_causal_square", "gqa_causal_chunked",
         "decode_mqa", "custom_scale"]


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _case(golden, name):
    g = {k.split("/", 1)[1]: v for k, v in golden.items() if k.startswith(name + "/")}
    b, hq, hkv, sq, sk, d, causal = (int(x) for x in g["meta"])
    return g, bool(causal), float(g["scale"])


@pytest.mark.parametrize("name", CASES)
def test_forward_matches_golden(golden, name):
    g, causal, scale = _case(golden, name)
    out, lse = orc.attention_forward(g["q"], g["k"], g["v"], causal, scale)
    np.testing.assert_allclose(out, g["out"], atol=1e-12, rtol=0)
    assert np.array_equal(np.isneginf(lse), np.isneginf(g["lse"]))
    fin = np.isfinite(g["lse"])
    np.testing.assert_allclose(lse[fin], g["lse"][fin], atol=1e-12, rtol=0)


@pytest.mark.parametrize("name", CASES)
def test_backward_matches_golden(golden, name):
    g, causal, scale = _case(golden, name)
    dq, dk, dv = orc.attention_backward(g["q"], g["k"], g["v"], g["do"], causal, scale)
    np.testing.assert_allclose(dq, g["dq"], atol=1e-11, rtol=0)
    np.testing.assert_allclose(dk, g["dk"], atol=1e-11, rtol=0)
    np.testing.assert_allclose(dv, g["dv"], atol=1e-11, rtol=0)


def test_golden_decode_case(golden):
    g, _, scale = _case(golden, "decode_mqa")
    np.testing.assert_allclose(orc.decode(g["q"], g["k"], g["v"], scale), g["out"], atol=1e-12)


def test_planted_top_left_mask_is_caught(golden):
    """A plausible slip -- top-left instead of bottom-right causal alignment -- fails golden."""
    g, _, scale = _case(golden, "gqa_causal_prefix")  # S_q=8 < S_k=24: alignments differ
    q, k, v = g["q"], g["k"], g["v"]
    sq, sk = q.shape[2], k.shape[2]
    kk = orc.repeat_kv(k, q.shape[1] // k.shape[1])
    vv = orc.repeat_kv(v, q.shape[1] // k.shape[1])
    s = np.einsum("bhid,bhjd->bhij", q, kk) * scale
    top_left = np.arange(sk)[None, :] <= np.arange(sq)[:, None]
    s = np.where(top_left, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    wrong = (p / p.sum(-1, keepdims=True)) @ vv
    assert np.abs(wrong - g["out"]).max() > 1e-2


def _rand(rng, *shape):
    return rng.standard_normal(shape)


@pytest.mark.parametrize("hq,hkv,sq,sk,causal", [
    (2, 2, 3, 3, False), (2, 1, 3, 5, True), (4, 2, 5, 3, True), (2, 2, 1, 4, True), (3, 1, 4, 4, True),
])
def test_forward_matches_loops(hq, hkv, sq, sk, causal):
    rng = np.random.default_rng(1)
    q, k, v = _rand(rng, 2, hq, sq, 4), _rand(rng, 2, hkv, sk, 4), _rand(rng, 2, hkv, sk, 4)
    o1, l1 = orc.attention_forward(q, k, v, causal)
    o2, l2 = orc.attention_forward_loops(q, k, v, causal)
    np.testing.assert_allclose(o1, o2, atol=1e-12)
    np.testing.assert_array_equal(np.isneginf(l1), np.isneginf(l2))
    np.testing.assert_allclose(l1[np.isfinite(l2)], l2[np.isfinite(l2)], atol=1e-12)


@pytest.mark.parametrize("hq,hkv,sq,sk,causal", [(2, 1, 3, 4, True), (2, 2, 4, 2, True), (4, 2, 3, 3, False)])
def test_backward_matches_finite_differences(hq, hkv, sq, sk, causal):
    rng = np.random.default_rng(2)
    d = 3
    q, k, v = _rand(rng, 1, hq, sq, d), _rand(rng, 1, hkv, sk, d), _rand(rng, 1, hkv, sk, d)
    do = _rand(rng, 1, hq, sq, d)
    dq, dk, dv = orc.attention_backward(q, k, v, do, causal)

    def loss(q_, k_, v_):
        return float((orc.attention_forward(q_, k_, v_, causal)[0] * do).sum())

    eps = 1e-6
    for arr, grad, idx in ((q, dq, 0), (k, dk, 1), (v, dv, 2)):
        num = np.zeros_like(arr)
        it = np.nditer(arr, flags=["multi_index"])
        for _ in it:
            mi = it.multi_index
            args = [q.copy(), k.copy(), v.copy()]
            args[idx][mi] += eps
            up = loss(*args)
            args[idx][mi] -= 2 * eps
            dn = loss(*args)
            num[mi] = (up - dn) / (2 * eps)
        np.testing.assert_allclose(grad, num, atol=1e-6)


def test_softmax_rows_sum_to_one():
    rng = np.random.default_rng(3)
    p = orc.softmax_probs(_rand(rng, 1, 2, 6, 4), _rand(rng, 1, 2, 9, 4), is_causal=True)
    np.testing.assert_allclose(p.sum(-1), 1.0, atol=1e-12)


def test_gqa_equals_mha_on_repeated_kv_and_grads_sum_per_group():
    rng = np.random.default_rng(4)
    q, k, v = _rand(rng, 2, 6, 5, 4), _rand(rng, 2, 2, 7, 4), _rand(rng, 2, 2, 7, 4)
    do = _rand(rng, 2, 6, 5, 4)
    kr, vr = np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1)
    o_gqa, _ = orc.attention_forward(q, k, v, True)
    o_mha, _ = orc.attention_forward(q, kr, vr, True)
    np.testing.assert_allclose(o_gqa, o_mha, atol=1e-12)
    _, dk_g, dv_g = orc.attention_backward(q, k, v, do, True)
    _, dk_m, dv_m = orc.attention_backward(q, kr, vr, do, True)
    np.testing.assert_allclose(dk_g, dk_m.reshape(2, 2, 3, 7, 4).sum(2), atol=1e-12)
    np.testing.assert_allclose(dv_g, dv_m.reshape(2, 2, 3, 7, 4).sum(2), atol=1e-12)
    # head h reads KV head h // group (repeat_interleave), not h % H_kv
    alt = np.tile(k, (1, 3, 1, 1))
    o_alt, _ = orc.attention_forward(q, alt, np.tile(v, (1, 3, 1, 1)), True)
    assert np.abs(o_alt - o_gqa).max() > 1e-3


def test_causal_row_ignores_hidden_keys():
    rng = np.random.default_rng(5)
    q, k, v = _rand(rng, 1, 1, 4, 4), _rand(rng, 1, 1, 6, 4), _rand(rng, 1, 1, 6, 4)
    o1, _ = orc.attention_forward(q, k, v, True)
    k2, v2 = k.copy(), v.copy()
    # row 1 sees keys j <= 1 + 2 = 3; perturb keys 4, 5
    k2[..., 4:, :] += 10.0
    v2[..., 4:, :] -= 7.0
    o2, _ = orc.attention_forward(q, k2, v2, True)
    np.testing.assert_allclose(o1[..., :2, :], o2[..., :2, :], atol=1e-12)
    assert np.abs(o1[..., 3, :] - o2[..., 3, :]).max() > 1e-3


def test_single_key_gives_v_and_score():
    rng = np.random.default_rng(6)
    q, k, v = _rand(rng, 1, 2, 3, 4), _rand(rng, 1, 2, 1, 4), _rand(rng, 1, 2, 1, 4)
    o, lse = orc.attention_forward(q, k, v, False, 0.7)
    np.testing.assert_allclose(o, np.broadcast_to(v, o.shape), atol=1e-12)
    np.testing.assert_allclose(lse, 0.7 * (q * k).sum(-1), atol=1e-12)


def test_zero_query_gives_mean_of_visible_values():
    rng = np.random.default_rng(7)
    q = np.zeros((1, 1, 3, 4))
    k, v = _rand(rng, 1, 1, 5, 4), _rand(rng, 1, 1, 5, 4)
    o, lse = orc.attention_forward(q, k, v, True)
    for i in range(3):
        vis = i + 2 + 1  # keys 0 .. i + (5 - 3)
        np.testing.assert_allclose(o[0, 0, i], v[0, 0, :vis].mean(0), atol=1e-12)
        np.testing.assert_allclose(lse[0, 0, i], np.log(vis), atol=1e-12)


def test_fully_masked_rows():
    rng = np.random.default_rng(8)
    q, k, v = _rand(rng, 1, 2, 6, 4), _rand(rng, 1, 1, 2, 4), _rand(rng, 1, 1, 2, 4)
    do = _rand(rng, 1, 2, 6, 4)
    o, lse = orc.attention_forward(q, k, v, True)
    assert np.all(o[:, :, :4] == 0) and np.all(np.isneginf(lse[:, :, :4]))
    dq, dk, dv = orc.attention_backward(q, k, v, do, True)
    assert np.all(dq[:, :, :4] == 0)
    do2 = do.copy()
    do2[:, :, :4] = 123.0  # gradients flowing into dead rows change nothing
    _, dk2, dv2 = orc.attention_backward(q, k, v, do2, True)
    np.testing.assert_allclose(dk, dk2, atol=1e-12)
    np.testing.assert_allclose(dv, dv2, atol=1e-12)


def test_empty_keys():
    o, lse = orc.attention_forward(np.ones((1, 1, 2, 4)), np.ones((1, 1, 0, 4)), np.ones((1, 1, 0, 4)))
    assert np.all(o == 0) and np.all(np.isneginf(lse))


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 16])
def test_split_combine_invariant(splits):
    rng = np.random.default_rng(9)
    q, k, v = _rand(rng, 2, 4, 1, 8), _rand(rng, 2, 2, 37, 8), _rand(rng, 2, 2, 37, 8)
    ref, ref_lse = orc.attention_forward(q, k, v, False)
    o, lse = orc.combine_partials(*orc.split_partials(q, k, v, splits))
    np.testing.assert_allclose(o, ref, atol=1e-12)
    np.testing.assert_allclose(lse, ref_lse[..., 0], atol=1e-12)


def test_decode_is_noncausal_forward_and_causal_with_one_query():
    rng = np.random.default_rng(10)
    q, k, v = _rand(rng, 1, 4, 1, 8), _rand(rng, 1, 2, 9, 8), _rand(rng, 1, 2, 9, 8)
    o = orc.decode(q, k, v)
    np.testing.assert_allclose(o, orc.attention_forward(q, k, v, False)[0], atol=1e-12)
    np.testing.assert_allclose(o, orc.attention_forward(q, k, v, True)[0], atol=1e-12)


# ---- per-row cache lengths and the KV-cache append -------------------------

def _dec_inputs(seed, b=3, hq=4, hkv=2, sk=19, d=8):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((b, hq, 1, d)), rng.standard_normal((b, hkv, sk, d)),
            rng.standard_normal((b, hkv, sk, d)))


def test_decode_varlen_full_rows_equal_decode():
    q, k, v = _dec_inputs(0)
    np.testing.assert_allclose(orc.decode_varlen(q, k, v, [19, 19, 19]), orc.decode(q, k, v),
                               rtol=0, atol=1e-15)


def test_decode_varlen_rows_equal_forward_on_sliced_cache():
    # attention_forward is pinned by the golden vectors; each row must be it on its own slice
    q, k, v = _dec_inputs(1)
    lens = [5, 1, 19]
    out = orc.decode_varlen(q, k, v, lens, 0.3)
    for b, n in enumerate(lens):
        ref, _ = orc.attention_forward(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n], False, 0.3)
        np.testing.assert_allclose(out[b:b + 1], ref, rtol=0, atol=1e-15)


def test_decode_varlen_matches_loops():
    q, k, v = _dec_inputs(2, b=2, hq=2, hkv=1, sk=6, d=4)
    out = orc.decode_varlen(q, k, v, [4, 6])
    for b, n in enumerate([4, 6]):
        ref, _ = orc.attention_forward_loops(q[b:b + 1], k[b:b + 1, :, :n], v[b:b + 1, :, :n])
        np.testing.assert_allclose(out[b:b + 1], ref, rtol=1e-12, atol=1e-12)


def test_decode_varlen_empty_and_overlong_rows():
    q, k, v = _dec_inputs(3)
    out = orc.decode_varlen(q, k, v, [0, -3, 1000])
    assert np.all(out[0] == 0) and np.all(out[1] == 0)
    np.testing.assert_allclose(out[2:], orc.decode(q[2:], k[2:], v[2:]), rtol=0, atol=1e-15)
    # a single visible key gives O = V of that key (softmax over one element)
    one = orc.decode_varlen(q, k, v, [1, 1, 1])
    np.testing.assert_allclose(one[:, :, 0], np.repeat(v[:, :, 0], 2, axis=1), rtol=0, atol=1e-15)


def test_kv_cache_update_matches_loops():
    rng = np.random.default_rng(4)
    b, h, t, s, d = 2, 3, 5, 9, 4
    k, v = rng.standard_normal((b, h, t, d)), rng.standard_normal((b, h, t, d))
    kc, vc = rng.standard_normal((b, h, s, d)), rng.standard_normal((b, h, s, d))
    slots = np.array([[3, 0, -1, 8, 5], [9, 2, 4, 100, 1]])
    nk, nv = orc.kv_cache_update(k, v, kc, vc, slots)
    ek, ev = kc.copy(), vc.copy()
    for bi in range(b):
        for ti in range(t):
            sl = slots[bi, ti]
            if 0 <= sl < s:
                for hi in range(h):
                    for di in range(d):
                        ek[bi, hi, sl, di] = k[bi, hi, ti, di]
                        ev[bi, hi, sl, di] = v[bi, hi, ti, di]
    assert np.array_equal(nk, ek) and np.array_equal(nv, ev)
    # untouched rows keep their contents; the inputs are not modified
    assert np.array_equal(nk[0, :, 1], kc[0, :, 1]) and not np.array_equal(nk, kc)


# ---- paged pools ---------------------------------------------------------------

def _pool_inputs(seed, b=3, hq=4, hkv=2, pages=6, ps=4, d=8, mp=3):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, hq, 1, d))
    kp, vp = rng.standard_normal((pages, hkv, ps, d)), rng.standard_normal((pages, hkv, ps, d))
    table = np.stack([rng.permutation(pages)[:mp] for _ in range(b)])
    return q, kp, vp, table


def test_decode_paged_equals_varlen_on_assembled_caches():
    q, kp, vp, table = _pool_inputs(5)
    lens = np.array([5, 12, 0])
    ps = kp.shape[2]
    # assemble each row's cache page by page with explicit loops
    k = np.zeros((3, 2, 12, 8))
    v = np.zeros((3, 2, 12, 8))
    for b in range(3):
        for j in range(12):
            page = table[b, j // ps]
            k[b, :, j] = kp[page, :, j % ps]
            v[b, :, j] = vp[page, :, j % ps]
    np.testing.assert_allclose(orc.decode_paged(q, kp, vp, table, lens, 0.5),
                               orc.decode_varlen(q, k, v, lens, 0.5), rtol=0, atol=1e-15)


def test_decode_paged_out_of_pool_page_masks_its_keys():
    q, kp, vp, table = _pool_inputs(6)
    table[1, 1] = 99  # outside the 6-page pool
    lens = np.array([12, 12, 12])
    out = orc.decode_paged(q, kp, vp, table, lens)
    # row 1 sees its pages 0 and 2 only
    k = np.concatenate([kp[table[1, 0]], kp[table[1, 2]]], axis=1)[None]
    v = np.concatenate([vp[table[1, 0]], vp[table[1, 2]]], axis=1)[None]
    np.testing.assert_allclose(out[1:2], orc.decode(q[1:2], k, v), rtol=0, atol=1e-15)


def test_kv_cache_update_paged_matches_loops():
    rng = np.random.default_rng(7)
    k, v = rng.standard_normal((2, 3, 4, 5)), rng.standard_normal((2, 3, 4, 5))
    kp, vp = rng.standard_normal((4, 3, 8, 5)), rng.standard_normal((4, 3, 8, 5))
    slots = np.array([[0, 9, -1, 31], [17, 40, 2, 8]])
    nk, nv = orc.kv_cache_update_paged(k, v, kp, vp, slots)
    ek, ev = kp.copy(), vp.copy()
    for b in range(2):
        for t in range(4):
            s = slots[b, t]
            if 0 <= s < 32:
                for h in range(3):
                    for d in range(5):
                        ek[s // 8, h, s % 8, d] = k[b, h, t, d]
                        ev[s // 8, h, s % 8, d] = v[b, h, t, d]
    assert np.array_equal(nk, ek) and np.array_equal(nv, ev)


# ---------------------------------------------------------------- RoPE pins

def test_rope_tables_entries_closed_form():
    d, n = 64, 40
    cos, sin = orc.rope_tables(d, n)
    assert cos.shape == sin.shape == (n, d)
    half = d // 2
    for t in (0, 1, 7, 39):
        for i in (0, 1, 5, half - 1):
            ang = t / 10000.0 ** (i / half)
            assert cos[t, i] == pytest.approx(math.cos(ang), abs=1e-12)
            assert sin[t, i] == pytest.approx(math.sin(ang), abs=1e-12)
    np.testing.assert_array_equal(cos[:, :half], cos[:, half:])
    np.testing.assert_array_equal(sin[:, :half], sin[:, half:])
    np.testing.assert_array_equal(cos[0], np.ones(d))
    np.testing.assert_array_equal(sin[0], np.zeros(d))


def _rope_complex(x, cos, sin, pos):
    """The rotation as a complex product (x_d + i x_{d+D/2}) * (cos + i sin), float64."""
    x = np.asarray(x, dtype=np.float64)
    half = x.shape[-1] // 2
    z = x[..., :half] + 1j * x[..., half:]
    c = np.asarray(cos, dtype=np.float64)[pos][:, None, :, :half]
    s = np.asarray(sin, dtype=np.float64)[pos][:, None, :, :half]
    w = z * (c + 1j * s)
    return np.concatenate([w.real, w.imag], axis=-1)


@pytest.mark.parametrize("start_pos", [0, 15, 23, 31, 64])
def test_rope_rotate_matches_complex_product(start_pos):
    rng = np.random.default_rng(start_pos)
    b, h, s, d = 2, 3, 8, 64
    x = rng.standard_normal((b, h, s, d)).astype(np.float32)
    cos, sin = orc.rope_tables(d, start_pos + s + 64)
    pos = orc.rope_positions(start_pos, b, s)
    got = orc.rope_rotate(x, cos, sin, pos)
    want = _rope_complex(x, cos, sin, pos)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def test_rope_rotate_matches_loops_bitwise():
    rng = np.random.default_rng(1)
    b, h, s, d = 2, 2, 5, 32
    x = rng.standard_normal((b, h, s, d)).astype(np.float32)
    cos, sin = (t.astype(np.float32) for t in orc.rope_tables(d, 16))
    pos = np.array([[0, 3, 9, 15, 2], [1, 1, 4, 7, 11]])
    got = orc.rope_rotate(x, cos, sin, pos)
    half = d // 2
    for bi in range(b):
        for hi in range(h):
            for si in range(s):
                p = pos[bi, si]
                for j in range(d):
                    if j < half:
                        other = np.float32(-x[bi, hi, si, j + half])
                    else:
                        other = x[bi, hi, si, j - half]
                    a = np.float32(x[bi, hi, si, j] * cos[p, j])
                    c = np.float32(other * sin[p, j])
                    assert got[bi, hi, si, j] == np.float32(a + c)


def test_rope_rotate_invariants():
    rng = np.random.default_rng(2)
    b, h, s, d = 1, 2, 6, 128
    x = rng.standard_normal((b, h, s, d)).astype(np.float32)
    cos, sin = orc.rope_tables(d, 200)
    half = d // 2
    # position 0 is the identity
    zero = orc.rope_rotate(x, cos, sin, np.zeros((b, s), dtype=np.int64))
    np.testing.assert_array_equal(zero, x)
    # each (d, d + D/2) pair keeps its norm
    pos = orc.rope_positions(37, b, s)
    y = orc.rope_rotate(x, cos, sin, pos).astype(np.float64)
    xn = np.hypot(x[..., :half].astype(np.float64), x[..., half:])
    yn = np.hypot(y[..., :half], y[..., half:])
    np.testing.assert_allclose(yn, xn, rtol=1e-5, atol=1e-6)
    # rotation by p1 then by p2 is rotation by p1 + p2
    p1 = orc.rope_positions(11, b, s) * 0 + 11
    p2 = orc.rope_positions(0, b, s) + 50
    two = orc.rope_rotate(orc.rope_rotate(x, cos, sin, p1), cos, sin, p2)
    one = orc.rope_rotate(x, cos, sin, p1 + p2)
    np.testing.assert_allclose(two, one, rtol=0, atol=2e-5)


def test_rope_rotate_out_of_table_positions_leave_tokens():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 1, 3, 16)).astype(np.float32)
    cos, sin = orc.rope_tables(16, 10)
    pos = np.array([[-1, 4, 10], [9, 12, 0]])
    y = orc.rope_rotate(x, cos, sin, pos)
    np.testing.assert_array_equal(y[0, :, 0], x[0, :, 0])
    np.testing.assert_array_equal(y[0, :, 2], x[0, :, 2])
    np.testing.assert_array_equal(y[1, :, 1], x[1, :, 1])
    assert not np.array_equal(y[0, :, 1], x[0, :, 1])


def test_planted_rope_sign_slip_is_caught():
    """A rotation that negates the wrong half fails the complex-product pin."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 1, 4, 32)).astype(np.float32)
    cos, sin = orc.rope_tables(32, 20)
    pos = orc.rope_positions(5, 1, 4)
    half = 16
    c = cos[pos][:, None]
    s = sin[pos][:, None]
    wrong = x * c + np.concatenate([x[..., half:], -x[..., :half]], axis=-1) * s
    assert np.abs(wrong - _rope_complex(x, cos, sin, pos)).max() > 1e-2


def test_rope_adjoint_is_the_transpose():
    """<R x, y> = <x, R^T y> for tables whose two halves differ (so a sine taken from
    the wrong half, or a wrong sign, breaks the identity), in float64."""
    rng = np.random.default_rng(6)
    b, h, s, d = 2, 2, 5, 32
    cos = rng.standard_normal((12, d))
    sin = rng.standard_normal((12, d))
    x = rng.standard_normal((b, h, s, d))
    y = rng.standard_normal((b, h, s, d))
    pos = np.array([[0, 3, 11, 7, 2], [5, 5, 1, 9, 4]])
    rx = orc.rope_rotate(x, cos, sin, pos).astype(np.float64)
    rty = orc.rope_rotate_adjoint(y, cos, sin, pos, dtype=np.float64)
    lhs = (rx * y).sum(axis=-1)
    rhs = (x * rty).sum(axis=-1)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-5, atol=1e-5)
    # the same identity fails for the rotation itself in place of its adjoint
    wrong = orc.rope_rotate(y, cos, sin, pos).astype(np.float64)
    assert np.abs((x * wrong).sum(axis=-1) - lhs).max() > 1e-1


def test_rope_adjoint_undoes_the_rotation_and_matches_the_reference_formula():
    """With real tables R is orthogonal, so R^T R x = x; and for precompute_freqs tables
    (equal halves) the adjoint is the reference's backward formula
    dx = dy * cos - rotate_half(dy) * sin, bit for bit in float32."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(7)
    b, h, s, d = 2, 3, 6, 64
    cos, sin = orc.rope_tables(d, 100)
    x = rng.standard_normal((b, h, s, d)).astype(np.float32)
    pos = orc.rope_positions(np.array([3, 40]), b, s)
    back = orc.rope_rotate_adjoint(orc.rope_rotate(x, cos, sin, pos), cos, sin, pos)
    np.testing.assert_allclose(back, x, rtol=0, atol=1e-5)
    c32, s32 = cos.astype(np.float32), sin.astype(np.float32)
    dy = torch.from_numpy(x)
    cs = torch.from_numpy(c32[pos][:, None])
    sn = torch.from_numpy(s32[pos][:, None])
    half = d // 2
    rot = torch.cat((-dy[..., half:], dy[..., :half]), dim=-1)
    ref = (dy * cs) - (rot * sn)
    np.testing.assert_array_equal(orc.rope_rotate_adjoint(x, c32, s32, pos), ref.numpy())
    # positions outside the table leave their tokens
    out = orc.rope_rotate_adjoint(x, cos, sin, np.full((b, s), 100))
    np.testing.assert_array_equal(out, x)


def test_round_to_matches_torch_casts():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32) * 3
    # exact ties for bf16: low 16 bits 0x8000 with even and odd kept bits
    ties = (np.array([0x3F808000, 0x3F818000, 0xBF808000, 0x40008000], dtype=np.uint32)
            .view(np.float32))
    x = np.concatenate([x, ties, np.array([0.0, -0.0, 1e-40], dtype=np.float32)])
    t = torch.from_numpy(x)
    np.testing.assert_array_equal(orc.round_to(x, "bf16"), t.to(torch.bfloat16).float().numpy())
    np.testing.assert_array_equal(orc.round_to(x, "f16"), t.to(torch.float16).float().numpy())
    np.testing.assert_array_equal(orc.round_to(x, "f32"), x)
