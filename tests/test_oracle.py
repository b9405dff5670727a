"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each oracle function is checked against (a) the committed golden vectors
(float64 closed forms, cross-checked with torch float64 SDPA when written),
and (b) properties the mathematics fixes, chosen so that a plausible mistake
-- a dropped term, a wrong sign or index, a transposed operand, a wrong head
mapping -- fails at least one of them.  The last tests plant such mistakes in
the oracle's inputs/outputs on the CPU and show the checks catch them.
"""
import numpy as np
import pytest

import nne_testlib as T

TIGHT = dict(atol=3e-6, rtol=3e-5)


def rnd(seed, *shape, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


# ---------------------------------------------------------------- golden -----

@pytest.mark.parametrize("name", T.golden_names("flash"))
def test_flash_oracle_matches_golden(name):
    g = T.load_golden(name)
    out = T.ref_flash(g["q"], g["k"], g["v"], bool(g["causal"]))
    T.assert_close(out, g["out"], what=name, **TIGHT)


@pytest.mark.parametrize("name", T.golden_names("gqa") + T.golden_names("cross"))
def test_standard_oracle_matches_golden(name):
    g = T.load_golden(name)
    out = T.ref_standard(g["q"], g["k"], g["v"], masked=bool(g["causal"]),
                         start_pos=int(g["q_offset"]))
    T.assert_close(out, g["out"], what=name, **TIGHT)


def test_decode_oracle_matches_golden():
    g = T.load_golden("decode_ragged_b5g2d16")
    out, kc, vc, lens = T.ref_decode_step(g["q"], g["k_cache"], g["v_cache"], g["lens"],
                                          g["k_new"], g["v_new"])
    T.assert_close(out, g["out"], what="decode", **TIGHT)
    assert (lens == g["lens"] + 1).all()


# ----------------------------------------------------- flash invariants -----

def test_flash_block_size_invariance():
    q, k, v = rnd(1, 1, 2, 77, 24), rnd(2, 1, 2, 77, 24), rnd(3, 1, 2, 77, 24)
    base = T.ref_flash(q, k, v, True, br=64, bc=64)
    for br, bc in [(16, 16), (16, 32), (32, 64), (8, 8)]:   # 8 clamps to 16 (:51-52)
        np.testing.assert_allclose(T.ref_flash(q, k, v, True, br=br, bc=bc), base, **TIGHT)


def test_flash_causal_first_row_is_v0():
    q, k, v = rnd(4, 2, 3, 20, 16), rnd(5, 2, 3, 20, 16), rnd(6, 2, 3, 20, 16)
    out = T.ref_flash(q, k, v, True)
    assert np.array_equal(out[:, :, 0, :], v[:, :, 0, :])


def test_flash_constant_v_gives_constant_output():
    q, k = rnd(7, 1, 2, 40, 32), rnd(8, 1, 2, 40, 32)
    v = np.full((1, 2, 40, 32), 0.375, np.float32)
    for causal in (False, True):
        np.testing.assert_allclose(T.ref_flash(q, k, v, causal), v, rtol=1e-6, atol=1e-6)


def test_flash_uniform_scores_average_visible_rows():
    q = np.zeros((1, 1, 33, 8), np.float32)
    k, v = rnd(9, 1, 1, 33, 8), rnd(10, 1, 1, 33, 8)
    nc = T.ref_flash(q, k, v, False)
    np.testing.assert_allclose(nc[0, 0], np.broadcast_to(v[0, 0].mean(0), (33, 8)), atol=1e-6)
    ca = T.ref_flash(q, k, v, True)
    want = np.cumsum(v[0, 0].astype(np.float64), axis=0) / np.arange(1, 34)[:, None]
    np.testing.assert_allclose(ca[0, 0], want, atol=1e-6)


def test_flash_noncausal_key_permutation_invariance():
    q, k, v = rnd(11, 1, 2, 19, 16), rnd(12, 1, 2, 45, 16), rnd(13, 1, 2, 45, 16)
    perm = np.random.default_rng(14).permutation(45)
    a = T.ref_flash(q, k, v, False)
    b = T.ref_flash(q, k[:, :, perm], v[:, :, perm], False)
    np.testing.assert_allclose(a, b, **TIGHT)


def test_flash_empty_keys_gives_zero():
    q = rnd(15, 1, 2, 5, 16)
    k = np.zeros((1, 2, 0, 16), np.float32)
    assert not T.ref_flash(q, k, k, False).any()


def test_flash_explicit_scale():
    q, k, v = rnd(16, 1, 1, 9, 8), rnd(17, 1, 1, 9, 8), rnd(18, 1, 1, 9, 8)
    s = q[0, 0].astype(np.float64) @ k[0, 0].T.astype(np.float64) * np.float32(0.3)
    p = np.exp(s - s.max(1, keepdims=True))
    want = (p / p.sum(1, keepdims=True)) @ v[0, 0]
    np.testing.assert_allclose(T.ref_flash(q, k, v, False, scale=0.3)[0, 0], want, **TIGHT)


# -------------------------------------------------- standard / GQA -----------

def test_gqa_equals_mha_on_repeated_kv():
    b, hq, hkv, t, d = 2, 8, 2, 11, 16
    q, k, v = rnd(20, b, hq, t, d), rnd(21, b, hkv, t, d), rnd(22, b, hkv, t, d)
    g = hq // hkv
    gqa = T.ref_standard(q, k, v, masked=True)
    mha = T.ref_standard(q, np.repeat(k, g, axis=1), np.repeat(v, g, axis=1), masked=True)
    assert np.array_equal(gqa, mha)


@pytest.mark.parametrize("start_pos", [0, 3])
def test_standard_mask_enumerated(start_pos):
    """Row r depends exactly on keys c <= start_pos + r (llama.rs:280-283)."""
    tq, d = 4, 8
    tk = tq + start_pos
    q, k, v = rnd(23, 1, 1, tq, d), rnd(24, 1, 1, tk, d), rnd(25, 1, 1, tk, d)
    base = T.ref_standard(q, k, v, masked=True, start_pos=start_pos)
    for c in range(tk):
        k2, v2 = k.copy(), v.copy()
        k2[0, 0, c] += 1.0
        v2[0, 0, c] += 1.0
        out = T.ref_standard(q, k2, v2, masked=True, start_pos=start_pos)
        for r in range(tq):
            changed = not np.array_equal(out[0, 0, r], base[0, 0, r])
            assert changed == (c <= start_pos + r), (c, r)


def test_flash_equals_standard_causal():
    """Two independent algorithms (tiled online softmax vs materialised softmax)."""
    q, k, v = rnd(26, 1, 3, 70, 32), rnd(27, 1, 3, 70, 32), rnd(28, 1, 3, 70, 32)
    np.testing.assert_allclose(T.ref_flash(q, k, v, True), T.ref_standard(q, k, v, True),
                               **TIGHT)


# ------------------------------------------------------- cache / decode ------

def test_kv_append_readback_is_concatenation():
    b, h, cap, d = 3, 2, 10, 8
    kc, vc = np.zeros((b, h, cap, d), np.float32), np.zeros((b, h, cap, d), np.float32)
    lens = np.array([0, 4, 7], np.int32)
    kc[:, :, :7] = rnd(30, b, h, 7, d)
    vc[:, :, :7] = rnd(31, b, h, 7, d)
    kn, vn = rnd(32, b, h, 3, d), rnd(33, b, h, 3, d)
    rc, kc2, vc2, lens2 = T.ref_kv_append(kc, vc, lens, kn, vn)
    assert rc == 0 and (lens2 == lens + 3).all()
    for i in range(b):
        L = lens[i]
        assert np.array_equal(kc2[i, :, :L + 3], np.concatenate([kc[i, :, :L], kn[i]], axis=1))
        assert np.array_equal(vc2[i, :, :L + 3], np.concatenate([vc[i, :, :L], vn[i]], axis=1))
    rc, *_ = T.ref_kv_append(kc2, vc2, lens2, kn, vn)    # 7 + 3 + 3 > 10
    assert rc == 3


def test_decode_equals_last_row_of_causal_prefill():
    """The cached-vs-full pattern of tests/nn/kv_cache_tests.rs:68-103."""
    b, hq, hkv, t, d, cap = 2, 4, 2, 9, 16, 16
    q, k, v = rnd(34, b, hq, t, d), rnd(35, b, hkv, t, d), rnd(36, b, hkv, t, d)
    full = T.ref_standard(q, k, v, masked=True)
    kc = np.zeros((b, hkv, cap, d), np.float32)
    vc = np.zeros((b, hkv, cap, d), np.float32)
    lens = np.zeros(b, np.int32)
    for step in range(t):
        out, kc, vc, lens = T.ref_decode_step(q[:, :, step:step + 1], kc, vc, lens,
                                              k[:, :, step:step + 1], v[:, :, step:step + 1])
        np.testing.assert_allclose(out[:, :, 0], full[:, :, step], rtol=1e-5, atol=2e-6)


# ------------------------------------------------ planted mistakes -----------

def test_checks_catch_wrong_scale():
    g = T.load_golden("flash_causal_b2h4t16d32")
    d = g["q"].shape[-1]
    bad = T.ref_flash(g["q"], g["k"], g["v"], True, scale=1.02 / np.sqrt(d))
    with pytest.raises(AssertionError):
        T.assert_close(bad, g["out"], **TIGHT)


def test_checks_catch_wrong_gqa_head_mapping():
    g = T.load_golden("gqa_g4_b2tq5tk9d32_start4")
    # hq % Hkv instead of hq // G: emulate by interleaving the query heads
    hq = g["q"].shape[1]
    hkv = g["k"].shape[1]
    grp = hq // hkv
    perm = np.array([(h % hkv) * grp + h // hkv for h in range(hq)])
    bad = T.ref_standard(g["q"][:, perm], g["k"], g["v"], True, start_pos=4)[:, np.argsort(perm)]
    with pytest.raises(AssertionError):
        T.assert_close(bad, g["out"], **TIGHT)


def test_checks_catch_off_by_one_mask():
    g = T.load_golden("gqa_g4_b2tq5tk9d32_start4")
    bad = T.ref_standard(g["q"], g["k"], g["v"], True, start_pos=5)
    with pytest.raises(AssertionError):
        T.assert_close(bad, g["out"], **TIGHT)


def test_checks_catch_transposed_kv():
    g = T.load_golden("flash_noncausal_b1h2t32d16")
    bad = T.ref_flash(g["q"], g["v"], g["k"], False)
    with pytest.raises(AssertionError):
        T.assert_close(bad, g["out"], **TIGHT)
