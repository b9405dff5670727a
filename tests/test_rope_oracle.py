"""Pins the oracle's decode-prologue functions (RoPE tables, RoPE apply,
Linear, the fused q/k/v projection) before they are trusted as checkers.

RotaryEmbedding (src/models/llama.rs:64-158) has no golden vectors in the
reference; these checks fix it from the mathematics: the float64 closed form
of each rotation, norm preservation, identity at position 0, composition of
rotations, and the relative-position property of q.k.  The planted-mistake
tests at the end show a wrong sign, a swapped half or an off-by-one position
fails them.
"""
import numpy as np
import pytest

import nne_testlib as T


def rnd(seed, *shape, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def f64_tables(max_seq_len, d, theta=10000.0):
    i = np.arange(d // 2, dtype=np.float64)
    inv = theta ** (-(2.0 * i) / d)
    ang = np.arange(max_seq_len, dtype=np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    return np.concatenate([c, c], 1), np.concatenate([s, s], 1)


def f64_rope(x, cos, sin, start_pos):
    """float64 rotation of each (i, i + d/2) pair with the given f32 tables."""
    x = x.astype(np.float64)
    b, h, t, d = x.shape
    half = d // 2
    out = np.empty_like(x)
    for bi in range(b):
        p = int(np.broadcast_to(start_pos, (b,))[bi])
        c = cos[p:p + t].astype(np.float64)[None]
        s = sin[p:p + t].astype(np.float64)[None]
        x1, x2 = x[bi, :, :, :half], x[bi, :, :, half:]
        out[bi, :, :, :half] = x1 * c[..., :half] - x2 * s[..., :half]
        out[bi, :, :, half:] = x2 * c[..., half:] + x1 * s[..., half:]
    return out


@pytest.mark.parametrize("d,theta", [(16, 10000.0), (64, 10000.0), (128, 500000.0)])
def test_rope_tables_match_float64(d, theta):
    n = 4096
    cos, sin = T.ref_rope_tables(n, d, theta)
    c64, s64 = f64_tables(n, d, theta)
    # f32 rounding of inv_freq and of p * inv_freq moves the angle by up to a
    # few ulp of p * inv_freq; cos/sin move by at most that much.
    tol = 1e-6 + 4.0 * np.arange(n)[:, None] * 2.0 ** -24
    assert (np.abs(cos - c64) <= tol).all()
    assert (np.abs(sin - s64) <= tol).all()
    assert np.array_equal(cos[:, : d // 2], cos[:, d // 2:])
    assert np.array_equal(sin[:, : d // 2], sin[:, d // 2:])
    assert (cos[0] == 1.0).all() and (sin[0] == 0.0).all()


def test_rope_apply_matches_float64_rotation():
    cos, sin = T.ref_rope_tables(300, 32)
    x = rnd(1, 3, 4, 9, 32)
    sp = np.array([0, 17, 290], np.int32)
    out = T.ref_rope_apply(x, cos, sin, sp)
    T.assert_close(out, f64_rope(x, cos, sin, sp), atol=1e-6, rtol=1e-6, what="rope")


def test_rope_apply_preserves_pair_norms_and_is_identity_at_zero():
    cos, sin = T.ref_rope_tables(64, 64)
    x = rnd(2, 2, 3, 40, 64)
    out = T.ref_rope_apply(x, cos, sin, 0)
    h = 32
    n_in = x[..., :h].astype(np.float64) ** 2 + x[..., h:].astype(np.float64) ** 2
    n_out = out[..., :h].astype(np.float64) ** 2 + out[..., h:].astype(np.float64) ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=2e-6, atol=1e-9)
    assert np.array_equal(out[:, :, 0], x[:, :, 0])        # position 0: cos 1, sin 0


def test_rope_rotations_compose():
    cos, sin = T.ref_rope_tables(128, 16)
    x = rnd(3, 1, 2, 1, 16)
    twice = T.ref_rope_apply(T.ref_rope_apply(x, cos, sin, 23), cos, sin, 41)
    once = T.ref_rope_apply(x, cos, sin, 64)
    np.testing.assert_allclose(twice, once, rtol=1e-5, atol=2e-6)


def test_rope_scores_depend_on_position_difference_only():
    cos, sin = T.ref_rope_tables(512, 64)
    q, k = rnd(4, 1, 1, 1, 64), rnd(5, 1, 1, 1, 64)
    s = []
    for shift in (0, 37, 300):
        qr = T.ref_rope_apply(q, cos, sin, 10 + shift).astype(np.float64)
        kr = T.ref_rope_apply(k, cos, sin, 3 + shift).astype(np.float64)
        s.append(float((qr * kr).sum()))
    np.testing.assert_allclose(s, s[0], rtol=2e-5, atol=1e-5)


def test_linear_matches_float64():
    x, w, b = rnd(6, 5, 33), rnd(7, 12, 33), rnd(8, 12)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    T.assert_close(T.ref_linear(x, w), ref, atol=1e-5, rtol=1e-5, what="linear")
    T.assert_close(T.ref_linear(x, w, b), ref + b, atol=1e-5, rtol=1e-5, what="linear+bias")


def test_qkv_rope_is_projection_split_then_rotation():
    b, t, c, hq, hkv, d = 2, 3, 24, 4, 2, 8
    x = rnd(9, b, t, c)
    wq, wk, wv = rnd(10, hq * d, c), rnd(11, hkv * d, c), rnd(12, hkv * d, c)
    bq, bk, bv = rnd(13, hq * d), rnd(14, hkv * d), rnd(15, hkv * d)
    cos, sin = T.ref_rope_tables(32, d)
    sp = np.array([5, 20], np.int32)
    q, k, v = T.ref_qkv_rope(x, wq, wk, wv, bq, bk, bv, cos, sin, sp, hq, hkv)
    x64 = x.astype(np.float64).reshape(b * t, c)

    def heads(y, h):
        return y.reshape(b, t, h, d).transpose(0, 2, 1, 3)

    q64 = heads(x64 @ wq.T.astype(np.float64) + bq, hq)
    k64 = heads(x64 @ wk.T.astype(np.float64) + bk, hkv)
    v64 = heads(x64 @ wv.T.astype(np.float64) + bv, hkv)
    T.assert_close(q, f64_rope(q64, cos, sin, sp), atol=1e-5, rtol=1e-5, what="q")
    T.assert_close(k, f64_rope(k64, cos, sin, sp), atol=1e-5, rtol=1e-5, what="k")
    T.assert_close(v, v64, atol=1e-5, rtol=1e-5, what="v")


# ------------------------------------------------------ planted mistakes -----

def test_checks_catch_rope_sign_half_and_position_mistakes():
    cos, sin = T.ref_rope_tables(64, 16)
    x = rnd(16, 1, 2, 5, 16)
    out = T.ref_rope_apply(x, cos, sin, 7)
    h = 8
    wrong_sign = f64_rope(x, cos, -sin, 7)                 # rotate_half = [x2, -x1]
    swapped = f64_rope(np.concatenate([x[..., h:], x[..., :h]], -1), cos, sin, 7)
    off_by_one = f64_rope(x, cos, sin, 8)
    for bad in (wrong_sign, swapped, off_by_one):
        with pytest.raises(AssertionError):
            T.assert_close(out, bad, atol=1e-6, rtol=1e-6)
