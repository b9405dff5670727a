"""The CPU timing restatement (oracle/rayon_path.c) against the parity oracle.

bench.py times rayon_path.c as the reference's own CPU path for standard
attention (AVX2/FMA GEMM and GEMV kernels, Rayon splits, repeat-KV, additive
mask, fused softmax, Tensor::cat of the cache).  Its numbers only mean
something if it computes the same attention, so every driver and every
kernel remainder path is checked here against oracle.c within the parity
bar (|x - ref| <= 1e-4 + 1e-3 |ref|).  The shapes are picked to reach each
branch of the kernels: 6- and 4-row tiles with row remainders, 16-, 8- and
1-column tails, k not a multiple of 8 or 2, GEMV chunks ending in 8-, 4- and
1-row groups, and strided (non-contiguous) operands.
"""
import numpy as np
import pytest

import nne_testlib as T


def rnd(seed, *shape, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


@pytest.mark.parametrize("threads", [1, 3, 8])
@pytest.mark.parametrize("b,hq,hkv,tq,tk,d,start", [
    (1, 4, 1, 13, 23, 20, 10),      # row remainders, odd k, 4-col tail, G = 4
    (2, 6, 2, 7, 7, 16, 0),         # square causal prefill, G = 3
    (1, 2, 2, 200, 200, 128, 0),    # several 96-row chunks, 16-col tiles
    (1, 8, 2, 5, 300, 44, 295),     # few rows at the end of a long key range
])
def test_gqa_prefill_matches_oracle(threads, b, hq, hkv, tq, tk, d, start):
    q, k, v = rnd(1, b, hq, tq, d), rnd(2, b, hkv, tk, d), rnd(3, b, hkv, tk, d)
    out, times = T.rp_attention(q, k, v, mode="gqa", start_pos=start, threads=threads)
    ref = T.ref_standard(q, k, v, masked=True, start_pos=start)
    T.assert_close(out, ref, what="rayon gqa %s" % ((b, hq, hkv, tq, tk, d, start),))
    assert times["qk"] > 0 and times["pv"] > 0
    assert (times["repeat_kv"] > 0) == (hq > hkv)


@pytest.mark.parametrize("tk", [1, 9, 1003])
@pytest.mark.parametrize("d", [44, 100, 128])
def test_gqa_single_row_gemv_matches_oracle(tk, d):
    q, k, v = rnd(4, 2, 8, 1, d), rnd(5, 2, 2, tk, d), rnd(6, 2, 2, tk, d)
    out, _ = T.rp_attention(q, k, v, mode="gqa", start_pos=tk - 1, threads=3)
    T.assert_close(out, T.ref_standard(q, k, v, masked=False), what="rayon gemv")


def test_mha_strided_views_bottom_right_mask():
    b, h, tq, tk, d = 2, 3, 6, 31, 24
    q, k, v = rnd(7, b, h, tq, d), rnd(8, b, h, tk, d), rnd(9, b, h, tk, d)
    # the projections' memory order [B, T, H, d]; the driver reads them as
    # the transposed views the reference makes (non-contiguous).
    qt, kt, vt = (np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in (q, k, v))
    out, times = T.rp_attention(qt, kt, vt, mode="mha", causal=True, q_bthd=True, kv_bthd=True,
                                threads=4)
    T.assert_close(out, T.ref_standard(q, k, v, masked=True, start_pos=tk - tq), what="rayon mha")
    assert times["gather"] > 0 and times["mask"] > 0 and times["repeat_kv"] == 0
    out_nc, times_nc = T.rp_attention(qt, kt, vt, mode="mha", causal=False, q_bthd=True,
                                      kv_bthd=True, threads=4)
    T.assert_close(out_nc, T.ref_standard(q, k, v, masked=False), what="rayon mha non-causal")
    assert times_nc["mask"] < times["mask"]


def test_cross_attention_matches_oracle():
    b, h, tq, tk, d = 2, 5, 8, 150, 64
    q, k, v = rnd(10, b, h, tq, d), rnd(11, b, h, tk, d), rnd(12, b, h, tk, d)
    qt, kt, vt = (np.ascontiguousarray(x.transpose(0, 2, 1, 3)) for x in (q, k, v))
    out, _ = T.rp_attention(qt, kt, vt, mode="cross", q_bthd=True, kv_bthd=True, threads=5)
    T.assert_close(out, T.ref_standard(q, k, v, masked=False), what="rayon cross")


@pytest.mark.parametrize("mode,hq,hkv,d", [("gqa", 8, 2, 40), ("gqa", 4, 4, 128),
                                           ("mha", 3, 3, 64)])
def test_decode_run_matches_oracle_steps(mode, hq, hkv, d):
    """Every step's context and the final cache, against the oracle's decode
    step applied step by step (an empty slot takes the new row as it is)."""
    rng = np.random.default_rng(13)
    b, steps = 4, 5
    lens = np.array([0, 1, 37, 70], np.int32)
    cap = int(lens.max()) + steps
    kc = rng.standard_normal((b, hkv, cap, d)).astype(np.float32)
    vc = rng.standard_normal((b, hkv, cap, d)).astype(np.float32)
    qs = rng.standard_normal((steps, b, hq, d)).astype(np.float32)
    kns = rng.standard_normal((steps, b, hkv, d)).astype(np.float32)
    vns = rng.standard_normal((steps, b, hkv, d)).astype(np.float32)
    outs, times, kend, vend = T.rp_decode_run(qs, kc, vc, lens, kns, vns, mode=mode, threads=3,
                                              want_cache=True)
    ok, ov, ol = kc.copy(), vc.copy(), lens.copy()
    for s in range(steps):
        ref, ok, ov, ol = T.ref_decode_step(qs[s][:, :, None, :], ok, ov, ol,
                                            kns[s][:, :, None, :], vns[s][:, :, None, :])
        T.assert_close(outs[s], ref[:, :, 0, :], what="rayon decode %s step %d" % (mode, s))
    assert (ol == lens + steps).all()
    for bi in range(b):
        n = int(ol[bi])
        assert np.array_equal(kend[bi, :, :n], ok[bi, :, :n])
        assert np.array_equal(vend[bi, :, :n], ov[bi, :, :n])
    assert times["cat"] > 0 and (times["repeat_kv"] > 0) == (hq > hkv)


def test_decode_run_rejects_overfull_cache():
    kc = np.zeros((1, 1, 4, 8), np.float32)
    q = np.zeros((2, 1, 1, 8), np.float32)
    kn = np.zeros((2, 1, 1, 8), np.float32)
    with pytest.raises(AssertionError):
        T.rp_decode_run(q, kc, kc, np.array([3], np.int32), kn, kn)


@pytest.mark.parametrize("hq,hkv,d,c,bias,rope", [(4, 2, 16, 64, False, True),
                                                  (8, 8, 64, 512, True, False),
                                                  (6, 3, 24, 100, True, True)])
def test_qkv_rope_run_matches_oracle(hq, hkv, d, c, bias, rope):
    """The decode prologue restatement against the oracle's projection +
    head split + RoPE, at odd d_model (GEMV tails) and with and without
    biases and tables."""
    rng = np.random.default_rng(14)
    b = 5
    x = rng.standard_normal((b, c)).astype(np.float32)
    w = [rng.standard_normal((h * d, c)).astype(np.float32) * c ** -0.5 for h in (hq, hkv, hkv)]
    bs = [rng.standard_normal(h * d).astype(np.float32) if bias else None for h in (hq, hkv, hkv)]
    cos, sin = T.ref_rope_tables(600, d) if rope else (None, None)
    pos = rng.integers(0, 600, size=b).astype(np.int32)
    q, k, v, times = T.rp_qkv_rope_run(x, *w, *bs, cos, sin, pos, hq, hkv, threads=3)
    if rope:
        rq, rk, rv = T.ref_qkv_rope(x[:, None, :], *w, *bs, cos, sin, pos, hq, hkv)
    else:
        rq, rk, rv = T.ref_qkv_rope(x[:, None, :], *w, *bs, np.ones((1, d), np.float32),
                                    np.zeros((1, d), np.float32), np.zeros(b, np.int32), hq, hkv)
    for got, ref, n in ((q, rq, "q"), (k, rk, "k"), (v, rv, "v")):
        T.assert_close(got, ref[:, :, 0, :], what="rayon prologue " + n)
    assert times["linear"] > 0 and (times["rope"] > 0) == rope
