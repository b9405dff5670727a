"""GPU parity of the prefill path (MFMA FlashAttention kernel and, for few-query
problems, the split-K kernel) against the CPU oracle and the golden vectors.

Bar: per element |gpu - ref| <= 1e-4 + 1e-3 * |ref| (f32 vs the reference's
f32 path).  Inputs are seeded; every case prints its name before running.
"""
import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu


def rnd(seed, *shape, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * std).astype(np.float32)


def dev(x, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("name", T.golden_names("flash"))
def test_flash_golden(nne, cuda, name):
    print("case", name, flush=True)
    g = T.load_golden(name)
    out = nne.flash_attention_forward(dev(g["q"], cuda), dev(g["k"], cuda), dev(g["v"], cuda),
                                      bool(g["causal"]))
    got = host(out)
    T.assert_close(got, g["out"], what=name)
    T.assert_close(got, T.ref_flash(g["q"], g["k"], g["v"], bool(g["causal"])), what=name)


@pytest.mark.parametrize("name", T.golden_names("gqa") + T.golden_names("cross"))
def test_gqa_and_cross_golden(nne, cuda, name):
    print("case", name, flush=True)
    g = T.load_golden(name)
    causal = bool(g["causal"])
    out = nne.attention_forward(dev(g["q"], cuda), dev(g["k"], cuda), dev(g["v"], cuda), causal,
                                q_offset=int(g["q_offset"]))
    got = host(out)
    T.assert_close(got, g["out"], what=name)
    ref = T.ref_standard(g["q"], g["k"], g["v"], masked=causal, start_pos=int(g["q_offset"]))
    T.assert_close(got, ref, what=name)


def test_config1_causal_b1h4t256d64(nne, cuda):
    """Config 1 exactly: B=1, H=4, T=256, d=64, causal, N(0,1)."""
    q, k, v = rnd(0x5EED0001, 1, 4, 256, 64), rnd(0x5EED0002, 1, 4, 256, 64), rnd(0x5EED0003, 1, 4, 256, 64)
    got = host(nne.flash_attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True))
    T.assert_close(got, T.ref_flash(q, k, v, True), what="config1")


@pytest.mark.parametrize("b,h,tq,tk,d,causal", [
    (1, 2, 33, 33, 64, True), (2, 3, 64, 64, 128, False), (1, 1, 95, 95, 32, True),
    (1, 2, 200, 130, 64, False), (1, 1, 130, 200, 128, True), (1, 2, 1, 300, 64, True),
    (2, 1, 257, 257, 16, True), (1, 1, 64, 64, 8, False),
])
def test_flash_shapes(nne, cuda, b, h, tq, tk, d, causal):
    print("case", b, h, tq, tk, d, causal, flush=True)
    s = 1000 * tq + d
    q, k, v = rnd(s, b, h, tq, d), rnd(s + 1, b, h, tk, d), rnd(s + 2, b, h, tk, d)
    got = host(nne.flash_attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), causal))
    T.assert_close(got, T.ref_flash(q, k, v, causal), what="flash shape")


def test_flash_strided_views_match_contiguous(nne, cuda):
    """[B, T, H, d] projections read through strides (FlashAttention layer
    layout, flash_attention.rs:259-261), output written through strides."""
    import torch
    b, t, h, d = 2, 100, 4, 64
    x = rnd(5, b, t, h, d)
    y = rnd(6, b, t, h, d)
    z = rnd(7, b, t, h, d)
    qb, kb, vb = dev(x, cuda), dev(y, cuda), dev(z, cuda)
    q, k, v = qb.transpose(1, 2), kb.transpose(1, 2), vb.transpose(1, 2)
    out = torch.empty(b, t, h, d, device=cuda)
    nne.flash_attention_forward(q, k, v, True, out=out.transpose(1, 2))
    ref = T.ref_flash(x.transpose(0, 2, 1, 3), y.transpose(0, 2, 1, 3), z.transpose(0, 2, 1, 3), True)
    T.assert_close(host(out).transpose(0, 2, 1, 3), ref, what="strided")


def test_flash_scalar_path_odd_head_dim_and_dim_stride(nne, cuda):
    """d % 4 != 0 and a non-unit dim stride take the scalar-load kernel."""
    q, k, v = rnd(8, 1, 2, 70, 30), rnd(9, 1, 2, 70, 30), rnd(10, 1, 2, 70, 30)
    got = host(nne.flash_attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True))
    T.assert_close(got, T.ref_flash(q, k, v, True), what="d=30")
    big = rnd(11, 1, 2, 70, 64)
    view = dev(big, cuda)[..., ::2]        # dim stride 2 -> scalar path
    got = host(nne.flash_attention_forward(view, view, view, False))
    sub = np.ascontiguousarray(big[..., ::2])
    T.assert_close(got, T.ref_flash(sub, sub, sub, False), what="dim stride 2")


def test_explicit_scale(nne, cuda):
    q, k, v = rnd(12, 1, 2, 50, 64), rnd(13, 1, 2, 50, 64), rnd(14, 1, 2, 50, 64)
    got = host(nne.flash_attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), False,
                                           scale=0.05))
    T.assert_close(got, T.ref_flash(q, k, v, False, scale=0.05), what="scale")


def test_empty_keys_and_fully_masked_rows_are_zero(nne, cuda):
    import torch
    q = dev(rnd(15, 1, 2, 40, 64), cuda)
    e = torch.zeros(1, 2, 0, 64, device=cuda)
    out = nne.flash_attention_forward(q, e, e, False)
    assert not host(out).any()
    # negative offset: rows r < 5 see no key (c <= r - 5) and stay zero
    k, v = rnd(16, 1, 2, 40, 64), rnd(17, 1, 2, 40, 64)
    got = host(nne.attention_forward(q, dev(k, cuda), dev(v, cuda), True, q_offset=-5))
    assert not got[:, :, :5].any()
    qn = host(q)
    ref = T.ref_standard(qn[:, :, 5:], k, v, True, start_pos=0)
    T.assert_close(got[:, :, 5:], ref, what="negative offset")


@pytest.mark.parametrize("g", [1, 2, 4, 8, 3])
def test_gqa_group_sizes(nne, cuda, g):
    hkv, t, d = 2, 97, 64
    q, k, v = rnd(20 + g, 1, hkv * g, t, d), rnd(30 + g, 1, hkv, t, d), rnd(40 + g, 1, hkv, t, d)
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True))
    T.assert_close(got, T.ref_standard(q, k, v, True), what="gqa g=%d" % g)


def _config2_inputs(b, hq, hkv, t, d, seed):
    """Config 2 inputs: N(0,1) Q/K/V with a per-position scale in [0.5, 1.5]
    applied to Q and K (all heads, all dims)."""
    rng = np.random.default_rng(seed)
    s = rng.uniform(0.5, 1.5, size=t).astype(np.float32)
    q = rng.standard_normal((b, hq, t, d)).astype(np.float32) * s[None, None, :, None]
    k = rng.standard_normal((b, hkv, t, d)).astype(np.float32) * s[None, None, :, None]
    v = rng.standard_normal((b, hkv, t, d)).astype(np.float32)
    return q, k, v


def test_config2_reduced_gqa_prefill(nne, cuda):
    q, k, v = _config2_inputs(1, 8, 2, 512, 128, 0x5EED0002)
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True))
    T.assert_close(got, T.ref_standard(q, k, v, True), what="config2 reduced")


def test_config2_full_size_sampled_heads(nne, cuda):
    """Full config 2 (B=4, Hq=32, Hkv=8, T=2048, d=128): every output finite,
    causal row 0 equals V[0], and sampled heads match the oracle exactly-sized."""
    b, hq, hkv, t, d = 4, 32, 8, 2048, 128
    q, k, v = _config2_inputs(b, hq, hkv, t, d, 0x5EED0002)
    out = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True))
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out[:, :, 0], np.repeat(v[:, :, 0], hq // hkv, axis=1),
                               rtol=1e-6, atol=1e-6)
    for bi, h in [(0, 0), (3, 31), (1, 13)]:
        kv = h // (hq // hkv)
        ref = T.ref_standard(q[bi:bi + 1, h:h + 1], k[bi:bi + 1, kv:kv + 1],
                             v[bi:bi + 1, kv:kv + 1], True)
        T.assert_close(out[bi:bi + 1, h:h + 1], ref, what="config2 head (%d,%d)" % (bi, h))


def test_config4_reduced_long_causal(nne, cuda):
    q, k, v = (rnd(0x5EED0004 + i, 1, 2, 2048, 64, std=0.5) for i in range(3))
    got = host(nne.flash_attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True))
    T.assert_close(got, T.ref_flash(q, k, v, True), what="config4 reduced")


def test_config5_noncausal_t1500_and_cross(nne, cuda):
    q, k, v = (rnd(0x5EED0005 + i, 2, 2, 1500, 64) for i in range(3))
    got = host(nne.flash_attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), False))
    T.assert_close(got, T.ref_flash(q, k, v, False), what="config5a reduced")
    qx = rnd(0x5EED0015, 2, 2, 8, 64)
    got = host(nne.attention_forward(dev(qx, cuda), dev(k, cuda), dev(v, cuda), False))
    T.assert_close(got, T.ref_standard(qx, k, v, False), what="config5b reduced")


@pytest.mark.parametrize("g,tq,tk,d", [(1, 1, 300, 128), (2, 2, 77, 64), (4, 1, 1029, 128),
                                        (1, 4, 64, 96), (3, 1, 515, 32), (2, 3, 200, 128),
                                        (5, 3, 150, 64), (16, 1, 333, 128)])
def test_few_query_split_k_row_tiles(nne, cuda, g, tq, tk, d):
    """Few-query cross-attention runs on the split-K kernel: G*Tq <= 4 rows on
    the 4-row tile, up to 16 on the 16-row tile."""
    print("case g=%d tq=%d tk=%d d=%d" % (g, tq, tk, d), flush=True)
    hkv = 2
    q = rnd(700 + g + tq, 2, hkv * g, tq, d)
    k = rnd(701 + tk, 2, hkv, tk, d)
    v = rnd(702 + d, 2, hkv, tk, d)
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), False))
    T.assert_close(got, T.ref_standard(q, k, v, False), what="few-query g=%d tq=%d" % (g, tq))


@pytest.mark.parametrize("g,tq,tk,q_off,d", [
    (1, 9, 1000, 991, 64),     # cached multi-token MHA step (bottom-right mask)
    (4, 4, 700, 696, 128),     # GQA 4-token step, 16 rows
    (2, 2, 300, 298, 128),     # 4 rows: the 4x4 tile
    (1, 3, 40, 5, 64),         # only keys <= 7 visible to any row
    (2, 8, 100, -3, 64),       # rows t < 3 see no key
    (1, 16, 2000, 1984, 32),   # padded head dim
    (4, 1, 500, 10, 128),      # one row: keys <= 10, no per-row mask
])
def test_few_query_causal_rows(nne, cuda, g, tq, tk, q_off, d):
    """Causal problems with G*Tq <= 16 rows per KV head run on the split-K
    kernel over the keys any row can see, masking key c > q_off + t per row
    (llama.rs:277-292, attention.rs:101-108)."""
    print("case causal few-query g=%d tq=%d tk=%d q_off=%d d=%d" % (g, tq, tk, q_off, d), flush=True)
    hkv = 2
    q = rnd(800 + g + tq, 2, hkv * g, tq, d)
    k = rnd(801 + tk, 2, hkv, tk, d)
    v = rnd(802 + d, 2, hkv, tk, d)
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True, q_offset=q_off))
    r0 = max(0, -q_off)
    assert not got[:, :, :r0].any()
    ref = T.ref_standard(q[:, :, r0:], k, v, True, start_pos=q_off + r0)
    T.assert_close(got[:, :, r0:], ref, what="causal few-query g=%d tq=%d" % (g, tq))


# Problems with fewer work items (4 row blocks of 32 rows) than CUs and at
# least 4 key tiles, too long for the small prefill kernel, split every
# item's key tiles into chunks, one workgroup each; the last workgroup of an
# item merges the partial (max, sum, O) records.  Cases: 4 heads of 600
# (chunks of 2 tiles), one item of 16 chunks (cached multi-token step), the
# 16-chunk cap with an odd number of records to fold, GQA through strided
# [B, T, H, d] views on the scalar path, a negative offset (rows without
# keys), a padded head dim.
@pytest.mark.parametrize("b,hq,hkv,tq,tk,d,causal,q_off,strided", [
    (1, 4, 4, 600, 600, 64, True, 0, False),
    (1, 2, 1, 9, 1000, 128, True, 991, False),
    (1, 1, 1, 32, 4096, 64, False, 0, False),
    (2, 8, 2, 160, 700, 32, True, 540, True),
    (1, 3, 3, 200, 333, 128, True, -50, False),
    (1, 2, 2, 130, 450, 80, False, 0, False),
])
def test_key_split_small_problems(nne, cuda, b, hq, hkv, tq, tk, d, causal, q_off, strided):
    import torch
    print("case key split", b, hq, hkv, tq, tk, d, causal, q_off, strided, flush=True)
    s = 31 * tk + d
    q, k, v = rnd(s, b, hq, tq, d), rnd(s + 1, b, hkv, tk, d), rnd(s + 2, b, hkv, tk, d)
    if strided:
        qd, kd, vd = (dev(x.transpose(0, 2, 1, 3), cuda).transpose(1, 2) for x in (q, k, v))
        out = torch.zeros(b, tq, hq, d, device=cuda).transpose(1, 2)
        nne.attention_forward(qd, kd, vd, causal, q_offset=q_off, out=out)
    else:
        out = nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), causal, q_offset=q_off)
    got = host(out)
    r0 = max(0, -q_off) if causal else 0          # rows r < -q_off see no key
    assert not got[:, :, :r0].any()
    ref = T.ref_standard(q[:, :, r0:], k, v, causal, start_pos=q_off + r0)
    T.assert_close(got[:, :, r0:], ref, what="key split")


def test_key_split_workspace_reuse_is_deterministic(nne, cuda):
    """Back-to-back split launches of different shapes share the stream's
    workspace and arrival counters; every call leaves the counters at zero,
    so repeating a call reproduces its output bit for bit."""
    qa, ka, va = (dev(rnd(90 + i, 1, 4, 600, 64), cuda) for i in range(3))
    qb = dev(rnd(93, 1, 2, 9, 128), cuda)
    kb, vb = (dev(rnd(94 + i, 1, 1, 1000, 128), cuda) for i in range(2))
    first = host(nne.attention_forward(qa, ka, va, True))
    for _ in range(3):
        ob = host(nne.attention_forward(qb, kb, vb, True, q_offset=991))
        again = host(nne.attention_forward(qa, ka, va, True))
        assert np.array_equal(again, first)
    T.assert_close(ob, T.ref_standard(host(qb), host(kb), host(vb), True, start_pos=991),
                   what="key split reuse")


def test_linearity_in_v_full_config4_shape(nne, cuda):
    """O is linear in V: f(a V1 + b V2) = a f(V1) + b f(V2) at T = 16384."""
    t = 16384
    q, k = dev(rnd(50, 1, 2, t, 64, std=0.5), cuda), dev(rnd(51, 1, 2, t, 64, std=0.5), cuda)
    v1, v2 = dev(rnd(52, 1, 2, t, 64), cuda), dev(rnd(53, 1, 2, t, 64), cuda)
    o1 = nne.flash_attention_forward(q, k, v1, True)
    o2 = nne.flash_attention_forward(q, k, v2, True)
    o3 = nne.flash_attention_forward(q, k, 0.75 * v1 - 1.5 * v2, True)
    T.assert_close(host(o3), host(0.75 * o1 - 1.5 * o2), what="linearity")
    # the last rows (which see every key) against the oracle
    qn, kn, vn = host(q), host(k), host(v1)
    ref_rows = T.ref_standard(qn[:, :, -4:], kn, vn, True, start_pos=t - 4)
    T.assert_close(host(o1)[:, :, -4:], ref_rows, what="config4 last rows")


@pytest.mark.parametrize("c,h,t", [(64, 4, 16), (1024, 2, 40)])   # d = 16; d = 512 (deep kernel)
def test_flash_layer_matches_composition(nne, cuda, c, h, t):
    layer = nne.FlashAttention(c, h, True, device=cuda, seed=3)
    x = dev(rnd(60, 2, t, c), cuda)
    got = host(layer(x))
    # reference composition (flash_attention.rs:254-275) with the oracle core
    xs = host(x).astype(np.float64)
    def lin(p, a):
        return (a @ host(p[0]).astype(np.float64).T + host(p[1])).astype(np.float32)
    b, d = xs.shape[0], c // h
    q = lin(layer.q_proj, xs).reshape(b, t, h, d).transpose(0, 2, 1, 3)
    k = lin(layer.k_proj, xs).reshape(b, t, h, d).transpose(0, 2, 1, 3)
    v = lin(layer.v_proj, xs).reshape(b, t, h, d).transpose(0, 2, 1, 3)
    core = T.ref_flash(q, k, v, True).transpose(0, 2, 1, 3).reshape(b, t, c)
    T.assert_close(got, lin(layer.out_proj, core.astype(np.float64)), atol=2e-4, rtol=2e-3,
                   what="layer d=%d" % d)


def test_stream_release_frees_and_reallocates(nne, cuda):
    """nne_stream_release drops a stream's workspace and counters; the next
    call on the stream allocates them again and gives the same result."""
    import torch
    s = torch.cuda.Stream(device=cuda)
    q, k, v = (dev(rnd(400 + i, 1, 4, 600, 64), cuda) for i in range(3))   # key-split path
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        a = nne.attention_forward(q, k, v, True, stream=s)
    nne.release_stream(s)
    nne.release_stream(s)                       # nothing left to free: still OK
    with torch.cuda.stream(s):
        b = nne.attention_forward(q, k, v, True, stream=s)
    s.synchronize()
    assert np.array_equal(host(a), host(b))
    T.assert_close(host(b), T.ref_flash(host(q), host(k), host(v), True), what="after release")


@pytest.mark.parametrize("b,hq,hkv,tq,tk,d,causal,q_off", [
    (1, 2, 2, 200, 200, 256, True, 0),      # flash causal, d = 256
    (1, 1, 1, 300, 300, 256, False, 0),     # non-causal
    (2, 4, 2, 70, 90, 192, True, 20),       # GQA, bottom-right offset, padded dim
    (1, 3, 3, 33, 33, 160, True, 0),        # a 1-row block after a full one
    (2, 8, 2, 8, 500, 256, False, 0),       # 8 queries x G = 4: one 32-row unit per KV head
    (1, 2, 1, 40, 64, 256, True, -10),      # rows that see no key
    (1, 8, 2, 257, 257, 256, True, 0),      # GQA, units that straddle workgroups
    (3, 5, 5, 100, 37, 224, False, 0),      # Tk < Tq, padded dim
    (1, 4, 4, 64, 1000, 256, True, 936),    # a few rows at the end of a long cache
    (2, 4, 4, 3, 300, 256, True, 297),      # 3 rows per KV head: split-K kernel
    (1, 8, 2, 4, 100, 192, False, 0),       # 16 rows per KV head: split-K kernel
])
def test_head_dims_above_128(nne, cuda, b, hq, hkv, tq, tk, d, causal, q_off):
    """flash_attention_forward takes any head dim (flash_attention.rs:39-48):
    d in (128, 256] runs on the wave-pair MFMA kernel (each 32-row unit on two
    waves, one per half of the head dim) when its work items fill the device
    at d = 256, else on the deep kernel (its 2-wave form, or its key split for
    problems of few units), or on the split-K kernel when a KV head has at
    most 16 query rows.  (These shapes are small: all but the split-K ones
    take the deep kernel.)"""
    print("case wide head dim", b, hq, hkv, tq, tk, d, causal, q_off, flush=True)
    s = 17 * tq + d
    q, k, v = rnd(s, b, hq, tq, d), rnd(s + 1, b, hkv, tk, d), rnd(s + 2, b, hkv, tk, d)
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), causal,
                                     q_offset=q_off))
    r0 = max(0, -q_off) if causal else 0
    assert not got[:, :, :r0].any()
    ref = T.ref_standard(q[:, :, r0:], k, v, causal, start_pos=q_off + r0)
    T.assert_close(got[:, :, r0:], ref, what="d=%d" % d)
    if hq == hkv and tq == tk and q_off == 0:
        T.assert_close(got, T.ref_flash(q, k, v, causal), what="d=%d flash" % d)


@pytest.mark.parametrize("b,hq,hkv,tq,tk,d,causal,q_off", [
    (1, 2, 2, 200, 200, 512, True, 0),      # flash causal, d = 512
    (1, 1, 1, 150, 150, 260, False, 0),     # a last chunk with 4 valid dims of 8
    (2, 4, 2, 70, 90, 320, True, 20),       # GQA, bottom-right offset
    (1, 2, 1, 40, 64, 384, True, -10),      # rows that see no key
    (2, 8, 2, 8, 300, 512, False, 0),       # 8 queries x G = 4: one unit per KV head
    (1, 3, 3, 33, 33, 1024, True, 0),       # one 1024-dim output chunk on 8 waves
    (1, 2, 2, 70, 70, 1028, True, 0),       # two output chunks, Q^T beyond 128 dims per wave re-read
    (2, 8, 8, 300, 300, 768, True, 0),      # 160 units, unsplit, a partial last unit
    (1, 16, 4, 100, 130, 1024, True, 30),   # GQA above 512 dims, units straddling heads
    (1, 1, 1, 64, 100, 2048, False, 0),
    (3, 5, 5, 100, 37, 768, False, 0),      # Tk < Tq
    (2, 4, 4, 3, 300, 640, True, 297),      # a few rows at the end of a long cache
    (1, 8, 2, 257, 257, 512, True, 0),      # GQA, units that straddle query heads
    (1, 8, 2, 64, 96, 512, True, 32),       # GQA, units by query position blocks
])
def test_head_dims_above_256(nne, cuda, b, hq, hkv, tq, tk, d, causal, q_off):
    """Above 256 dims (the reference's attention takes any head dim,
    flash_attention.rs:39-48) the deep kernel runs: 8 waves per 32-row unit
    split S = Q K^T by dims and O = P V by output blocks."""
    print("case deep head dim", b, hq, hkv, tq, tk, d, causal, q_off, flush=True)
    s = 19 * tq + d
    q, k, v = rnd(s, b, hq, tq, d), rnd(s + 1, b, hkv, tk, d), rnd(s + 2, b, hkv, tk, d)
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), causal,
                                     q_offset=q_off))
    r0 = max(0, -q_off) if causal else 0
    assert not got[:, :, :r0].any()
    ref = T.ref_standard(q[:, :, r0:], k, v, causal, start_pos=q_off + r0)
    T.assert_close(got[:, :, r0:], ref, what="d=%d" % d)
    if hq == hkv and tq == tk and q_off == 0:
        T.assert_close(got, T.ref_flash(q, k, v, causal), what="d=%d flash" % d)


@pytest.mark.parametrize("b,hq,hkv,tq,tk,d,causal,q_off,layout", [
    (1, 24, 24, 1024, 1024, 512, True, 0, 0),    # 768 units, causal
    (1, 24, 24, 1024, 1024, 512, True, 0, 1),    # the same on [B, T, H, d] views
    (2, 32, 8, 512, 700, 320, True, 188, 0),     # GQA by query position blocks, offset
    (8, 32, 8, 100, 100, 512, True, 0, 0),       # GQA, units straddling query heads
    (1, 32, 32, 512, 600, 260, False, 0, 0),     # a last chunk with 4 valid dims of 8
    (2, 64, 8, 256, 256, 384, True, -10, 0),     # G = 8, rows that see no key
    (3, 24, 24, 230, 77, 448, False, 0, 1),      # Tk < Tq, a partial last unit, views
])
def test_deep_four_wave_form(nne, cuda, b, hq, hkv, tq, tk, d, causal, q_off, layout):
    """Prefill problems of more workgroups than CUs (causal: more than two
    per CU; 257+ and 513+ units on the 256-CU MI355X) run the deep kernel's
    4-wave form: two workgroups per CU, S from 4 partials, half of each
    wave's Q^T in LDS.  A second call gives the same bits."""
    print("case deep four-wave", b, hq, hkv, tq, tk, d, causal, q_off, layout, flush=True)
    s = 29 * tq + d
    q, k, v = rnd(s, b, hq, tq, d), rnd(s + 1, b, hkv, tk, d), rnd(s + 2, b, hkv, tk, d)
    if layout == 0:
        qd, kd, vd = dev(q, cuda), dev(k, cuda), dev(v, cuda)
    else:
        qd, kd, vd = (dev(x.transpose(0, 2, 1, 3), cuda).transpose(1, 2) for x in (q, k, v))
    got = host(nne.attention_forward(qd, kd, vd, causal, q_offset=q_off))
    assert np.array_equal(host(nne.attention_forward(qd, kd, vd, causal, q_offset=q_off)), got)
    r0 = max(0, -q_off) if causal else 0
    assert not got[:, :, :r0].any()
    ref = T.ref_standard(q[:, :, r0:], k, v, causal, start_pos=q_off + r0)
    T.assert_close(got[:, :, r0:], ref, what="d=%d four-wave" % d)


@pytest.mark.parametrize("b,hq,hkv,tq,tk,d,causal,q_off", [
    (2, 4, 4, 8, 3000, 512, False, 0),      # cross-attention: 8 queries, keys split in 8
    (1, 8, 2, 4, 2500, 384, True, 2496),    # 4 new rows at the end of a long cache, G = 4
    (1, 2, 1, 3, 1200, 1028, False, 0),     # two output chunks, each split
    (1, 4, 4, 64, 1500, 192, False, 0),     # 129-256 dims off the wave-pair kernel: 8 units split
])
def test_deep_key_split(nne, cuda, b, hq, hkv, tq, tk, d, causal, q_off):
    """Problems with too few query rows to fill the device split each unit's
    keys over up to 8 workgroups (partial records, then the combine kernel);
    with a workspace too small for any record the same call runs unsplit."""
    import torch
    print("case deep key split", b, hq, hkv, tq, tk, d, causal, q_off, flush=True)
    s = 23 * tq + d
    q, k, v = rnd(s, b, hq, tq, d), rnd(s + 1, b, hkv, tk, d), rnd(s + 2, b, hkv, tk, d)
    size = nne.attention_workspace_size(q.shape, k.shape, causal, q_off)
    assert size.records_bytes > 0 and size.n_counters == 0
    qd, kd, vd = dev(q, cuda), dev(k, cuda), dev(v, cuda)
    split = host(nne.attention_forward(qd, kd, vd, causal, q_offset=q_off,
                                       workspace=nne.Workspace(cuda)))
    ref = T.ref_standard(q, k, v, causal, start_pos=q_off)
    T.assert_close(split, ref, what="d=%d split" % d)
    # Through the C ABI with a 256-byte workspace: no record fits, no error.
    import ctypes
    i64 = lambda v: (ctypes.c_int64 * 4)(*[int(x) for x in v])
    buf = torch.empty(256, dtype=torch.uint8, device=cuda)
    tiny = nne.NneWorkspace(buf.data_ptr(), 256, None, 0)
    out = torch.empty_like(qd)
    rc = nne.lib().nne_attention_forward_ws(
        qd.data_ptr(), i64(qd.shape), i64(qd.stride()), kd.data_ptr(), i64(kd.shape),
        i64(kd.stride()), vd.data_ptr(), i64(vd.shape), i64(vd.stride()), out.data_ptr(),
        i64(out.stride()), int(causal), q_off, 0, 0.0, ctypes.byref(tiny),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == nne.NNE_OK, nne.lib().nne_last_error()
    T.assert_close(host(out), ref, what="d=%d unsplit" % d)


def test_deep_head_dim_strided_views_and_repeat(nne, cuda):
    """d = 512 on [B, T, H, d] views, output through a strided view; a second
    call gives the same bits."""
    import torch
    print("case deep head dim strided views", flush=True)
    b, h, t, d = 2, 3, 90, 512
    rng = np.random.default_rng(63)
    qt, kt, vt = (rng.standard_normal((b, t, h, d), dtype=np.float32) for _ in range(3))
    qv, kv, vv = (dev(x, cuda).transpose(1, 2) for x in (qt, kt, vt))
    out = torch.zeros(b, t, h, d, device=cuda)
    nne.attention_forward(qv, kv, vv, True, out=out.transpose(1, 2))
    first = host(out).copy()
    nne.attention_forward(qv, kv, vv, True, out=out.transpose(1, 2))
    assert np.array_equal(host(out), first)
    ref = T.ref_flash(qt.transpose(0, 2, 1, 3), kt.transpose(0, 2, 1, 3),
                      vt.transpose(0, 2, 1, 3), True)
    T.assert_close(first.transpose(0, 2, 1, 3), ref, what="d=512 strided")


@pytest.mark.parametrize("b,hq,hkv,tq,tk,d,causal,q_off,layout", [
    (2, 16, 16, 256, 256, 192, True, 0, 0),      # 256 units, unsplit
    (2, 16, 16, 256, 256, 192, True, 0, 1),      # the same on [B, T, H, d] views
    (2, 16, 4, 300, 350, 160, True, 50, 0),      # GQA, units straddling query heads, offset
    (1, 32, 8, 256, 256, 256, True, 0, 0),       # d = 256 with too few wave-pair items
    (3, 8, 8, 130, 90, 228, False, 0, 0),        # Tk < Tq, a half-valid last 8-dim chunk
    (1, 4, 4, 64, 1500, 192, False, 0, 0),       # 8 units: the 8-wave key split at d = 192
])
def test_deep_two_wave_form(nne, cuda, b, hq, hkv, tq, tk, d, causal, q_off, layout):
    """Head dims 129-256 that the wave-pair kernel does not take (dims other
    than 256, or too few of its 4-unit items to fill the device) run the deep
    kernel: its 2-wave form, four workgroups per CU (a wave pair per 32-row
    unit, Q^T half in LDS), or for few units its 8-wave key split.  A second
    call gives the same bits."""
    print("case deep two-wave", b, hq, hkv, tq, tk, d, causal, q_off, layout, flush=True)
    s = 31 * tq + d
    q, k, v = rnd(s, b, hq, tq, d), rnd(s + 1, b, hkv, tk, d), rnd(s + 2, b, hkv, tk, d)
    if layout == 0:
        qd, kd, vd = dev(q, cuda), dev(k, cuda), dev(v, cuda)
    else:
        qd, kd, vd = (dev(x.transpose(0, 2, 1, 3), cuda).transpose(1, 2) for x in (q, k, v))
    got = host(nne.attention_forward(qd, kd, vd, causal, q_offset=q_off))
    assert np.array_equal(host(nne.attention_forward(qd, kd, vd, causal, q_offset=q_off)), got)
    r0 = max(0, -q_off) if causal else 0
    assert not got[:, :, :r0].any()
    ref = T.ref_standard(q[:, :, r0:], k, v, causal, start_pos=q_off + r0)
    T.assert_close(got[:, :, r0:], ref, what="d=%d two-wave" % d)


@pytest.mark.parametrize("d", [192, 256, 512, 1024])
def test_wide_and_deep_dims_empty_keys(nne, cuda, d):
    """No keys (Tk = 0) above 128 dims: every row is zero, on the deep
    kernel's forms as on the others."""
    import torch
    print("case empty keys d=%d" % d, flush=True)
    q = dev(rnd(74, 1, 2, 40, d), cuda)
    e = torch.zeros(1, 2, 0, d, device=cuda)
    for causal in (False, True):
        out = torch.full((1, 2, 40, d), float("nan"), device=cuda)
        nne.attention_forward(q, e, e, causal, out=out)
        assert not host(out).any()


def test_wide_dims_kv_row_stride_beyond_deep_kernel(nne, cuda):
    """At 129-256 dims, K/V views whose row stride is beyond the deep kernel's
    32-bit tile offsets (2^25 floats) stay on the wave-pair kernel."""
    import torch
    print("case wide dims huge kv row stride", flush=True)
    d, tk, tq = 192, 3, 40
    q, k, v = rnd(71, 1, 1, tq, d), rnd(72, 1, 1, tk, d), rnd(73, 1, 1, tk, d)
    st = 1 << 25
    kv_buf = torch.zeros(2, (tk - 1) * st + d, device=cuda)
    for i in range(tk):
        kv_buf[0, i * st:i * st + d] = torch.from_numpy(k[0, 0, i])
        kv_buf[1, i * st:i * st + d] = torch.from_numpy(v[0, 0, i])
    kd = kv_buf[0].as_strided((1, 1, tk, d), (tk * st, tk * st, st, 1))
    vd = kv_buf[1].as_strided((1, 1, tk, d), (tk * st, tk * st, st, 1))
    got = host(nne.attention_forward(dev(q, cuda), kd, vd, True, q_offset=tk - tq))
    r0 = tq - tk
    assert not got[:, :, :r0].any()
    ref = T.ref_standard(q[:, :, r0:], k, v, True, start_pos=0)
    T.assert_close(got[:, :, r0:], ref, what="d=192 huge row stride")


@pytest.mark.parametrize("b,hq,hkv,t,causal", [
    (2, 16, 16, 1024, False),    # 256 items of 4 units: the wave-pair kernel
    (1, 32, 8, 1024, True),      # GQA, 256 items
])
def test_wave_pair_kernel_full_device(nne, cuda, b, hq, hkv, t, causal):
    """d = 256 problems whose wave-pair items fill the device stay on the
    wave-pair kernel: sampled rows of sampled heads against the oracle, every
    output finite."""
    print("case wave-pair full device", b, hq, hkv, t, causal, flush=True)
    d = 256
    rng = np.random.default_rng(b * hq * t + causal)
    q, k, v = (rng.standard_normal((b, h, t, d), dtype=np.float32) for h in (hq, hkv, hkv))
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), causal))
    assert np.isfinite(got).all()
    g = hq // hkv
    for bi in {0, b - 1}:
        for h in (0, hq - 1):
            for r0 in (0, t // 2 - 32, t - 64):
                rows = slice(r0, r0 + 64)
                ref = T.ref_standard(q[bi:bi + 1, h:h + 1, rows], k[bi:bi + 1, h // g:h // g + 1],
                                     v[bi:bi + 1, h // g:h // g + 1], causal, start_pos=r0)
                T.assert_close(got[bi:bi + 1, h:h + 1, rows], ref,
                               what="wave pair b %d head %d rows %d" % (bi, h, r0))


def test_wide_head_dim_strided_views_and_repeat(nne, cuda):
    """d = 256 on [B, T, H, d] views (the FlashAttention layer's projections),
    output written through a strided view; a second call gives the same bits."""
    import torch
    print("case wide head dim strided views", flush=True)
    b, h, t, d = 2, 3, 150, 256
    rng = np.random.default_rng(61)
    qt, kt, vt = (rng.standard_normal((b, t, h, d), dtype=np.float32) for _ in range(3))
    qv, kv, vv = (dev(x, cuda).transpose(1, 2) for x in (qt, kt, vt))
    out = torch.zeros(b, t, h, d, device=cuda)
    nne.attention_forward(qv, kv, vv, True, out=out.transpose(1, 2))
    first = host(out).copy()
    nne.attention_forward(qv, kv, vv, True, out=out.transpose(1, 2))
    assert np.array_equal(host(out), first)
    ref = T.ref_flash(qt.transpose(0, 2, 1, 3), kt.transpose(0, 2, 1, 3),
                      vt.transpose(0, 2, 1, 3), True)
    T.assert_close(first.transpose(0, 2, 1, 3), ref, what="d=256 strided")


def test_wide_head_dim_long_causal_prefill(nne, cuda):
    """Causal GQA prefill at T = 4096, d = 256 (Hq = 8, Hkv = 2): rows at the
    start, middle and end of sampled heads against the oracle (each row over
    every key it can see), row 0 == V[0] for every head, all finite."""
    print("case wide head dim T=4096", flush=True)
    b, hq, hkv, t, d = 1, 8, 2, 4096, 256
    rng = np.random.default_rng(62)
    q, k, v = (rng.standard_normal((b, h, t, d), dtype=np.float32) for h in (hq, hkv, hkv))
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True))
    assert np.isfinite(got).all()
    g = hq // hkv
    np.testing.assert_allclose(got[0, :, 0], v[0, np.arange(hq) // g, 0], rtol=1e-6, atol=1e-6)
    for h in (0, 5):
        for r0 in (0, 2000, 4032):
            rows = slice(r0, r0 + 64)
            ref = T.ref_standard(q[:, h:h + 1, rows], k[:, h // g:h // g + 1],
                                 v[:, h // g:h // g + 1], True, start_pos=r0)
            T.assert_close(got[:, h:h + 1, rows], ref, what="T=4096 d=256 head %d rows %d" % (h, r0))


@pytest.mark.parametrize("hq,hkv,t,d", [
    (32, 8, 2048, 128),     # two workgroups on every CU, complementary lengths
    (8, 8, 6144, 64),       # 48 items per XCD: 16 CUs with one, 16 with two
    (8, 8, 2048, 128),      # fewer items than CUs
    (8, 8, 12288, 64),      # beyond two per CU: longest first
])
def test_causal_item_order_without_pairing(nne, cuda, hq, hkv, t, d):
    """Causal problems too small for paired items run one item per workgroup
    in the longest-first order, with complementary lengths on the CUs that
    take two.  Sampled rows (start, middle, end) of sampled heads against the
    oracle, every output finite, row 0 = V[0]."""
    print("case causal item order", hq, hkv, t, d, flush=True)
    rng = np.random.default_rng(hq * t + d)
    q, k, v = (rng.standard_normal((1, h, t, d), dtype=np.float32) for h in (hq, hkv, hkv))
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True))
    assert np.isfinite(got).all()
    g = hq // hkv
    np.testing.assert_allclose(got[0, :, 0], v[0, np.arange(hq) // g, 0], rtol=1e-6, atol=1e-6)
    for h in (0, hq - 1):
        for r0 in (0, t // 2 - 32, t - 64):
            rows = slice(r0, r0 + 64)
            ref = T.ref_standard(q[:, h:h + 1, rows], k[:, h // g:h // g + 1],
                                 v[:, h // g:h // g + 1], True, start_pos=r0)
            T.assert_close(got[:, h:h + 1, rows], ref, what="order head %d rows %d" % (h, r0))


# Problems of at most one workgroup per CU (one per sequence, query head and
# 16-row block) with at most two 16-key tiles per wave run on the small
# prefill kernel: the waves of a workgroup take one row block's key tiles and
# merge in LDS.  Row counts that are not multiples of 16, GQA, offsets of both
# signs (rows that see no key), Tk < Tq and Tk > Tq, padded head dims.  Up to
# half as many row blocks as CUs, two workgroups share a block (each computes
# S and the softmax, and half of P V); the last two shapes have more blocks
# (240 and 132), one workgroup each.
@pytest.mark.parametrize("b,hq,hkv,tq,tk,d,causal,q_off", [
    (1, 4, 4, 256, 256, 64, True, 0),      # config 1
    (2, 6, 2, 37, 37, 64, True, 0),
    (1, 8, 1, 100, 300, 32, True, 200),
    (1, 2, 2, 90, 60, 48, True, -20),
    (1, 3, 3, 70, 450, 64, False, 0),
    (2, 4, 4, 64, 64, 128, True, 0),
    (1, 2, 1, 130, 250, 96, False, 0),
    (1, 5, 5, 17, 200, 128, True, 183),
    (2, 8, 4, 240, 240, 64, True, 0),
    (1, 12, 3, 176, 176, 128, False, 0),
])
def test_small_prefill_kernel_shapes(nne, cuda, b, hq, hkv, tq, tk, d, causal, q_off):
    print("case small prefill", b, hq, hkv, tq, tk, d, causal, q_off, flush=True)
    s = 53 * tq + tk + d
    q, k, v = rnd(s, b, hq, tq, d), rnd(s + 1, b, hkv, tk, d), rnd(s + 2, b, hkv, tk, d)
    got = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), causal,
                                     q_offset=q_off))
    r0 = max(0, -q_off) if causal else 0
    assert not got[:, :, :r0].any()
    ref = T.ref_standard(q[:, :, r0:], k, v, causal, start_pos=q_off + r0)
    T.assert_close(got[:, :, r0:], ref, what="small prefill")
    # the same call again gives the same bits (no state between calls)
    again = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), causal,
                                       q_offset=q_off))
    assert np.array_equal(again, got)
