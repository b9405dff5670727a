"""GPU parity of the decode prologue: RoPE (RotaryEmbedding, llama.rs:64-158),
the fused q/k/v projection + RoPE (llama.rs:226-235), and the whole
GroupedQueryAttention::forward_gqa_cached step (llama.rs:205-300) built on
them and on the decode / prefill kernels.

Bars: RoPE on given inputs is bit-exact (the kernel rounds like the
reference's three tensor ops); everything that includes a projection GEMM is
held to |gpu - ref| <= 1e-4 + 1e-3 |ref|; cache lengths exact.
"""
import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu


def rnd(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)


def dev(x, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def weights(rng, out_f, in_f):
    bound = 1.0 / np.sqrt(in_f)
    return rng.uniform(-bound, bound, (out_f, in_f)).astype(np.float32)


# ----------------------------------------------------------------- RoPE ------

@pytest.mark.parametrize("b,h,t,d,starts", [
    (1, 1, 1, 2, [0]),
    (2, 3, 17, 64, [0, 5]),
    (3, 4, 9, 128, [100, 0, 3000]),
])
def test_rope_apply_bit_exact(nne, cuda, b, h, t, d, starts):
    rng = np.random.default_rng(7 + d)
    rope = nne.RotaryEmbedding(d, 4096, device=cuda)
    assert np.array_equal(rope.cos_host, T.ref_rope_tables(4096, d)[0])
    x = rnd(rng, b, h, t, d)
    out = rope.apply(dev(x, cuda), np.array(starts, np.int32))
    ref = T.ref_rope_apply(x, rope.cos_host, rope.sin_host, np.array(starts, np.int32))
    assert np.array_equal(host(out), ref)


def test_rope_apply_strided_view_and_in_place(nne, cuda):
    """The reference rotates q/k as [B, T, H, d] -> [B, H, T, d] views
    (llama.rs:231-235); the kernel reads that view and may write in place."""
    rng = np.random.default_rng(11)
    b, t, h, d = 2, 13, 3, 32
    rope = nne.RotaryEmbedding(d, 64, device=cuda)
    x = rnd(rng, b, t, h, d)
    xd = dev(x, cuda)
    view = xd.transpose(1, 2)                     # [B, H, T, d], strided
    ref = T.ref_rope_apply(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), rope.cos_host,
                           rope.sin_host, np.array([4, 9], np.int32))
    out = rope.apply(view, [4, 9])
    assert np.array_equal(host(out), ref)
    rope.apply(view, [4, 9], out=view)            # in place through the same strides
    assert np.array_equal(host(xd).transpose(0, 2, 1, 3), ref)


# ------------------------------------------------------ fused projection -----

@pytest.mark.parametrize("b,c,hq,hkv,d,bias", [
    (1, 64, 1, 1, 64, False),        # one chunk: no split of C
    (3, 192, 2, 1, 64, True),
    (5, 768, 12, 12, 64, True),      # GPT-2 / Whisper-style MHA widths
    (70, 128, 2, 1, 64, False),      # more than 64 rows: two launches
    (17, 1024, 8, 2, 128, False),    # C split across workgroups, merged in-launch
    (33, 2048, 4, 4, 192, True),     # three 64-column tiles per head
])
def test_qkv_rope_matches_oracle(nne, cuda, b, c, hq, hkv, d, bias):
    rng = np.random.default_rng(b * 1000 + c)
    x = rnd(rng, b, c)
    wq, wk, wv = weights(rng, hq * d, c), weights(rng, hkv * d, c), weights(rng, hkv * d, c)
    bq, bk, bv = ((rnd(rng, hq * d, scale=0.1), rnd(rng, hkv * d, scale=0.1),
                   rnd(rng, hkv * d, scale=0.1)) if bias else (None, None, None))
    max_len = 512
    pos = rng.integers(0, max_len, b).astype(np.int32)
    rope = nne.RotaryEmbedding(d, max_len, device=cuda)
    packed = nne.qkv_pack(dev(wq, cuda), dev(wk, cuda), dev(wv, cuda), hq, hkv)
    q, k, v = nne.qkv_rope(dev(x, cuda), packed,
                           None if bq is None else dev(bq, cuda),
                           None if bk is None else dev(bk, cuda),
                           None if bv is None else dev(bv, cuda), rope, dev(pos, cuda), pos, hq,
                           hkv)
    rq, rk, rv = T.ref_qkv_rope(x[:, None, :], wq, wk, wv, bq, bk, bv, rope.cos_host,
                                rope.sin_host, pos, hq, hkv)
    T.assert_close(host(q), rq, what="q")
    T.assert_close(host(k), rk, what="k")
    T.assert_close(host(v), rv, what="v")


@pytest.mark.parametrize("seed", range(12))
def test_qkv_rope_random_shapes(nne, cuda, seed):
    """Seeded random prologue shapes: d_model any multiple of 64 up to 3072 (one
    chunk to 48, so C splits into 1 to 8 slices), head dims 64 to 256 (1 to 4
    tiles per head), 1 to 4 KV heads with group sizes 1, 2 and 4, 1 to 100 rows
    (more than 64: two launches), with and without bias."""
    rng = np.random.default_rng(9000 + seed)
    b = int(rng.integers(1, 101))
    c = 64 * int(rng.integers(1, 49))
    d = int(rng.choice([64, 128, 192, 256]))
    hkv = int(rng.integers(1, 5))
    hq = hkv * int(rng.choice([1, 2, 4]))
    bias = bool(rng.random() < 0.5)
    print("case seed=%d b=%d c=%d hq=%d hkv=%d d=%d bias=%d" % (seed, b, c, hq, hkv, d, bias),
          flush=True)
    x = rnd(rng, b, c)
    wq, wk, wv = weights(rng, hq * d, c), weights(rng, hkv * d, c), weights(rng, hkv * d, c)
    bq, bk, bv = ((rnd(rng, hq * d, scale=0.1), rnd(rng, hkv * d, scale=0.1),
                   rnd(rng, hkv * d, scale=0.1)) if bias else (None, None, None))
    max_len = 300
    pos = rng.integers(0, max_len, b).astype(np.int32)
    rope = nne.RotaryEmbedding(d, max_len, device=cuda)
    packed = nne.qkv_pack(dev(wq, cuda), dev(wk, cuda), dev(wv, cuda), hq, hkv)
    q, k, v = nne.qkv_rope(dev(x, cuda), packed,
                           None if bq is None else dev(bq, cuda),
                           None if bk is None else dev(bk, cuda),
                           None if bv is None else dev(bv, cuda), rope, dev(pos, cuda), pos, hq,
                           hkv)
    rq, rk, rv = T.ref_qkv_rope(x[:, None, :], wq, wk, wv, bq, bk, bv, rope.cos_host,
                                rope.sin_host, pos, hq, hkv)
    T.assert_close(host(q), rq, what="q seed %d" % seed)
    T.assert_close(host(k), rk, what="k seed %d" % seed)
    T.assert_close(host(v), rv, what="v seed %d" % seed)


def test_qkv_rope_llama7b_shapes(nne, cuda):
    """Config-3 projection shapes: B = 32, C = 4096, Hq = 32, Hkv = 8, d = 128."""
    rng = np.random.default_rng(3)
    b, c, hq, hkv, d = 32, 4096, 32, 8, 128
    x = rnd(rng, b, c)
    wq, wk, wv = weights(rng, hq * d, c), weights(rng, hkv * d, c), weights(rng, hkv * d, c)
    pos = rng.integers(512, 4096, b).astype(np.int32)
    rope = nne.RotaryEmbedding(d, 4160, device=cuda)
    packed = nne.qkv_pack(dev(wq, cuda), dev(wk, cuda), dev(wv, cuda), hq, hkv)
    q, k, v = nne.qkv_rope(dev(x, cuda), packed, None, None, None, rope, dev(pos, cuda), pos, hq,
                           hkv)
    # the same packed weights serve a second, different batch (x and positions)
    x2 = rnd(rng, b, c)
    pos2 = rng.integers(0, 4096, b).astype(np.int32)
    q2, _, v2 = nne.qkv_rope(dev(x2, cuda), packed, None, None, None, rope, dev(pos2, cuda), pos2,
                             hq, hkv)
    rq2, _, rv2 = T.ref_qkv_rope(x2[:, None, :], wq, wk, wv, None, None, None, rope.cos_host,
                                 rope.sin_host, pos2, hq, hkv)
    T.assert_close(host(q2), rq2, what="q (second batch)")
    T.assert_close(host(v2), rv2, what="v (second batch)")
    rq, rk, rv = T.ref_qkv_rope(x[:, None, :], wq, wk, wv, None, None, None, rope.cos_host,
                                rope.sin_host, pos, hq, hkv)
    T.assert_close(host(q), rq, what="q")
    T.assert_close(host(k), rk, what="k")
    T.assert_close(host(v), rv, what="v")


# --------------------------------------------------- whole attention step ----

def oracle_gqa_step(layer, x, cache_k, cache_v, lens):
    """forward_gqa_cached with t = 1 on the oracle: projections + RoPE, append,
    attend (no mask), output projection."""
    wq, wk, wv, wo = (host(w) for w in (layer.wq, layer.wk, layer.wv, layer.wo))
    q, k, v = T.ref_qkv_rope(x, wq, wk, wv, None, None, None, layer.rope.cos_host,
                             layer.rope.sin_host, lens, layer.num_heads, layer.num_kv_heads)
    out, kc, vc, lens2 = T.ref_decode_step(q, cache_k, cache_v, lens, k, v)
    b = x.shape[0]
    y = T.ref_linear(out.reshape(b, -1), wo).reshape(b, 1, -1)
    return y, kc, vc, lens2


@pytest.mark.parametrize("b,c,hq,hkv,lens", [
    (4, 256, 4, 2, [0, 3, 17, 64]),
    (3, 512, 8, 8, [5, 129, 300]),
    # unpacked projections (d not a multiple of 64), ragged lengths: d = 32,
    # d = 80 on the fused append + attend kernel, d = 30 on the general kernels
    (4, 128, 4, 2, [0, 3, 17, 64]),
    (3, 160, 2, 1, [5, 129, 300]),
    (3, 60, 2, 2, [1, 40, 7]),
])
def test_gqa_decode_step_matches_oracle(nne, cuda, b, c, hq, hkv, lens):
    rng = np.random.default_rng(21 + b)
    layer = nne.GroupedQueryAttention(c, hq, hkv, max_seq_len=512, device=cuda, seed=b)
    d = c // hq
    cap = 400
    lens = np.array(lens, np.int32)
    cache = nne.KVCache(1, b, hkv, cap, d, device=cuda)
    kc = np.zeros((b, hkv, cap, d), np.float32)
    vc = np.zeros_like(kc)
    for i, L in enumerate(lens):
        kc[i, :, :L] = rnd(rng, hkv, L, d)
        vc[i, :, :L] = rnd(rng, hkv, L, d)
    cache.k[0].copy_(dev(kc, cuda))
    cache.v[0].copy_(dev(vc, cuda))
    cache.set_lengths(0, lens)
    x = rnd(rng, b, 1, c)
    y = layer.forward_gqa_cached(dev(x, cuda), lens, cache, 0)
    ry, rkc, rvc, rlens = oracle_gqa_step(layer, x, kc, vc, lens)
    T.assert_close(host(y), ry, what="gqa decode output")
    assert list(cache.lens_host[0]) == list(rlens)
    assert list(host(cache.lens_dev[0])) == list(rlens)
    for i, L in enumerate(lens):        # the appended rows are the projected k, v
        T.assert_close(host(cache.k[0])[i, :, L], rkc[i, :, L], what="k row")
        T.assert_close(host(cache.v[0])[i, :, L], rvc[i, :, L], what="v row")


def test_gqa_prefill_then_decode_equals_full_prefill(nne, cuda):
    """The cached-vs-full pattern of tests/nn/kv_cache_tests.rs:30-103: a
    prefill of T tokens followed by one decode step reproduces the last row
    of a single causal prefill over T + 1 tokens."""
    rng = np.random.default_rng(5)
    b, c, hq, hkv, t = 2, 256, 4, 2, 23
    d = c // hq
    layer = nne.GroupedQueryAttention(c, hq, hkv, max_seq_len=64, device=cuda, seed=9)
    assert layer.w_packed is not None          # the decode step takes the fused path
    x = rnd(rng, b, t + 1, c)
    full = host(layer.forward_gqa_cached(dev(x, cuda), 0))
    cache = nne.KVCache(1, b, hkv, 64, d, device=cuda)
    pre = host(layer.forward_gqa_cached(dev(x[:, :t], cuda), 0, cache, 0))
    step = host(layer.forward_gqa_cached(dev(x[:, t:], cuda), t, cache, 0))
    T.assert_close(pre, full[:, :t], what="prefill rows")
    T.assert_close(step, full[:, t:], what="decode row")
    assert list(cache.lens_host[0]) == [t + 1] * b


def test_gqa_prefill_matches_oracle(nne, cuda):
    """Multi-token step with a non-empty cache: projections, RoPE at
    start_pos, append, the -1e4-masked attention (llama.rs:277-292) and the
    output projection, against the oracle."""
    rng = np.random.default_rng(8)
    b, c, hq, hkv, t, start = 2, 128, 4, 2, 9, 6
    d = c // hq
    layer = nne.GroupedQueryAttention(c, hq, hkv, max_seq_len=32, device=cuda, seed=2)
    cache = nne.KVCache(1, b, hkv, 32, d, device=cuda)
    kc = np.zeros((b, hkv, 32, d), np.float32)
    vc = np.zeros_like(kc)
    kc[:, :, :start] = rnd(rng, b, hkv, start, d)
    vc[:, :, :start] = rnd(rng, b, hkv, start, d)
    cache.k[0].copy_(dev(kc, cuda))
    cache.v[0].copy_(dev(vc, cuda))
    cache.set_lengths(0, [start] * b)
    x = rnd(rng, b, t, c)
    y = host(layer.forward_gqa_cached(dev(x, cuda), start, cache, 0))
    wq, wk, wv, wo = (host(w) for w in (layer.wq, layer.wk, layer.wv, layer.wo))
    q, k, v = T.ref_qkv_rope(x, wq, wk, wv, None, None, None, layer.rope.cos_host,
                             layer.rope.sin_host, np.array([start] * b, np.int32), hq, hkv)
    k_all = np.concatenate([kc[:, :, :start], k], 2)
    v_all = np.concatenate([vc[:, :, :start], v], 2)
    ctx = T.ref_standard(q, k_all, v_all, masked=True, start_pos=start)
    ry = T.ref_linear(ctx.transpose(0, 2, 1, 3).reshape(b * t, c), wo).reshape(b, t, c)
    T.assert_close(y, ry, what="gqa prefill")
