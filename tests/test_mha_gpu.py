"""GPU parity of the MultiHeadAttention paths of GPT-2 and Whisper
(src/nn/attention.rs:9-210; call sites gpt2.rs:141, whisper.rs:169-176) and of
the WhisperKVCache slots (whisper.rs:325-350), built on the same kernels: the
fused projection (without RoPE) feeding the append + attend launch for
self-attention decode steps, the prefill kernel with the bottom-right mask
(q_offset = L - T, attention.rs:101-108) for multi-token steps, and the
few-query kernel for cross-attention over cached memory K/V.

Bar: |gpu - ref| <= 1e-4 + 1e-3 |ref| against the oracle (projections with
bias: oracle_linear; attention: oracle_standard_attention with the reference's
-1e4 mask); cache lengths exact.
"""
import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu


def rnd(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


def dev(x, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def weights(layer):
    return {n: (host(getattr(layer, n)[0]), host(getattr(layer, n)[1]))
            for n in ("q_proj", "k_proj", "v_proj", "out_proj")}


def heads(y, b, t, h, d):
    return np.ascontiguousarray(y.reshape(b, t, h, d).transpose(0, 2, 1, 3))


def oracle_self(w, x, k_cache, v_cache, h, causal):
    """attention.rs:51-129 on the oracle: projections, cat onto the cached
    rows, -1e4 mask with start = L - T (only for T > 1), softmax, PV, out."""
    b, t, c = x.shape
    d = c // h
    x2 = x.reshape(b * t, c)
    q = heads(T.ref_linear(x2, *w["q_proj"]), b, t, h, d)
    k = heads(T.ref_linear(x2, *w["k_proj"]), b, t, h, d)
    v = heads(T.ref_linear(x2, *w["v_proj"]), b, t, h, d)
    k_all = k if k_cache is None else np.concatenate([k_cache, k], 2)
    v_all = v if v_cache is None else np.concatenate([v_cache, v], 2)
    total = k_all.shape[2]
    ctx = T.ref_standard(q, k_all, v_all, masked=causal and t > 1, start_pos=total - t)
    y = T.ref_linear(ctx.transpose(0, 2, 1, 3).reshape(b * t, c), *w["out_proj"])
    return y.reshape(b, t, c), k_all, v_all


@pytest.mark.parametrize("c,h", [(256, 4), (192, 6), (1024, 2)])   # d = 64 (fused decode), 32 (GEMM path), 512 (deep kernel)
def test_mha_self_attention_cached_steps_match_oracle(nne, cuda, c, h):
    rng = np.random.default_rng(c + h)
    b, t0, steps = 3, 9, 4
    d = c // h
    layer = nne.MultiHeadAttention(c, h, True, device=cuda, seed=4)
    assert (layer.w_packed is not None) == (d % 64 == 0)
    w = weights(layer)
    cache = nne.KVCache(1, b, h, 32, d, device=cuda)
    x = rnd(rng, b, t0 + steps, c)
    kc = vc = None
    for s in range(steps + 1):
        lo, hi = (0, t0) if s == 0 else (t0 + s - 1, t0 + s)
        y = layer.forward_attention_cached(dev(x[:, lo:hi], cuda), cache, 0)
        ry, kc, vc = oracle_self(w, x[:, lo:hi], kc, vc, h, True)
        T.assert_close(host(y), ry, what="mha step %d" % s)
    assert list(cache.lens_host[0]) == [t0 + steps] * b
    # the cache holds exactly the projected rows
    T.assert_close(host(cache.k[0])[:, :, :t0 + steps], kc, what="cached K")
    T.assert_close(host(cache.v[0])[:, :, :t0 + steps], vc, what="cached V")


def test_mha_cached_equals_full_sequence(nne, cuda):
    """gpt2_tests.rs:42-86 pattern: token-by-token cached decoding reproduces
    the full causal forward within 1e-4."""
    rng = np.random.default_rng(3)
    b, t, c, h = 2, 12, 128, 2
    layer = nne.MultiHeadAttention(c, h, True, device=cuda, seed=1)
    x = rnd(rng, b, t, c)
    full = host(layer.forward_attention(dev(x, cuda)))
    cache = nne.KVCache(1, b, h, 16, c // h, device=cuda)
    for s in range(t):
        y = host(layer.forward_attention_cached(dev(x[:, s:s + 1], cuda), cache, 0))
        assert np.abs(y[:, 0] - full[:, s]).max() < 1e-4


def test_mha_non_causal_matches_oracle(nne, cuda):
    rng = np.random.default_rng(6)
    b, t, c, h = 2, 37, 128, 2
    layer = nne.MultiHeadAttention(c, h, False, device=cuda, seed=2)
    x = rnd(rng, b, t, c)
    ry, _, _ = oracle_self(weights(layer), x, None, None, h, False)
    T.assert_close(host(layer.forward_attention(dev(x, cuda))), ry, what="mha non-causal")


@pytest.mark.parametrize("tq", [1, 3])
def test_cross_attention_cached_matches_oracle(nne, cuda, tq):
    """forward_cross_attention_cached: the first call projects the memory and
    fills the slot, later calls reuse it (attention.rs:174-191)."""
    rng = np.random.default_rng(20 + tq)
    b, tkv, c, h, layers = 2, 150, 128, 2, 2
    d = c // h
    layer = nne.MultiHeadAttention(c, h, False, device=cuda, seed=7)
    w = weights(layer)
    mem = rnd(rng, b, tkv, c)
    cache = nne.WhisperKVCache(layers, b, h, 16, d, device=cuda)
    k = heads(T.ref_linear(mem.reshape(b * tkv, c), *w["k_proj"]), b, tkv, h, d)
    v = heads(T.ref_linear(mem.reshape(b * tkv, c), *w["v_proj"]), b, tkv, h, d)
    for step in range(3):
        x = rnd(rng, b, tq, c)
        y = layer.forward_cross_attention_cached(dev(x, cuda), dev(mem, cuda), cache.cross_attn, 1)
        q = heads(T.ref_linear(x.reshape(b * tq, c), *w["q_proj"]), b, tq, h, d)
        ctx = T.ref_standard(q, k, v, masked=False)
        ry = T.ref_linear(ctx.transpose(0, 2, 1, 3).reshape(b * tq, c), *w["out_proj"])
        T.assert_close(host(y), ry.reshape(b, tq, c), what="cross step %d" % step)
        assert cache.cross_attn[0] is None and cache.cross_attn[1] is not None
    # uncached call agrees with the cached one
    y2 = layer.forward_cross_attention(dev(x, cuda), dev(mem, cuda))
    T.assert_close(host(y2), host(y), what="uncached cross")
    cache.reset()
    assert cache.cross_attn == [None] * layers and cache.self_attn.current_seq_len(0) == 0


def test_mha_shape_errors_match_reference(nne, cuda):
    layer = nne.MultiHeadAttention(64, 2, True, device=cuda)
    import torch
    with pytest.raises(nne.EngineError, match=r"MultiHeadAttention forward \(expected 3D input"):
        layer.forward_attention(torch.zeros(2, 64, device=cuda))
    with pytest.raises(nne.EngineError, match="batch size and channel dim must match"):
        layer.forward_cross_attention(torch.zeros(2, 3, 64, device=cuda),
                                      torch.zeros(3, 5, 64, device=cuda))
    with pytest.raises(nne.InvalidArgument, match=r"d_model \(30\) must be divisible by "
                                                  r"num_heads \(4\)"):
        nne.MultiHeadAttention(30, 4, True, device=cuda)


@pytest.mark.parametrize("c,h", [(128, 4), (160, 2), (120, 4)])   # d = 32, 80, 30
def test_mha_ragged_decode_step_matches_oracle(nne, cuda, c, h):
    """A single-token step over a cache whose sequences have different
    lengths, with projections that do not take the packed launch: every
    sequence attends to its own rows only (the reference runs such a batch
    as separate B = 1 calls, attention.rs:79-122)."""
    rng = np.random.default_rng(c + 7 * h)
    b, cap = 3, 64
    d = c // h
    lens = np.array([5, 40, 17], np.int32)
    layer = nne.MultiHeadAttention(c, h, True, device=cuda, seed=11)
    assert layer.w_packed is None
    w = weights(layer)
    cache = nne.KVCache(1, b, h, cap, d, device=cuda)
    kc = np.zeros((b, h, cap, d), np.float32)
    vc = np.zeros_like(kc)
    for i, L in enumerate(lens):
        kc[i, :, :L] = rnd(rng, h, L, d)
        vc[i, :, :L] = rnd(rng, h, L, d)
    cache.k[0].copy_(dev(kc, cuda))
    cache.v[0].copy_(dev(vc, cuda))
    cache.set_lengths(0, lens)
    x = rnd(rng, b, 1, c)
    y = host(layer.forward_attention_cached(dev(x, cuda), cache, 0))
    for i, L in enumerate(lens):
        ry, rk, rv = oracle_self(w, x[i:i + 1], kc[i:i + 1, :, :L], vc[i:i + 1, :, :L], h, True)
        T.assert_close(y[i:i + 1], ry, what="ragged mha decode seq %d (d=%d)" % (i, d))
        T.assert_close(host(cache.k[0])[i:i + 1, :, :L + 1], rk, what="cached K seq %d" % i)
    assert list(cache.lens_host[0]) == list(lens + 1)
    assert list(host(cache.lens_dev[0])) == list(lens + 1)


def test_mha_ragged_multi_token_step_is_refused_before_append(nne, cuda):
    layer = nne.MultiHeadAttention(128, 2, True, device=cuda, seed=12)
    cache = nne.KVCache(1, 2, 2, 16, 64, device=cuda)
    cache.set_lengths(0, [3, 5])
    import torch
    with pytest.raises(nne.InvalidArgument, match="equal cached lengths"):
        layer.forward_attention_cached(torch.zeros(2, 2, 128, device=cuda), cache, 0)
    assert list(cache.lens_host[0]) == [3, 5]
