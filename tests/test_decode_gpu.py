"""GPU parity of the KV cache (in-place append) and single-token decode.

Reference semantics: llama.rs:239-296 with t = 1 -- append the new K/V row,
then attend to all L rows of the sequence with no mask; ragged batches are
separate B = 1 problems in the reference.  Bar: |gpu - ref| <= 1e-4 +
1e-3 |ref|; cache contents bit-exact.
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
    return t.cpu().numpy()


def make_cache(nne, cuda, b, hkv, cap, d, lens, rng):
    cache = nne.KVCache(1, b, hkv, cap, d, device=cuda)
    kc = np.zeros((b, hkv, cap, d), np.float32)
    vc = np.zeros((b, hkv, cap, d), np.float32)
    for i, L in enumerate(lens):
        kc[i, :, :L] = rnd(rng, hkv, L, d)
        vc[i, :, :L] = rnd(rng, hkv, L, d)
    cache.k[0].copy_(dev(kc, cuda))
    cache.v[0].copy_(dev(vc, cuda))
    cache.set_lengths(0, lens)
    return cache, kc, vc


def test_decode_golden(nne, cuda):
    g = T.load_golden("decode_ragged_b5g2d16")
    b, hkv, cap, d = g["k_cache"].shape
    cache = nne.KVCache(1, b, hkv, cap, d, device=cuda)
    cache.k[0].copy_(dev(g["k_cache"], cuda))
    cache.v[0].copy_(dev(g["v_cache"], cuda))
    cache.set_lengths(0, g["lens"])
    out = cache.decode_step(0, dev(g["q"], cuda), dev(g["k_new"], cuda), dev(g["v_new"], cuda))
    T.assert_close(host(out), g["out"], what="decode golden")
    assert list(cache.lens_host[0]) == list(g["lens"] + 1)
    assert list(host(cache.lens_dev[0])) == list(g["lens"] + 1)


def test_append_is_bit_exact_and_capacity_checked(nne, cuda):
    rng = np.random.default_rng(1)
    b, hkv, cap, d = 3, 2, 12, 16
    lens = np.array([0, 5, 9], np.int32)
    cache, kc, vc = make_cache(nne, cuda, b, hkv, cap, d, lens, rng)
    kn, vn = rnd(rng, b, hkv, 3, d), rnd(rng, b, hkv, 3, d)
    k_all, v_all = cache.update(0, dev(kn, cuda), dev(vn, cuda))
    rc, kc2, vc2, lens2 = T.ref_kv_append(kc, vc, lens, kn, vn)
    assert rc == 0
    assert np.array_equal(host(cache.k[0]), kc2) and np.array_equal(host(cache.v[0]), vc2)
    assert list(host(cache.lens_dev[0])) == list(lens2)
    assert tuple(k_all.shape) == (b, hkv, 12, d)
    with pytest.raises(nne.CapacityError):
        cache.update(0, dev(kn[:, :, :1], cuda), dev(vn[:, :, :1], cuda))   # 12 + 1 > 12
    assert list(cache.lens_host[0]) == list(lens2)
    # strided new rows ([B, T, H, d] projection layout)
    cache2, kc, vc = make_cache(nne, cuda, b, hkv, cap, d, np.array([1, 2, 3], np.int32), rng)
    kt, vt = rnd(rng, b, 2, hkv, d), rnd(rng, b, 2, hkv, d)
    cache2.update(0, dev(kt, cuda).transpose(1, 2), dev(vt, cuda).transpose(1, 2))
    _, kc3, vc3, _ = T.ref_kv_append(kc, vc, np.array([1, 2, 3], np.int32),
                                     kt.transpose(0, 2, 1, 3), vt.transpose(0, 2, 1, 3))
    assert np.array_equal(host(cache2.k[0]), kc3) and np.array_equal(host(cache2.v[0]), vc3)


@pytest.mark.parametrize("g,d", [(4, 128), (1, 64), (8, 64), (16, 32), (2, 16), (3, 96),
                                 (1, 128), (4, 64), (2, 128)])
def test_decode_ragged_group_sizes(nne, cuda, g, d):
    print("case g=%d d=%d" % (g, d), flush=True)
    rng = np.random.default_rng(100 + g + d)
    b, hkv, cap = 6, 2, 1200
    lens = np.array([1, 63, 64, 65, 700, 1100], np.int32)
    cache, kc, vc = make_cache(nne, cuda, b, hkv, cap, d, lens, rng)
    q = rnd(rng, b, hkv * g, 1, d)
    out = host(cache.attend(0, dev(q, cuda)))
    T.assert_close(out, T.ref_decode_attend(q, kc, vc, lens), what="decode g=%d d=%d" % (g, d))


def test_decode_zero_length_sequence_gives_zero(nne, cuda):
    rng = np.random.default_rng(7)
    lens = np.array([0, 3000], np.int32)
    cache, kc, vc = make_cache(nne, cuda, 2, 1, 4096, 64, lens, rng)
    q = rnd(rng, 2, 4, 1, 64)
    out = host(cache.attend(0, dev(q, cuda)))
    assert not out[0].any()
    T.assert_close(out[1:], T.ref_decode_attend(q, kc, vc, lens)[1:], what="len 3000")


def test_config3_multi_step_decode(nne, cuda):
    """Config 3 geometry (Hq=32, Hkv=8, d=128, ragged L in [512, 4096]) at
    B=4 over 6 steps; every step checked against the oracle's append+attend."""
    rng = np.random.default_rng(0x5EED0003)
    b, hq, hkv, d, steps = 4, 32, 8, 128, 6
    lens = rng.integers(512, 4097, size=b).astype(np.int32)
    cap = int(lens.max()) + steps
    cache, kc, vc = make_cache(nne, cuda, b, hkv, cap, d, lens, rng)
    for s in range(steps):
        q, kn, vn = rnd(rng, b, hq, 1, d), rnd(rng, b, hkv, 1, d), rnd(rng, b, hkv, 1, d)
        out = host(cache.decode_step(0, dev(q, cuda), dev(kn, cuda), dev(vn, cuda)))
        ref, kc, vc, lens = T.ref_decode_step(q, kc, vc, lens, kn, vn)
        T.assert_close(out, ref, what="config3 step %d" % s)
        assert list(host(cache.lens_dev[0])) == list(lens)
    assert list(cache.lens_host[0]) == list(lens)
    assert np.array_equal(host(cache.k[0]), kc) and np.array_equal(host(cache.v[0]), vc)


def test_config3_full_batch_one_step(nne, cuda):
    """Full config 3 batch: B=32 sequences, Hq=32, Hkv=8, d=128, L ~ U[512, 4096]."""
    rng = np.random.default_rng(0x5EED0033)
    b, hq, hkv, d = 32, 32, 8, 128
    lens = rng.integers(512, 4097, size=b).astype(np.int32)
    cap = 4096 + 64
    cache, kc, vc = make_cache(nne, cuda, b, hkv, cap, d, lens, rng)
    q, kn, vn = rnd(rng, b, hq, 1, d), rnd(rng, b, hkv, 1, d), rnd(rng, b, hkv, 1, d)
    out = host(cache.decode_step(0, dev(q, cuda), dev(kn, cuda), dev(vn, cuda)))
    ref, *_ = T.ref_decode_step(q, kc, vc, lens, kn, vn)
    T.assert_close(out, ref, what="config3 full batch")


def oracle_step_in_place(q, kc, vc, lens, kn, vn):
    """The oracle's append + attend, updating kc, vc and lens in place (no
    copies of the 545 MB caches per step)."""
    b, hq, _, d = q.shape
    hkv, cap = kc.shape[1], kc.shape[2]
    out = np.zeros((b, hq, 1, d), np.float32)
    rc = T.oracle().oracle_decode_step(T._p(q), T._p(kc), T._p(vc), lens.ctypes.data_as(T._i32),
                                       T._p(kn), T._p(vn), T._p(out), b, hq, hkv, cap, d, 0, 0.0,
                                       T._threads())
    assert rc == 0
    return out


@pytest.mark.parametrize("hq", [32, 64])
def test_bench_decode_sequence_against_oracle(nne, cuda, hq):
    """The exact sequence bench.py times for config 3 (Hq = 32) and the G = 8
    line (Hq = 64): B = 32, Hkv = 8, d = 128, L0 ~ U[512, 4096], 64 append +
    attend steps queued back to back with no host synchronisation between
    them, on the bench's own seeded inputs.  Every step's output against the
    oracle; the cache and lengths bit-exact after the last step.  The cut
    chunks are re-planned every step as the lengths grow."""
    import torch
    seed = 0x5EED0003 if hq == 32 else 0x5EED0016
    print("case bench decode sequence hq=%d" % hq, flush=True)
    b, hkv, d, steps, warmup = 32, 8, 128, 64, 4
    rng = np.random.default_rng(seed)
    lens0 = rng.integers(512, 4097, size=b).astype(np.int32)
    cap = 4096 + steps + warmup
    cache = nne.KVCache(1, b, hkv, cap, d, device=cuda)
    g = torch.Generator(device=cuda).manual_seed(seed)
    cache.k[0].normal_(generator=g)
    cache.v[0].normal_(generator=g)
    qs = torch.randn(steps, b, hq, 1, d, generator=g, device=cuda)
    kn = torch.randn(steps, b, hkv, 1, d, generator=g, device=cuda)
    vn = torch.randn(steps, b, hkv, 1, d, generator=g, device=cuda)
    kc, vc = host(cache.k[0]), host(cache.v[0])
    cache.set_lengths(0, lens0)
    outs = torch.empty(steps, b, hq, 1, d, device=cuda)
    for i in range(steps):
        cache.decode_step(0, qs[i], kn[i], vn[i], out=outs[i])
    got = host(outs)
    qs_h, kn_h, vn_h = host(qs), host(kn), host(vn)
    lens = lens0.copy()
    for i in range(steps):
        ref = oracle_step_in_place(qs_h[i], kc, vc, lens, kn_h[i], vn_h[i])
        T.assert_close(got[i], ref, what="bench decode hq=%d step %d" % (hq, i))
    assert (lens == lens0 + steps).all()
    assert list(cache.lens_host[0]) == list(lens)
    assert list(host(cache.lens_dev[0])) == list(lens)
    assert np.array_equal(host(cache.k[0]), kc) and np.array_equal(host(cache.v[0]), vc)


def test_decode_matches_last_row_of_gpu_prefill(nne, cuda):
    """Cached decode == the corresponding row of the causal prefill kernel
    (kv_cache_tests.rs:68-103 pattern), across the two GPU kernels."""
    rng = np.random.default_rng(9)
    b, hq, hkv, t, d = 2, 8, 2, 300, 64
    q, k, v = rnd(rng, b, hq, t, d), rnd(rng, b, hkv, t, d), rnd(rng, b, hkv, t, d)
    full = host(nne.attention_forward(dev(q, cuda), dev(k, cuda), dev(v, cuda), True))
    cache = nne.KVCache(1, b, hkv, t, d, device=cuda)
    cache.update(0, dev(k[:, :, :t - 1], cuda), dev(v[:, :, :t - 1], cuda))
    out = host(cache.decode_step(0, dev(q[:, :, t - 1:], cuda), dev(k[:, :, t - 1:], cuda),
                                 dev(v[:, :, t - 1:], cuda)))
    T.assert_close(out[:, :, 0], full[:, :, t - 1], what="decode vs prefill row")


def test_workspace_argument_paths(nne, cuda):
    """Library workspace (NULL), a caller workspace (records + zeroed
    counters), and undersized caller workspaces, which are refused."""
    import ctypes
    import torch
    rng = np.random.default_rng(11)
    b, hq, hkv, d, cap = 2, 8, 2, 64, 5000
    lens = np.array([4000, 4990], np.int32)
    cache, kc, vc = make_cache(nne, cuda, b, hkv, cap, d, lens, rng)
    q = dev(rnd(rng, b, hq, 1, d), cuda)
    ref = T.ref_decode_attend(host(q), kc, vc, lens)
    lib = nne.lib()
    i32p = ctypes.POINTER(ctypes.c_int32)
    size = nne.NneWorkspaceSize()
    assert lib.nne_decode_workspace_size(b, hq, hkv, d, ctypes.byref(size)) == nne.NNE_OK
    caller = nne.Workspace(cuda).reserve(size)
    buf = torch.zeros(16, dtype=torch.int32, device=cuda)
    short_records = nne.NneWorkspace(buf.data_ptr(), 16, buf.data_ptr(), 16)
    short_counters = nne.NneWorkspace(caller.records.data_ptr(), caller.records.numel(),
                                      buf.data_ptr(), 1)
    outs = {}
    for name, ws in (("library", None), ("caller", caller.struct()[0]),
                     ("short records", ctypes.byref(short_records)),
                     ("short counters", ctypes.byref(short_counters))):
        print("case workspace", name, flush=True)
        out = torch.empty_like(q)
        rc = lib.nne_decode_attention(q.data_ptr(), None, cache.k[0].data_ptr(),
                                      cache.v[0].data_ptr(), cache.lens_dev[0].data_ptr(),
                                      cache.lens_host[0].ctypes.data_as(i32p), out.data_ptr(),
                                      None, b, hq, hkv, cap, d, 0, 0.0, ws, nne._stream())
        if name.startswith("short"):
            assert rc == nne.NNE_EINVAL
        else:
            assert rc == 0
            outs[name] = host(out)
            T.assert_close(outs[name], ref, what=name + " workspace")
    assert np.array_equal(outs["library"], outs["caller"])


def test_split_head_handoff_alternating_inputs(nne, cuda):
    """Heads split across workgroups are merged inside the launch by the last
    workgroup to arrive.  Back-to-back calls on one stream alternate between
    two unrelated caches and queries with the same geometry, with no host
    synchronisation between them, so a merge that read another call's partial
    records would not match its own reference."""
    import torch
    rng = np.random.default_rng(21)
    b, hq, hkv, d = 3, 16, 4, 128
    lens = np.array([9000, 17, 6000], np.int32)
    cap = 9100
    caches = [make_cache(nne, cuda, b, hkv, cap, d, lens, rng) for _ in range(2)]
    qs = [rnd(rng, b, hq, 1, d) for _ in range(2)]
    refs = [T.ref_decode_attend(qs[i], caches[i][1], caches[i][2], lens) for i in range(2)]
    qd = [dev(q, cuda) for q in qs]
    outs = [torch.empty(b, hq, 1, d, device=cuda) for _ in range(12)]
    for j, o in enumerate(outs):
        caches[j % 2][0].attend(0, qd[j % 2], out=o)
    for j, o in enumerate(outs):
        T.assert_close(host(o), refs[j % 2], what="alternating call %d" % j)


def test_few_query_handoff_alternating_inputs(nne, cuda):
    """The same check for few-query cross-attention (prefill entry point)."""
    import torch
    rng = np.random.default_rng(22)
    q = [rnd(rng, 2, 8, 2, 64) for _ in range(2)]
    k = [rnd(rng, 2, 4, 7000, 64) for _ in range(2)]
    v = [rnd(rng, 2, 4, 7000, 64) for _ in range(2)]
    refs = [T.ref_standard(q[i], k[i], v[i], False) for i in range(2)]
    qd, kd, vd = ([dev(x, cuda) for x in xs] for xs in (q, k, v))
    outs = [torch.empty(2, 8, 2, 64, device=cuda) for _ in range(10)]
    for j, o in enumerate(outs):
        nne.attention_forward(qd[j % 2], kd[j % 2], vd[j % 2], False, out=o)
    for j, o in enumerate(outs):
        T.assert_close(host(o), refs[j % 2], what="alternating cross call %d" % j)


def test_large_batch_uses_combine_kernel(nne, cuda):
    """More than 128 sequences: the prefix is scanned on the GPU and a second
    kernel merges the split heads; includes empty sequences and a decode step."""
    rng = np.random.default_rng(23)
    b, hq, hkv, d = 150, 8, 2, 64
    lens = rng.integers(0, 700, size=b).astype(np.int32)
    lens[[3, 77]] = 0
    lens[10] = 3000
    cap = 3100
    cache, kc, vc = make_cache(nne, cuda, b, hkv, cap, d, lens, rng)
    q = rnd(rng, b, hq, 1, d)
    out = host(cache.attend(0, dev(q, cuda)))
    T.assert_close(out, T.ref_decode_attend(q, kc, vc, lens), what="B=150 attend")
    kn, vn = rnd(rng, b, hkv, 1, d), rnd(rng, b, hkv, 1, d)
    out = host(cache.decode_step(0, dev(q, cuda), dev(kn, cuda), dev(vn, cuda)))
    ref, kc, vc, lens = T.ref_decode_step(q, kc, vc, lens, kn, vn)
    T.assert_close(out, ref, what="B=150 step")
    assert list(host(cache.lens_dev[0])) == list(lens)


def test_kv_cache_layers_slot_view(nne, cuda):
    """KVCache.layers (kv_cache.rs:13) with the models' idioms: engage every
    slot with empty tensors (llama.rs:501-503), fill through the cache, read
    the slot back as [B, Hkv, L, d] views, assign Some((k, v)), None, reset."""
    import torch
    rng = np.random.default_rng(41)
    b, hkv, cap, d = 2, 2, 32, 16
    cache = nne.KVCache(2, b, hkv, cap, d, device=cuda)
    assert len(cache.layers) == 2 and list(cache.layers) == [None, None]
    for i in range(len(cache.layers)):
        cache.layers[i] = (torch.zeros(0, device=cuda), torch.zeros(0, device=cuda))
    assert all(kv is not None and kv[0].shape[2] == 0 for kv in cache.layers)
    k1, v1 = rnd(rng, b, hkv, 5, d), rnd(rng, b, hkv, 5, d)
    cache.update(1, dev(k1, cuda), dev(v1, cuda))
    k_view, v_view = cache.layers[1]
    assert k_view.shape == (b, hkv, 5, d) and k_view.data_ptr() == cache.k[1].data_ptr()
    assert np.array_equal(host(k_view), k1) and np.array_equal(host(v_view), v1)
    cache.layers[0] = (dev(k1, cuda), dev(v1, cuda))            # *slot = Some((k, v))
    assert cache.current_seq_len(0) == 5 and np.array_equal(host(cache.layers[0][0]), k1)
    q = rnd(rng, b, 4, 1, d)
    out = host(cache.attend(0, dev(q, cuda)))
    T.assert_close(out, T.ref_decode_attend(q, np.pad(k1, ((0, 0), (0, 0), (0, cap - 5), (0, 0))),
                                            np.pad(v1, ((0, 0), (0, 0), (0, cap - 5), (0, 0))),
                                            [5, 5]), what="attend after slot assignment")
    with pytest.raises(nne.ShapeMismatch):
        cache.layers[0] = (dev(k1[:, :1], cuda), dev(v1[:, :1], cuda))
    assert cache.current_seq_len(0) == 5                       # refused, slot unchanged
    cache.layers[1] = None
    assert cache.layers[1] is None and cache.current_seq_len(1) == 0
    cache.reset()
    assert list(cache.layers) == [None, None]
    with pytest.raises(IndexError):
        cache.layers[2]
