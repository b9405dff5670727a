"""Every entry point driven with caller-owned buffers, on a stream of its own:
the library must hold no device memory for that stream afterwards
(nne_stream_resource_bytes == 0), and the results must equal those of the
same calls on the library's per-stream workspace (same kernels, same split,
so bit for bit), and the oracle.

The reference's caller owns all state (src/nn/kv_cache.rs:11-14; inputs
borrowed, outputs owned by the caller); here that extends to the scratch of
the split computations: records plus arrival counters zeroed once.
"""
import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu


def rnd(seed, *shape):
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)


def test_every_entry_point_on_caller_buffers_allocates_nothing(nne, cuda):
    import torch
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    s = torch.cuda.Stream(device=cuda)
    ws = nne.Workspace(cuda)
    got, ref = {}, {}

    # prefill: key split, persistent (no workspace), few-query cross
    q1, k1, v1 = (dev(rnd(900 + i, 1, 4, 600, 64)) for i in range(3))
    q2, k2, v2 = dev(rnd(903, 2, 8, 300, 64)), dev(rnd(904, 2, 4, 300, 64)), dev(rnd(905, 2, 4, 300, 64))
    qx, kx, vx = dev(rnd(906, 2, 6, 8, 64)), dev(rnd(907, 2, 6, 500, 64)), dev(rnd(908, 2, 6, 500, 64))
    # decode prologue + step over a ragged cache
    b, hq, hkv, d, c, cap = 4, 8, 2, 64, 512, 300
    lens = np.array([7, 150, 31, 260], np.int32)
    layer = nne.GroupedQueryAttention(c, hq, hkv, max_seq_len=cap, device=cuda, seed=31)
    assert layer.w_packed is not None
    kc, vc = rnd(909, b, hkv, cap, d), rnd(910, b, hkv, cap, d)
    x = dev(rnd(911, b, c))
    torch.cuda.synchronize()

    def run(stream, workspace, tag):
        with torch.cuda.stream(stream):
            out = {}
            out["flash"] = nne.flash_attention_forward(q1, k1, v1, True, stream=stream,
                                                       workspace=workspace)
            out["gqa"] = nne.attention_forward(q2, k2, v2, True, stream=stream,
                                               workspace=workspace)
            out["cross"] = nne.attention_forward(qx, kx, vx, False, stream=stream,
                                                 workspace=workspace)
            # the library leg's cache passes no workspace, so its decode
            # calls run on the library's per-stream records and counters
            cache = nne.KVCache(1, b, hkv, cap, d, device=cuda,
                                own_workspace=workspace is not None)
            cache.k[0].copy_(dev(kc))
            cache.v[0].copy_(dev(vc))
            cache.set_lengths(0, lens)
            lens_dev = cache.lens_dev[0]
            q, kn, vn = nne.qkv_rope(x, layer.w_packed, None, None, None, layer.rope, lens_dev,
                                     lens, hq, hkv, stream=stream, workspace=workspace)
            out["q"] = q
            out["attend"] = cache.attend(0, q, stream=stream)
            out["step"] = cache.decode_step(0, q, kn, vn, stream=stream)
            out["cache_k"] = cache.k[0]
            out["lens"] = cache.lens_dev[0]
        stream.synchronize()
        return {k: v.cpu().numpy() for k, v in out.items()}

    print("case caller buffers on a fresh stream", flush=True)
    got = run(s, ws, "caller")
    assert nne.stream_resource_bytes(s) == 0
    print("case the same calls on the library's workspace", flush=True)
    lib_stream = torch.cuda.Stream(device=cuda)
    ref = run(lib_stream, None, "library")
    assert nne.stream_resource_bytes(lib_stream) > 0
    nne.release_stream(lib_stream)
    for key in got:
        assert np.array_equal(got[key], ref[key]), key
    # and against the oracle
    qn = lambda t: t.cpu().numpy()
    T.assert_close(got["flash"], T.ref_flash(qn(q1), qn(k1), qn(v1), True), what="flash")
    T.assert_close(got["gqa"], T.ref_standard(qn(q2), qn(k2), qn(v2), True), what="gqa")
    T.assert_close(got["cross"], T.ref_standard(qn(qx), qn(kx), qn(vx), False), what="cross")
    T.assert_close(got["attend"], T.ref_decode_attend(got["q"], kc, vc, lens), what="attend")
    assert np.array_equal(got["lens"], lens + 1)
    nne.release_stream(s)
    assert nne.stream_resource_bytes(s) == 0


def test_library_workspace_is_reported_and_released(nne, cuda):
    """Without a caller workspace the library holds memory for the stream
    until nne_stream_release."""
    import torch
    s = torch.cuda.Stream(device=cuda)
    q, k, v = (torch.randn(1, 4, 600, 64, device=cuda) for _ in range(3))   # key split
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        nne.flash_attention_forward(q, k, v, True, stream=s)
    s.synchronize()
    assert nne.stream_resource_bytes(s) > 0
    nne.release_stream(s)
    assert nne.stream_resource_bytes(s) == 0
