"""Concurrent callers of the C ABI (include/nne_attn.h, "Threads").

Four host threads issue attention calls at once -- each on its own stream,
then all on the shared default stream -- with shapes that make the library
grow a stream's workspace while other threads are using it (the default
stream's workspace is released first, so it starts empty).  The reference's
functions may be called from several threads (Module: Send + Sync,
src/nn/module.rs:7; the Rayon pool of flash_attention.rs:69 is re-entrant).

Every output must equal, bit for bit, the same call made alone on a fresh
stream: the key-split and split-K merges fold their records in a fixed
order.  The lone calls are checked against the oracle (llama.rs:253-296)
at the usual bar, |gpu - ref| <= 1e-4 + 1e-3 |ref|.
"""
import threading

import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu

# (b, hq, hkv, tq, tk, d, causal, q_off): small-problem key split (4 heads
# of 600), few-query split-K with the causal row mask, a cached 9-token GQA
# step (key split, 16 chunks), and a larger key split that needs a bigger
# workspace.
CASES = [
    (1, 4, 4, 600, 600, 64, True, 0),
    (2, 8, 2, 4, 1000, 128, True, 996),
    (1, 12, 3, 9, 1000, 64, True, 991),
    (1, 12, 12, 1024, 1024, 64, True, 0),
]
N_THREADS, N_ITERS = 4, 6


def _inputs(cuda):
    import torch
    out = []
    for i, (b, hq, hkv, tq, tk, d, causal, q_off) in enumerate(CASES):
        rng = np.random.default_rng(3000 + i)
        h = [rng.standard_normal(s).astype(np.float32)
             for s in ((b, hq, tq, d), (b, hkv, tk, d), (b, hkv, tk, d))]
        out.append(([torch.from_numpy(x).to(cuda) for x in h], causal, q_off, h))
    return out


@pytest.mark.parametrize("own_streams", [True, False])
def test_concurrent_callers(nne, cuda, own_streams):
    import torch
    inputs = _inputs(cuda)
    lone = torch.cuda.Stream()
    with torch.cuda.stream(lone):
        refs = [nne.attention_forward(*dev, causal, q_offset=q_off) for dev, causal, q_off, _ in inputs]
    lone.synchronize()
    refs = [r.cpu().numpy() for r in refs]
    nne.release_stream(lone)
    for (_, causal, q_off, (q, k, v)), r in zip(inputs, refs):
        T.assert_close(r, T.ref_standard(q, k, v, causal, start_pos=q_off), what="lone call")

    torch.cuda.synchronize()
    if not own_streams:
        nne.release_stream(torch.cuda.default_stream())
    errors = []

    def worker(tid):
        try:
            stream = torch.cuda.Stream() if own_streams else torch.cuda.default_stream()
            with torch.cuda.stream(stream):
                outs = [torch.empty_like(dev[0]) for dev, _, _, _ in inputs]
                for it in range(N_ITERS):
                    # Rotated order: the threads reach the large case at different times.
                    for j in np.roll(np.arange(len(inputs)), tid + it):
                        dev, causal, q_off, _ = inputs[j]
                        nne.attention_forward(*dev, causal, q_offset=q_off, out=outs[j])
                    stream.synchronize()
                    for j, o in enumerate(outs):
                        if not np.array_equal(o.cpu().numpy(), refs[j]):
                            errors.append("thread %d iteration %d case %d differs" % (tid, it, j))
            if own_streams:
                nne.release_stream(stream)
        except Exception as e:  # reported by the main thread
            errors.append("thread %d: %r" % (tid, e))

    print("case concurrent callers own_streams=%d threads=%d" % (own_streams, N_THREADS), flush=True)
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(N_THREADS)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=90)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors[:5]
