"""Seeded random sweep over the attention entry points on the GPU.

Each case draws a shape, a layout and a mask at random (numpy's generator,
the case number is the seed), so the sweep crosses the dispatch boundaries
of the library: the few-query kernel (causal or not), the key split of small
prefill problems, the persistent schedule, the 16-byte and the scalar load
paths, ragged decode batches with and without the append.  References: the
oracle's masked standard attention (llama.rs:253-296 with the -1e4 mask,
rows without a visible key compared as zero, which is what the flash
algorithm gives them, flash_attention.rs:186-194) and its decode step.

Bar: |gpu - ref| <= 1e-4 + 1e-3 |ref|; cache contents and lengths exact.
"""
import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu

HEAD_DIMS = [8, 16, 20, 32, 48, 64, 80, 96, 100, 128]


def draw_attention_case(seed):
    rng = np.random.default_rng(1000 + seed)
    b = int(rng.integers(1, 4))
    hkv = int(rng.integers(1, 5))
    g = int(rng.choice([1, 1, 2, 3, 4, 8]))
    kind = rng.integers(0, 3)                 # 0: few rows, 1: small, 2: medium
    tq = int(rng.integers(1, 5) if kind == 0 else rng.integers(5, 130) if kind == 1
             else rng.integers(130, 700))
    tk = int(rng.integers(1, 1500)) if rng.random() < 0.7 else tq
    if kind == 2:                             # keep the oracle's work to a few GFLOP
        b, hkv, g = 1, min(hkv, 2), min(g, 4)
    d = int(rng.choice(HEAD_DIMS))
    causal = bool(rng.random() < 0.6)
    q_off = 0
    if causal:
        q_off = int(rng.choice([0, tk - tq, int(rng.integers(-20, max(1, tk)))]))
    layout = int(rng.integers(0, 3))          # 0 contiguous, 1 [B,T,H,d] views, 2 dim stride 2
    return b, hkv, g, tq, tk, d, causal, q_off, layout


def view(x, layout, cuda):
    """Device tensor holding x [B, H, T, d] in the drawn layout."""
    import torch
    if layout == 0:
        return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    if layout == 1:
        return torch.from_numpy(np.ascontiguousarray(x.transpose(0, 2, 1, 3))).to(cuda).transpose(1, 2)
    wide = np.zeros(x.shape[:3] + (2 * x.shape[3],), np.float32)
    wide[..., ::2] = x
    return torch.from_numpy(wide).to(cuda)[..., ::2]


@pytest.mark.parametrize("seed", range(64))
def test_random_attention_forward(nne, cuda, seed):
    import torch
    b, hkv, g, tq, tk, d, causal, q_off, layout = draw_attention_case(seed)
    print("case seed=%d b=%d hkv=%d g=%d tq=%d tk=%d d=%d causal=%d q_off=%d layout=%d"
          % (seed, b, hkv, g, tq, tk, d, causal, q_off, layout), flush=True)
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((b, hkv * g, tq, d)).astype(np.float32)
    k = rng.standard_normal((b, hkv, tk, d)).astype(np.float32)
    v = rng.standard_normal((b, hkv, tk, d)).astype(np.float32)
    out = torch.full((b, hkv * g, tq, d), float("nan"), device=cuda)
    nne.attention_forward(view(q, layout, cuda), view(k, layout, cuda), view(v, layout, cuda),
                          causal, q_offset=q_off, out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    r0 = min(tq, max(0, -q_off)) if causal else 0      # rows that see no key
    assert not got[:, :, :r0].any()
    if r0 < tq:
        ref = T.ref_standard(q[:, :, r0:], k, v, causal, start_pos=q_off + r0)
        T.assert_close(got[:, :, r0:], ref, what="seed %d" % seed)


@pytest.mark.parametrize("seed", range(24))
def test_random_decode_steps(nne, cuda, seed):
    import torch
    rng = np.random.default_rng(2000 + seed)
    b = int(rng.integers(1, 40))
    hkv = int(rng.integers(1, 9))
    g = int(rng.choice([1, 2, 4, 5, 8]))
    d = int(rng.choice([16, 32, 64, 96, 128]))
    lens = rng.integers(0, 900, size=b).astype(np.int32)
    cap = int(lens.max()) + 4
    steps = int(rng.integers(1, 4))
    append = bool(rng.random() < 0.7)
    print("case seed=%d b=%d hkv=%d g=%d d=%d steps=%d append=%d max_len=%d"
          % (seed, b, hkv, g, d, steps, append, lens.max()), flush=True)
    cache = nne.KVCache(1, b, hkv, cap, d, device=cuda)
    kc = np.zeros((b, hkv, cap, d), np.float32)
    vc = np.zeros((b, hkv, cap, d), np.float32)
    for i, L in enumerate(lens):
        kc[i, :, :L] = rng.standard_normal((hkv, L, d))
        vc[i, :, :L] = rng.standard_normal((hkv, L, d))
    cache.k[0].copy_(torch.from_numpy(kc).to(cuda))
    cache.v[0].copy_(torch.from_numpy(vc).to(cuda))
    cache.set_lengths(0, lens)
    for s in range(steps):
        q = rng.standard_normal((b, hkv * g, 1, d)).astype(np.float32)
        if append:
            kn = rng.standard_normal((b, hkv, 1, d)).astype(np.float32)
            vn = rng.standard_normal((b, hkv, 1, d)).astype(np.float32)
            out = cache.decode_step(0, torch.from_numpy(q).to(cuda), torch.from_numpy(kn).to(cuda),
                                    torch.from_numpy(vn).to(cuda))
            ref, kc, vc, lens = T.ref_decode_step(q, kc, vc, lens, kn, vn)
        else:
            out = cache.attend(0, torch.from_numpy(q).to(cuda))
            ref = T.ref_decode_attend(q, kc, vc, lens)
        torch.cuda.synchronize()
        T.assert_close(out.cpu().numpy(), ref, what="seed %d step %d" % (seed, s))
    assert list(cache.lens_host[0]) == list(lens)
    assert list(cache.lens_dev[0].cpu().numpy()) == list(lens)
    assert np.array_equal(cache.k[0].cpu().numpy(), kc)
    assert np.array_equal(cache.v[0].cpu().numpy(), vc)


def draw_wide_decode_case(seed):
    """Wider ragged decode batches than test_random_decode_steps: up to 160
    sequences (past 128 the flattened prefix is not in the kernel arguments
    and the launch cuts equal chunks), lengths up to 5000, batches of short
    heads with empty ones, or one long head among short ones; the split-K
    layout is whichever the launch chooses (whole heads, cut chunks, equal
    chunks).  Dense cache arrays stay under 600 MB."""
    rng = np.random.default_rng(5000 + seed)
    b = int(rng.integers(1, 161))
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 8]))
    d = int(rng.choice([64, 128]))
    kind = int(rng.integers(0, 3))
    if kind == 0:
        lens = rng.integers(0, 5000, size=b)
    elif kind == 1:
        lens = np.where(rng.random(b) < 0.1, 0, rng.integers(1, 300, size=b))
    else:
        lens = rng.integers(1, 400, size=b)
        lens[int(rng.integers(0, b))] = int(rng.integers(8000, 20000))
    lens = lens.astype(np.int32)
    while b > 1 and b * hkv * (int(lens.max()) + 2) * d > 1.5e8:
        b = max(1, b // 2)
        lens = lens[:b].copy()
        if kind == 2 and lens.max() < 8000:
            lens[0] = 8000
    append = bool(rng.random() < 0.7)
    return b, hkv, g, d, lens, append


@pytest.mark.parametrize("seed", range(12))
def test_random_wide_decode(nne, cuda, seed):
    b, hkv, g, d, lens, append = draw_wide_decode_case(seed)
    print("case seed=%d b=%d hkv=%d g=%d d=%d max_len=%d keys=%d append=%d"
          % (seed, b, hkv, g, d, lens.max(), lens.sum(), append), flush=True)
    T.decode_vs_oracle(nne, cuda, b, hkv * g, hkv, d, lens, append, 7000 + seed, "wide seed %d" % seed)
