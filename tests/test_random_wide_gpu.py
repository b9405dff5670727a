"""Seeded random sweep over head dims above 128 on the GPU.

Each case draws a head dim in (128, 1028], a shape, a layout and a mask at
random (numpy's generator, the case number is the seed), so the sweep crosses
the routing of wide head dims: the wave-pair prefill kernel (d = 256 with the
device full), the deep kernel's 2-wave form (other dims up to 256), its
8-wave form and key split (few units), its 4-wave form (d <= 512 with more
workgroups than CUs), its 1024-dim output chunks (d > 512) and, for decode
steps, its ragged split.  One case in four is a large problem compared on
sampled heads and rows.  References: the oracle's masked standard attention
(llama.rs:253-296, rows without a visible key compared as zero) and its
decode step.

Bar: |gpu - ref| <= 1e-4 + 1e-3 |ref|; cache contents and lengths exact.
"""
import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu

WIDE_DIMS = [132, 160, 192, 228, 256, 260, 320, 384, 448, 512, 640, 768, 1024, 1028]


def draw_case(seed):
    rng = np.random.default_rng(7000 + seed)
    d = int(rng.choice(WIDE_DIMS))
    large = seed % 4 == 3
    if large:                                  # enough units for the 4-wave and 2-wave forms
        b = 1
        hkv = int(rng.choice([8, 16]))
        g = int(rng.choice([1, 2]))
        tq = int(rng.integers(900, 1400))
        tk = tq if rng.random() < 0.7 else int(rng.integers(600, 1600))
    else:
        b = int(rng.integers(1, 4))
        hkv = int(rng.integers(1, 5))
        g = int(rng.choice([1, 2, 4, 8]))
        tq = int(rng.integers(1, 300))
        tk = int(rng.integers(1, 600))
        while b * hkv * g * tq * tk * d > 1.5e9:   # keep the oracle's work to a few GFLOP
            tq = max(1, tq // 2)
            tk = max(1, tk // 2)
    causal = bool(rng.random() < 0.6)
    q_off = 0
    if causal:
        q_off = int(rng.choice([0, tk - tq, int(rng.integers(-20, max(1, tk)))]))
    layout = int(rng.integers(0, 2))           # 0 contiguous, 1 [B, T, H, d] views
    return b, hkv, g, tq, tk, d, causal, q_off, layout, large


def dev_view(x, layout, cuda):
    import torch
    if layout == 0:
        return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    return torch.from_numpy(np.ascontiguousarray(x.transpose(0, 2, 1, 3))).to(cuda).transpose(1, 2)


@pytest.mark.parametrize("seed", range(32))
def test_random_wide_attention_forward(nne, cuda, seed):
    import torch
    b, hkv, g, tq, tk, d, causal, q_off, layout, large = draw_case(seed)
    print("case seed=%d b=%d hkv=%d g=%d tq=%d tk=%d d=%d causal=%d q_off=%d layout=%d large=%d"
          % (seed, b, hkv, g, tq, tk, d, causal, q_off, layout, large), flush=True)
    rng = np.random.default_rng(seed)
    hq = hkv * g
    q = rng.standard_normal((b, hq, tq, d)).astype(np.float32)
    k = rng.standard_normal((b, hkv, tk, d)).astype(np.float32)
    v = rng.standard_normal((b, hkv, tk, d)).astype(np.float32)
    out = torch.full((b, hq, tq, d), float("nan"), device=cuda)
    nne.attention_forward(dev_view(q, layout, cuda), dev_view(k, layout, cuda),
                          dev_view(v, layout, cuda), causal, q_offset=q_off, out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    r0 = min(tq, max(0, -q_off)) if causal else 0      # rows that see no key
    assert not got[:, :, :r0].any()
    if r0 == tq:
        return
    if not large:
        ref = T.ref_standard(q[:, :, r0:], k, v, causal, start_pos=q_off + r0)
        T.assert_close(got[:, :, r0:], ref, what="seed %d" % seed)
        return
    assert np.isfinite(got).all()
    for h in sorted({0, hq // 2, hq - 1}):
        for s0 in sorted({r0, (r0 + tq) // 2, max(r0, tq - 48)}):
            rows = slice(s0, min(tq, s0 + 48))
            kv = h // g
            ref = T.ref_standard(q[:, h:h + 1, rows], k[:, kv:kv + 1], v[:, kv:kv + 1], causal,
                                 start_pos=q_off + s0)
            T.assert_close(got[:, h:h + 1, rows], ref, what="seed %d head %d rows %d" % (seed, h, s0))


@pytest.mark.parametrize("seed", range(16))
def test_random_wide_decode_steps(nne, cuda, seed):
    """Decode steps above 256 dims through the cache: unsplit, equal-part and
    ragged key splits, and batches with more (sequence, KV head) pairs than
    CUs."""
    import torch
    rng = np.random.default_rng(8000 + seed)
    d = int(rng.choice([260, 320, 384, 512, 640, 1028]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    g = int(rng.choice([1, 2, 4, 8]))
    b = int(rng.integers(1, 81))
    lens = rng.integers(0, 3000, size=b).astype(np.int32)
    if rng.random() < 0.3:
        lens[int(rng.integers(0, b))] = int(rng.integers(3000, 6000))
    cap = int(lens.max()) + 4
    while b > 1 and b * hkv * cap * d > 1.2e8:      # dense host copies under 500 MB each
        b //= 2
        lens = lens[:b]
        cap = int(lens.max()) + 4
    steps = int(rng.integers(1, 3))
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
    assert np.array_equal(cache.k[0].cpu().numpy(), kc)
    assert np.array_equal(cache.v[0].cpu().numpy(), vc)
