"""Decode shapes beyond the common ones, against the CPU oracle.

The reference's GQA only requires that Hkv divides Hq (llama.rs:181-185) and
its attention takes any head dim (flash_attention.rs:39-48); its decode batch
is unbounded.  On the split-K kernel these cases take:

* 17-64 query rows per KV head: the waves split into 2 or 4 row groups of 16
  rows over the same K/V blocks (32- and 64-row tiles);
* more than 64 rows (32 at d = 256): several launches of row ranges, the
  first appending the new row and the later ones reading it from the cache;
* d up to 256 (16-row tiles with a one-block ring); above 256 the append
  kernel, then the deep kernel (8 waves per 32-row unit);
* more than 2048 sequences: launches of 2048 sequences in stream order.

Bar: |gpu - ref| <= 1e-4 + 1e-3 |ref|; cache contents and lengths bit-exact.
"""
import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu


def rnd(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float32)


def run_case(nne, cuda, b, hq, hkv, d, lens, append, seed, cap=None):
    import torch
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    cap = cap or int(lens.max()) + 3
    kc, vc = rnd(rng, b, hkv, cap, d), rnd(rng, b, hkv, cap, d)
    q = rnd(rng, b, hq, 1, d)
    cache = nne.KVCache(1, b, hkv, cap, d, device=cuda)
    cache.k[0].copy_(torch.from_numpy(kc))
    cache.v[0].copy_(torch.from_numpy(vc))
    cache.set_lengths(0, lens)
    qd = torch.from_numpy(q).to(cuda)
    if append:
        kn, vn = rnd(rng, b, hkv, 1, d), rnd(rng, b, hkv, 1, d)
        out = cache.decode_step(0, qd, torch.from_numpy(kn).to(cuda), torch.from_numpy(vn).to(cuda))
        ref, rkc, rvc, rlens = T.ref_decode_step(q, kc, vc, lens, kn, vn)
        torch.cuda.synchronize()
        assert np.array_equal(cache.lens_host[0], rlens)
        assert np.array_equal(cache.lens_dev[0].cpu().numpy(), rlens)
        # the whole cache: the appended rows and every row that must not move
        assert np.array_equal(cache.k[0].cpu().numpy(), rkc)
        assert np.array_equal(cache.v[0].cpu().numpy(), rvc)
    else:
        out = cache.attend(0, qd)
        ref = T.ref_decode_attend(q, kc, vc, lens)
    torch.cuda.synchronize()
    T.assert_close(out.cpu().numpy(), ref, what="decode b=%d hq=%d hkv=%d d=%d" % (b, hq, hkv, d))


@pytest.mark.parametrize("b,hq,hkv,d,append", [
    (3, 32, 1, 64, True),      # MQA, 32 rows: 2 row groups
    (2, 64, 1, 128, False),    # 64 rows: 4 row groups
    (2, 96, 1, 64, True),      # 96 rows: a 64-row launch, then a 32-row one
    (2, 40, 2, 128, True),     # G = 20 over 2 KV heads
    (3, 8, 2, 256, True),      # d = 256, G = 4
    (2, 12, 12, 256, False),   # d = 256, MHA
    (2, 48, 1, 256, True),     # d = 256, 48 rows: a 32-row launch, then a 16-row one
    (1, 130, 1, 80, True),     # 130 rows over three launches, padded head dim
])
def test_decode_group_sizes_and_head_dims(nne, cuda, b, hq, hkv, d, append):
    print("case decode b=%d hq=%d hkv=%d d=%d append=%s" % (b, hq, hkv, d, append), flush=True)
    rng = np.random.default_rng(hq * 7 + d)
    lens = rng.integers(1, 700, size=b)
    lens[0] = 1100                     # one long head split over several workgroups
    run_case(nne, cuda, b, hq, hkv, d, lens, append, seed=hq + d)


@pytest.mark.parametrize("b,hq,hkv,d,append", [
    (3, 8, 2, 512, True),      # G = 4
    (2, 4, 4, 320, False),     # MHA
    (2, 16, 1, 1028, True),    # MQA, two output chunks
    (4, 64, 8, 384, True),     # G = 8
    (32, 16, 4, 384, True),    # 128 ragged pairs: the long sequence in several parts
    (40, 32, 8, 512, True),    # 320 pairs, more than the CUs: no ragged split
])
def test_decode_head_dims_above_256(nne, cuda, b, hq, hkv, d, append):
    print("case decode deep b=%d hq=%d hkv=%d d=%d append=%s" % (b, hq, hkv, d, append), flush=True)
    rng = np.random.default_rng(hq * 11 + d)
    lens = rng.integers(1, 400, size=b)
    lens[0] = 700
    if not append:
        lens[-1] = 0                   # an empty sequence attends to nothing: zeros
    run_case(nne, cuda, b, hq, hkv, d, lens, append, seed=hq + 3 * d)


def test_decode_long_sequences_above_256_dims(nne, cuda):
    """Few (sequence, KV head) pairs with long caches at d = 512: each head's
    keys split over workgroups, merged by the combine kernel."""
    print("case decode deep long", flush=True)
    rng = np.random.default_rng(65)
    lens = rng.integers(1000, 3000, size=4)
    run_case(nne, cuda, 4, 16, 4, 512, lens, True, seed=66)
    run_case(nne, cuda, 4, 16, 4, 512, lens, False, seed=67)


def test_decode_steps_above_256_dims(nne, cuda):
    """Four decode steps in a row at d = 512 through the cache: each step's
    output, the whole cache and the lengths against the oracle's steps."""
    import torch
    print("case decode deep steps", flush=True)
    b, hq, hkv, d, cap = 3, 8, 2, 512, 200
    rng = np.random.default_rng(64)
    lens = np.array([5, 120, 33], np.int32)
    kc, vc = rnd(rng, b, hkv, cap, d), rnd(rng, b, hkv, cap, d)
    cache = nne.KVCache(1, b, hkv, cap, d, device=cuda)
    cache.k[0].copy_(torch.from_numpy(kc))
    cache.v[0].copy_(torch.from_numpy(vc))
    cache.set_lengths(0, lens)
    for step in range(4):
        q, kn, vn = rnd(rng, b, hq, 1, d), rnd(rng, b, hkv, 1, d), rnd(rng, b, hkv, 1, d)
        out = cache.decode_step(0, dev(q, cuda), dev(kn, cuda), dev(vn, cuda))
        ref, kc, vc, lens = T.ref_decode_step(q, kc, vc, lens, kn, vn)
        torch.cuda.synchronize()
        T.assert_close(out.cpu().numpy(), ref, what="d=512 step %d" % step)
        assert np.array_equal(cache.lens_host[0], lens)
        assert np.array_equal(cache.k[0].cpu().numpy(), kc)
        assert np.array_equal(cache.v[0].cpu().numpy(), vc)


def dev(x, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


@pytest.mark.parametrize("b,hq,hkv,d", [
    (130, 20, 1, 64),      # 20 rows: the 32-row tile
    (145, 64, 1, 128),     # 64 rows: 4 row groups
    (160, 96, 1, 64),      # 96 rows: a 64-row launch, then a 32-row one
    (150, 96, 1, 128),
    (140, 8, 2, 256),      # d = 256, G = 4
    (135, 48, 1, 256),     # d = 256, 48 rows: a 32-row launch, then a 16-row one
])
@pytest.mark.parametrize("append", [True, False])
def test_decode_wide_rows_beyond_128_sequences(nne, cuda, b, hq, hkv, d, append):
    """More than 128 sequences: the flattened prefix is scanned on the GPU and
    a second kernel merges split heads, zero-fills empty sequences and
    advances lens.  With row-range launches the later launches read lens
    after that kernel of the first launch has advanced it."""
    print("case decode wide b=%d hq=%d hkv=%d d=%d append=%s" % (b, hq, hkv, d, append), flush=True)
    rng = np.random.default_rng(b * 31 + hq + d)
    lens = rng.integers(1, 400, size=b)
    lens[rng.integers(0, b, size=5)] = 0
    lens[3] = 1500                     # one long head split over several workgroups
    run_case(nne, cuda, b, hq, hkv, d, lens, append, seed=b + hq + d)


@pytest.mark.parametrize("append", [True, False])
def test_decode_batch_beyond_2048_sequences(nne, cuda, append):
    """2100 sequences: a launch of 2048 and one of 52, ragged short lengths
    (empty sequences included)."""
    print("case decode b=2100 append=%s" % append, flush=True)
    rng = np.random.default_rng(77)
    lens = rng.integers(0, 40, size=2100)
    run_case(nne, cuda, 2100, 4, 2, 64, lens, append, seed=78, cap=48)


def test_decode_llama70b_groups_config3_lengths(nne, cuda):
    """G = 8 at d = 128 (LLaMA-2-70B-style Hq = 64, Hkv = 8) at config-3
    batch and lengths: B = 32, L ~ U[512, 4096], append then attend."""
    print("case decode b=32 hq=64 hkv=8 d=128", flush=True)
    rng = np.random.default_rng(0x5EED0003)
    lens = rng.integers(512, 4097, size=32)
    run_case(nne, cuda, 32, 64, 8, 128, lens, True, seed=0x5EED0033, cap=4100)
