"""Whole-head packing of the split-K launch, against the CPU oracle.

When every head is short next to the launch, or the heads are few, long and
even, the split-K launch groups whole heads into at most one workgroup per CU
instead of cutting the flattened keys into equal chunks: no head is split, so
no partial records, arrivals or merges exist.  The choice is a cost estimate
(longest group at one CU's streaming rate against the device's rate plus the
hand-off of split heads); the shapes below sit far on one side of it:

* the GPT-2-small decode attend (B = 32, 12 heads, d = 64, L ~ U[128, 1024]):
  384 heads paired into 256 workgroups (the 128 longest alone, the rest
  longest with shortest), packed ~15 us against ~21 us chunked;
* a uniform batch (B = 32, Hkv = 8, d = 128, L = 1000): one head per CU;
* short ragged heads with empty sequences among them (zero rows out);
* config 3's ragged lengths stay chunked (its longest head alone would take a
  CU ~110 us against ~100 us for the whole launch chunked) and are covered by
  test_decode_gpu.py; config 5b (160 heads of 1500 keys, one per workgroup)
  by test_configs_fullsize_gpu.py.

Reference: llama.rs:239-296 (t = 1 decode), gpt2.rs:249-263 (MHA decode).
Bar: |gpu - ref| <= 1e-4 + 1e-3 |ref|; cache rows and lengths bit-exact.
"""
import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu


def run(nne, cuda, b, hq, hkv, d, lens, append, seed):
    T.decode_vs_oracle(nne, cuda, b, hq, hkv, d, lens, append, seed, "packed")


@pytest.mark.parametrize("append", [False, True])
def test_gpt2_decode_attend_shape(nne, cuda, append):
    print("case gpt2 attend append=%s" % append, flush=True)
    lens = np.random.default_rng(0x5EED0015).integers(128, 1025, size=32)
    run(nne, cuda, 32, 12, 12, 64, lens, append, seed=15)


@pytest.mark.parametrize("append", [False, True])
def test_uniform_batch_one_head_per_workgroup(nne, cuda, append):
    print("case uniform b=32 hkv=8 d=128 append=%s" % append, flush=True)
    run(nne, cuda, 32, 32, 8, 128, np.full(32, 1000), append, seed=16)


def test_short_heads_with_empty_sequences(nne, cuda):
    print("case short ragged heads with empty sequences", flush=True)
    lens = np.random.default_rng(17).integers(0, 90, size=24)
    lens[[0, 5, 6, 23]] = 0
    run(nne, cuda, 24, 8, 2, 64, lens, False, seed=17)
    run(nne, cuda, 24, 8, 2, 64, lens, True, seed=18)
