"""Cut chunks of the split-K launch, against the CPU oracle.

A chunked split-K launch (heads too uneven to pack whole) cuts the flattened
(sequence, KV head, key) rows into one range per workgroup.  The host cuts
them so that a workgroup's keys plus a fixed cost for every segment after its
first are about equal: workgroups that cross head boundaries get fewer keys.
Ranges therefore start and end anywhere inside a head, a head is shared by a
variable number of workgroups, and the in-launch merge finds the first and
last workgroup of a head by searching the cut.  The shapes below exercise:

* a few long heads among many tiny ones (d = 128, 4-row tile): workgroups
  with several segments next to workgroups inside one long head;
* one long head per sequence on the 16-row tile (Hq = 16 per KV head): every
  head split, the largest records;
* the G = 8 decode (Hq = 64, Hkv = 8, d = 128) with config 3's ragged lengths
  at a quarter of its batch;
* repeat attends bit-identical (records merge in workgroup order, whichever
  workgroup arrives last).

Reference: llama.rs:239-296 (t = 1 decode: append, then attend to all rows).
Bar: |gpu - ref| <= 1e-4 + 1e-3 |ref|; cache rows and lengths bit-exact.
"""
import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu


def long_and_tiny_lengths():
    lens = np.random.default_rng(31).integers(1, 201, size=48)
    lens[[0, 13, 14, 40]] = 3000
    return lens


@pytest.mark.parametrize("append", [False, True])
def test_long_and_tiny_heads(nne, cuda, append):
    print("case long+tiny b=48 hq=8 hkv=2 d=128 append=%s" % append, flush=True)
    T.decode_vs_oracle(nne, cuda, 48, 8, 2, 128, long_and_tiny_lengths(), append, 31, "cut")


@pytest.mark.parametrize("append", [False, True])
def test_split_heads_on_16_row_tile(nne, cuda, append):
    print("case 16-row tile b=2 hq=32 hkv=2 d=64 append=%s" % append, flush=True)
    T.decode_vs_oracle(nne, cuda, 2, 32, 2, 64, [20000, 7], append, 32, "cut")


def test_g8_ragged_decode(nne, cuda):
    print("case G=8 b=8 hq=64 hkv=8 d=128 L~U[512,4096]", flush=True)
    lens = np.random.default_rng(0x5EED0008).integers(512, 4097, size=8)
    T.decode_vs_oracle(nne, cuda, 8, 64, 8, 128, lens, True, 33, "cut")
    T.decode_vs_oracle(nne, cuda, 8, 64, 8, 128, lens, False, 34, "cut")
