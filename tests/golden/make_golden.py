"""Writes the golden attention fixtures under tests/golden/*.npz.

The reference (elvin-mark/neural-network-engine) ships no attention fixtures and
its tests draw unseeded inputs (src/tensor/mod.rs:110-116), so the vectors here
are produced from seeded inputs and the mathematical definition of each
reference function, evaluated in float64:

* flash  (src/nn/flash_attention.rs:19-199): softmax(scale * Q K^T + M) V with
  M = -inf where c > r (top-left causal, :113) -- the same formula the
  reference's own test builds as its expected value
  (tests/nn/flash_attention_tests.rs:18-37).  Rows with no visible key are 0
  (:186-194).
* standard / GQA (src/models/llama.rs:253-296, src/nn/attention.rs:93-122):
  K/V head for query head hq is hq // G; additive -1e4 where c > start_pos + r
  when Tq > 1; softmax; times V.
* decode (llama.rs:239-296 with t = 1): append one row, attend to all rows.

Each float64 result is cross-checked against torch's float64
scaled_dot_product_attention before it is written.  Run from the repo root:
    python tests/golden/make_golden.py
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def softmax64(s):
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    return e / e.sum(axis=-1, keepdims=True)


def attention64(q, k, v, mask_mode, q_offset=0, scale=None):
    """q [B,Hq,Tq,d]; k,v [B,Hkv,Tk,d]; mask_mode in {'none','inf','1e4'}."""
    q = q.astype(np.float64)
    k = k.astype(np.float64)
    v = v.astype(np.float64)
    b, hq, tq, d = q.shape
    hkv, tk = k.shape[1], k.shape[2]
    g = hq // hkv
    kk = np.repeat(k, g, axis=1)          # head hq reads kv head hq // g
    vv = np.repeat(v, g, axis=1)
    sc = (1.0 / np.sqrt(np.float32(d))) if scale is None else scale
    sc = float(np.float32(sc))
    s = np.einsum("bhrd,bhcd->bhrc", q, kk) * sc
    r = np.arange(tq)[:, None]
    c = np.arange(tk)[None, :]
    above = c > (r + q_offset)
    out = np.zeros((b, hq, tq, d))
    if mask_mode == "inf":
        s = np.where(above, -np.inf, s)
        visible = (~above).any(axis=1)
        p = np.zeros_like(s)
        if visible.any():
            p[:, :, visible, :] = softmax64(s[:, :, visible, :])
        out = p @ vv
    else:
        if mask_mode == "1e4":
            s = s + np.where(above, -1e4, 0.0)
        out = softmax64(s) @ vv if tk > 0 else out
    # cross-check with torch float64 SDPA
    tq_ = torch.from_numpy(q)
    tk_ = torch.from_numpy(kk)
    tv_ = torch.from_numpy(vv)
    if mask_mode == "inf":
        m = torch.from_numpy(np.where(above, -np.inf, 0.0))
    elif mask_mode == "1e4":
        m = torch.from_numpy(np.where(above, -1e4, 0.0))
    else:
        m = None
    if tk > 0 and (mask_mode != "inf" or (~above).any(axis=1).all()):
        ref = torch.nn.functional.scaled_dot_product_attention(
            tq_, tk_, tv_, attn_mask=m, scale=sc).numpy()
        assert np.allclose(ref, out, atol=1e-12, rtol=1e-10), "torch cross-check failed"
    return out


def randn(rng, shape, std=1.0):
    return (rng.standard_normal(shape) * std).astype(np.float32)


def main():
    cases = {}
    # --- flash (a1-a3) --------------------------------------------------
    # shapes of tests/nn/flash_attention_tests.rs:5-8 and :63-66
    for name, (b, h, tq, tk, d, causal, seed) in {
        "flash_causal_b2h4t16d32": (2, 4, 16, 16, 32, True, 11),
        "flash_noncausal_b1h2t32d16": (1, 2, 32, 32, 16, False, 12),
        "flash_causal_b1h2t37d16": (1, 2, 37, 37, 16, True, 13),
        "flash_noncausal_b1h2t37d16": (1, 2, 37, 37, 16, False, 14),
        "flash_causal_b1h2t100d64": (1, 2, 100, 100, 64, True, 15),
        "flash_noncausal_b2h1t150d64": (2, 1, 150, 150, 64, False, 16),
        "flash_causal_b1h1t70d128": (1, 1, 70, 70, 128, True, 17),
        "flash_causal_tq40_tk24_d32": (1, 2, 40, 24, 32, True, 18),
        "flash_noncausal_tq5_tk90_d48": (1, 3, 5, 90, 48, False, 19),
    }.items():
        rng = np.random.default_rng(seed)
        q, k, v = randn(rng, (b, h, tq, d)), randn(rng, (b, h, tk, d)), randn(rng, (b, h, tk, d))
        out = attention64(q, k, v, "inf" if causal else "none")
        cases[name] = dict(kind="flash", q=q, k=k, v=v, out=out, causal=int(causal),
                           q_offset=0)
    # --- GQA standard path (a5): LlamaConfig::mini heads (llama.rs:28-46) --
    for name, (b, hq, hkv, tq, tk, d, start, seed) in {
        "gqa_g2_b1t6d16": (1, 4, 2, 6, 6, 16, 0, 21),
        "gqa_g4_b2tq5tk9d32_start4": (2, 8, 2, 5, 9, 32, 4, 22),
        "gqa_g4_b1t67d128": (1, 4, 1, 67, 67, 128, 0, 23),
        "gqa_g8_b1t33d64": (1, 8, 1, 33, 33, 64, 0, 24),
    }.items():
        rng = np.random.default_rng(seed)
        q = randn(rng, (b, hq, tq, d))
        k, v = randn(rng, (b, hkv, tk, d)), randn(rng, (b, hkv, tk, d))
        out = attention64(q, k, v, "1e4" if tq > 1 else "none", q_offset=start)
        cases[name] = dict(kind="gqa", q=q, k=k, v=v, out=out, causal=int(tq > 1),
                           q_offset=start)
    # --- cross-attention (a8): Tq query rows onto a longer memory ---------
    rng = np.random.default_rng(31)
    b, h, tq, tk, d = 2, 3, 8, 150, 64
    q, k, v = randn(rng, (b, h, tq, d)), randn(rng, (b, h, tk, d)), randn(rng, (b, h, tk, d))
    cases["cross_b2h3tq8tk150d64"] = dict(kind="cross", q=q, k=k, v=v,
                                          out=attention64(q, k, v, "none"), causal=0,
                                          q_offset=0)
    # --- decode (a6/a7): ragged lengths, append one row then attend -------
    rng = np.random.default_rng(41)
    b, hq, hkv, d, cap = 5, 4, 2, 16, 80
    lens = np.array([1, 5, 63, 64, 65], dtype=np.int32)
    kc = np.zeros((b, hkv, cap, d), np.float32)
    vc = np.zeros((b, hkv, cap, d), np.float32)
    for i, L in enumerate(lens):
        kc[i, :, :L] = randn(rng, (hkv, L, d))
        vc[i, :, :L] = randn(rng, (hkv, L, d))
    kn, vn = randn(rng, (b, hkv, 1, d)), randn(rng, (b, hkv, 1, d))
    q = randn(rng, (b, hq, 1, d))
    out = np.zeros((b, hq, 1, d))
    for i, L in enumerate(lens):
        kk = np.concatenate([kc[i:i + 1, :, :L], kn[i:i + 1]], axis=2)
        vv = np.concatenate([vc[i:i + 1, :, :L], vn[i:i + 1]], axis=2)
        out[i:i + 1] = attention64(q[i:i + 1], kk, vv, "none")
    cases["decode_ragged_b5g2d16"] = dict(kind="decode", q=q, k_cache=kc, v_cache=vc,
                                          lens=lens, k_new=kn, v_new=vn, out=out, cap=cap)
    for name, c in cases.items():
        c = {key: (np.asarray(val) if not isinstance(val, str) else np.array(val))
             for key, val in c.items()}
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **c)
        print("wrote", name)


if __name__ == "__main__":
    main()
