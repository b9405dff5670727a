"""Test-side helpers: load the product package and the CPU oracle.

The oracle (oracle/liboracle.so) is the checker only; the product library never
loads it.  Tolerances follow the north-star parity bar: per element
|gpu - ref| <= 1e-4 + 1e-3 * |ref|.
"""
import ctypes
import importlib.util
import os
import subprocess
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "neural-network-engine_amd")
HEADER = os.path.join(ROOT, "include", "nne_attn.h")
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_LIB = os.path.join(ORACLE_DIR, "liboracle.so")
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")

ATOL = 1e-4
RTOL = 1e-3


def load_package():
    name = "nne_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(
        name, os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


_oracle = None
_f = ctypes.POINTER(ctypes.c_float)
_i32 = ctypes.POINTER(ctypes.c_int32)
_I = ctypes.c_int64


def oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_LIB):
            subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)
        o = ctypes.CDLL(ORACLE_LIB)
        o.oracle_flash_forward.argtypes = [_f, _f, _f, _f, _I, _I, _I, _I, _I, ctypes.c_int,
                                           ctypes.c_int, ctypes.c_float, _I, _I, ctypes.c_int]
        o.oracle_flash_forward.restype = None
        o.oracle_standard_attention.argtypes = [_f, _f, _f, _f, _I, _I, _I, _I, _I, _I,
                                                ctypes.c_int, _I, ctypes.c_int, ctypes.c_float,
                                                ctypes.c_int]
        o.oracle_standard_attention.restype = None
        o.oracle_kv_append.argtypes = [_f, _f, _i32, _f, _f, _I, _I, _I, _I, _I]
        o.oracle_kv_append.restype = ctypes.c_int
        o.oracle_decode_step.argtypes = [_f, _f, _f, _i32, _f, _f, _f, _I, _I, _I, _I, _I,
                                         ctypes.c_int, ctypes.c_float, ctypes.c_int]
        o.oracle_decode_step.restype = ctypes.c_int
        o.oracle_decode_attend.argtypes = [_f, _f, _f, _i32, _f, _I, _I, _I, _I, _I,
                                           ctypes.c_int, ctypes.c_float, ctypes.c_int]
        o.oracle_decode_attend.restype = None
        o.oracle_rope_tables.argtypes = [_f, _f, _I, _I, ctypes.c_float]
        o.oracle_rope_tables.restype = None
        o.oracle_rope_apply.argtypes = [_f, _f, _f, _f, _I, _I, _I, _I, _i32]
        o.oracle_rope_apply.restype = None
        o.oracle_linear.argtypes = [_f, _f, _f, _f, _I, _I, _I]
        o.oracle_linear.restype = None
        o.oracle_qkv_rope.argtypes = [_f, _f, _f, _f, _f, _f, _f, _f, _f, _i32, _f, _f, _f, _I,
                                      _I, _I, _I, _I, _I]
        o.oracle_qkv_rope.restype = None
        _oracle = o
    return _oracle


def _p(a):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(_f)


def _threads():
    return min(8, os.cpu_count() or 1)


def ref_flash(q, k, v, causal, scale=None, br=64, bc=64, threads=None):
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    b, h, tq, d = q.shape
    tk = k.shape[2]
    out = np.zeros((b, h, tq, d), np.float32)
    oracle().oracle_flash_forward(_p(q), _p(k), _p(v), _p(out), b, h, tq, tk, d, int(causal),
                                  int(scale is not None), float(scale or 0.0), br, bc,
                                  threads or _threads())
    return out


def ref_standard(q, k, v, masked, start_pos=0, scale=None, threads=None):
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    b, hq, tq, d = q.shape
    hkv, tk = k.shape[1], k.shape[2]
    out = np.zeros((b, hq, tq, d), np.float32)
    oracle().oracle_standard_attention(_p(q), _p(k), _p(v), _p(out), b, hq, hkv, tq, tk, d,
                                       int(masked), start_pos, int(scale is not None),
                                       float(scale or 0.0), threads or _threads())
    return out


def ref_decode_attend(q, kc, vc, lens, scale=None, threads=None):
    q, kc, vc = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, kc, vc))
    lens = np.ascontiguousarray(lens, dtype=np.int32)
    b, hq, _, d = q.shape
    hkv, cap = kc.shape[1], kc.shape[2]
    out = np.zeros((b, hq, 1, d), np.float32)
    oracle().oracle_decode_attend(_p(q), _p(kc), _p(vc), lens.ctypes.data_as(_i32), _p(out), b,
                                  hq, hkv, cap, d, int(scale is not None), float(scale or 0.0),
                                  threads or _threads())
    return out


def ref_decode_step(q, kc, vc, lens, kn, vn, scale=None, threads=None):
    """Returns (out, kc', vc', lens') -- inputs are not modified."""
    q, kn, vn = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, kn, vn))
    kc, vc = kc.astype(np.float32, copy=True), vc.astype(np.float32, copy=True)
    lens = np.array(lens, dtype=np.int32, copy=True)
    b, hq, _, d = q.shape
    hkv, cap = kc.shape[1], kc.shape[2]
    out = np.zeros((b, hq, 1, d), np.float32)
    rc = oracle().oracle_decode_step(_p(q), _p(kc), _p(vc), lens.ctypes.data_as(_i32), _p(kn),
                                     _p(vn), _p(out), b, hq, hkv, cap, d, int(scale is not None),
                                     float(scale or 0.0), threads or _threads())
    assert rc == 0
    return out, kc, vc, lens


def ref_kv_append(kc, vc, lens, kn, vn):
    kc, vc = kc.astype(np.float32, copy=True), vc.astype(np.float32, copy=True)
    lens = np.array(lens, dtype=np.int32, copy=True)
    kn, vn = (np.ascontiguousarray(x, dtype=np.float32) for x in (kn, vn))
    b, hkv, cap, d = kc.shape
    rc = oracle().oracle_kv_append(_p(kc), _p(vc), lens.ctypes.data_as(_i32), _p(kn), _p(vn), b,
                                   hkv, cap, d, kn.shape[2])
    return rc, kc, vc, lens


def _po(a):
    return None if a is None else _p(a)


def ref_rope_tables(max_seq_len, d, theta=10000.0):
    cos = np.zeros((max_seq_len, d), np.float32)
    sin = np.zeros((max_seq_len, d), np.float32)
    oracle().oracle_rope_tables(_p(cos), _p(sin), max_seq_len, d, float(theta))
    return cos, sin


def ref_rope_apply(x, cos, sin, start_pos):
    x = np.ascontiguousarray(x, dtype=np.float32)
    b, h, t, d = x.shape
    sp = np.ascontiguousarray(np.broadcast_to(np.asarray(start_pos, np.int32), (b,)))
    assert (sp >= 0).all() and (sp + t <= cos.shape[0]).all()
    out = np.zeros_like(x)
    oracle().oracle_rope_apply(_p(x), _p(out), _p(np.ascontiguousarray(cos)),
                               _p(np.ascontiguousarray(sin)), b, h, t, d,
                               sp.ctypes.data_as(_i32))
    return out


def ref_linear(x, w, bias=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.zeros((m, n), np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    oracle().oracle_linear(_p(x), _p(w), _po(bias), _p(y), m, k, n)
    return y


def ref_qkv_rope(x, wq, wk, wv, bq, bk, bv, cos, sin, start_pos, hq, hkv):
    """x [B, T, C] -> (q [B, Hq, T, d], k [B, Hkv, T, d], v [B, Hkv, T, d])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b, t, c = x.shape
    d = wq.shape[0] // hq
    sp = np.ascontiguousarray(np.broadcast_to(np.asarray(start_pos, np.int32), (b,)))
    q = np.zeros((b, hq, t, d), np.float32)
    k = np.zeros((b, hkv, t, d), np.float32)
    v = np.zeros((b, hkv, t, d), np.float32)
    ws = [np.ascontiguousarray(a, dtype=np.float32) for a in (wq, wk, wv)]
    bs = [None if a is None else np.ascontiguousarray(a, dtype=np.float32) for a in (bq, bk, bv)]
    oracle().oracle_qkv_rope(_p(x), _p(ws[0]), _p(ws[1]), _p(ws[2]), _po(bs[0]), _po(bs[1]),
                             _po(bs[2]), _p(np.ascontiguousarray(cos)),
                             _p(np.ascontiguousarray(sin)), sp.ctypes.data_as(_i32), _p(q),
                             _p(k), _p(v), b, t, c, hq, hkv, d)
    return q, k, v


RAYON_LIB = os.path.join(ORACLE_DIR, "librayon_path.so")
RP_COMPONENTS = ("repeat_kv", "gather", "qk", "scale", "mask", "softmax", "pv", "cat", "free",
                 "linear", "rope")
RP_MODES = {"gqa": 0, "mha": 1, "cross": 2}
_rayon = None


def rayon_path():
    """oracle/librayon_path.so: the timing restatement of the reference's CPU
    standard-attention path (AVX2/FMA GEMMs, Rayon splits); bench.py's
    cpu_baseline legs time it.  Checked against the oracle in
    tests/test_rayon_path.py."""
    global _rayon
    if _rayon is None:
        if not os.path.exists(RAYON_LIB):
            subprocess.run(["make", "-s", "-C", ORACLE_DIR, "librayon_path.so"], check=True)
        r = ctypes.CDLL(RAYON_LIB)
        _d = ctypes.POINTER(ctypes.c_double)
        _c = ctypes.c_int
        r.rp_set_threads.argtypes = [_c]
        r.rp_set_threads.restype = None
        r.rp_max_threads.restype = _c
        r.rp_components.restype = _c
        r.rp_attention.argtypes = [_f, _f, _f, _f] + [_c] * 11 + [_d]
        r.rp_attention.restype = _c
        r.rp_decode_run.argtypes = [_f, _f, _f, _i32, _f, _f, _f] + [_c] * 7 + [_f, _f, _d]
        r.rp_decode_run.restype = _c
        r.rp_qkv_rope_run.argtypes = [_f] * 9 + [_i32] + [_c] * 5 + [_f, _f, _f, _d]
        r.rp_qkv_rope_run.restype = _c
        assert r.rp_components() == len(RP_COMPONENTS)
        _rayon = r
    return _rayon


def _rp_times(t):
    return {n: float(t[i]) for i, n in enumerate(RP_COMPONENTS)}


def rp_attention(q, k, v, mode="gqa", causal=True, start_pos=0, q_bthd=False, kv_bthd=False,
                 threads=None):
    """The reference's standard attention on the CPU path it really runs
    (llama.rs:253-296 for "gqa", attention.rs:93-122 for "mha",
    attention.rs:193-203 for "cross").  q [B, Hq, Tq, d], k/v [B, Hkv, Tk, d]
    as logical shapes; *_bthd passes them as the reference's transposed views
    of [B, T, H, d] buffers (give the arrays in that memory order).  Returns
    (context [B, Hq, Tq, d], seconds per component)."""
    q, k, v = (np.ascontiguousarray(x, dtype=np.float32) for x in (q, k, v))
    if q_bthd:
        b, tq, hq, d = q.shape
    else:
        b, hq, tq, d = q.shape
    if kv_bthd:
        hkv, tk = k.shape[2], k.shape[1]
    else:
        hkv, tk = k.shape[1], k.shape[2]
    r = rayon_path()
    if threads:
        r.rp_set_threads(int(threads))
    out = np.zeros((b, hq, tq, d), np.float32)
    t = (ctypes.c_double * len(RP_COMPONENTS))()
    rc = r.rp_attention(_p(q), _p(k), _p(v), _p(out), b, hq, hkv, tq, tk, d, int(q_bthd),
                        int(kv_bthd), int(start_pos), RP_MODES[mode], int(causal), t)
    assert rc == 0, rc
    return out, _rp_times(t)


def rp_decode_run(qs, kc, vc, lens, kns, vns, mode="gqa", threads=None, want_cache=False):
    """steps decode steps (t = 1) as the reference runs a ragged batch: one
    B = 1 call per sequence, each Tensor::cat-ing its slot, then attending.
    qs [steps, B, Hq, d]; kc/vc [B, Hkv, cap, d]; kns/vns [steps, B, Hkv, d].
    Returns (outs [steps, B, Hq, d], seconds per component[, kc', vc'])."""
    qs, kns, vns, kc, vc = (np.ascontiguousarray(x, dtype=np.float32)
                            for x in (qs, kns, vns, kc, vc))
    lens = np.ascontiguousarray(lens, dtype=np.int32)
    steps, b, hq, d = qs.shape
    hkv, cap = kc.shape[1], kc.shape[2]
    r = rayon_path()
    if threads:
        r.rp_set_threads(int(threads))
    outs = np.zeros((steps, b, hq, d), np.float32)
    t = (ctypes.c_double * len(RP_COMPONENTS))()
    kend = np.zeros_like(kc) if want_cache else None
    vend = np.zeros_like(vc) if want_cache else None
    rc = r.rp_decode_run(_p(qs), _p(kc), _p(vc), lens.ctypes.data_as(_i32), _p(kns), _p(vns),
                         _p(outs), b, hq, hkv, cap, d, steps, RP_MODES[mode], _po(kend),
                         _po(vend), t)
    assert rc == 0, rc
    if want_cache:
        return outs, _rp_times(t), kend, vend
    return outs, _rp_times(t)


def rp_qkv_rope_run(x, wq, wk, wv, bq, bk, bv, cos, sin, pos, hq, hkv, threads=None):
    """The decode prologue as the reference runs a ragged batch: per
    sequence, the three Linear projections (gemv_a_bt_m1 + bias) and RoPE
    through its elementwise ops.  x [B, C]; cos/sin [max_pos, d] or None.
    Returns (q [B, Hq, d], k [B, Hkv, d], v [B, Hkv, d], seconds per
    component)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b, c = x.shape
    d = wq.shape[0] // hq
    ws = [np.ascontiguousarray(a, dtype=np.float32) for a in (wq, wk, wv)]
    bs = [None if a is None else np.ascontiguousarray(a, dtype=np.float32) for a in (bq, bk, bv)]
    tabs = [None if a is None else np.ascontiguousarray(a, dtype=np.float32) for a in (cos, sin)]
    pos = np.ascontiguousarray(np.broadcast_to(np.asarray(pos, np.int32), (b,)))
    r = rayon_path()
    if threads:
        r.rp_set_threads(int(threads))
    q = np.zeros((b, hq, d), np.float32)
    k = np.zeros((b, hkv, d), np.float32)
    v = np.zeros((b, hkv, d), np.float32)
    t = (ctypes.c_double * len(RP_COMPONENTS))()
    rc = r.rp_qkv_rope_run(_p(x), _p(ws[0]), _p(ws[1]), _p(ws[2]), _po(bs[0]), _po(bs[1]),
                           _po(bs[2]), _po(tabs[0]), _po(tabs[1]), pos.ctypes.data_as(_i32), b, c,
                           hq, hkv, d, _p(q), _p(k), _p(v), t)
    assert rc == 0, rc
    return q, k, v, _rp_times(t)


def assert_close(got, ref, atol=ATOL, rtol=RTOL, what=""):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.isfinite(got).all(), what + ": non-finite output"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err - bound), err.shape)
        raise AssertionError("%s: %d/%d elements out of tolerance; worst at %s: got %r ref %r "
                             "(max abs err %.3g)" % (what, bad.sum(), bad.size, i, got[i], ref[i],
                                                     err.max()))


def error_stats(got, ref):
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    big = np.abs(ref) >= 1e-3
    return {"max_abs": float(err.max()) if err.size else 0.0,
            "max_rel": float((err[big] / np.abs(ref[big])).max()) if big.any() else 0.0}


def load_golden(name):
    with np.load(os.path.join(GOLDEN_DIR, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def golden_names(kind=None):
    out = []
    for f in sorted(os.listdir(GOLDEN_DIR)):
        if f.endswith(".npz"):
            n = f[:-4]
            if kind is None or str(load_golden(n)["kind"]) == kind:
                out.append(n)
    return out


def header_symbols():
    """Function names declared in include/nne_attn.h."""
    import re
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(nne_[a-z0-9_]+)\s*\(", txt)))


def decode_vs_oracle(nne, cuda, b, hq, hkv, d, lens, append, seed, what):
    """One decode step (append) or attend over a KVCache with the given
    lengths, against the oracle; repeat attends must be bit-identical and the
    appended rows and lengths bit-exact."""
    import torch
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int32)
    cap = int(lens.max()) + 2
    kc = rng.standard_normal((b, hkv, cap, d), dtype=np.float32)
    vc = rng.standard_normal((b, hkv, cap, d), dtype=np.float32)
    q = rng.standard_normal((b, hq, 1, d), dtype=np.float32)
    cache = nne.KVCache(1, b, hkv, cap, d, device=cuda)
    cache.k[0].copy_(torch.from_numpy(kc))
    cache.v[0].copy_(torch.from_numpy(vc))
    cache.set_lengths(0, lens)
    qd = torch.from_numpy(q).to(cuda)
    if append:
        kn = rng.standard_normal((b, hkv, 1, d), dtype=np.float32)
        vn = rng.standard_normal((b, hkv, 1, d), dtype=np.float32)
        out = cache.decode_step(0, qd, torch.from_numpy(kn).to(cuda), torch.from_numpy(vn).to(cuda))
        ref, rkc, _, rlens = ref_decode_step(q, kc, vc, lens, kn, vn)
        torch.cuda.synchronize()
        assert np.array_equal(cache.lens_host[0], rlens)
        assert np.array_equal(cache.lens_dev[0].cpu().numpy(), rlens)
        rows = np.arange(b)
        assert np.array_equal(cache.k[0].cpu().numpy()[rows, :, lens], rkc[rows, :, lens])
    else:
        out = cache.attend(0, qd)
        ref = ref_decode_attend(q, kc, vc, lens)
        again = cache.attend(0, qd)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), again.cpu().numpy()), "repeat calls differ"
    torch.cuda.synchronize()
    assert_close(out.cpu().numpy(), ref, what="%s b=%d hq=%d hkv=%d d=%d" % (what, b, hq, hkv, d))
