"""nne_decode_step_noalloc (the decode step on the library's static device
scratch) against nne_decode_step (caller workspace: records and counters),
both through the C ABI, and against the CPU oracle's decode step.

Two calls in a row on the same scratch, the second with a smaller input
(fewer sequences, fewer heads, a smaller head dim), so a call that read the
previous call's records or counters would show.  Outputs must agree to the
parity bar |a - b| <= 1e-4 + 1e-3 |b| (the kernels and their split are the
same, so in practice bit for bit); the caches and lengths must agree exactly.
"""
import ctypes

import numpy as np
import pytest

import nne_testlib as T

pytestmark = pytest.mark.gpu

_i32p = ctypes.POINTER(ctypes.c_int32)


def _case(nne, cuda, seed, b, hq, hkv, d, cap, lo, hi):
    import torch
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=b).astype(np.int32)
    kc = torch.from_numpy(rng.standard_normal((b, hkv, cap, d), dtype=np.float32)).to(cuda)
    vc = torch.from_numpy(rng.standard_normal((b, hkv, cap, d), dtype=np.float32)).to(cuda)
    q = torch.from_numpy(rng.standard_normal((b, hq, 1, d), dtype=np.float32)).to(cuda)
    kn = torch.from_numpy(rng.standard_normal((b, hkv, 1, d), dtype=np.float32)).to(cuda)
    vn = torch.from_numpy(rng.standard_normal((b, hkv, 1, d), dtype=np.float32)).to(cuda)
    return lens, kc, vc, q, kn, vn


def _step(nne, fn, lens, kc, vc, q, kn, vn, cuda, workspace=None):
    import torch
    b, hq, _, d = q.shape
    hkv, cap = kc.shape[1], kc.shape[2]
    lens_host = lens.copy()
    lens_dev = torch.from_numpy(lens_host.copy()).to(cuda)
    o = torch.empty_like(q)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = [q.data_ptr(), None, kc.data_ptr(), vc.data_ptr(), lens_dev.data_ptr(),
            lens_host.ctypes.data_as(_i32p), kn.data_ptr(), None, vn.data_ptr(), None,
            o.data_ptr(), None, b, hq, hkv, cap, d, 0, 0.0]
    keep = None
    if workspace is not None:
        wsp, keep = workspace.struct()
        args += [wsp]
    rc = fn(*args, s)
    assert rc == nne.NNE_OK, nne.lib().nne_last_error()
    torch.cuda.synchronize()
    return o.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy(), lens_host, lens_dev.cpu().numpy()


@pytest.mark.parametrize("order", ["noalloc_first", "reference_first"])
def test_noalloc_decode_step_matches_decode_step(nne, cuda, order):
    import torch
    lib = nne.lib()
    cases = [
        # config-3 geometry (B=32, Hq=32, Hkv=8, d=128), ragged lengths
        dict(seed=71, b=32, hq=32, hkv=8, d=128, cap=1200, lo=300, hi=1100),
        # then a smaller input on the same scratch: 16-row tile, d = 64
        dict(seed=72, b=5, hq=16, hkv=2, d=64, cap=700, lo=1, hi=650),
        # above 256 dims: the append kernel and the deep kernel, no scratch
        dict(seed=73, b=3, hq=8, hkv=2, d=512, cap=300, lo=1, hi=250),
    ]
    for c in cases:
        print("case noalloc", order, c, flush=True)
        base = _case(nne, cuda, c["seed"], c["b"], c["hq"], c["hkv"], c["d"], c["cap"], c["lo"],
                     c["hi"])
        lens, kc, vc, q, kn, vn = base
        size = nne.NneWorkspaceSize()
        assert lib.nne_decode_workspace_size(c["b"], c["hq"], c["hkv"], c["d"],
                                             ctypes.byref(size)) == nne.NNE_OK
        ws = nne.Workspace(cuda).reserve(size)
        runs = {}
        names = ["noalloc", "reference"] if order == "noalloc_first" else ["reference", "noalloc"]
        for name in names:
            kc_i, vc_i = kc.clone(), vc.clone()
            if name == "noalloc":
                runs[name] = _step(nne, lib.nne_decode_step_noalloc, lens, kc_i, vc_i, q, kn, vn,
                                   cuda)
            else:
                runs[name] = _step(nne, lib.nne_decode_step, lens, kc_i, vc_i, q, kn, vn, cuda,
                                   workspace=ws)
        a, r = runs["noalloc"], runs["reference"]
        T.assert_close(a[0], r[0], what="noalloc output")
        ref, rkc, rvc, rlens = T.ref_decode_step(q.cpu().numpy(), kc.cpu().numpy(),
                                                 vc.cpu().numpy(), lens, kn.cpu().numpy(),
                                                 vn.cpu().numpy())
        T.assert_close(a[0], ref, what="noalloc output against the oracle")
        assert np.array_equal(a[1], rkc) and np.array_equal(a[2], rvc)
        assert np.array_equal(a[3], rlens)
        assert np.array_equal(a[1], r[1]) and np.array_equal(a[2], r[2])
        assert np.array_equal(a[3], lens + 1) and np.array_equal(a[4], lens + 1)
        assert np.array_equal(r[3], lens + 1)


def test_noalloc_rejects_steps_beyond_its_scratch(nne, cuda):
    """Refused on the host, before any device work.  Only k_new and v_new are
    real (small) device tensors; every other pointer is NULL, so if the
    scratch check ever moved after the argument checks the call would fail
    on a host NULL check, never on the device."""
    import torch
    lib = nne.lib()
    lens = np.full(2048, 5, np.int32)
    kn = torch.zeros(16, device=cuda)
    vn = torch.zeros(16, device=cuda)
    rc = lib.nne_decode_step_noalloc(None, None, None, None, None, lens.ctypes.data_as(_i32p),
                                     kn.data_ptr(), None, vn.data_ptr(), None, None, None, 2048,
                                     128, 8, 64, 128, 0, 0.0, None)
    assert rc == nne.NNE_EINVAL
    assert "scratch" in lib.nne_last_error().decode()
    assert (lens == 5).all()
