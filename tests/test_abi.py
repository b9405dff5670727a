"""C-ABI checks that need no GPU: the library loads, exports every symbol
include/nne_attn.h declares, and rejects bad arguments on the host with the
error classes of the reference (src/error.rs) before touching the device."""
import ctypes

import numpy as np
import pytest

import nne_testlib as T

FAKE = ctypes.c_void_p(4096)   # never dereferenced: validation fails first


def i64(*v):
    return (ctypes.c_int64 * 4)(*v)


def test_library_exports_header_symbols(nne):
    lib = nne.lib()
    declared = T.header_symbols()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
        assert name in nne.SIGNATURES, name
    assert lib.nne_abi_version() == 4


def test_flash_shape_mismatch_is_shape_error(nne):
    lib = nne.lib()
    rc = lib.nne_flash_attention_forward(FAKE, i64(2, 4, 16, 32), None, FAKE, i64(2, 2, 16, 32),
                                         None, FAKE, i64(2, 2, 16, 32), None, FAKE, None, 1, 0,
                                         0.0, 64, 64, None)
    assert rc == nne.NNE_ESHAPE
    msg = lib.nne_last_error().decode()
    # the reference reports expected [b, h, t_k, d] vs actual [k_b, k_h, t_k, k_d] (:44-47)
    assert "expected shape [2, 4, 16, 32], got [2, 2, 16, 32]" in msg


def test_flash_rejects_head_count_mismatch_but_gqa_entry_accepts_division(nne):
    lib = nne.lib()
    rc = lib.nne_attention_forward(FAKE, i64(1, 6, 8, 16), None, FAKE, i64(1, 4, 8, 16), None,
                                   FAKE, i64(1, 4, 8, 16), None, FAKE, None, 1, 0, 0, 0.0, None)
    assert rc == nne.NNE_ESHAPE          # 4 does not divide 6


def test_value_length_mismatch(nne):
    lib = nne.lib()
    rc = lib.nne_flash_attention_forward(FAKE, i64(1, 2, 8, 16), None, FAKE, i64(1, 2, 8, 16),
                                         None, FAKE, i64(1, 2, 9, 16), None, FAKE, None, 0, 0,
                                         0.0, 64, 64, None)
    assert rc == nne.NNE_ESHAPE


def test_wide_head_dims_need_vector_views(nne):
    """Above 128 dims every kernel (split-K, wave pair, and above 256 the
    deep kernel) reads 16-byte vector rows; other views are refused before
    any launch."""
    lib = nne.lib()
    odd = ctypes.c_void_p(4096 + 4)   # 4-byte, not 16-byte, aligned
    s = i64(1, 1, 4, 260)
    rc = lib.nne_flash_attention_forward(odd, s, None, FAKE, s, None, FAKE, s, None, FAKE, None,
                                         0, 0, 0.0, 64, 64, None)
    assert rc == nne.NNE_EINVAL
    assert "head dim 260 > 128" in lib.nne_last_error().decode()
    s = i64(1, 1, 4, 1030)
    rc = lib.nne_flash_attention_forward(FAKE, s, None, FAKE, s, None, FAKE, s, None, FAKE, None,
                                         0, 0, 0.0, 64, 64, None)
    assert rc == nne.NNE_EINVAL
    assert "multiple of 4" in lib.nne_last_error().decode()
    s = i64(1, 1, 4, 130)
    rc = lib.nne_flash_attention_forward(FAKE, s, None, FAKE, s, None, FAKE, s, None, FAKE, None,
                                         0, 0, 0.0, 64, 64, None)
    assert rc == nne.NNE_EINVAL
    assert "multiple of 4" in lib.nne_last_error().decode()


def test_kv_append_capacity_error_leaves_lengths(nne):
    lib = nne.lib()
    lens = np.array([3, 9], np.int32)
    rc = lib.nne_kv_append(FAKE, FAKE, FAKE, lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                           FAKE, None, FAKE, None, 2, 2, 10, 16, 2, None)
    assert rc == nne.NNE_ECAPACITY
    assert list(lens) == [3, 9]


def test_decode_rejects_bad_geometry(nne):
    lib = nne.lib()
    lens = np.array([1], np.int32)
    lp = lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    # Hq not divisible by Hkv
    rc = lib.nne_decode_attention(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, 1, 6, 4, 8, 16,
                                  0, 0.0, None, None)
    assert rc == nne.NNE_EINVAL
    # head dim not a multiple of 4
    rc = lib.nne_decode_attention(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, 1, 4, 4, 8, 18,
                                  0, 0.0, None, None)
    assert rc == nne.NNE_EINVAL
    # head dim beyond 256 (the deep kernel): q must be a 16-byte vector view
    rc = lib.nne_decode_attention(ctypes.c_void_p(4096 + 4), None, FAKE, FAKE, FAKE, lp, FAKE,
                                  None, 1, 4, 4, 8, 260, 0, 0.0, None, None)
    assert rc == nne.NNE_EINVAL
    assert "16-byte" in lib.nne_last_error().decode()
    # length beyond capacity
    lens[0] = 9
    rc = lib.nne_decode_attention(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, 1, 4, 4, 8, 16,
                                  0, 0.0, None, None)
    assert rc == nne.NNE_EINVAL


def test_decode_workspace_size(nne):
    lib = nne.lib()
    assert lib.nne_decode_workspace_bytes(1, 4, 3, 64, 100) == 0   # 3 does not divide 4
    assert lib.nne_decode_workspace_bytes(1, 4, 4, 260, 100) == 0  # > 256, 4 tiles: no split
    assert lib.nne_decode_workspace_bytes(1, 4, 4, 30, 100) == 0   # head dim not a multiple of 4
    assert lib.nne_decode_workspace_bytes(1, 4, 4, 256, 100) > 0
    # any group size: rows beyond one launch's 64 go in further launches that
    # reuse the workspace, so 128 rows need what 64 need
    g64 = lib.nne_decode_workspace_bytes(1, 64, 1, 64, 100)
    assert g64 > 0 and lib.nne_decode_workspace_bytes(1, 128, 1, 64, 100) == g64
    # batches beyond 2048 sequences run 2048 at a time
    assert lib.nne_decode_workspace_bytes(5000, 8, 8, 64, 10) == \
        lib.nne_decode_workspace_bytes(2048, 8, 8, 64, 10)
    small = lib.nne_decode_workspace_bytes(2, 4, 2, 64, 4160)
    big = lib.nne_decode_workspace_bytes(32, 32, 8, 128, 4160)
    assert 0 < small < big
    # partial records for (workgroups + heads) slots of 4 rows x (128 + 2)
    # floats; one workgroup per CU (256 on MI355X, and the count assumed
    # where no device is visible)
    assert big >= (256 + 32 * 8) * 4 * 130 * 4


def test_decode_step_capacity_error_leaves_lengths(nne):
    lib = nne.lib()
    lens = np.array([3, 8], np.int32)
    lp = lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    rc = lib.nne_decode_step(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, FAKE, None, FAKE, None,
                             2, 4, 2, 8, 16, 0, 0.0, None, None)
    assert rc == nne.NNE_ECAPACITY
    assert list(lens) == [3, 8]


def test_python_mirror_rejects_non_4d(nne):
    import torch
    x = torch.zeros(2, 3, 4)
    with pytest.raises(nne.InvalidArgument):
        nne.flash_attention_forward(x, x, x, True)


def test_layer_divisibility_check(nne):
    with pytest.raises(nne.InvalidArgument):
        nne.FlashAttention(30, 4, True, device="cpu")


# ---------------------------------------------------------- decode prologue --

def test_rope_tables_are_the_reference_tables(nne):
    """nne_rope_tables runs on the host: bit-identical to the oracle's
    restatement of RotaryEmbedding::new (llama.rs:74-107)."""
    lib = nne.lib()
    for d, n, theta in [(64, 300, 10000.0), (128, 4096, 10000.0), (16, 5, 500000.0)]:
        cos = np.zeros((n, d), np.float32)
        sin = np.zeros((n, d), np.float32)
        assert lib.nne_rope_tables(cos.ctypes.data, sin.ctypes.data, n, d, theta) == nne.NNE_OK
        rc, rs = T.ref_rope_tables(n, d, theta)
        assert np.array_equal(cos, rc) and np.array_equal(sin, rs)


def test_rope_tables_reject_odd_head_dim(nne):
    lib = nne.lib()
    cos = np.zeros(16, np.float32)
    assert lib.nne_rope_tables(cos.ctypes.data, cos.ctypes.data, 2, 7, 10000.0) == nne.NNE_EINVAL
    assert "RoPE head_dim (7) must be even" in lib.nne_last_error().decode()


def test_rope_apply_host_checks(nne):
    lib = nne.lib()
    sp = np.array([0, 250], np.int32)
    # head dim differs from the table's: ShapeMismatch {expected [64], actual [32]} (:119-124)
    rc = lib.nne_rope_apply(FAKE, i64(2, 4, 8, 32), None, FAKE, None, FAKE, FAKE, 256, 64, FAKE,
                            sp.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), None)
    assert rc == nne.NNE_ESHAPE
    assert "expected shape [64], got [32]" in lib.nne_last_error().decode()
    # [250, 258) runs past max_seq_len 256 (:131-139)
    rc = lib.nne_rope_apply(FAKE, i64(2, 4, 8, 64), None, FAKE, None, FAKE, FAKE, 256, 64, FAKE,
                            sp.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), None)
    assert rc == nne.NNE_EINVAL
    assert "Sequence range [250, 258) exceeds RoPE max_seq_len 256" in lib.nne_last_error().decode()


def test_qkv_rope_host_checks(nne):
    lib = nne.lib()
    pos = np.array([3, 7], np.int32)
    pp = pos.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))

    def call(C=256, Hq=4, Hkv=2, d=64, table_d=64, max_len=8, x=FAKE, stride=256):
        return lib.nne_qkv_rope(x, stride, FAKE, None, None, None, FAKE, FAKE, max_len, table_d,
                                FAKE, pp, FAKE, FAKE, FAKE, 2, C, Hq, Hkv, d, None)

    assert call(table_d=128) == nne.NNE_ESHAPE
    assert call(d=48, table_d=48) == nne.NNE_EINVAL            # d % 64
    assert call(C=200, stride=200) == nne.NNE_EINVAL           # C % 64
    assert call(max_len=7) == nne.NNE_EINVAL                   # position 7 needs 8 rows
    assert "Sequence range [7, 8) exceeds RoPE max_seq_len 7" in lib.nne_last_error().decode()
    assert call(x=ctypes.c_void_p(4100)) == nne.NNE_EINVAL     # x rows not 16-byte aligned
    assert call(stride=200) == nne.NNE_EINVAL                  # row stride < d_model


def test_qkv_packed_bytes(nne):
    lib = nne.lib()
    assert lib.nne_qkv_packed_bytes(4096, 32, 8, 128) == 4 * 4096 * 48 * 128
    assert lib.nne_qkv_packed_bytes(768, 12, 12, 64) == 4 * 768 * 36 * 64
    assert lib.nne_qkv_packed_bytes(100, 4, 2, 64) == 0        # C % 64
    assert lib.nne_qkv_packed_bytes(256, 4, 2, 32) == 0        # d % 64
    assert lib.nne_qkv_pack(FAKE, FAKE, FAKE, FAKE, 256, 4, 2, 32, None) == nne.NNE_EINVAL


def test_decode_and_append_reject_null_device_pointers(nne):
    """A NULL device pointer with work to do is an InvalidArgument on the
    host, never a launch that would fault."""
    lib = nne.lib()
    lens = np.array([3, 4], np.int32)
    lp = lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    for bad in range(5):
        ptrs = [FAKE] * 5
        ptrs[bad] = None
        kc, vc, ld, kn, vn = ptrs
        assert lib.nne_kv_append(kc, vc, ld, lp, kn, None, vn, None, 2, 2, 16, 16, 1,
                                 None) == nne.NNE_EINVAL
        assert "null tensor pointer" in lib.nne_last_error().decode()
    assert list(lens) == [3, 4]
    for bad in range(7):
        ptrs = [FAKE] * 7
        ptrs[bad] = None
        q, kc, vc, ld, kn, vn, o = ptrs
        rc = lib.nne_decode_step(q, None, kc, vc, ld, lp, kn, None, vn, None, o, None, 2, 4, 2,
                                 16, 16, 0, 0.0, None, None)
        assert rc == nne.NNE_EINVAL, bad
    assert list(lens) == [3, 4]
    # attention only: q, caches, lengths and output
    for bad in range(5):
        ptrs = [FAKE] * 5
        ptrs[bad] = None
        q, kc, vc, ld, o = ptrs
        rc = lib.nne_decode_attention(q, None, kc, vc, ld, lp, o, None, 2, 4, 2, 16, 16, 0, 0.0,
                                      None, None)
        assert rc == nne.NNE_EINVAL, bad


def test_decode_16_row_tile_needs_vector_q(nne):
    """More than 4 query heads per KV head read q as 16-byte vectors: a
    misaligned q or strides that are not multiples of 4 are refused."""
    lib = nne.lib()
    lens = np.array([3], np.int32)
    lp = lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    misaligned = ctypes.c_void_p(4096 + 4)
    rc = lib.nne_decode_attention(misaligned, None, FAKE, FAKE, FAKE, lp, FAKE, None, 1, 8, 1, 16,
                                  16, 0, 0.0, None, None)
    assert rc == nne.NNE_EINVAL
    assert "16-byte alignment" in lib.nne_last_error().decode()
    odd = i64(8 * 16, 18, 16, 1)       # head stride 18 floats
    rc = lib.nne_decode_attention(FAKE, odd, FAKE, FAKE, FAKE, lp, FAKE, None, 1, 8, 1, 16, 16, 0,
                                  0.0, None, None)
    assert rc == nne.NNE_EINVAL


def test_workspace_size_queries(nne):
    """What each split computation needs from a caller workspace."""
    lib = nne.lib()
    size = nne.NneWorkspaceSize()
    # config 1 (4 work items on 256 CUs): key split, records and counters
    assert lib.nne_attention_workspace_size(i64(1, 4, 256, 64), i64(1, 4, 256, 64), 1, 0,
                                            ctypes.byref(size)) == nne.NNE_OK
    assert size.records_bytes > 0 and size.n_counters > 0
    # config 2 fills the device: no workspace
    assert lib.nne_attention_workspace_size(i64(4, 32, 2048, 128), i64(4, 8, 2048, 128), 1, 0,
                                            ctypes.byref(size)) == nne.NNE_OK
    assert (size.records_bytes, size.n_counters) == (0, 0)
    # few-query cross-attention: one counter per (sequence, KV head)
    assert lib.nne_attention_workspace_size(i64(8, 20, 8, 64), i64(8, 20, 1500, 64), 0, 0,
                                            ctypes.byref(size)) == nne.NNE_OK
    assert size.records_bytes > 0 and size.n_counters >= 8 * 20
    # 129-256 dims: d = 256 with the device full stays on the wave-pair kernel
    # (no workspace); a d = 192 prefill of few units takes the deep kernel's
    # key split: records only (4 heads x 2 units x 8 parts of 32 rows x
    # (512 + 2) floats, 256 CUs assumed without a device)
    assert lib.nne_attention_workspace_size(i64(1, 32, 2048, 256), i64(1, 8, 2048, 256), 1, 0,
                                            ctypes.byref(size)) == nne.NNE_OK
    assert (size.records_bytes, size.n_counters) == (0, 0)
    assert lib.nne_attention_workspace_size(i64(1, 4, 64, 192), i64(1, 4, 1500, 192), 0, 0,
                                            ctypes.byref(size)) == nne.NNE_OK
    assert (size.records_bytes, size.n_counters) == (8 * 8 * 32 * 514 * 4, 0)
    # shapes the call would refuse
    assert lib.nne_attention_workspace_size(i64(1, 6, 8, 16), i64(1, 4, 8, 16), 1, 0,
                                            ctypes.byref(size)) == nne.NNE_ESHAPE
    assert lib.nne_decode_workspace_size(32, 32, 8, 128, ctypes.byref(size)) == nne.NNE_OK
    assert size.n_counters == 32 * 8
    assert size.records_bytes == lib.nne_decode_workspace_bytes(32, 32, 8, 128, 4160)
    assert lib.nne_decode_workspace_size(1, 4, 4, 30, ctypes.byref(size)) == nne.NNE_EINVAL
    # above 256 dims: the records of the deep kernel's key split, no counters --
    # up to 8 parts of each (sequence, KV head) (8 pairs x 8 parts x 4 rows x
    # (512 + 2) floats), or for ragged lengths one record of 4 rows per CU
    # (256 CUs, the count assumed without a device); none for a batch too
    # large for either split
    assert lib.nne_decode_workspace_size(4, 8, 2, 512, ctypes.byref(size)) == nne.NNE_OK
    assert (size.records_bytes, size.n_counters) == (max(8 * 8, 256) * 4 * 514 * 4, 0)
    assert lib.nne_decode_workspace_bytes(4, 8, 2, 512, 100) == 0     # 4 tiles: no split
    assert lib.nne_decode_workspace_size(1024, 8, 2, 512, ctypes.byref(size)) == nne.NNE_OK
    assert (size.records_bytes, size.n_counters) == (0, 0)
    assert lib.nne_decode_workspace_size(4, 8, 3, 512, ctypes.byref(size)) == nne.NNE_EINVAL
    assert lib.nne_qkv_workspace_size(4096, 32, 8, 128, ctypes.byref(size)) == nne.NNE_OK
    assert size.records_bytes > 0 and size.n_counters == 48 * 128 // 64
    assert lib.nne_qkv_workspace_size(100, 4, 2, 64, ctypes.byref(size)) == nne.NNE_EINVAL


def test_undersized_caller_workspace_is_refused_before_launch(nne):
    lib = nne.lib()
    lens = np.array([3, 5], np.int32)
    lp = lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    small = nne.NneWorkspace(records=4096, records_bytes=64, counters=4096, n_counters=16)
    rc = lib.nne_decode_step(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, FAKE, None, FAKE, None,
                             2, 4, 2, 16, 16, 0, 0.0, ctypes.byref(small), None)
    assert rc == nne.NNE_EINVAL
    assert "record bytes" in lib.nne_last_error().decode()
    assert list(lens) == [3, 5]
    few = nne.NneWorkspace(records=4096, records_bytes=1 << 30, counters=4096, n_counters=1)
    rc = lib.nne_decode_attention(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, 2, 4, 2, 16, 16,
                                  0, 0.0, ctypes.byref(few), None)
    assert rc == nne.NNE_EINVAL
    assert "counters" in lib.nne_last_error().decode()


def test_misaligned_caller_workspace_is_refused_before_launch(nne):
    lib = nne.lib()
    lens = np.array([3, 5], np.int32)
    lp = lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    for rec, cnt in ((4096 + 8, 4096), (4096, 4096 + 2)):
        ws = nne.NneWorkspace(records=rec, records_bytes=1 << 30, counters=cnt, n_counters=1 << 20)
        rc = lib.nne_decode_step(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, FAKE, None, FAKE,
                                 None, 2, 4, 2, 16, 16, 0, 0.0, ctypes.byref(ws), None)
        assert rc == nne.NNE_EINVAL
        assert "aligned" in lib.nne_last_error().decode()
        assert list(lens) == [3, 5]


def test_integration_build_lists_every_source():
    """The Rust build script in INTEGRATION.md compiles the same sources as
    neural-network-engine_amd/build.py (a missing one would leave symbols
    undefined at link time)."""
    import os
    import re
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    build_py = open(os.path.join(root, "neural-network-engine_amd", "build.py")).read()
    sources = re.search(r"^SOURCES = \[(.*)\]$", build_py, re.M).group(1)
    sources = re.findall(r'"([^"]+)"', sources)
    doc = open(os.path.join(root, "INTEGRATION.md")).read()
    args = re.search(r'\.args\(\[("prefill\.hip"[^\]]*)\]', doc).group(1)
    assert re.findall(r'"([^"]+)"', args) == sources
    for s in sources:
        assert "csrc/" + s in doc.split("## 1.")[0], s


def test_integration_declares_every_entry_point():
    """INTEGRATION.md's `lib.rs` declares each function of include/nne_attn.h
    once, and nothing else."""
    import os
    import re
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    header = open(os.path.join(root, "include", "nne_attn.h")).read()
    declared = set(re.findall(r"\b(nne_[a-z0-9_]+)\s*\(", header))
    doc = open(os.path.join(root, "INTEGRATION.md")).read()
    bound = re.findall(r"pub fn (nne_[a-z0-9_]+)\s*\(", doc)
    assert len(bound) == len(set(bound))
    assert set(bound) == declared
