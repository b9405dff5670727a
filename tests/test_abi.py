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
    assert lib.nne_abi_version() == 1


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


def test_head_dim_too_large_is_invalid_argument(nne):
    lib = nne.lib()
    s = i64(1, 1, 4, 256)
    rc = lib.nne_flash_attention_forward(FAKE, s, None, FAKE, s, None, FAKE, s, None, FAKE, None,
                                         0, 0, 0.0, 64, 64, None)
    assert rc == nne.NNE_EINVAL
    assert "head dim" in lib.nne_last_error().decode()


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
                                  0, 0.0, None, 0, None)
    assert rc == nne.NNE_EINVAL
    # head dim not a multiple of 4
    rc = lib.nne_decode_attention(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, 1, 4, 4, 8, 18,
                                  0, 0.0, None, 0, None)
    assert rc == nne.NNE_EINVAL
    # more than 16 query rows per KV head
    rc = lib.nne_decode_attention(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, 1, 32, 1, 8, 16,
                                  0, 0.0, None, 0, None)
    assert rc == nne.NNE_EINVAL
    # length beyond capacity
    lens[0] = 9
    rc = lib.nne_decode_attention(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, 1, 4, 4, 8, 16,
                                  0, 0.0, None, 0, None)
    assert rc == nne.NNE_EINVAL


def test_decode_workspace_size(nne):
    lib = nne.lib()
    assert lib.nne_decode_workspace_bytes(1, 4, 3, 64, 100) == 0   # 3 does not divide 4
    assert lib.nne_decode_workspace_bytes(1, 4, 4, 256, 100) == 0  # head dim > 128
    assert lib.nne_decode_workspace_bytes(1, 32, 1, 64, 100) == 0  # 32 rows per KV head > 16
    small = lib.nne_decode_workspace_bytes(2, 4, 2, 64, 4160)
    big = lib.nne_decode_workspace_bytes(32, 32, 8, 128, 4160)
    assert 0 < small < big
    # partial records for (workgroups + heads) slots of 4 rows x (128 + 2) floats
    assert big >= (2048 + 32 * 8) * 4 * 130 * 4


def test_decode_step_capacity_error_leaves_lengths(nne):
    lib = nne.lib()
    lens = np.array([3, 8], np.int32)
    lp = lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    rc = lib.nne_decode_step(FAKE, None, FAKE, FAKE, FAKE, lp, FAKE, None, FAKE, None, FAKE, None,
                             2, 4, 2, 8, 16, 0, 0.0, None, 0, None)
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
