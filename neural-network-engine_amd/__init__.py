"""Python host mirror of the MI355X attention hot path.

Binds the C ABI of lib/libnne_attn.so (declared in include/nne_attn.h) with
ctypes and exposes it with the names and argument meanings of the reference
engine's attention API (elvin-mark/neural-network-engine):

* ``flash_attention_forward(q, k, v, is_causal, scale, block_size_r,
  block_size_c)``  -- src/nn/flash_attention.rs:19-199
* ``attention_forward(q, k, v, is_causal, q_offset, scale)`` -- the GQA /
  offset generalisation behind GroupedQueryAttention (src/models/llama.rs:253-296)
  and MultiHeadAttention (src/nn/attention.rs:51-210)
* ``KVCache`` -- src/nn/kv_cache.rs:11-74, stored on the device head-major
  and appended in place
* ``FlashAttention`` layer -- src/nn/flash_attention.rs:202-292
* ``RotaryEmbedding`` -- src/models/llama.rs:64-158
* ``qkv_rope`` -- the fused decode prologue (q/k/v projections + RoPE) of
  GroupedQueryAttention::forward_gqa_cached (llama.rs:226-235)
* ``GroupedQueryAttention`` -- src/models/llama.rs:160-300
* ``MultiHeadAttention`` -- src/nn/attention.rs:9-210 (GPT-2 / Whisper self- and
  cross-attention) and ``WhisperKVCache`` -- src/models/whisper.rs:325-350

Tensors are torch tensors on the GPU (torch is used only for device memory and
streams).  Errors raise the EngineError variant the reference would return.
There is no CPU path: if the HIP library is missing, importing works but every
call raises.
"""
import ctypes
import math
import os

import numpy as np

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libnne_attn.so")

NNE_OK, NNE_EINVAL, NNE_ESHAPE, NNE_ECAPACITY, NNE_EHIP = 0, 1, 2, 3, 4


class EngineError(RuntimeError):
    """Base of the reference's error enum (src/error.rs:9-52)."""


class InvalidArgument(EngineError):
    pass


class ShapeMismatch(EngineError):
    pass


class GpuError(EngineError):
    pass


class CapacityError(GpuError):
    pass


_ERRORS = {NNE_EINVAL: InvalidArgument, NNE_ESHAPE: ShapeMismatch,
           NNE_ECAPACITY: CapacityError, NNE_EHIP: GpuError}

_lib = None

_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p


class NneWorkspace(ctypes.Structure):
    """nne_workspace_t: caller-owned records buffer and zeroed counters."""
    _fields_ = [("records", ctypes.c_void_p), ("records_bytes", ctypes.c_uint64),
                ("counters", ctypes.c_void_p), ("n_counters", ctypes.c_uint64)]


class NneWorkspaceSize(ctypes.Structure):
    """nne_workspace_size_t."""
    _fields_ = [("records_bytes", ctypes.c_uint64), ("n_counters", ctypes.c_uint64)]


_wsp = ctypes.POINTER(NneWorkspace)
_wszp = ctypes.POINTER(NneWorkspaceSize)

# exported symbol -> (restype, argtypes); mirrors include/nne_attn.h
SIGNATURES = {
    "nne_abi_version": (ctypes.c_int, []),
    "nne_last_error": (ctypes.c_char_p, []),
    "nne_dev_alloc": (ctypes.c_int, [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint64]),
    "nne_dev_free": (ctypes.c_int, [_vp]),
    "nne_memcpy_h2d": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64, _vp]),
    "nne_memcpy_d2h": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64, _vp]),
    "nne_memcpy_d2d": (ctypes.c_int, [_vp, _vp, ctypes.c_uint64, _vp]),
    "nne_stream_sync": (ctypes.c_int, [_vp]),
    "nne_stream_release": (ctypes.c_int, [_vp]),
    "nne_stream_resource_bytes": (ctypes.c_uint64, [_vp]),
    "nne_counters_init": (ctypes.c_int, [_vp, ctypes.c_uint64, _vp]),
    "nne_flash_attention_forward": (ctypes.c_int, [
        _vp, _i64p, _i64p, _vp, _i64p, _i64p, _vp, _i64p, _i64p, _vp, _i64p,
        ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int64, ctypes.c_int64, _vp]),
    "nne_attention_forward": (ctypes.c_int, [
        _vp, _i64p, _i64p, _vp, _i64p, _i64p, _vp, _i64p, _i64p, _vp, _i64p,
        ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_float, _vp]),
    "nne_flash_attention_forward_ws": (ctypes.c_int, [
        _vp, _i64p, _i64p, _vp, _i64p, _i64p, _vp, _i64p, _i64p, _vp, _i64p,
        ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int64, ctypes.c_int64, _wsp, _vp]),
    "nne_attention_forward_ws": (ctypes.c_int, [
        _vp, _i64p, _i64p, _vp, _i64p, _i64p, _vp, _i64p, _i64p, _vp, _i64p,
        ctypes.c_int, ctypes.c_int64, ctypes.c_int, ctypes.c_float, _wsp, _vp]),
    "nne_attention_workspace_size": (ctypes.c_int, [_i64p, _i64p, ctypes.c_int, ctypes.c_int64,
                                                    _wszp]),
    "nne_kv_append": (ctypes.c_int, [
        _vp, _vp, _vp, _i32p, _vp, _i64p, _vp, _i64p, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _vp]),
    "nne_decode_workspace_bytes": (ctypes.c_uint64, [
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]),
    "nne_decode_workspace_size": (ctypes.c_int, [
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _wszp]),
    "nne_decode_attention": (ctypes.c_int, [
        _vp, _i64p, _vp, _vp, _vp, _i32p, _vp, _i64p, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_float, _wsp,
        _vp]),
    "nne_decode_step": (ctypes.c_int, [
        _vp, _i64p, _vp, _vp, _vp, _i32p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int, ctypes.c_float, _wsp, _vp]),
    "nne_decode_step_noalloc": (ctypes.c_int, [
        _vp, _i64p, _vp, _vp, _vp, _i32p, _vp, _i64p, _vp, _i64p, _vp, _i64p,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int, ctypes.c_float, _vp]),
    "nne_rope_tables": (ctypes.c_int, [_vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_float]),
    "nne_rope_apply": (ctypes.c_int, [
        _vp, _i64p, _i64p, _vp, _i64p, _vp, _vp, ctypes.c_int64, ctypes.c_int64, _vp, _i32p,
        _vp]),
    "nne_qkv_packed_bytes": (ctypes.c_uint64, [
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]),
    "nne_qkv_pack": (ctypes.c_int, [
        _vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _vp]),
    "nne_qkv_rope": (ctypes.c_int, [
        _vp, ctypes.c_int64, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int64,
        ctypes.c_int64, _vp, _i32p, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _vp]),
    "nne_qkv_workspace_size": (ctypes.c_int, [
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _wszp]),
    "nne_qkv_rope_ws": (ctypes.c_int, [
        _vp, ctypes.c_int64, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int64,
        ctypes.c_int64, _vp, _i32p, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64,
        ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _wsp, _vp]),
}


def lib():
    """The loaded HIP library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise GpuError("HIP attention library not built: %s is missing "
                           "(run neural-network-engine_amd/build.py)" % LIB_PATH)
        l = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _lib = l
    return _lib


def check(rc):
    if rc != NNE_OK:
        msg = lib().nne_last_error().decode(errors="replace")
        raise _ERRORS.get(rc, EngineError)(msg)


def _i64(vals):
    arr = (ctypes.c_int64 * 4)(*[int(x) for x in vals])
    return arr


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def release_stream(stream=None):
    """Frees the workspace and counters the library keeps for ``stream``
    (default: the current stream) after waiting for it; the next call on the
    stream allocates them again."""
    check(lib().nne_stream_release(_stream(stream)))


def stream_resource_bytes(stream=None):
    """Bytes the library holds for ``stream`` (0 when every call on it
    brought its own workspace)."""
    return int(lib().nne_stream_resource_bytes(_stream(stream)))


class Workspace:
    """A caller-owned workspace (nne_workspace_t): a records buffer and an
    array of arrival counters zeroed once (every call leaves them zeroed),
    both torch tensors on ``device``, grown on demand by ``reserve``.  One
    workspace serves every entry point; calls that share it must not overlap
    in time (calls on one stream never do)."""

    def __init__(self, device="cuda"):
        self.device = device
        self.records = None
        self.counters = None

    def reserve(self, size, stream=None):
        """Grows the buffers to at least ``size`` (an NneWorkspaceSize)."""
        import torch
        if size.records_bytes and (self.records is None or
                                   self.records.numel() < size.records_bytes):
            self.records = torch.empty(int(size.records_bytes), dtype=torch.uint8,
                                       device=self.device)
        if size.n_counters and (self.counters is None or
                                self.counters.numel() < size.n_counters):
            self.counters = torch.empty(int(size.n_counters), dtype=torch.int32,
                                        device=self.device)
            check(lib().nne_counters_init(self.counters.data_ptr(), self.counters.numel(),
                                          _stream(stream)))
        return self

    def struct(self):
        w = NneWorkspace()
        if self.records is not None:
            w.records, w.records_bytes = self.records.data_ptr(), self.records.numel()
        if self.counters is not None:
            w.counters, w.n_counters = self.counters.data_ptr(), self.counters.numel()
        return ctypes.byref(w), w


def _ws_arg(workspace, size, stream):
    """(pointer argument, keep-alive) for an optional Workspace."""
    if workspace is None:
        return None, None
    workspace.reserve(size, stream)
    return workspace.struct()


def _require_f32_cuda(*ts):
    import torch
    for t in ts:
        if not t.is_cuda or t.dtype != torch.float32:
            raise InvalidArgument("Invalid configuration or argument: expected float32 GPU tensors")


def _shape4(t, what):
    if t.dim() != 4:
        raise InvalidArgument(
            "Invalid configuration or argument: FlashAttention expects 4D tensors "
            "[Batch, Heads, SeqLen, Dim], got %s:%s" % (what, list(t.shape)))
    return t.shape, t.stride()


def attention_workspace_size(q_shape, k_shape, is_causal, q_offset=0):
    size = NneWorkspaceSize()
    check(lib().nne_attention_workspace_size(_i64(q_shape), _i64(k_shape), int(bool(is_causal)),
                                             int(q_offset), ctypes.byref(size)))
    return size


def flash_attention_forward(q, k, v, is_causal, scale=None, block_size_r=64, block_size_c=64,
                            out=None, stream=None, workspace=None):
    """flash_attention_forward (src/nn/flash_attention.rs:19-199) on the GPU.

    q, k, v: float32 CUDA tensors [B, H, T, d] with any strides.  Returns a new
    contiguous [B, H, Tq, d] tensor (or fills ``out``).  ``workspace``: a
    Workspace the call uses instead of the library's per-stream one."""
    import torch
    qs, qst = _shape4(q, "Q")
    ks, kst = _shape4(k, "K")
    vs, vst = _shape4(v, "V")
    _require_f32_cuda(q, k, v)
    if out is None:
        out = torch.empty(tuple(qs), dtype=torch.float32, device=q.device)
    wsp, keep = None, None
    if workspace is not None and qs[1] == ks[1]:
        wsp, keep = _ws_arg(workspace, attention_workspace_size(qs, ks, is_causal), stream)
    check(lib().nne_flash_attention_forward_ws(
        q.data_ptr(), _i64(qs), _i64(qst), k.data_ptr(), _i64(ks), _i64(kst),
        v.data_ptr(), _i64(vs), _i64(vst), out.data_ptr(), _i64(out.stride()),
        int(bool(is_causal)), int(scale is not None), float(scale or 0.0),
        int(block_size_r), int(block_size_c), wsp, _stream(stream)))
    return out


def attention_forward(q, k, v, is_causal, q_offset=0, scale=None, out=None, stream=None,
                      workspace=None):
    """GQA-capable attention: q [B, Hq, Tq, d], k/v [B, Hkv, Tk, d], Hkv | Hq.

    Query head hq reads KV head hq // (Hq // Hkv) (src/models/llama.rs:256-266);
    with is_causal, key c is visible to row r iff c <= r + q_offset.
    ``workspace``: a Workspace the call uses instead of the library's
    per-stream one."""
    import torch
    qs, qst = _shape4(q, "Q")
    ks, kst = _shape4(k, "K")
    vs, vst = _shape4(v, "V")
    _require_f32_cuda(q, k, v)
    if out is None:
        out = torch.empty(tuple(qs), dtype=torch.float32, device=q.device)
    wsp, keep = None, None
    if workspace is not None:
        wsp, keep = _ws_arg(workspace, attention_workspace_size(qs, ks, is_causal, q_offset),
                            stream)
    check(lib().nne_attention_forward_ws(
        q.data_ptr(), _i64(qs), _i64(qst), k.data_ptr(), _i64(ks), _i64(kst),
        v.data_ptr(), _i64(vs), _i64(vst), out.data_ptr(), _i64(out.stride()),
        int(bool(is_causal)), int(q_offset), int(scale is not None), float(scale or 0.0),
        wsp, _stream(stream)))
    return out


class _LayerSlots:
    """``KVCache.layers`` -- the reference's ``pub layers:
    Vec<Option<(Tensor, Tensor)>>`` (kv_cache.rs:13) over the device cache.
    Item i is None or (K, V) views [B, Hkv, L, d] of the filled rows
    (L = the longest sequence), materialised when read, with no copy.
    Assigning None empties the layer; assigning (k, v) [B, Hkv, L, d] makes
    them its rows 0..L (zero-element k, v give an engaged, empty slot, as
    llama.rs:501-503 sets up before the prompt)."""

    def __init__(self, cache):
        self._c = cache

    def __len__(self):
        return self._c.num_layers()

    def _index(self, i):
        n = len(self)
        i = i + n if i < 0 else i
        if not 0 <= i < n:
            raise IndexError("KVCache layer index %d out of range (total layers: %d)" % (i, n))
        return i

    def __getitem__(self, i):
        c = self._c
        i = self._index(i)
        if not c._engaged[i]:
            return None
        L = c.current_seq_len(i)
        return c.k[i][:, :, :L], c.v[i][:, :, :L]

    def __setitem__(self, i, kv):
        c = self._c
        i = self._index(i)
        if kv is not None:
            k, v = kv
            if k.numel() or v.numel():
                want = [c.batch, c.num_kv_heads, k.shape[2] if k.dim() == 4 else 0, c.head_dim]
                if list(k.shape) != want or list(v.shape) != want:
                    raise ShapeMismatch("Shape mismatch error: expected shape %s, got %s"
                                        % (want, list(k.shape)))
                if want[2] > c.capacity:
                    raise CapacityError("GPU compute error: KV cache slot of %d rows exceeds "
                                        "capacity %d" % (want[2], c.capacity))
        c.lens_dev[i].zero_()
        c.lens_host[i][:] = 0
        c._engaged[i] = False
        if kv is not None:
            if kv[0].numel():
                c.update(i, kv[0], kv[1])
            c._engaged[i] = True

    def __iter__(self):
        return (self[i] for i in range(len(self)))


class KVCache:
    """Device-resident KV cache (src/nn/kv_cache.rs:11-74).

    Per layer: K and V buffers [B, Hkv, capacity, d] (head-major, rows appended
    in place) and per-sequence lengths kept on the device (read by kernels) and
    on the host (validation, launch sizing).  Sequences may be ragged.
    ``layers`` is the reference's per-layer slot vector over these buffers.
    With own_workspace=False the decode calls pass no workspace and run on the
    library's per-stream one instead of the cache's."""

    def __init__(self, num_layers, batch, num_kv_heads, capacity, head_dim, device="cuda",
                 own_workspace=True):
        import torch
        self.batch, self.num_kv_heads = int(batch), int(num_kv_heads)
        self.capacity, self.head_dim = int(capacity), int(head_dim)
        shape = (self.batch, self.num_kv_heads, self.capacity, self.head_dim)
        self.k = [torch.zeros(shape, dtype=torch.float32, device=device) for _ in range(num_layers)]
        self.v = [torch.zeros(shape, dtype=torch.float32, device=device) for _ in range(num_layers)]
        self.lens_dev = [torch.zeros(self.batch, dtype=torch.int32, device=device)
                         for _ in range(num_layers)]
        self.lens_host = [np.zeros(self.batch, dtype=np.int32) for _ in range(num_layers)]
        self._ws = Workspace(device) if own_workspace else None
        self._engaged = [False] * num_layers    # Some(..) in the reference's slot vector

    @property
    def layers(self):
        return _LayerSlots(self)

    # kv_cache.rs:25-29
    def reset(self):
        for i in range(self.num_layers()):
            self.lens_dev[i].zero_()
            self.lens_host[i][:] = 0
            self._engaged[i] = False

    # kv_cache.rs:32-34
    def num_layers(self):
        return len(self.k)

    # kv_cache.rs:37-44 (0 for an out-of-range layer; with ragged sequences the
    # longest one)
    def current_seq_len(self, layer_idx):
        if layer_idx >= self.num_layers():
            return 0
        return int(self.lens_host[layer_idx].max()) if self.batch else 0

    def set_lengths(self, layer_idx, lens):
        """Declares that rows [0, lens[b]) of each sequence are filled."""
        import torch
        lens = np.asarray(lens, dtype=np.int32)
        if lens.shape != (self.batch,) or (lens < 0).any() or (lens > self.capacity).any():
            raise InvalidArgument("Invalid configuration or argument: bad lengths")
        self.lens_host[layer_idx][:] = lens
        self.lens_dev[layer_idx].copy_(torch.from_numpy(lens))
        self._engaged[layer_idx] = True

    def _check_layer(self, layer_idx):
        if layer_idx >= self.num_layers():
            raise InvalidArgument(
                "Invalid configuration or argument: KVCache layer index %d out of range "
                "(total layers: %d)" % (layer_idx, self.num_layers()))

    # kv_cache.rs:49-74: append along the sequence axis; returns views of all rows
    def update(self, layer_idx, k_new, v_new, stream=None):
        self._check_layer(layer_idx)
        _require_f32_cuda(k_new, v_new)
        b, h, t, d = k_new.shape
        if (b, h, d) != (self.batch, self.num_kv_heads, self.head_dim) or v_new.shape != k_new.shape:
            raise ShapeMismatch("Shape mismatch error: expected shape %s, got %s" % (
                [self.batch, self.num_kv_heads, t, self.head_dim], list(k_new.shape)))
        lh = self.lens_host[layer_idx]
        check(lib().nne_kv_append(
            self.k[layer_idx].data_ptr(), self.v[layer_idx].data_ptr(),
            self.lens_dev[layer_idx].data_ptr(), lh.ctypes.data_as(_i32p),
            k_new.data_ptr(), _i64(k_new.stride()), v_new.data_ptr(), _i64(v_new.stride()),
            self.batch, self.num_kv_heads, self.capacity, self.head_dim, t, _stream(stream)))
        self._engaged[layer_idx] = True
        L = int(lh.max()) if self.batch else 0
        return self.k[layer_idx][:, :, :L], self.v[layer_idx][:, :, :L]

    def workspace(self, num_heads, stream=None):
        """The cache's own decode workspace (records and zeroed counters),
        grown to what num_heads query heads need: (pointer argument,
        keep-alive).  The library allocates nothing for these calls."""
        if self._ws is None:
            return None, None      # the library's per-stream workspace
        size = NneWorkspaceSize()
        rc = lib().nne_decode_workspace_size(self.batch, num_heads, self.num_kv_heads,
                                             self.head_dim, ctypes.byref(size))
        if rc != NNE_OK:
            return None, None      # the call itself reports the geometry error
        self._ws.reserve(size, stream)
        return self._ws.struct()

    def attend(self, layer_idx, q, out=None, scale=None, stream=None):
        """Decode attention of q [B, Hq, 1, d] over the cached rows."""
        import torch
        self._check_layer(layer_idx)
        _require_f32_cuda(q)
        hq = q.shape[1]
        if out is None:
            out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
        wsp, keep = self.workspace(hq, stream)
        check(lib().nne_decode_attention(
            q.data_ptr(), _i64(q.stride()), self.k[layer_idx].data_ptr(),
            self.v[layer_idx].data_ptr(), self.lens_dev[layer_idx].data_ptr(),
            self.lens_host[layer_idx].ctypes.data_as(_i32p), out.data_ptr(), _i64(out.stride()),
            self.batch, hq, self.num_kv_heads, self.capacity, self.head_dim,
            int(scale is not None), float(scale or 0.0), wsp, _stream(stream)))
        return out

    def decode_step(self, layer_idx, q, k_new, v_new, out=None, scale=None, stream=None):
        """Append one row per sequence, then attend (llama.rs:239-296, t = 1).

        Every sequence attends to its own rows only, whatever the other
        sequences' lengths.  Geometries the fused decode kernel does not take
        (a head dim that is not a multiple of 4) append with the append kernel
        and attend with the attention kernel, one call per distinct length."""
        import torch
        self._check_layer(layer_idx)
        _require_f32_cuda(q, k_new, v_new)
        hq = q.shape[1]
        if out is None:
            out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
        if not decode_kernel_fits(self.batch, hq, self.num_kv_heads, self.head_dim):
            return self._append_then_attend(layer_idx, q, k_new, v_new, out, scale, stream)
        wsp, keep = self.workspace(hq, stream)
        check(lib().nne_decode_step(
            q.data_ptr(), _i64(q.stride()), self.k[layer_idx].data_ptr(),
            self.v[layer_idx].data_ptr(), self.lens_dev[layer_idx].data_ptr(),
            self.lens_host[layer_idx].ctypes.data_as(_i32p), k_new.data_ptr(),
            _i64(k_new.stride()), v_new.data_ptr(), _i64(v_new.stride()), out.data_ptr(),
            _i64(out.stride()), self.batch, hq, self.num_kv_heads, self.capacity, self.head_dim,
            int(scale is not None), float(scale or 0.0), wsp, _stream(stream)))
        self._engaged[layer_idx] = True
        return out

    def _append_then_attend(self, layer_idx, q, k_new, v_new, out, scale, stream):
        # The same semantics as decode_step on the general kernels: append,
        # then attend sequence b to its first lens[b] rows (no mask for t = 1,
        # llama.rs:277), batching the sequences that share a length.
        self.update(layer_idx, k_new, v_new, stream=stream)
        lens = self.lens_host[layer_idx]
        kl, vl = self.k[layer_idx], self.v[layer_idx]
        for L in np.unique(lens):
            idx = np.nonzero(lens == L)[0]
            if len(idx) == self.batch:
                attention_forward(q, kl[:, :, :L], vl[:, :, :L], False, scale=scale, out=out,
                                  stream=stream, workspace=self._ws)
                break
            for bi in idx:
                bi = int(bi)
                attention_forward(q[bi:bi + 1], kl[bi:bi + 1, :, :L], vl[bi:bi + 1, :, :L], False,
                                  scale=scale, out=out[bi:bi + 1], stream=stream,
                                  workspace=self._ws)
        return out


def decode_kernel_fits(batch, num_heads, num_kv_heads, head_dim):
    """True when the decode step entry point takes this geometry (the library's
    decode workspace query accepts it)."""
    size = NneWorkspaceSize()
    return lib().nne_decode_workspace_size(max(int(batch), 1), int(num_heads),
                                           int(num_kv_heads), int(head_dim),
                                           ctypes.byref(size)) == NNE_OK


class FlashAttention:
    """FlashAttention layer (src/nn/flash_attention.rs:202-292), forward only.

    The four d_model x d_model projections are plain GEMMs (torch); the
    attention core runs on the HIP kernel and reads the projected [B, T, H, d]
    activations through strides, so no transpose copies are made."""

    def __init__(self, d_model, num_heads, is_causal, device="cuda", seed=0):
        import torch
        if d_model % num_heads != 0:
            raise InvalidArgument("d_model (%d) must be divisible by num_heads (%d)"
                                  % (d_model, num_heads))
        self.d_model, self.num_heads = d_model, num_heads
        self.head_dim = d_model // num_heads
        self.is_causal = is_causal
        self.block_size = 64
        g = torch.Generator(device="cpu").manual_seed(seed)
        bound = 1.0 / math.sqrt(d_model)

        def lin():
            w = (torch.rand(d_model, d_model, generator=g) * 2 - 1) * bound
            b = (torch.rand(d_model, generator=g) * 2 - 1) * bound
            return w.to(device), b.to(device)

        self.q_proj, self.k_proj, self.v_proj, self.out_proj = lin(), lin(), lin(), lin()

    def forward(self, x):
        import torch
        if x.dim() != 3:
            raise EngineError("Incompatible shapes for operation FlashAttention forward "
                              "(expected 3D input [B, T, C]): %s" % [list(x.shape)])
        b, t, _ = x.shape
        h, d = self.num_heads, self.head_dim
        q = torch.nn.functional.linear(x, *self.q_proj).view(b, t, h, d).transpose(1, 2)
        k = torch.nn.functional.linear(x, *self.k_proj).view(b, t, h, d).transpose(1, 2)
        v = torch.nn.functional.linear(x, *self.v_proj).view(b, t, h, d).transpose(1, 2)
        out = torch.empty((b, t, h, d), dtype=torch.float32, device=x.device)
        flash_attention_forward(q, k, v, self.is_causal, None, self.block_size, self.block_size,
                                out=out.transpose(1, 2))
        return torch.nn.functional.linear(out.view(b, t, self.d_model), *self.out_proj)

    __call__ = forward


class RotaryEmbedding:
    """RotaryEmbedding (src/models/llama.rs:64-158).

    The cos/sin tables are computed on the host in f32 exactly as the
    reference's ``new`` (:74-107) and kept on the device; ``apply`` rotates a
    [B, H, T, d] tensor on the GPU with the reference's roundings."""

    def __init__(self, head_dim, max_seq_len, theta=10000.0, device="cuda"):
        import torch
        self.head_dim, self.max_seq_len = int(head_dim), int(max_seq_len)
        cos = np.zeros((max(self.max_seq_len, 0), max(self.head_dim, 0)), np.float32)
        sin = np.zeros_like(cos)
        check(lib().nne_rope_tables(cos.ctypes.data, sin.ctypes.data, self.max_seq_len,
                                    self.head_dim, float(theta)))
        self.cos_host, self.sin_host = cos, sin
        self.cos = torch.from_numpy(cos).to(device)
        self.sin = torch.from_numpy(sin).to(device)

    def _starts(self, start_pos, b, device):
        import torch
        sp = np.ascontiguousarray(np.broadcast_to(np.asarray(start_pos, np.int32), (b,)))
        return sp, torch.from_numpy(sp.copy()).to(device)

    def apply(self, x, start_pos, out=None, stream=None):
        """x [B, H, T, d] (any strides); row t of sequence b uses position
        start_pos[b] + t (start_pos: an int or B ints).  Returns ``out``
        (a new contiguous tensor by default; may be ``x`` itself)."""
        import torch
        if x.dim() != 4:
            raise InvalidArgument(
                "Invalid configuration or argument: RoPE apply expects 4D tensor [Batch, Heads, "
                "SeqLen, HeadDim], got rank %d with shape %s" % (x.dim(), list(x.shape)))
        _require_f32_cuda(x)
        if out is None:
            out = torch.empty(tuple(x.shape), dtype=torch.float32, device=x.device)
        sp_h, sp_d = self._starts(start_pos, x.shape[0], x.device)
        check(lib().nne_rope_apply(
            x.data_ptr(), _i64(x.shape), _i64(x.stride()), out.data_ptr(), _i64(out.stride()),
            self.cos.data_ptr(), self.sin.data_ptr(), self.max_seq_len, self.head_dim,
            sp_d.data_ptr(), sp_h.ctypes.data_as(_i32p), _stream(stream)))
        return out


def qkv_pack(wq, wk, wv, num_heads, num_kv_heads, stream=None):
    """Packs q_proj / k_proj / v_proj weights ([H * d, C]) for ``qkv_rope``
    (once per layer: the weights are static)."""
    import torch
    _require_f32_cuda(wq, wk, wv)
    c = wq.shape[1]
    d = wq.shape[0] // num_heads
    nbytes = lib().nne_qkv_packed_bytes(c, num_heads, num_kv_heads, d)
    if nbytes == 0:
        raise InvalidArgument("Invalid configuration or argument: the fused projection needs a "
                              "head dim and a d_model that are multiples of 64")
    packed = torch.empty(int(nbytes) // 4, dtype=torch.float32, device=wq.device)
    check(lib().nne_qkv_pack(wq.contiguous().data_ptr(), wk.contiguous().data_ptr(),
                             wv.contiguous().data_ptr(), packed.data_ptr(), c, num_heads,
                             num_kv_heads, d, _stream(stream)))
    return packed


def qkv_rope(x, w_packed, bq, bk, bv, rope, pos_dev, pos_host, num_heads, num_kv_heads,
             q_out=None, k_out=None, v_out=None, stream=None, head_dim=None, workspace=None):
    """Fused decode prologue: x [B, C] (or [B, 1, C]) -> q [B, Hq, 1, d] and
    k, v [B, Hkv, 1, d] with q = RoPE(x Wq^T + bq), k = RoPE(x Wk^T + bk),
    v = x Wv^T + bv at positions pos (int32, device and host copies);
    ``w_packed`` comes from ``qkv_pack``.  With rope=None nothing is rotated
    (the MultiHeadAttention projections) and ``head_dim`` gives d.
    ``workspace``: a Workspace the call uses instead of the library's
    per-stream one."""
    import torch
    x2 = x.reshape(x.shape[0], x.shape[-1]) if x.dim() == 3 else x
    _require_f32_cuda(x2, w_packed)
    b, c = x2.shape
    d = rope.head_dim if rope is not None else int(head_dim)
    dev = x2.device
    if q_out is None:
        q_out = torch.empty((b, num_heads, 1, d), dtype=torch.float32, device=dev)
    if k_out is None:
        k_out = torch.empty((b, num_kv_heads, 1, d), dtype=torch.float32, device=dev)
    if v_out is None:
        v_out = torch.empty((b, num_kv_heads, 1, d), dtype=torch.float32, device=dev)
    def ptr(t):
        return None if t is None else t.data_ptr()

    for t in (q_out, k_out, v_out):
        if not t.is_contiguous():
            raise InvalidArgument("Invalid configuration or argument: outputs must be contiguous")
    if rope is not None:
        pos_host = np.ascontiguousarray(pos_host, dtype=np.int32)
        tables = (rope.cos.data_ptr(), rope.sin.data_ptr(), rope.max_seq_len, rope.head_dim,
                  pos_dev.data_ptr(), pos_host.ctypes.data_as(_i32p))
    else:
        tables = (None, None, 0, d, None, None)
    wsp, keep = None, None
    if workspace is not None:
        size = NneWorkspaceSize()
        check(lib().nne_qkv_workspace_size(c, num_heads, num_kv_heads, d, ctypes.byref(size)))
        wsp, keep = _ws_arg(workspace, size, stream)
    check(lib().nne_qkv_rope_ws(
        x2.data_ptr(), x2.stride(0), w_packed.data_ptr(), ptr(bq), ptr(bk), ptr(bv), *tables,
        q_out.data_ptr(), k_out.data_ptr(), v_out.data_ptr(), b, c, num_heads, num_kv_heads, d,
        wsp, _stream(stream)))
    return q_out, k_out, v_out


class GroupedQueryAttention:
    """GroupedQueryAttention (src/models/llama.rs:160-300), forward only.

    Decode steps (T = 1 with a cache) run the fused prologue (projections +
    RoPE in one launch, on weights packed at construction) and the fused
    append + attend launch; the output projection is a plain GEMM.  Longer
    inputs (and head dims or widths that are not multiples of 64) project with
    GEMMs, rotate with ``RotaryEmbedding.apply``, append to the cache and run
    the attention kernel with q_offset = start_pos (:277-292)."""

    def __init__(self, d_model, num_heads, num_kv_heads, max_seq_len, rope_theta=10000.0,
                 device="cuda", seed=0):
        import torch
        if d_model % num_heads != 0:
            raise InvalidArgument("d_model must be divisible by num_heads")
        if num_heads % num_kv_heads != 0:
            raise InvalidArgument("num_heads must be divisible by num_kv_heads for GQA")
        self.num_heads, self.num_kv_heads = num_heads, num_kv_heads
        self.head_dim = d_model // num_heads
        self.d_model = d_model
        kv_dim = num_kv_heads * self.head_dim
        g = torch.Generator(device="cpu").manual_seed(seed)

        def w(out_f, in_f):   # Linear::without_bias, Kaiming-uniform range
            bound = math.sqrt(6.0 / in_f)
            return ((torch.rand(out_f, in_f, generator=g) * 2 - 1) * bound).to(device)

        self.wq, self.wk = w(d_model, d_model), w(kv_dim, d_model)
        self.wv, self.wo = w(kv_dim, d_model), w(d_model, d_model)
        self.rope = RotaryEmbedding(self.head_dim, max_seq_len, rope_theta, device)
        self.w_packed = None
        if self.head_dim % 64 == 0 and d_model % 64 == 0:
            self.w_packed = qkv_pack(self.wq, self.wk, self.wv, num_heads, num_kv_heads)

    def forward_gqa_cached(self, x, start_pos, cache=None, layer_idx=0, stream=None):
        """x [B, T, C].  With a cache, start_pos must be each sequence's cached
        length (an int for equal lengths, or B ints)."""
        import torch
        if x.dim() != 3:
            raise EngineError("Incompatible shapes for operation GroupedQueryAttention forward "
                              "(expected 3D input [B, T, C]): %s" % [list(x.shape)])
        b, t, c = x.shape
        hq, hkv, d = self.num_heads, self.num_kv_heads, self.head_dim
        sp = np.ascontiguousarray(np.broadcast_to(np.asarray(start_pos, np.int32), (b,)))
        if cache is not None:
            cache._check_layer(layer_idx)
            if not np.array_equal(sp, cache.lens_host[layer_idx]):
                raise InvalidArgument("Invalid configuration or argument: start_pos must equal "
                                      "the cached length of every sequence")
            # Checked before anything is appended, so a refused step leaves
            # the cache as it was.
            if t > 1 and b > 1 and not (sp == sp[0]).all():
                raise InvalidArgument("Invalid configuration or argument: multi-token steps need "
                                      "equal cached lengths")
        if cache is not None and t == 1:
            if self.w_packed is not None:
                q, k_new, v_new = qkv_rope(x, self.w_packed, None, None, None, self.rope,
                                           cache.lens_dev[layer_idx], sp, hq, hkv, stream=stream,
                                           workspace=cache._ws)
            else:
                q = torch.nn.functional.linear(x, self.wq).view(b, 1, hq, d).transpose(1, 2)
                k_new = torch.nn.functional.linear(x, self.wk).view(b, 1, hkv, d).transpose(1, 2)
                v_new = torch.nn.functional.linear(x, self.wv).view(b, 1, hkv, d).transpose(1, 2)
                q = self.rope.apply(q, sp, stream=stream)
                k_new = self.rope.apply(k_new, sp, stream=stream)
                v_new = v_new.contiguous()
            # append, then attend each sequence to its own rows (ragged lengths)
            ctx = cache.decode_step(layer_idx, q, k_new, v_new, stream=stream)
            return torch.nn.functional.linear(ctx.view(b, 1, hq * d), self.wo)
        q = torch.nn.functional.linear(x, self.wq).view(b, t, hq, d).transpose(1, 2)
        k = torch.nn.functional.linear(x, self.wk).view(b, t, hkv, d).transpose(1, 2)
        v = torch.nn.functional.linear(x, self.wv).view(b, t, hkv, d).transpose(1, 2)
        q = self.rope.apply(q, sp, stream=stream)
        k = self.rope.apply(k, sp, stream=stream)
        if cache is not None:
            k_all, v_all = cache.update(layer_idx, k, v, stream=stream)
        else:
            k_all, v_all = k, v
        out = torch.empty((b, t, hq, d), dtype=torch.float32, device=x.device)
        attention_forward(q, k_all, v_all, t > 1, q_offset=int(sp[0]) if b else 0,
                          out=out.transpose(1, 2), stream=stream)
        return torch.nn.functional.linear(out.view(b, t, hq * d), self.wo)


class MultiHeadAttention:
    """MultiHeadAttention (src/nn/attention.rs:9-210), forward only: biased
    q/k/v/out projections (Linear::new), causal self-attention with an
    optional KV cache and cross-attention whose projected memory K/V are
    cached once.

    Self-attention decode steps (T = 1 with a cache, head dim and d_model
    multiples of 64) run the fused projection launch (no RoPE) and the fused
    append + attend launch; other inputs project with GEMMs, append, and run
    the attention kernel with the reference's bottom-right mask
    (q_offset = L - T, attention.rs:101-108)."""

    def __init__(self, d_model, num_heads, is_causal, device="cuda", seed=0):
        import torch
        if d_model % num_heads != 0:
            raise InvalidArgument("d_model (%d) must be divisible by num_heads (%d)"
                                  % (d_model, num_heads))
        self.d_model, self.num_heads = d_model, num_heads
        self.head_dim = d_model // num_heads
        self.is_causal = is_causal
        g = torch.Generator(device="cpu").manual_seed(seed)

        def lin():   # Linear::new: Kaiming-uniform weight, U(-1/sqrt(in), 1/sqrt(in)) bias
            w = (torch.rand(d_model, d_model, generator=g) * 2 - 1) * math.sqrt(6.0 / d_model)
            bb = (torch.rand(d_model, generator=g) * 2 - 1) / math.sqrt(d_model)
            return w.to(device), bb.to(device)

        self.q_proj, self.k_proj, self.v_proj, self.out_proj = lin(), lin(), lin(), lin()
        self.w_packed = None
        if self.head_dim % 64 == 0 and d_model % 64 == 0:
            self.w_packed = qkv_pack(self.q_proj[0], self.k_proj[0], self.v_proj[0], num_heads,
                                     num_heads)

    def _heads(self, y, b, t):
        return y.view(b, t, self.num_heads, self.head_dim).transpose(1, 2)

    def forward_attention(self, x, stream=None):
        return self.forward_attention_cached(x, None, stream=stream)

    def forward_attention_cached(self, x, cache=None, layer_idx=0, stream=None):
        """x [B, T, C]; cache a KVCache whose layer ``layer_idx`` holds this
        layer's self-attention rows (attention.rs:78-91)."""
        import torch
        if x.dim() != 3:
            raise EngineError("Incompatible shapes for operation MultiHeadAttention forward "
                              "(expected 3D input [B, T, C]): %s" % [list(x.shape)])
        b, t, c = x.shape
        h, d = self.num_heads, self.head_dim
        if cache is not None:
            cache._check_layer(layer_idx)
            lens = cache.lens_host[layer_idx]
            if t > 1 and b > 1 and not (lens == lens[0]).all():
                raise InvalidArgument("Invalid configuration or argument: multi-token steps need "
                                      "equal cached lengths")
        if cache is not None and t == 1:
            if self.w_packed is not None:
                q, k_new, v_new = qkv_rope(x, self.w_packed, self.q_proj[1], self.k_proj[1],
                                           self.v_proj[1], None, None, None, h, h, stream=stream,
                                           head_dim=d, workspace=cache._ws)
            else:
                q = self._heads(torch.nn.functional.linear(x, *self.q_proj), b, 1)
                k_new = self._heads(torch.nn.functional.linear(x, *self.k_proj), b, 1).contiguous()
                v_new = self._heads(torch.nn.functional.linear(x, *self.v_proj), b, 1).contiguous()
            # append, then attend each sequence to its own rows (ragged lengths)
            ctx = cache.decode_step(layer_idx, q, k_new, v_new, stream=stream)
            return torch.nn.functional.linear(ctx.view(b, 1, c), *self.out_proj)
        q = self._heads(torch.nn.functional.linear(x, *self.q_proj), b, t)
        k = self._heads(torch.nn.functional.linear(x, *self.k_proj), b, t)
        v = self._heads(torch.nn.functional.linear(x, *self.v_proj), b, t)
        if cache is not None:
            k_all, v_all = cache.update(layer_idx, k.contiguous(), v.contiguous(), stream=stream)
            total = int(cache.lens_host[layer_idx][0]) if b else 0
        else:
            k_all, v_all, total = k, v, t
        out = torch.empty((b, t, h, d), dtype=torch.float32, device=x.device)
        attention_forward(q, k_all, v_all, self.is_causal and t > 1, q_offset=max(total - t, 0),
                          out=out.transpose(1, 2), stream=stream)
        return torch.nn.functional.linear(out.view(b, t, c), *self.out_proj)

    def forward_cross_attention(self, x, memory, stream=None):
        return self.forward_cross_attention_cached(x, memory, None, stream=stream)

    def forward_cross_attention_cached(self, x, memory, slots=None, layer_idx=0, stream=None):
        """Queries from x [B, T_q, C], keys/values from memory [B, T_kv, C];
        with ``slots`` (e.g. WhisperKVCache.cross_attn) the projected memory
        K/V [B, H, T_kv, d] are computed once and reused (attention.rs:139-191)."""
        import torch
        if x.dim() != 3 or memory.dim() != 3:
            raise EngineError("Incompatible shapes for operation MultiHeadAttention cross-attention "
                              "(expected 3D query [B, T_q, C] and 3D memory [B, T_kv, C]): %s"
                              % [list(x.shape), list(memory.shape)])
        if x.shape[0] != memory.shape[0] or x.shape[2] != memory.shape[2]:
            raise EngineError("Incompatible shapes for operation MultiHeadAttention cross-attention "
                              "(batch size and channel dim must match): %s"
                              % [list(x.shape), list(memory.shape)])
        b, tq, c = x.shape
        tkv = memory.shape[1]
        h, d = self.num_heads, self.head_dim
        q = self._heads(torch.nn.functional.linear(x, *self.q_proj), b, tq)
        kv = slots[layer_idx] if slots is not None else None
        if kv is None:
            k = self._heads(torch.nn.functional.linear(memory, *self.k_proj), b, tkv).contiguous()
            v = self._heads(torch.nn.functional.linear(memory, *self.v_proj), b, tkv).contiguous()
            kv = (k, v)
            if slots is not None:
                slots[layer_idx] = kv
        out = torch.empty((b, tq, h, d), dtype=torch.float32, device=x.device)
        attention_forward(q, kv[0], kv[1], False, out=out.transpose(1, 2), stream=stream)
        return torch.nn.functional.linear(out.view(b, tq, c), *self.out_proj)


class WhisperKVCache:
    """WhisperKVCache (src/models/whisper.rs:325-350): per decoder layer a
    self-attention cache (a device KVCache layer) and a cross-attention slot
    holding the projected encoder memory K/V (None until the first step)."""

    def __init__(self, num_layers, batch, num_heads, capacity, head_dim, device="cuda"):
        self.self_attn = KVCache(num_layers, batch, num_heads, capacity, head_dim, device=device)
        self.cross_attn = [None] * num_layers

    def reset(self):
        self.self_attn.reset()
        self.cross_attn = [None] * len(self.cross_attn)
