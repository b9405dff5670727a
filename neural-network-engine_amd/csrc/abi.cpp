// extern "C" boundary of the attention hot path (declared in include/nne_attn.h).
//
// This layer validates shapes the way the reference does, picks the kernel
// and fills the launch-parameter structs; it never computes attention itself.
// There is no CPU fallback: every compute entry point either launches a HIP
// kernel or returns an error.
#include <atomic>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "nne_abi_internal.hpp"
#include "nne_attn.h"
#include "nne_launch.hpp"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(NNE_EHIP, "GPU compute error: %s: %s", what, hipGetErrorString(e));
}

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

void contiguous_strides(const int64_t* shape, int64_t* st) {
    st[3] = 1;
    st[2] = shape[3];
    st[1] = shape[2] * shape[3];
    st[0] = shape[1] * st[1];
}

std::string shape_str(const int64_t* s) {
    char buf[128];
    snprintf(buf, sizeof(buf), "[%lld, %lld, %lld, %lld]", (long long)s[0], (long long)s[1],
             (long long)s[2], (long long)s[3]);
    return buf;
}

bool dims_ok(const int64_t* s) {
    for (int i = 0; i < 4; ++i)
        if (s[i] < 0 || s[i] > INT32_MAX) return false;
    return true;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int device_cus();   // CUs of the current device (cached per device)

// Per-stream resources of the split-K kernel, one set per (device, stream) --
// per calling thread for the per-thread default stream.  Launches on one
// stream run in order, so they share the set:
//   * arrival counters of the in-launch combine, zeroed by a fill kernel when
//     allocated and left zeroed by every launch;
//   * the workspace used when the caller passes none.
// Both grow on demand (stream-ordered allocation).  A replaced buffer is
// retired, not freed: another thread that took it for a launch on the same
// stream (the null stream is shared by all threads) may not have queued that
// launch yet.  Sizes double, so the retired buffers together are smaller than
// the live one.  Everything is kept until nne_stream_release or the end of
// the process.
struct StreamResources {
    int dev;
    hipStream_t stream;
    std::thread::id thread;
    uint32_t* counters;
    int64_t n_counters;
    void* ws;
    uint64_t ws_bytes;
    std::vector<void*> retired;
    uint64_t retired_bytes;
};
std::mutex g_res_mu;
std::vector<StreamResources> g_res;

// Counters for n heads and, when ws_bytes > 0, a workspace of that size.
hipError_t stream_resources(int64_t n, uint64_t ws_bytes, hipStream_t s, uint32_t** counters,
                            void** ws) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const std::thread::id th =
        s == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    std::lock_guard<std::mutex> lock(g_res_mu);
    StreamResources* r = nullptr;
    for (auto& x : g_res)
        if (x.dev == dev && x.stream == s && x.thread == th) r = &x;
    if (!r) {
        g_res.push_back(StreamResources{dev, s, th, nullptr, 0, nullptr, 0, {}, 0});
        r = &g_res.back();
    }
    if (r->n_counters < n) {
        int64_t cap = 1 << 16;
        while (cap < n) cap <<= 1;
        uint32_t* p = nullptr;
        e = hipMallocAsync(reinterpret_cast<void**>(&p), (size_t)cap * 4, s);
        if (e != hipSuccess) return e;
        e = nne::zero_counters(p, cap, s);
        if (e != hipSuccess) return e;
        if (r->counters) {
            r->retired.push_back(r->counters);
            r->retired_bytes += (uint64_t)r->n_counters * 4;
        }
        r->counters = p;
        r->n_counters = cap;
    }
    *counters = r->counters;
    if (ws_bytes > 0) {
        if (r->ws_bytes < ws_bytes) {
            uint64_t cap = 1u << 20;
            while (cap < ws_bytes) cap <<= 1;
            void* p = nullptr;
            e = hipMallocAsync(&p, cap, s);
            if (e != hipSuccess) return e;
            if (r->ws) {
                r->retired.push_back(r->ws);
                r->retired_bytes += r->ws_bytes;
            }
            r->ws = p;
            r->ws_bytes = cap;
        }
        *ws = r->ws;
    }
    return hipSuccess;
}

// Records and counters of one call: the caller's workspace, checked against
// what the call needs, or (ws == NULL) the stream's library-side ones.
int call_workspace(const nne_workspace_t* ws, uint64_t need_bytes, int64_t need_counters,
                   hipStream_t s, void** records, uint32_t** counters, const char* what) {
    if (ws) {
        if ((ws->records && reinterpret_cast<uintptr_t>(ws->records) % 16) ||
            (ws->counters && reinterpret_cast<uintptr_t>(ws->counters) % 4))
            return fail(NNE_EINVAL, "Invalid configuration or argument: %s workspace records must "
                                    "be 16-byte aligned and counters 4-byte aligned", what);
        if (need_bytes > 0 && (!ws->records || ws->records_bytes < need_bytes))
            return fail(NNE_EINVAL, "Invalid configuration or argument: %s workspace holds %llu "
                                    "record bytes, the call needs %llu", what,
                        (unsigned long long)(ws->records ? ws->records_bytes : 0),
                        (unsigned long long)need_bytes);
        if (need_counters > 0 && (!ws->counters || ws->n_counters < (uint64_t)need_counters))
            return fail(NNE_EINVAL, "Invalid configuration or argument: %s workspace holds %llu "
                                    "counters, the call needs %lld", what,
                        (unsigned long long)(ws->counters ? ws->n_counters : 0),
                        (long long)need_counters);
        *records = ws->records;
        *counters = ws->counters;
        return NNE_OK;
    }
    const hipError_t e = stream_resources(need_counters, need_bytes, s, counters, records);
    return e == hipSuccess ? NNE_OK : hip_fail(e, what);
}

// 16-byte vector access is valid for this view: unit dim stride and every
// other stride a multiple of 4 floats, 16-byte aligned base.
bool vec_view(const void* p, const int64_t* st) {
    return aligned16(p) && st[3] == 1 && st[0] % 4 == 0 && st[1] % 4 == 0 && st[2] % 4 == 0;
}

nne::View4 make_view(const float* p, const int64_t* st) {
    nne::View4 v;
    v.p = p;
    v.sb = st[0]; v.sh = st[1]; v.st = st[2]; v.sd = st[3];
    return v;
}

nne::OutView4 make_out(float* p, const int64_t* st) {
    nne::OutView4 v;
    v.p = p;
    v.sb = st[0]; v.sh = st[1]; v.st = st[2]; v.sd = st[3];
    return v;
}

float softmax_scale(int has_scale, float scale, int64_t d) {
    // scale.unwrap_or(1.0 / (d as f32).sqrt())  (flash_attention.rs:50, llama.rs:273)
    return has_scale ? scale : 1.0f / std::sqrt((float)d);
}

// Query rows per launch when the split-K kernel serves a prefill of head
// dim above 128: causal steps take the 16-row tile with per-row masks.
int wide_rows_per_launch(int d, bool causal) {
    return causal ? 16 : nne::splitk_rows_per_launch(d);
}

// Key tiles of the longest unit of a deep-kernel problem: the keys some row
// can see.
int deep_max_tiles(int64_t Tk, bool causal, int64_t qoff, int64_t Tq) {
    const int64_t tk = causal ? std::max<int64_t>(0, std::min<int64_t>(Tk, qoff + Tq)) : Tk;
    return (int)std::min<int64_t>((tk + 31) / 32, INT32_MAX);
}

// Key split of a deep-kernel launch and its records: the caller's workspace
// caps the split (a smaller workspace gives fewer parts, never an error for
// its size), the stream's own workspace is grown to the plan.
int deep_workspace(nne::DeepParams& p, int max_tiles, const nne_workspace_t* wsp,
                   hipStream_t stream, const int32_t* seq_keys = nullptr) {
    const uint64_t avail = wsp ? (wsp->records ? wsp->records_bytes : 0) : UINT64_MAX;
    uint64_t bytes = seq_keys ? nne::deep_ragged_plan(p, seq_keys, device_cus(), avail) : 0;
    if (bytes == 0) bytes = nne::deep_split_plan(p, max_tiles, device_cus(), avail);
    if (bytes == 0) return NNE_OK;
    void* ws = nullptr;
    uint32_t* counters = nullptr;
    const int rc = call_workspace(wsp, bytes, 0, stream, &ws, &counters, "deep attention key split");
    if (rc != NNE_OK) return rc;
    p.ws = static_cast<float*>(ws);
    return NNE_OK;
}

// Head dims 129-256 with more query rows per KV head than the split-K kernel
// takes: the wave-pair kernel at d = 256 when its work items (4 units of 32
// rows each) fill the device, else the deep kernel's 2-wave form, which pads
// no dims to 256 and spreads (or key-splits) small problems over the CUs.
// (Measured: d = 192 B = 8, H = 20, T = 1500 3.32 -> 2.56 ms; d = 256 causal
// B = 1, H = 8, T = 1024 0.28 -> 0.17 ms; at d = 256 with the device full the
// wave-pair kernel is level or up to 2 % faster.)
bool wide_on_deep(int64_t B, int64_t Hkv, int64_t G, int64_t Tq, int d) {
    if (nne::prefill_padded_dim(d) != 0 || nne::splitk_padded_dim(d) == 0) return false;
    if (G * Tq <= nne::splitk_max_rows()) return false;
    if (d != 256) return true;
    const int64_t items = B * Hkv * ((G * ((Tq + 31) / 32) + 3) / 4);
    return items < device_cus();
}

// Records of the largest key split a deep-kernel problem of these shapes
// takes (max_tiles: tiles of its longest unit; 0 when unknown).  A decode
// step (Tq = 1) may take the ragged split instead: at most one record of its
// rows per CU.
uint64_t deep_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t d,
                              int max_tiles, bool decode = false) {
    nne::DeepParams p{};
    p.B = (int)B; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.G = (int)(Hq / Hkv); p.Tq = (int)Tq;
    p.d = (int)d;
    uint64_t bytes = nne::deep_split_plan(p, max_tiles > 0 ? max_tiles : (1 << 24), device_cus(), UINT64_MAX);
    const int64_t rows = (Hq / Hkv) * Tq;
    if (decode && rows <= 32 && d <= nne::kDeepChunk && B * Hkv <= nne::kDeepMaxHeads &&
        B * Hkv <= device_cus() && (max_tiles <= 0 || max_tiles >= 5))   // shorter sequences never split
        bytes = std::max<uint64_t>(bytes, (uint64_t)device_cus() * (uint64_t)rows *
                                              (nne::kDeepChunk + 2) * 4u);
    return bytes;
}

// Shared body of the two prefill entry points.  Shapes were validated.
int run_attention(const float* q, const int64_t* qs_, const int64_t* qst, const float* k,
                  const int64_t* ks_, const int64_t* kst, const float* v, const int64_t* vst,
                  float* o, const int64_t* ost, bool causal, int64_t q_offset, float scale,
                  const nne_workspace_t* wsp, hipStream_t stream) {
    const int B = (int)qs_[0], Hq = (int)qs_[1], Tq = (int)qs_[2], d = (int)qs_[3];
    const int Hkv = (int)ks_[1], Tk = (int)ks_[2];
    if ((int64_t)B * Hq * Tq == 0 || d == 0) return NNE_OK;
    // Head dims above 128 (d <= 256) run on the wave-pair MFMA kernel or the
    // deep kernel's 2-wave form (wide_on_deep), or on the split-K kernel when a
    // KV head has few query rows; above 256 on the deep kernel.
    const bool wide = nne::prefill_padded_dim(d) == 0;
    // (At 129-256 dims K/V row strides outside the deep kernel's 32-bit tile
    // offsets keep the wave-pair kernel.)
    const bool deep_strides = kst[2] >= 0 && vst[2] >= 0 && kst[2] < (1 << 25) && vst[2] < (1 << 25);
    const bool deep = wide && (nne::splitk_padded_dim(d) == 0 ||
                               (deep_strides && wide_on_deep(B, Hkv, Hq / Hkv, Tq, d)));
    // Offsets beyond +-2^30 cannot change visibility for int32 lengths.
    const int qoff = (int)std::max<int64_t>(-(1 << 30), std::min<int64_t>(q_offset, 1 << 30));
    const bool vec = d % 4 == 0 && vec_view(q, qst) && vec_view(k, kst) && vec_view(v, vst) &&
                     vec_view(o, ost);
    if (wide && !vec)
        return fail(NNE_EINVAL, "Invalid configuration or argument: head dim %d > 128 needs a "
                                "multiple of 4, unit dim strides, strides that are multiples of 4 "
                                "and 16-byte aligned tensors", d);
    if (deep) {
        // The deep kernel addresses 32 K/V rows of a tile with 32-bit byte offsets.
        if (kst[2] < 0 || vst[2] < 0 || kst[2] >= (1 << 25) || vst[2] >= (1 << 25))
            return fail(NNE_EINVAL, "Invalid configuration or argument: K/V row strides must lie in "
                                    "[0, 2^25) floats at head dim %d", d);
        nne::DeepParams p{};
        p.q = make_view(q, qst);
        p.k = make_view(k, kst);
        p.v = make_view(v, vst);
        p.o = make_out(o, ost);
        p.lens = nullptr;
        p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.G = Hq / Hkv; p.Tq = Tq; p.Tk = Tk; p.d = d;
        p.q_offset = qoff;
        p.qscale = scale * nne::kLog2e;
        const int rc = deep_workspace(p, deep_max_tiles(Tk, causal, qoff, Tq), wsp, stream);
        if (rc != NNE_OK) return rc;
        hipError_t e = nne::launch_deep(p, causal, device_cus(), stream);
        if (e != hipSuccess) return hip_fail(e, "deep head-dim attention launch");
        return NNE_OK;
    }
    const int G = Hq / Hkv;
    const int64_t rows = (int64_t)G * Tq;
    // Few query rows per KV head (decode-like steps, cross-attention, a few
    // new tokens over a cache) go to the split-K kernel.  With a causal mask
    // only the first tk keys are visible to any row (the last row sees keys
    // <= qoff + Tq - 1), and rows see different prefixes of them when
    // qoff < tk - 1.
    const int64_t tk = causal ? std::max<int64_t>(0, std::min<int64_t>(Tk, (int64_t)qoff + Tq)) : Tk;
    const bool masked = causal && (int64_t)qoff < tk - 1;
    // The split-K kernel addresses a head's rows with 32-bit byte offsets.
    const bool fits32 = (int64_t)B * Hkv * Tk < INT32_MAX && (int64_t)Tk * kst[2] < (1LL << 30) &&
                        (int64_t)Tk * vst[2] < (1LL << 30);
    if (wide && rows > nne::splitk_max_rows()) {
        nne::PrefillParams p{};
        p.q = make_view(q, qst);
        p.k = make_view(k, kst);
        p.v = make_view(v, vst);
        p.o = make_out(o, ost);
        p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.Tq = Tq; p.Tk = Tk; p.d = d;
        p.q_offset = qoff;
        p.qscale = scale * nne::kLog2e;
        hipError_t e = nne::launch_prefill_wide(p, causal, stream);
        if (e != hipSuccess) return hip_fail(e, "wide prefill attention launch");
        return NNE_OK;
    }
    if (wide && !fits32)
        return fail(NNE_EINVAL, "Invalid configuration or argument: head dim %d > 128 with %lld "
                                "keys per call exceeds the split-K kernel's limits (2^31 keys per call, 2^30 "
                                "floats per head)", d,
                    (long long)((int64_t)B * Hkv * Tk));

    if (vec && fits32 && (wide || (rows <= nne::splitk_max_rows() && tk > 0))) {
        nne::SplitKParams p{};
        p.q = make_view(q, qst);
        p.k = k; p.v = v;
        p.ksb = kst[0]; p.ksh = kst[1]; p.kst = kst[2];
        p.vsb = vst[0]; p.vsh = vst[1]; p.vst = vst[2];
        p.lens = nullptr;
        p.o = make_out(o, ost);
        p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.Tq = Tq; p.d = d;
        p.qscale = scale * nne::kLog2e;
        p.q_off = qoff;
        const int rp = wide ? wide_rows_per_launch(d, causal) : (int)rows;
        const nne::SplitKWorkspace w = nne::splitk_workspace_layout(
            std::min(B, nne::splitk_max_seqs()), Hkv, (int)std::min<int64_t>(rows, rp), d);
        uint32_t* counters = nullptr;
        void* ws = nullptr;
        const int rc = call_workspace(wsp, w.total_bytes,
                                      (int64_t)std::min(B, nne::splitk_max_seqs()) * Hkv, stream,
                                      &ws, &counters, "few-query attention");
        if (rc != NNE_OK) return rc;
        // One launch per range of rp rows, each over the keys its rows can see.
        for (int64_t r0 = 0; r0 < rows; r0 += rp) {
            const int R = (int)std::min<int64_t>(rp, rows - r0);
            int64_t tkp = tk;
            bool maskp = masked;
            if (wide && causal) {
                int tmin = Tq, tmax = -1;
                for (int64_t rr = r0; rr < r0 + R; ++rr) {
                    tmin = std::min(tmin, (int)(rr % Tq));
                    tmax = std::max(tmax, (int)(rr % Tq));
                }
                tkp = std::max<int64_t>(0, std::min<int64_t>(Tk, (int64_t)qoff + tmax + 1));
                maskp = (int64_t)qoff + tmin < tkp - 1;
            }
            p.tk = (int)tkp;
            p.max_keys = (int)tkp;
            p.masked = maskp ? 1 : 0;
            hipError_t e = nne::launch_splitk(p, (int64_t)B * Hkv * tkp, (int)tkp, ws, stream,
                                              nullptr, counters, (int)r0, R);
            if (e != hipSuccess) return hip_fail(e, "split-K attention launch");
        }
        return NNE_OK;
    }

    nne::PrefillParams p{};
    p.q = make_view(q, qst);
    p.k = make_view(k, kst);
    p.v = make_view(v, vst);
    p.o = make_out(o, ost);
    p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.Tq = Tq; p.Tk = Tk; p.d = d;
    p.q_offset = qoff;
    p.qscale = scale * nne::kLog2e;
    // Small problems: one workgroup per 16-row block, waves over its key
    // tiles, merged in LDS.
    const int cus = device_cus();
    if (nne::small_prefill_fits(p, vec, cus)) {
        hipError_t e = nne::launch_small_prefill(p, causal, cus, stream);
        if (e != hipSuccess) return hip_fail(e, "small prefill launch");
        return NNE_OK;
    }
    // Other problems too small to fill the device split their key range
    // across workgroups, with partial records in the workspace.
    const nne::PrefillSplit plan = nne::prefill_split_plan(p, causal, vec);
    if (p.n_chunks > 1) {
        uint32_t* counters = nullptr;
        void* ws = nullptr;
        const int rc = call_workspace(wsp, plan.ws_bytes, plan.n_counters, stream, &ws, &counters,
                                      "prefill key split");
        if (rc != NNE_OK) return rc;
        p.ws = static_cast<float*>(ws);
        p.cnt = counters;
    }
    hipError_t e = nne::launch_prefill(p, causal, vec, stream);
    if (e != hipSuccess) return hip_fail(e, "prefill attention launch");
    return NNE_OK;
}

// Upper bound on the workspace of a prefill call: the few-query layout and
// the key-split plan of the same shapes (which one runs depends on strides).
nne_workspace_size_t attention_workspace(const int64_t* qs_, const int64_t* ks_, bool causal,
                                         int64_t q_offset) {
    nne_workspace_size_t r{0, 0};
    const int B = (int)qs_[0], Hq = (int)qs_[1], Tq = (int)qs_[2], d = (int)qs_[3];
    const int Hkv = (int)ks_[1], Tk = (int)ks_[2];
    if ((int64_t)B * Hq * Tq == 0 || d == 0 || Hkv == 0) return r;
    const int qoff = (int)std::max<int64_t>(-(1 << 30), std::min<int64_t>(q_offset, 1 << 30));
    // The deep kernel's key split: above 256 dims, and head dims 129-256 on its
    // 2-wave form.
    if (nne::splitk_padded_dim(d) == 0 || (Hq % Hkv == 0 && wide_on_deep(B, Hkv, Hq / Hkv, Tq, d))) {
        if (d % 4 == 0 && Hq % Hkv == 0)
            r.records_bytes = deep_workspace_bytes(B, Hq, Hkv, Tq, d, deep_max_tiles(Tk, causal, qoff, Tq));
        return r;
    }
    const bool wide = nne::prefill_padded_dim(d) == 0;
    const int64_t rows = (int64_t)(Hq / Hkv) * Tq;
    const int64_t tk = causal ? std::min<int64_t>(Tk, (int64_t)qoff + Tq) : Tk;
    // Wide head dims with more rows per KV head take the wave-pair kernel,
    // which needs no workspace.
    const bool wide_mfma = wide && rows > nne::splitk_max_rows();
    if (d % 4 == 0 && !wide_mfma && (wide || (rows <= nne::splitk_max_rows() && tk > 0))) {
        const int rp = wide ? wide_rows_per_launch(d, causal) : (int)rows;
        const int Bl = std::min(B, nne::splitk_max_seqs());
        const nne::SplitKWorkspace w =
            nne::splitk_workspace_layout(Bl, Hkv, (int)std::min<int64_t>(rows, rp), d);
        r.records_bytes = w.total_bytes;
        r.n_counters = (uint64_t)Bl * Hkv;
    }
    if (wide) return r;
    nne::PrefillParams p{};
    p.B = B; p.Hq = Hq; p.Hkv = Hkv; p.Tq = Tq; p.Tk = Tk; p.d = d;
    p.q_offset = qoff;
    const nne::PrefillSplit plan = nne::prefill_split_plan(p, causal, true);
    if (p.n_chunks > 1) {
        r.records_bytes = std::max<uint64_t>(r.records_bytes, plan.ws_bytes);
        r.n_counters = std::max<uint64_t>(r.n_counters, (uint64_t)plan.n_counters);
    }
    return r;
}

struct Resolved {
    int64_t q[4], k[4], v[4], o[4];
};

void resolve_strides(Resolved& r, const int64_t* qs_, const int64_t* qst, const int64_t* ks_,
                     const int64_t* kst, const int64_t* vs_, const int64_t* vst, const int64_t* ost) {
    int64_t c[4];
    contiguous_strides(qs_, c);
    for (int i = 0; i < 4; ++i) r.q[i] = qst ? qst[i] : c[i];
    for (int i = 0; i < 4; ++i) r.o[i] = ost ? ost[i] : c[i];
    contiguous_strides(ks_, c);
    for (int i = 0; i < 4; ++i) r.k[i] = kst ? kst[i] : c[i];
    contiguous_strides(vs_, c);
    for (int i = 0; i < 4; ++i) r.v[i] = vst ? vst[i] : c[i];
}

// Cache geometry; `decode` adds the decode kernel's head-dim limits (the
// append kernel is element-wise and takes any head dim).
int check_kv_cache_args(int64_t B, int64_t Hq, int64_t Hkv, int64_t capacity, int64_t d, bool decode) {
    if (B < 0 || Hq < 0 || Hkv <= 0 || capacity < 0 || d <= 0 || B > INT32_MAX ||
        Hq > INT32_MAX || Hkv > INT32_MAX || capacity > INT32_MAX || d > INT32_MAX)
        return fail(NNE_EINVAL, "Invalid configuration or argument: bad KV cache geometry "
                                "B=%lld Hq=%lld Hkv=%lld capacity=%lld d=%lld",
                    (long long)B, (long long)Hq, (long long)Hkv, (long long)capacity, (long long)d);
    if (Hq % Hkv != 0)
        return fail(NNE_EINVAL, "Invalid configuration or argument: num_heads (%lld) must be "
                                "divisible by num_kv_heads (%lld) for GQA",
                    (long long)Hq, (long long)Hkv);
    if (decode && d % 4 != 0)
        return fail(NNE_EINVAL, "Invalid configuration or argument: KV cache head dim %lld must be "
                                "a multiple of 4", (long long)d);
    return NNE_OK;
}

}  // namespace

namespace nne {

int fail_message(int code, const char* msg) { return fail(code, "%s", msg); }

int fail_hip(hipError_t e, const char* what) { return hip_fail(e, what); }

}  // namespace nne

extern "C" {

int nne_abi_version(void) { return NNE_ABI_VERSION; }

const char* nne_last_error(void) { return g_err.c_str(); }

int nne_dev_alloc(void** ptr, uint64_t bytes) {
    if (!ptr) return fail(NNE_EINVAL, "Invalid configuration or argument: null output pointer");
    *ptr = nullptr;
    if (bytes == 0) return NNE_OK;
    hipError_t e = hipMalloc(ptr, bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc");
    return NNE_OK;
}

int nne_dev_free(void* ptr) {
    if (!ptr) return NNE_OK;
    hipError_t e = hipFree(ptr);
    if (e != hipSuccess) return hip_fail(e, "hipFree");
    return NNE_OK;
}

int nne_memcpy_h2d(void* dst, const void* src, uint64_t bytes, void* stream) {
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, as_stream(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(as_stream(stream));
    return e == hipSuccess ? NNE_OK : hip_fail(e, "hipMemcpy H2D");
}

int nne_memcpy_d2h(void* dst, const void* src, uint64_t bytes, void* stream) {
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, as_stream(stream));
    if (e == hipSuccess) e = hipStreamSynchronize(as_stream(stream));
    return e == hipSuccess ? NNE_OK : hip_fail(e, "hipMemcpy D2H");
}

int nne_memcpy_d2d(void* dst, const void* src, uint64_t bytes, void* stream) {
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, as_stream(stream));
    return e == hipSuccess ? NNE_OK : hip_fail(e, "hipMemcpy D2D");
}

int nne_stream_sync(void* stream) {
    hipError_t e = hipStreamSynchronize(as_stream(stream));
    return e == hipSuccess ? NNE_OK : hip_fail(e, "hipStreamSynchronize");
}

int nne_stream_release(void* stream) {
    const hipStream_t s = as_stream(stream);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    const std::thread::id th =
        s == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    std::lock_guard<std::mutex> lock(g_res_mu);
    for (size_t i = 0; i < g_res.size(); ++i) {
        StreamResources& r = g_res[i];
        if (r.dev != dev || r.stream != s || r.thread != th) continue;
        if (r.counters) e = hipFree(r.counters);
        if (e == hipSuccess && r.ws) e = hipFree(r.ws);
        for (void* old : r.retired)
            if (e == hipSuccess) e = hipFree(old);
        g_res.erase(g_res.begin() + (std::ptrdiff_t)i);
        return e == hipSuccess ? NNE_OK : hip_fail(e, "hipFree");
    }
    return NNE_OK;
}

namespace {

// flash_attention_forward's checks (flash_attention.rs:32-48).
int check_flash_shapes(const int64_t* q_shape, const int64_t* k_shape, const int64_t* v_shape) {
    if (!q_shape || !k_shape || !v_shape)
        return fail(NNE_EINVAL, "Invalid configuration or argument: FlashAttention expects 4D "
                                "tensors [Batch, Heads, SeqLen, Dim]");
    if (!dims_ok(q_shape) || !dims_ok(k_shape) || !dims_ok(v_shape))
        return fail(NNE_EINVAL, "Invalid configuration or argument: FlashAttention dims out of "
                                "range, got Q:%s, K:%s, V:%s", shape_str(q_shape).c_str(),
                    shape_str(k_shape).c_str(), shape_str(v_shape).c_str());
    const int64_t b = q_shape[0], h = q_shape[1], d = q_shape[3];
    const int64_t kb = k_shape[0], kh = k_shape[1], tk = k_shape[2], kd = k_shape[3];
    const int64_t vb = v_shape[0], vh = v_shape[1], vt = v_shape[2], vd = v_shape[3];
    if (b != kb || b != vb || h != kh || h != vh || d != kd || d != vd || tk != vt) {
        const int64_t expected[4] = {b, h, tk, d};
        const int64_t actual[4] = {kb, kh, tk, kd};
        return fail(NNE_ESHAPE, "Shape mismatch error: expected shape %s, got %s",
                    shape_str(expected).c_str(), shape_str(actual).c_str());
    }
    return NNE_OK;
}

// The grouped-query entry's checks: K/V agree with each other and with Q in
// batch and head dim, and Hkv divides Hq.
int check_attention_shapes(const int64_t* q_shape, const int64_t* k_shape, const int64_t* v_shape) {
    if (!q_shape || !k_shape || !v_shape)
        return fail(NNE_EINVAL, "Invalid configuration or argument: attention expects 4D "
                                "tensors [Batch, Heads, SeqLen, Dim]");
    if (!dims_ok(q_shape) || !dims_ok(k_shape) || !dims_ok(v_shape))
        return fail(NNE_EINVAL, "Invalid configuration or argument: attention dims out of range, "
                                "got Q:%s, K:%s, V:%s", shape_str(q_shape).c_str(),
                    shape_str(k_shape).c_str(), shape_str(v_shape).c_str());
    const int64_t b = q_shape[0], hq = q_shape[1], d = q_shape[3];
    const int64_t kb = k_shape[0], hkv = k_shape[1], tk = k_shape[2], kd = k_shape[3];
    if (b != kb || b != v_shape[0] || hkv != v_shape[1] || d != kd || d != v_shape[3] ||
        tk != v_shape[2] || hkv == 0 || hq % hkv != 0) {
        const int64_t expected[4] = {b, hkv > 0 && hq % hkv == 0 ? hkv : hq, tk, d};
        const int64_t actual[4] = {kb, hkv, tk, kd};
        return fail(NNE_ESHAPE, "Shape mismatch error: expected shape %s, got %s",
                    shape_str(expected).c_str(), shape_str(actual).c_str());
    }
    return NNE_OK;
}

int attention_entry(const float* q, const int64_t* q_shape, const int64_t* q_strides, const float* k,
                    const int64_t* k_shape, const int64_t* k_strides, const float* v,
                    const int64_t* v_shape, const int64_t* v_strides, float* o,
                    const int64_t* o_strides, bool causal, int64_t q_offset, int has_scale,
                    float scale, const nne_workspace_t* ws, hipStream_t stream) {
    if (q_shape[0] * q_shape[1] * q_shape[2] > 0 && k_shape[2] > 0 && (!q || !k || !v || !o))
        return fail(NNE_EINVAL, "Invalid configuration or argument: null tensor pointer");
    Resolved r;
    resolve_strides(r, q_shape, q_strides, k_shape, k_strides, v_shape, v_strides, o_strides);
    return run_attention(q, q_shape, r.q, k, k_shape, r.k, v, r.v, o, r.o, causal, q_offset,
                         softmax_scale(has_scale, scale, q_shape[3]), ws, stream);
}

}  // namespace

int nne_flash_attention_forward_ws(const float* q, const int64_t q_shape[4], const int64_t q_strides[4],
                                   const float* k, const int64_t k_shape[4], const int64_t k_strides[4],
                                   const float* v, const int64_t v_shape[4], const int64_t v_strides[4],
                                   float* o, const int64_t o_strides[4], int is_causal, int has_scale,
                                   float scale, int64_t block_size_r, int64_t block_size_c,
                                   const nne_workspace_t* ws, void* stream) {
    const int rc = check_flash_shapes(q_shape, k_shape, v_shape);
    if (rc != NNE_OK) return rc;
    (void)block_size_r;   // br, bc = max(arg, 16) (:51-52) only order the reference's loops
    (void)block_size_c;
    return attention_entry(q, q_shape, q_strides, k, k_shape, k_strides, v, v_shape, v_strides, o,
                           o_strides, is_causal != 0, 0, has_scale, scale, ws, as_stream(stream));
}

int nne_flash_attention_forward(const float* q, const int64_t q_shape[4], const int64_t q_strides[4],
                                const float* k, const int64_t k_shape[4], const int64_t k_strides[4],
                                const float* v, const int64_t v_shape[4], const int64_t v_strides[4],
                                float* o, const int64_t o_strides[4], int is_causal, int has_scale,
                                float scale, int64_t block_size_r, int64_t block_size_c,
                                void* stream) {
    return nne_flash_attention_forward_ws(q, q_shape, q_strides, k, k_shape, k_strides, v, v_shape,
                                          v_strides, o, o_strides, is_causal, has_scale, scale,
                                          block_size_r, block_size_c, nullptr, stream);
}

int nne_attention_forward_ws(const float* q, const int64_t q_shape[4], const int64_t q_strides[4],
                             const float* k, const int64_t k_shape[4], const int64_t k_strides[4],
                             const float* v, const int64_t v_shape[4], const int64_t v_strides[4],
                             float* o, const int64_t o_strides[4], int is_causal, int64_t q_offset,
                             int has_scale, float scale, const nne_workspace_t* ws, void* stream) {
    const int rc = check_attention_shapes(q_shape, k_shape, v_shape);
    if (rc != NNE_OK) return rc;
    return attention_entry(q, q_shape, q_strides, k, k_shape, k_strides, v, v_shape, v_strides, o,
                           o_strides, is_causal != 0, q_offset, has_scale, scale, ws,
                           as_stream(stream));
}

int nne_attention_forward(const float* q, const int64_t q_shape[4], const int64_t q_strides[4],
                          const float* k, const int64_t k_shape[4], const int64_t k_strides[4],
                          const float* v, const int64_t v_shape[4], const int64_t v_strides[4],
                          float* o, const int64_t o_strides[4], int is_causal, int64_t q_offset,
                          int has_scale, float scale, void* stream) {
    return nne_attention_forward_ws(q, q_shape, q_strides, k, k_shape, k_strides, v, v_shape,
                                    v_strides, o, o_strides, is_causal, q_offset, has_scale, scale,
                                    nullptr, stream);
}

int nne_attention_workspace_size(const int64_t q_shape[4], const int64_t k_shape[4], int is_causal,
                                 int64_t q_offset, nne_workspace_size_t* out) {
    if (!out) return fail(NNE_EINVAL, "Invalid configuration or argument: null output pointer");
    *out = nne_workspace_size_t{0, 0};
    const int rc = check_attention_shapes(q_shape, k_shape, k_shape);
    if (rc != NNE_OK) return rc;
    *out = attention_workspace(q_shape, k_shape, is_causal != 0, q_offset);
    return NNE_OK;
}

int nne_counters_init(uint32_t* counters, uint64_t n, void* stream) {
    if (n == 0) return NNE_OK;
    if (!counters) return fail(NNE_EINVAL, "Invalid configuration or argument: null counters");
    const hipError_t e = nne::zero_counters(counters, (int64_t)n, as_stream(stream));
    return e == hipSuccess ? NNE_OK : hip_fail(e, "counter fill");
}

uint64_t nne_stream_resource_bytes(void* stream) {
    const hipStream_t s = as_stream(stream);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    const std::thread::id th =
        s == hipStreamPerThread ? std::this_thread::get_id() : std::thread::id();
    std::lock_guard<std::mutex> lock(g_res_mu);
    uint64_t total = 0;
    for (const auto& r : g_res)
        if (r.dev == dev && r.stream == s && r.thread == th)
            total += (uint64_t)r.n_counters * 4 + r.ws_bytes + r.retired_bytes;
    return total;
}

int nne_kv_append(float* k_cache, float* v_cache, int32_t* lens_dev, int32_t* lens_host,
                  const float* k_new, const int64_t k_new_strides[4], const float* v_new,
                  const int64_t v_new_strides[4], int64_t B, int64_t Hkv, int64_t capacity,
                  int64_t d, int64_t t_new, void* stream) {
    int rc = check_kv_cache_args(B, Hkv, Hkv, capacity, d, false);
    if (rc) return rc;
    if (t_new < 0 || t_new > INT32_MAX)
        return fail(NNE_EINVAL, "Invalid configuration or argument: t_new = %lld", (long long)t_new);
    if (B > 0 && !lens_host)
        return fail(NNE_EINVAL, "Invalid configuration or argument: lens_host is null");
    for (int64_t b = 0; b < B; ++b) {
        if (lens_host[b] < 0 || (int64_t)lens_host[b] + t_new > capacity)
            return fail(NNE_ECAPACITY, "GPU compute error: KV cache append of %lld rows to "
                                       "sequence %lld of length %d exceeds capacity %lld",
                        (long long)t_new, (long long)b, lens_host[b], (long long)capacity);
    }
    if (B == 0 || t_new == 0) return NNE_OK;
    if (!k_cache || !v_cache || !lens_dev || !k_new || !v_new)
        return fail(NNE_EINVAL, "Invalid configuration or argument: null tensor pointer");
    const int64_t shape[4] = {B, Hkv, t_new, d};
    int64_t c[4];
    contiguous_strides(shape, c);
    nne::View4 kn = make_view(k_new, k_new_strides ? k_new_strides : c);
    nne::View4 vn = make_view(v_new, v_new_strides ? v_new_strides : c);
    hipError_t e = nne::launch_kv_append(k_cache, v_cache, lens_dev, kn, vn, (int)B, (int)Hkv,
                                         (int)capacity, (int)d, (int)t_new, as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "KV append launch");
    for (int64_t b = 0; b < B; ++b) lens_host[b] += (int32_t)t_new;
    return NNE_OK;
}

uint64_t nne_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t d, int64_t max_len) {
    if (B <= 0 || Hkv <= 0 || Hq <= 0 || Hq % Hkv != 0 || d <= 0 || d % 4 != 0 || max_len < 0 ||
        B > INT32_MAX || Hq > INT32_MAX || d > INT32_MAX)
        return 0;
    if (nne::splitk_padded_dim((int)d) == 0)   // above 256 dims: the deep kernel's key split
        return deep_workspace_bytes(B, Hq, Hkv, 1, d, max_len > 0 ? (int)((max_len + 31) / 32) : 0, true);
    // One launch's worth: batches and rows beyond one launch run as several.
    const int Bl = (int)std::min<int64_t>(B, nne::splitk_max_seqs());
    const int Rl = (int)std::min<int64_t>(Hq / Hkv, nne::splitk_rows_per_launch((int)d));
    if ((int64_t)Bl * Hkv > INT32_MAX) return 0;
    return nne::splitk_workspace_layout(Bl, (int)Hkv, Rl, (int)d).total_bytes;
}

}  // extern "C"

namespace nne {

// Decode at head dims above 256 (lengths validated, max_len the longest
// sequence after the step): the step's row is appended by the append kernel
// (which advances lens_dev), then the deep kernel attends every sequence to
// its first lens_dev[b] rows, its keys split over several workgroups when the
// batch has too few (sequence, KV head) pairs to fill the device.
int run_decode_deep(const float* q, const int64_t* q_strides, const float* k_cache,
                    const float* v_cache, const int32_t* lens_dev, int32_t* lens_dev_w,
                    const float* k_new, const int64_t* kn_strides, const float* v_new,
                    const int64_t* vn_strides, float* o, const int64_t* o_strides, int64_t B,
                    int64_t Hq, int64_t Hkv, int64_t capacity, int64_t d, int has_scale,
                    float scale, int max_len, const int32_t* seq_keys, const nne_workspace_t* wsp,
                    hipStream_t s) {
    const int64_t qshape[4] = {B, Hq, 1, d};
    const int64_t kvshape[4] = {B, Hkv, 1, d};
    int64_t c[4], ckv[4];
    contiguous_strides(qshape, c);
    contiguous_strides(kvshape, ckv);
    const int64_t* qst = q_strides ? q_strides : c;
    const int64_t* ost = o_strides ? o_strides : c;
    if (!vec_view(q, qst) || !vec_view(o, ost))
        return fail(NNE_EINVAL, "Invalid configuration or argument: decode q/o at head dim %lld "
                                "need unit dim stride, 16-byte alignment and strides that are "
                                "multiples of 4", (long long)d);
    if (!aligned16(k_cache) || !aligned16(v_cache))
        return fail(NNE_EINVAL, "Invalid configuration or argument: KV cache must be 16-byte aligned");
    if (d >= (1 << 25))   // 32 cache rows of a tile are addressed with 32-bit byte offsets
        return fail(NNE_EINVAL, "Invalid configuration or argument: KV cache head dim %lld", (long long)d);
    if (k_new) {
        const nne::View4 kn = make_view(k_new, kn_strides ? kn_strides : ckv);
        const nne::View4 vn = make_view(v_new, vn_strides ? vn_strides : ckv);
        hipError_t e = nne::launch_kv_append(const_cast<float*>(k_cache), const_cast<float*>(v_cache),
                                             lens_dev_w, kn, vn, (int)B, (int)Hkv, (int)capacity,
                                             (int)d, 1, s);
        if (e != hipSuccess) return hip_fail(e, "decode append launch");
    }
    nne::DeepParams p{};
    p.q = make_view(q, qst);
    const int64_t kst[4] = {Hkv * capacity * d, capacity * d, d, 1};
    p.k = make_view(k_cache, kst);
    p.v = make_view(v_cache, kst);
    p.o = make_out(o, ost);
    p.lens = lens_dev;
    p.B = (int)B; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.G = (int)(Hq / Hkv); p.Tq = 1;
    p.Tk = (int)capacity; p.d = (int)d;
    p.qscale = softmax_scale(has_scale, scale, d) * nne::kLog2e;
    const int rc = deep_workspace(p, (max_len + 31) / 32, wsp, s, seq_keys);
    if (rc != NNE_OK) return rc;
    hipError_t e = nne::launch_deep(p, false, device_cus(), s);
    if (e != hipSuccess) return hip_fail(e, "decode attention launch");
    return NNE_OK;
}

// Shared body of the decode entry points.  With a NULL workspace or NULL
// counters the stream's library-side ones are used.
int run_decode(const float* q, const int64_t* q_strides, const float* k_cache, const float* v_cache,
               const int32_t* lens_dev, int32_t* lens_dev_w, int32_t* lens_host, const float* k_new,
               const int64_t* kn_strides, const float* v_new, const int64_t* vn_strides, float* o,
               const int64_t* o_strides, int64_t B, int64_t Hq, int64_t Hkv, int64_t capacity,
               int64_t d, int has_scale, float scale, const nne_workspace_t* wsp, hipStream_t s) {
    int rc = check_kv_cache_args(B, Hq, Hkv, capacity, d, true);
    if (rc) return rc;
    if (B == 0 || Hq == 0) return NNE_OK;
    if (!lens_host)
        return fail(NNE_EINVAL, "Invalid configuration or argument: lens_host is null");
    const bool append = k_new != nullptr;
    if (!q || !o || !k_cache || !v_cache || !lens_dev || (append && !v_new))
        return fail(NNE_EINVAL, "Invalid configuration or argument: null tensor pointer");
    int max_len = 0;
    int64_t total_keys = 0;
    std::vector<int32_t> seq_lens((size_t)B);
    for (int64_t b = 0; b < B; ++b) {
        const int64_t L = (int64_t)lens_host[b] + (append ? 1 : 0);
        if (lens_host[b] < 0 || L > capacity) {
            if (append)
                return fail(NNE_ECAPACITY, "GPU compute error: KV cache append of 1 row to sequence "
                                           "%lld of length %d exceeds capacity %lld",
                            (long long)b, lens_host[b], (long long)capacity);
            return fail(NNE_EINVAL, "Invalid configuration or argument: sequence %lld length %d "
                                    "outside [0, %lld]", (long long)b, lens_host[b],
                        (long long)capacity);
        }
        max_len = std::max(max_len, (int)L);
        total_keys += L * Hkv;
        seq_lens[(size_t)b] = (int32_t)L;
    }
    if (nne::splitk_padded_dim((int)d) == 0) {
        rc = run_decode_deep(q, q_strides, k_cache, v_cache, lens_dev, lens_dev_w, k_new,
                             kn_strides, v_new, vn_strides, o, o_strides, B, Hq, Hkv, capacity, d,
                             has_scale, scale, max_len, seq_lens.data(), wsp, s);
        if (rc == NNE_OK && append)
            for (int64_t b = 0; b < B; ++b) lens_host[b] += 1;
        return rc;
    }
    if (capacity * d >= (1LL << 30))
        return fail(NNE_EINVAL, "Invalid configuration or argument: KV cache rows of one head "
                                "(capacity %lld x d %lld) exceed 2^30 floats",
                    (long long)capacity, (long long)d);
    if (total_keys >= INT32_MAX)
        return fail(NNE_EINVAL, "Invalid configuration or argument: %lld cached rows exceed the "
                                "decode kernel's 2^31 limit", (long long)total_keys);
    const int64_t qshape[4] = {B, Hq, 1, d};
    const int64_t kvshape[4] = {B, Hkv, 1, d};
    int64_t c[4], ckv[4];
    contiguous_strides(qshape, c);
    contiguous_strides(kvshape, ckv);
    const int64_t* qst = q_strides ? q_strides : c;
    const int64_t* ost = o_strides ? o_strides : c;
    const int64_t* knst = kn_strides ? kn_strides : ckv;
    const int64_t* vnst = vn_strides ? vn_strides : ckv;
    if (qst[3] != 1 || ost[3] != 1)
        return fail(NNE_EINVAL, "Invalid configuration or argument: decode q/o need unit dim stride");
    // The 16-row tiles (more than 4 query heads per KV head, or d > 128) read
    // q rows as 16-byte vectors.
    if ((Hq / Hkv > 4 || d > 128) && !vec_view(q, qst))
        return fail(NNE_EINVAL, "Invalid configuration or argument: decode q needs 16-byte alignment "
                                "and strides that are multiples of 4");
    if (!aligned16(k_cache) || !aligned16(v_cache))
        return fail(NNE_EINVAL, "Invalid configuration or argument: KV cache must be 16-byte aligned");
    if (append && (!vec_view(k_new, knst) || !vec_view(v_new, vnst)))
        return fail(NNE_EINVAL, "Invalid configuration or argument: new K/V rows need unit dim "
                                "stride, 16-byte alignment and strides that are multiples of 4");

    nne::SplitKParams p{};
    p.q = make_view(q, qst);
    p.k = k_cache; p.v = v_cache;
    p.ksb = Hkv * capacity * d; p.ksh = capacity * d; p.kst = d;
    p.vsb = p.ksb; p.vsh = p.ksh; p.vst = p.kst;
    p.lens = lens_dev;
    p.tk = 0;
    p.max_keys = max_len;
    p.o = make_out(o, ost);
    p.B = (int)B; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.Tq = 1; p.d = (int)d;
    p.qscale = softmax_scale(has_scale, scale, d) * nne::kLog2e;
    if (append) {
        p.k_new = k_new; p.v_new = v_new;
        p.kn_sb = knst[0]; p.kn_sh = knst[1];
        p.vn_sb = vnst[0]; p.vn_sh = vnst[1];
        p.lens_w = lens_dev_w;
    }
    nne_workspace_size_t need{0, 0};
    rc = nne_decode_workspace_size(B, Hq, Hkv, d, &need);
    if (rc != NNE_OK) return rc;
    void* ws = nullptr;
    uint32_t* counters = nullptr;
    rc = call_workspace(wsp, need.records_bytes, (int64_t)need.n_counters, s, &ws, &counters,
                        "decode");
    if (rc != NNE_OK) return rc;
    hipError_t e = nne::launch_splitk(p, total_keys, max_len, ws, s, seq_lens.data(), counters);
    if (e != hipSuccess) return hip_fail(e, "decode attention launch");
    if (append)
        for (int64_t b = 0; b < B; ++b) lens_host[b] += 1;
    return NNE_OK;
}

}  // namespace nne

extern "C" {


int nne_decode_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t d,
                              nne_workspace_size_t* out) {
    if (!out) return fail(NNE_EINVAL, "Invalid configuration or argument: null output pointer");
    *out = nne_workspace_size_t{0, 0};
    // Head dims above 256 (the deep kernel): records of its key split (zero
    // for batches that fill the device without one), no counters.
    if (B > 0 && Hkv > 0 && Hq > 0 && Hq % Hkv == 0 && d > 256 && d % 4 == 0 && B <= INT32_MAX &&
        Hq <= INT32_MAX && d <= INT32_MAX) {
        out->records_bytes = nne_decode_workspace_bytes(B, Hq, Hkv, d, 0);
        return NNE_OK;
    }
    const uint64_t bytes = nne_decode_workspace_bytes(B, Hq, Hkv, d, 0);
    if (bytes == 0)
        return fail(NNE_EINVAL, "Invalid configuration or argument: no decode kernel for B=%lld "
                                "Hq=%lld Hkv=%lld d=%lld", (long long)B, (long long)Hq,
                    (long long)Hkv, (long long)d);
    out->records_bytes = bytes;
    out->n_counters = (uint64_t)std::min<int64_t>(B, nne::splitk_max_seqs()) * (uint64_t)Hkv;
    return NNE_OK;
}

int nne_decode_attention(const float* q, const int64_t q_strides[4], const float* k_cache,
                         const float* v_cache, const int32_t* lens_dev, const int32_t* lens_host,
                         float* o, const int64_t o_strides[4], int64_t B, int64_t Hq, int64_t Hkv,
                         int64_t capacity, int64_t d, int has_scale, float scale,
                         const nne_workspace_t* ws, void* stream) {
    return nne::run_decode(q, q_strides, k_cache, v_cache, lens_dev, nullptr,
                           const_cast<int32_t*>(lens_host), nullptr, nullptr, nullptr, nullptr, o,
                           o_strides, B, Hq, Hkv, capacity, d, has_scale, scale, ws,
                           as_stream(stream));
}

int nne_decode_step(const float* q, const int64_t q_strides[4], float* k_cache, float* v_cache,
                    int32_t* lens_dev, int32_t* lens_host, const float* k_new,
                    const int64_t k_new_strides[4], const float* v_new,
                    const int64_t v_new_strides[4], float* o, const int64_t o_strides[4],
                    int64_t B, int64_t Hq, int64_t Hkv, int64_t capacity, int64_t d,
                    int has_scale, float scale, const nne_workspace_t* ws, void* stream) {
    if (!k_new || !v_new)
        return fail(NNE_EINVAL, "Invalid configuration or argument: decode step needs k_new and v_new");
    return nne::run_decode(q, q_strides, k_cache, v_cache, lens_dev, lens_dev, lens_host, k_new,
                           k_new_strides, v_new, v_new_strides, o, o_strides, B, Hq, Hkv, capacity,
                           d, has_scale, scale, ws, as_stream(stream));
}

// ---- decode prologue: projections and rotary position embedding ----------

int nne_rope_tables(float* cos_out, float* sin_out, int64_t max_seq_len, int64_t head_dim,
                    float theta) {
    // RotaryEmbedding::new (llama.rs:74-107); the reference asserts an even
    // head_dim (:75).
    if (head_dim <= 0 || head_dim % 2 != 0)
        return fail(NNE_EINVAL, "Invalid configuration or argument: RoPE head_dim (%lld) must be "
                                "even", (long long)head_dim);
    if (max_seq_len < 0)
        return fail(NNE_EINVAL, "Invalid configuration or argument: RoPE max_seq_len %lld",
                    (long long)max_seq_len);
    if (max_seq_len > 0 && (!cos_out || !sin_out))
        return fail(NNE_EINVAL, "Invalid configuration or argument: null table pointer");
    nne::rope_tables_host(cos_out, sin_out, max_seq_len, head_dim, theta);
    return NNE_OK;
}

namespace {

// RotaryEmbedding::apply's checks (llama.rs:115-139) for rows
// [start, start + t) of every sequence.
int check_rope_range(const int32_t* start_host, int64_t B, int64_t t, int64_t max_seq_len) {
    if (B > 0 && !start_host)
        return fail(NNE_EINVAL, "Invalid configuration or argument: start positions are null");
    for (int64_t b = 0; b < B; ++b) {
        const int64_t s = start_host[b];
        if (s < 0 || s + t > max_seq_len)
            return fail(NNE_EINVAL, "Invalid configuration or argument: Sequence range [%lld, %lld) "
                                    "exceeds RoPE max_seq_len %lld",
                        (long long)s, (long long)(s + t), (long long)max_seq_len);
    }
    return NNE_OK;
}

}  // namespace

int nne_rope_apply(const float* x, const int64_t x_shape[4], const int64_t x_strides[4], float* out,
                   const int64_t out_strides[4], const float* cos_table, const float* sin_table,
                   int64_t max_seq_len, int64_t table_head_dim, const int32_t* start_dev,
                   const int32_t* start_host, void* stream) {
    if (!x_shape)
        return fail(NNE_EINVAL, "Invalid configuration or argument: RoPE apply expects 4D tensor "
                                "[Batch, Heads, SeqLen, HeadDim]");
    if (!dims_ok(x_shape))
        return fail(NNE_EINVAL, "Invalid configuration or argument: RoPE dims out of range, got %s",
                    shape_str(x_shape).c_str());
    const int64_t B = x_shape[0], H = x_shape[1], T = x_shape[2], d = x_shape[3];
    if (d != table_head_dim)   // llama.rs:119-124
        return fail(NNE_ESHAPE, "Shape mismatch error: expected shape [%lld], got [%lld]",
                    (long long)table_head_dim, (long long)d);
    if (d % 2 != 0)
        return fail(NNE_EINVAL, "Invalid configuration or argument: RoPE head_dim (%lld) must be "
                                "even", (long long)d);
    int rc = check_rope_range(start_host, B, T, max_seq_len);
    if (rc) return rc;
    if (B * H * T * d == 0) return NNE_OK;
    if (!x || !out || !cos_table || !sin_table || !start_dev)
        return fail(NNE_EINVAL, "Invalid configuration or argument: null tensor pointer");
    int64_t c[4];
    contiguous_strides(x_shape, c);
    hipError_t e = nne::launch_rope_apply(make_view(x, x_strides ? x_strides : c),
                                          make_out(out, out_strides ? out_strides : c), (int)B,
                                          (int)H, (int)T, (int)d, cos_table, sin_table, start_dev,
                                          as_stream(stream));
    return e == hipSuccess ? NNE_OK : hip_fail(e, "RoPE launch");
}

namespace {

// Shared checks of the packed-projection entry points.
int check_qkv_geometry(int64_t C, int64_t Hq, int64_t Hkv, int64_t d) {
    if (C <= 0 || Hq <= 0 || Hkv <= 0 || d <= 0 || C > INT32_MAX || Hq > INT32_MAX ||
        Hkv > INT32_MAX || (Hq + 2 * Hkv) * d > INT32_MAX || (Hq + 2 * Hkv) * d * C > INT64_MAX / 8)
        return fail(NNE_EINVAL, "Invalid configuration or argument: bad projection geometry "
                                "C=%lld Hq=%lld Hkv=%lld d=%lld", (long long)C, (long long)Hq,
                    (long long)Hkv, (long long)d);
    if (d % 64 != 0 || C % 64 != 0)
        return fail(NNE_EINVAL, "Invalid configuration or argument: the fused projection needs a "
                                "head dim (got %lld) and a d_model (got %lld) that are multiples "
                                "of 64", (long long)d, (long long)C);
    return NNE_OK;
}

int device_cus() {
    static std::atomic<int> cached[64];   // callers on several threads may fill it at once
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int cus = cached[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cached[dev].store(cus, std::memory_order_relaxed);
    }
    return cus;
}

}  // namespace

uint64_t nne_qkv_packed_bytes(int64_t C, int64_t Hq, int64_t Hkv, int64_t d) {
    if (check_qkv_geometry(C, Hq, Hkv, d) != NNE_OK) return 0;
    return 4 * nne::qkv_packed_floats((int)C, (int)Hq, (int)Hkv, (int)d);
}

int nne_qkv_pack(const float* wq, const float* wk, const float* wv, float* packed, int64_t C,
                 int64_t Hq, int64_t Hkv, int64_t d, void* stream) {
    int rc = check_qkv_geometry(C, Hq, Hkv, d);
    if (rc) return rc;
    if (!wq || !wk || !wv || !packed)
        return fail(NNE_EINVAL, "Invalid configuration or argument: null tensor pointer");
    if (!aligned16(wq) || !aligned16(wk) || !aligned16(wv) || !aligned16(packed))
        return fail(NNE_EINVAL, "Invalid configuration or argument: weights must be 16-byte aligned");
    hipError_t e = nne::launch_qkv_pack(wq, wk, wv, packed, (int)C, (int)Hq, (int)Hkv, (int)d,
                                        as_stream(stream));
    return e == hipSuccess ? NNE_OK : hip_fail(e, "weight packing launch");
}

int nne_qkv_workspace_size(int64_t C, int64_t Hq, int64_t Hkv, int64_t d, nne_workspace_size_t* out) {
    if (!out) return fail(NNE_EINVAL, "Invalid configuration or argument: null output pointer");
    *out = nne_workspace_size_t{0, 0};
    const int rc = check_qkv_geometry(C, Hq, Hkv, d);
    if (rc) return rc;
    const nne::QkvWorkspace w = nne::qkv_workspace((int)C, (int)Hq, (int)Hkv, (int)d, device_cus());
    out->records_bytes = w.floats * 4;
    out->n_counters = (uint64_t)w.n_tiles;
    return NNE_OK;
}

int nne_qkv_rope(const float* x, int64_t x_row_stride, const float* w_packed, const float* bq,
                 const float* bk, const float* bv, const float* cos_table, const float* sin_table,
                 int64_t max_seq_len, int64_t table_head_dim, const int32_t* pos_dev,
                 const int32_t* pos_host, float* q_out, float* k_out, float* v_out, int64_t B,
                 int64_t C, int64_t Hq, int64_t Hkv, int64_t d, void* stream) {
    return nne_qkv_rope_ws(x, x_row_stride, w_packed, bq, bk, bv, cos_table, sin_table, max_seq_len,
                           table_head_dim, pos_dev, pos_host, q_out, k_out, v_out, B, C, Hq, Hkv, d,
                           nullptr, stream);
}

int nne_qkv_rope_ws(const float* x, int64_t x_row_stride, const float* w_packed, const float* bq,
                    const float* bk, const float* bv, const float* cos_table, const float* sin_table,
                    int64_t max_seq_len, int64_t table_head_dim, const int32_t* pos_dev,
                    const int32_t* pos_host, float* q_out, float* k_out, float* v_out, int64_t B,
                    int64_t C, int64_t Hq, int64_t Hkv, int64_t d, const nne_workspace_t* wsp,
                    void* stream) {
    if (B < 0 || B > INT32_MAX)
        return fail(NNE_EINVAL, "Invalid configuration or argument: batch %lld", (long long)B);
    const bool rope = cos_table || sin_table;
    if (rope && d != table_head_dim)   // llama.rs:119-124
        return fail(NNE_ESHAPE, "Shape mismatch error: expected shape [%lld], got [%lld]",
                    (long long)table_head_dim, (long long)d);
    int rc = check_qkv_geometry(C, Hq, Hkv, d);
    if (rc) return rc;
    if (rope) {
        rc = check_rope_range(pos_host, B, 1, max_seq_len);
        if (rc) return rc;
    }
    if (B == 0) return NNE_OK;
    if (!x || !w_packed || !q_out || !k_out || !v_out || (rope && (!cos_table || !sin_table || !pos_dev)))
        return fail(NNE_EINVAL, "Invalid configuration or argument: null tensor pointer");
    if (x_row_stride < C || x_row_stride % 4 != 0 || !aligned16(x) || !aligned16(w_packed))
        return fail(NNE_EINVAL, "Invalid configuration or argument: x rows and packed weights "
                                "must be 16-byte aligned with a row stride >= d_model and a "
                                "multiple of 4");
    const nne::QkvWorkspace w = nne::qkv_workspace((int)C, (int)Hq, (int)Hkv, (int)d, device_cus());
    uint32_t* counters = nullptr;
    void* ws = nullptr;
    rc = call_workspace(wsp, w.floats * 4, w.n_tiles, as_stream(stream), &ws, &counters,
                        "projection");
    if (rc != NNE_OK) return rc;
    nne::QkvParams p{};
    p.x = x;
    p.x_rs = x_row_stride;
    p.wp = w_packed;
    p.bias[0] = bq; p.bias[1] = bk; p.bias[2] = bv;
    p.cos = rope ? cos_table : nullptr;
    p.sin = rope ? sin_table : nullptr;
    p.pos = rope ? pos_dev : nullptr;
    p.out[0] = q_out; p.out[1] = k_out; p.out[2] = v_out;
    p.o_sb[0] = Hq * d; p.o_sh[0] = d;
    p.o_sb[1] = Hkv * d; p.o_sh[1] = d;
    p.o_sb[2] = Hkv * d; p.o_sh[2] = d;
    p.M = (int)B; p.C = (int)C; p.Hq = (int)Hq; p.Hkv = (int)Hkv; p.d = (int)d;
    p.n_tiles = w.n_tiles; p.S = w.S; p.kc_per_slice = w.kc_per_slice;
    p.ws = static_cast<float*>(ws);
    p.cnt = counters;
    const hipError_t e = nne::launch_qkv_rope(p, as_stream(stream));
    return e == hipSuccess ? NNE_OK : hip_fail(e, "q/k/v projection launch");
}

}  // extern "C"
