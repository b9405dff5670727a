// Decode step that allocates nothing: nne_decode_step_noalloc.
//
// nne_decode_step keeps its split-K partial records in a caller workspace or
// in memory the library allocates per stream, and its arrival counters in
// library-allocated memory.  Callers that cannot allocate device memory at
// call time (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc) use this variant instead: records and counters live
// in `scratch`, a file-scope device array of NNE_NOALLOC_SCRATCH_BYTES, of
// which every GPU the library runs on holds one copy until the process ends.
//
// In host code `scratch` names a host-side stand-in, not device memory: the
// device address of each GPU's copy is looked up once per device with
// hipGetSymbolAddress (with that device current) and only that address is
// handed to kernels.
//
// Every call on a GPU uses that GPU's one array, so calls that overlap in
// time on one GPU -- on any streams, from any threads -- race and must be
// serialised by the caller.  The array keeps the last call's contents; each
// call clears the arrival counters it uses with a fill kernel before its
// launch (a kernel, not a memset).  The call plans the step on the host from
// lens_host and advances lens_host itself, so a graph captured from one call
// replays that one step for the same lengths; it does not advance.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "nne_abi_internal.hpp"
#include "nne_attn.h"
#include "nne_launch.hpp"

namespace {

constexpr uint64_t kScratchBytes = NNE_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0, "scratch is carved in 256-byte units");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];   // device address of each GPU's `scratch`

// Device address of the current device's copy of `scratch`.
int scratch_address(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return nne::fail_hip(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return nne::fail_message(NNE_EINVAL, "Invalid configuration or argument: device index out "
                                             "of range for the no-allocation scratch");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return nne::fail_hip(e, "hipGetSymbolAddress(scratch)");
        if (!p)
            return nne::fail_message(NNE_EHIP, "GPU compute error: no device address for the "
                                               "no-allocation scratch");
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return NNE_OK;
}

}  // namespace

extern "C" int nne_decode_step_noalloc(const float* q, const int64_t q_strides[4], float* k_cache,
                                       float* v_cache, int32_t* lens_dev, int32_t* lens_host,
                                       const float* k_new, const int64_t k_new_strides[4],
                                       const float* v_new, const int64_t v_new_strides[4], float* o,
                                       const int64_t o_strides[4], int64_t B, int64_t Hq, int64_t Hkv,
                                       int64_t capacity, int64_t d, int has_scale, float scale,
                                       void* stream) {
    if (!k_new || !v_new)
        return nne::fail_message(NNE_EINVAL, "Invalid configuration or argument: decode step needs "
                                             "k_new and v_new");
    // [arrival counters (B * Hkv, 256-byte aligned)][split-K workspace].
    // Geometry the decode kernel does not take reports 0 bytes and is
    // refused by the validation in run_decode.
    nne_workspace_size_t need{0, 0};
    const uint64_t ws_bytes =
        nne_decode_workspace_size(B, Hq, Hkv, d, &need) == NNE_OK ? need.records_bytes : 0;
    const uint64_t cnt_bytes = ws_bytes ? (need.n_counters * 4 + 255) / 256 * 256 : 0;
    // Above 256 dims the records only allow a key split: a smaller scratch
    // gives fewer parts (none at worst), so those steps are never refused.
    const bool deep = d > 256;
    if (!deep && cnt_bytes + ws_bytes > kScratchBytes) {
        char msg[256];
        snprintf(msg, sizeof(msg),
                 "Invalid configuration or argument: decode step needs %llu bytes of scratch, more "
                 "than the no-allocation entry point's %llu (use nne_decode_step with a workspace)",
                 (unsigned long long)(cnt_bytes + ws_bytes), (unsigned long long)kScratchBytes);
        return nne::fail_message(NNE_EINVAL, msg);
    }
    void* base = nullptr;
    int rc = scratch_address(&base);
    if (rc != NNE_OK) return rc;
    uint32_t* counters = static_cast<uint32_t*>(base);
    void* ws = static_cast<char*>(base) + cnt_bytes;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (ws_bytes > 0 && need.n_counters > 0) {
        const hipError_t e = nne::zero_counters(counters, (int64_t)need.n_counters, s);
        if (e != hipSuccess) return nne::fail_hip(e, "no-allocation counter clear");
    }
    const nne_workspace_t scratch_ws{ws, kScratchBytes - cnt_bytes, counters,
                                     (uint64_t)(cnt_bytes / 4)};
    return nne::run_decode(q, q_strides, k_cache, v_cache, lens_dev, lens_dev, lens_host, k_new,
                           k_new_strides, v_new, v_new_strides, o, o_strides, B, Hq, Hkv, capacity,
                           d, has_scale, scale, &scratch_ws, s);
}
