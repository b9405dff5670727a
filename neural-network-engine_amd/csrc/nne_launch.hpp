// Host-side launchers of the attention kernels (called by the C ABI in abi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nne_common.hpp"

namespace nne {

// Head dims are padded to the next of {32, 64, 128}; 0 = unsupported.
int prefill_padded_dim(int d);
int splitk_padded_dim(int d);
int splitk_max_rows();

// `vec` selects 16-byte loads/stores: requires dim stride 1, d % 4 == 0,
// 16-byte aligned base pointers and row/head/batch strides that are multiples of 4.
hipError_t launch_prefill(PrefillParams p, bool causal, bool vec, hipStream_t stream);

// Split-K workspace: per-sequence prefix (B+1 ints) and partial records for
// up to splitk_max_workgroups() + B*Hkv (workgroup, head) pairs.
// Workspace: [prefix (B+1) int32][partial (max, sum)][partial O].
struct SplitKWorkspace {
    uint64_t ml_offset;
    uint64_t o_offset;
    uint64_t total_bytes;
};
int splitk_max_seqs();
int splitk_max_workgroups();
SplitKWorkspace splitk_workspace_layout(int B, int Hkv, int R, int d);
// Launches the split kernel over total_keys flattened (sequence, KV head, key)
// rows.  With counters (B*Hkv zeroed arrival counters, left zeroed) and at
// most kArgSeqs sequences, the last workgroup of each split head merges it;
// otherwise the per-head combine kernel follows.  max_len bounds every sequence.
// seq_lens (host) are this launch's key counts per sequence (including a
// decode step's new row), or null when every sequence has p.tk keys.
hipError_t launch_splitk(SplitKParams p, int64_t total_keys, int max_len, void* workspace,
                         hipStream_t stream, const int32_t* seq_lens, uint32_t* counters);

// Zeroes n counters with a fill kernel on the stream.
hipError_t zero_counters(uint32_t* counters, int64_t n, hipStream_t stream);

hipError_t launch_kv_append(float* kc, float* vc, int32_t* lens_dev, View4 kn, View4 vn, int B,
                            int Hkv, int cap, int d, int t_new, hipStream_t stream);

}  // namespace nne
