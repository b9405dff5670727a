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

// Keys handled by one split-K workgroup for a given longest sequence and
// number of (sequence, KV head) pairs.
int splitk_keys_per_split(int max_len, int n_heads);
uint64_t splitk_workspace_bytes(int B, int Hkv, int R, int d, int max_len, int keys_per_split);
hipError_t launch_splitk(SplitKParams p, int max_len, int keys_per_split, void* workspace,
                         hipStream_t stream);

hipError_t launch_kv_append(float* kc, float* vc, int32_t* lens_dev, View4 kn, View4 vn, int B,
                            int Hkv, int cap, int d, int t_new, hipStream_t stream);

}  // namespace nne
