// Pieces of the C ABI (abi.cpp) that other sources of the library share.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nne_attn.h"

namespace nne {

// Sets the calling thread's nne_last_error() message and returns `code`.
int fail_message(int code, const char* msg);
int fail_hip(hipError_t e, const char* what);

// Body of nne_decode_attention / nne_decode_step (k_new == NULL: attention
// only).  Validates every argument, then launches.  A NULL workspace makes
// the call use the stream's library-side one.
int run_decode(const float* q, const int64_t* q_strides, const float* k_cache, const float* v_cache,
               const int32_t* lens_dev, int32_t* lens_dev_w, int32_t* lens_host, const float* k_new,
               const int64_t* kn_strides, const float* v_new, const int64_t* vn_strides, float* o,
               const int64_t* o_strides, int64_t B, int64_t Hq, int64_t Hkv, int64_t capacity,
               int64_t d, int has_scale, float scale, const nne_workspace_t* ws, hipStream_t s);

}  // namespace nne
