// Shared device helpers of the attention kernels; the launch-parameter
// structs and layout conventions are in nne_params.hpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nne_params.hpp"

namespace nne {

typedef float floatx16 __attribute__((ext_vector_type(16)));
// Native 4-float vector for register tiles and 16-byte loads/stores.  (HIP's
// float4 is a struct whose copies lower to memcpy through private memory,
// which can keep register arrays of it out of registers.)
typedef float vf4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// Brings [B0, E0) and [B1, E1) of the kernel argument block into the scalar
// cache: one load per 64-byte line, all issued before a single wait.  The
// arguments read later then hit there instead of each first use paying a
// memory round trip in a dependent chain (about 1 us apiece at a launch).
template <int B0, int E0, int B1, int E1>
__device__ __forceinline__ void warm_kernargs() {
    typedef const __attribute__((address_space(4))) int kernarg_int;
    kernarg_int* kp = (kernarg_int*)__builtin_amdgcn_kernarg_segment_ptr();
    constexpr int N0 = (E0 - B0 + 63) / 64, N1 = (E1 - B1 + 63) / 64;
    int v[N0 + N1];
#pragma unroll
    for (int i = 0; i < N0; ++i) v[i] = kp[(B0 + 64 * i) / 4];
#pragma unroll
    for (int i = 0; i < N1; ++i) v[N0 + i] = kp[(B1 + 64 * i) / 4];
#pragma unroll
    for (int i = 0; i < N0 + N1; ++i) asm volatile("" ::"s"(v[i]));
}
template <int B0, int E0>
__device__ __forceinline__ void warm_kernargs() {
    warm_kernargs<B0, E0, E0, E0>();
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Partial records cross workgroups without a fence: they are written with
// agent-scope relaxed atomic stores (global_store sc1, written through to the
// device coherence point) and read with agent-scope relaxed atomic loads
// (global_load sc1, never served from a stale per-XCD L2 line).  A writer waits
// for its stores (vmcnt(0)) before its arrival is counted, and a reader loads
// only after the count says every writer has arrived.  An agent-scope
// release/acquire pair would also write back and invalidate the whole L2 of
// each XCD, which costs tens of microseconds per launch.
__device__ __forceinline__ void store_coherent(float* p, float x) {
    __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16-byte form of load_coherent: a buffer load with the same sc1 policy
// (buffer_load_dwordx4 ... sc1) from a range of `bytes` bytes at `base`
// (offsets past the range read as zero).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_range(const float* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ vf4 load_coherent4(__amdgpu_buffer_rsrc_t range, uint32_t byte_offset) {
    return __builtin_bit_cast(vf4, __builtin_amdgcn_raw_buffer_load_b128(range, byte_offset, 0, 16));
}
__device__ __forceinline__ float2 load_coherent2(__amdgpu_buffer_rsrc_t range, uint32_t byte_offset) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(range, byte_offset, 0, 16);
    return float2{__uint_as_float(v[0]), __uint_as_float(v[1])};
}
__device__ __forceinline__ void wait_stores_performed() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0), expcnt/lgkmcnt unconstrained
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}


// Swaps lanes 32..63 of `a` with lanes 0..31 of `b` (gfx950 v_permlane32_swap).
// Called with a == b == x, element 0 of the result holds x from lanes 0..31 in
// both halves and element 1 holds x from lanes 32..63 in both halves, so
// combining the two elements reduces over the lane pair (l, l ^ 32).
__device__ __forceinline__ float pair_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float pair_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace nne
