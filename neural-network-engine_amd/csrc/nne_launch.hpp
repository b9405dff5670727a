// Host-side launchers of the attention kernels (called by the C ABI in abi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "deep_plan.hpp"
#include "nne_common.hpp"

namespace nne {

// Head dims are padded to the next of {32, 64, 128} (prefill) or
// {64, 128, 256} (split-K); 0 = unsupported.
int prefill_padded_dim(int d);
int splitk_padded_dim(int d);
// Query rows per KV head the few-query prefill routes to the split-K kernel.
int splitk_max_rows();
// Query rows per KV head one split-K launch serves (more go in further launches).
int splitk_rows_per_launch(int d);

// `vec` selects 16-byte loads/stores: requires dim stride 1, d % 4 == 0,
// 16-byte aligned base pointers and row/head/batch strides that are multiples of 4.
hipError_t launch_prefill(PrefillParams p, bool causal, bool vec, hipStream_t stream);
// Head dims 129..256 (16-byte vector views): the wave-pair MFMA kernel.
hipError_t launch_prefill_wide(PrefillParams p, bool causal, hipStream_t stream);
// Head dims above 256 (deep.hip; d % 4 == 0, 16-byte vector views of Q, K,
// V and O): prefill, cross-attention and decode over a KV cache (p.lens).
// The key-split plans (deep_plan.hpp) fill p.n_split and its fields first;
// launch_deep fills the schedule fields and runs the kernel (and the combine
// kernel after a split) on a device of `cus` CUs.
hipError_t launch_deep(DeepParams p, bool causal, int cus, hipStream_t stream);
// Key-split plan for a prefill problem too small to fill the device (fills
// p.n_chunks / p.chunk_tiles; n_chunks stays 0 when the problem is large
// enough).  The caller then sets p.ws (ws_bytes) and p.cnt (n_counters zeroed
// counters) before launch_prefill; without them the split is not used.
struct PrefillSplit {
    uint64_t ws_bytes;
    int64_t n_counters;
};
PrefillSplit prefill_split_plan(PrefillParams& p, bool causal, bool vec);

// Prefill of a problem too small to fill the device (small.hip): one
// workgroup per (sequence, query head, 16-row block), whose waves split the
// block's key tiles and merge in LDS (no workspace).  small_prefill_fits says
// whether the problem is one (16-byte vector views, d <= 128, at most one
// workgroup per CU, at most two key tiles per wave).
bool small_prefill_fits(const PrefillParams& p, bool vec, int cus);
hipError_t launch_small_prefill(PrefillParams p, bool causal, int cus, hipStream_t stream);

// Split-K workspace of one launch (at most splitk_max_seqs() sequences and
// splitk_rows_per_launch() rows): per-sequence prefix (B+1 ints) and partial
// records for up to (workgroups of a launch) + B*Hkv (workgroup, head) pairs.
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
// Batches beyond splitk_max_seqs() and rows beyond splitk_rows_per_launch()
// take several launches in stream order, with the workspace and counters of
// one.
// seq_lens (host) are this launch's key counts per sequence (including a
// decode step's new row), or null when every sequence has p.tk keys.
// row_begin / row_count restrict the launch to a range of each KV head's
// G * Tq rows (row_count < 0: all of them).
hipError_t launch_splitk(SplitKParams p, int64_t total_keys, int max_len, void* workspace,
                         hipStream_t stream, const int32_t* seq_lens, uint32_t* counters,
                         int row_begin = 0, int row_count = -1);

// Zeroes n counters with a fill kernel on the stream.
hipError_t zero_counters(uint32_t* counters, int64_t n, hipStream_t stream);

hipError_t launch_kv_append(float* kc, float* vc, int32_t* lens_dev, View4 kn, View4 vn, int B,
                            int Hkv, int cap, int d, int t_new, hipStream_t stream);

// Decode prologue (qkv.hip).  Requires d % 64 == 0, C % 64 == 0, 16-byte
// aligned x rows; any M (launched in groups of qkv_max_rows_per_launch()).
int qkv_max_rows_per_launch();
uint64_t qkv_packed_floats(int C, int Hq, int Hkv, int d);
hipError_t launch_qkv_pack(const float* wq, const float* wk, const float* wv, float* packed, int C,
                           int Hq, int Hkv, int d, hipStream_t stream);
struct QkvWorkspace {
    int n_tiles, S, kc_per_slice;
    uint64_t floats;   // partial tiles (0 when S == 1)
};
QkvWorkspace qkv_workspace(int C, int Hq, int Hkv, int d, int cus);
hipError_t launch_qkv_rope(QkvParams p, hipStream_t stream);
// RoPE tables of RotaryEmbedding::new, computed on the host ([max_seq_len, d]).
void rope_tables_host(float* cos_out, float* sin_out, int64_t max_seq_len, int64_t d, float theta);
// RoPE on a strided [B, H, T, d] view (d even); row t of sequence b at table
// row pos[b] + t.  o may alias x with the same strides.
hipError_t launch_rope_apply(View4 x, OutView4 o, int B, int H, int T, int d, const float* cos_t,
                             const float* sin_t, const int32_t* pos, hipStream_t stream);

}  // namespace nne
