// Host-side layout of a split-K launch: whole heads packed per workgroup,
// cut chunks, or equal chunks of the flattened (sequence, KV head, key) rows.
// Plain C++ (no HIP), shared by splitk.hip and the planner's tests.
#pragma once

#include <stdint.h>

#include "nne_params.hpp"

namespace nne {

// Greedy grouping of the heads, in flattened order, into groups whose cost
// (keys + ovh per head) is at most x: the number of groups, and with `first`
// their first heads (first[groups] = B * Hkv).
int pack_groups(const SplitKParams& p, int64_t x, int64_t ovh, uint16_t* first);
// At most two whole heads per workgroup, the longest alone and the rest
// paired longest with shortest: the costliest workgroup (INT64_MAX if the
// heads with keys outnumber twice the slots), with `pairs` (2 per workgroup,
// 0xFFFF: none) and *n_wg.
int64_t pair_heads(const SplitKParams& p, int slots, int64_t ovh, uint16_t* pairs, int* n_wg);
// Whole-head packing when its estimate beats chunks (fused launches with the
// prefix in the arguments): sets packed (1: flattened runs, 2: pairs), n_wg,
// pack_head.
bool plan_packing(SplitKParams& p, int slots, int64_t total_keys);
// The cut with budget x: its workgroup count (with `ends`, their chunk ends),
// or max_wg + 1 if it needs more workgroups or gives a head more than
// max_parts of them.
int cut_chunks(const SplitKParams& p, int64_t x, int64_t ovh, int max_wg, int* ends);
// Cut chunks (fused launches with the prefix in the arguments): sets cut,
// chunk, n_wg, chunk_end.
bool plan_cut(SplitKParams& p, int slots, int64_t total_keys, int max_len);
// Equal chunks: sets chunk, n_wg.
void plan_equal(SplitKParams& p, int slots, int64_t total_keys, int max_len);
// packed, else cut, else equal chunks, over at most `slots` workgroups.
void plan_split_layout(SplitKParams& p, int slots, int64_t total_keys, int max_len);
// Per-segment cost of the cut, in keys at head dim d.
int64_t cut_segment_keys(int d);

}  // namespace nne
