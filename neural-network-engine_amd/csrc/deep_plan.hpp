// Host-side key-split plans of the deep kernel (head dims above 256, deep.hip):
// plain C++ (no HIP), shared by the C ABI and the planner's CPU tests.
#pragma once

#include <stdint.h>

#include "nne_params.hpp"

namespace nne {

// Equal key split of a problem with too few workgroups to fill the device:
// fills p.n_split / p.split_tiles / p.rpu for units of at most max_tiles
// 32-key tiles, with records of at most max_bytes, and returns the record
// bytes (0: no split; p.n_split = 1).  The caller sets p.ws when non-zero.
uint64_t deep_split_plan(DeepParams& p, int max_tiles, int cus, uint64_t max_bytes);
// Ragged key split of a decode step (seq_keys: host key counts per sequence
// after the step): fills p.ragged / p.part_prefix / p.split_tiles / p.rpu and
// returns the record bytes, or 0 (p.ragged = 0) when the step does not gain
// from it.
uint64_t deep_ragged_plan(DeepParams& p, const int32_t* seq_keys, int cus, uint64_t max_bytes);

}  // namespace nne
