// Key-split plans of the deep kernel (deep.hip), host side, plain C++.
#include "deep_plan.hpp"

namespace nne {

// Problems with at most half as many workgroups as CUs (decode steps of
// small batches, few-query cross-attention) split each unit's keys into up to
// kDeepMaxSplit parts of at least 4 tiles, one round of workgroups over the
// CUs, as far as max_bytes of records allow.  (Measured at d = 512, decode
// over L ~ U[512, 4096]: B = 8 601 -> 190 us with 4 parts; at B = 32, where
// every CU already has a head, 4 parts per head cost 667 -> 775 us: each
// extra workgroup pays its cold start, its record and the merge.)
uint64_t deep_split_plan(DeepParams& p, int max_tiles, int cus, uint64_t max_bytes) {
    p.n_split = 1;
    p.split_tiles = 0;
    const int64_t rows = (int64_t)p.G * p.Tq;
    p.rpu = (int)(rows < 32 ? rows : 32);
    const int64_t wg = (int64_t)p.B * p.Hkv * ((rows + 31) / 32) * ((p.d + kDeepChunk - 1) / kDeepChunk);
    if (wg == 0 || 2 * wg > (int64_t)cus || max_tiles < 8) return 0;
    int64_t sp = (int64_t)cus / wg;
    if (sp > kDeepMaxSplit) sp = kDeepMaxSplit;
    if (sp > max_tiles / 4) sp = max_tiles / 4;
    const uint64_t per = (uint64_t)wg * (uint64_t)p.rpu * (kDeepChunk + 2) * 4u;
    while (sp > 1 && per * (uint64_t)sp > max_bytes) --sp;
    if (sp <= 1) return 0;
    p.n_split = (int)sp;
    p.split_tiles = (int)((max_tiles + sp - 1) / sp);
    return per * (uint64_t)sp;
}

// Decode over ragged lengths (one unit and one output chunk per (sequence,
// KV head) pair, at most kDeepMaxHeads pairs and no more than the CUs): each
// pair's keys are cut into parts of `target` tiles -- at least 4, at most
// kDeepMaxSplit parts per pair, all parts in one round of workgroups over the
// CUs -- so a long sequence no longer sets the step's time on one CU while
// the others idle.  Used when that shortens the longest workgroup by a
// quarter or more.  (Measured at d = 512, L ~ U[512, 4096], Hq = 32,
// Hkv = 8: B = 8 571 -> 148 us, against 190 us for equal parts per pair;
// allowing two rounds, so that B = 32 could split too, made B = 8 261 us and
// B = 32 916 against 628 us unsplit: a part dispatched in the second round
// starts only when a CU's first one ends.)
uint64_t deep_ragged_plan(DeepParams& p, const int32_t* seq_keys, int cus, uint64_t max_bytes) {
    p.ragged = 0;
    const int64_t rows = (int64_t)p.G * p.Tq;
    const int64_t heads = (int64_t)p.B * p.Hkv;
    // With more pairs than CUs no part fits in the one round.
    if (rows > 32 || p.d > kDeepChunk || heads == 0 || heads > kDeepMaxHeads || heads > cus || !seq_keys)
        return 0;
    int64_t total = 0, longest = 0;
    for (int b = 0; b < p.B; ++b) {
        const int64_t t = ((int64_t)(seq_keys[b] > 0 ? seq_keys[b] : 0) + 31) / 32;
        total += t * p.Hkv;
        longest = longest > t ? longest : t;
    }
    auto parts = [](int64_t t, int64_t target) { return t > target ? (t + target - 1) / target : 1; };
    auto parts_of = [&](int64_t target) {
        int64_t n = 0;
        for (int b = 0; b < p.B; ++b)
            n += parts(((int64_t)(seq_keys[b] > 0 ? seq_keys[b] : 0) + 31) / 32, target) * p.Hkv;
        return n;
    };
    int64_t target = (total + cus - 1) / cus;
    if (target < 4) target = 4;
    if (target < (longest + kDeepMaxSplit - 1) / kDeepMaxSplit) target = (longest + kDeepMaxSplit - 1) / kDeepMaxSplit;
    // The smallest target whose parts fit the CUs (parts_of falls as target
    // grows; at target >= longest every pair is one part, and heads <= cus).
    if (parts_of(target) > cus) {
        int64_t lo = target, hi = longest > target ? longest : target;   // parts_of(hi) <= cus
        while (hi - lo > 1) {
            const int64_t mid = lo + (hi - lo) / 2;
            if (parts_of(mid) > cus) lo = mid;
            else hi = mid;
        }
        target = hi;
    }
    if (4 * longest < 5 * target) return 0;   // no pair's time shrinks enough to pay the split
    const int64_t n = parts_of(target);
    p.rpu = (int)(rows < 32 ? rows : 32);
    const uint64_t bytes = (uint64_t)n * (uint64_t)p.rpu * (kDeepChunk + 2) * 4u;
    if (bytes > max_bytes || n > 65535) return 0;
    int64_t at = 0;
    for (int b = 0; b < p.B; ++b) {
        const int64_t np = parts(((int64_t)(seq_keys[b] > 0 ? seq_keys[b] : 0) + 31) / 32, target);
        for (int k = 0; k < p.Hkv; ++k) {
            p.part_prefix[b * p.Hkv + k] = (uint16_t)at;
            at += np;
        }
    }
    p.part_prefix[heads] = (uint16_t)at;
    p.ragged = 1;
    p.n_split = kDeepMaxSplit;   // marks a split launch; parts per pair come from part_prefix
    p.split_tiles = (int)target;
    return bytes;
}

}  // namespace nne
