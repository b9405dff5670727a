// Host-side layout of a split-K launch (the kernel is in splitk.hip): which
// workgroup streams which of the flattened (sequence, KV head, key) rows.
// Plain C++ over SplitKParams, so the planner's tests build without HIP.
#include "splitk_plan.hpp"

#include <algorithm>
#include <climits>
#include <utility>
#include <vector>

namespace nne {

// Greedy grouping of the heads, in flattened order, into groups whose cost is
// at most x, a head of L keys costing L + ovh (ovh: the start and end of its
// segment in key-equivalents; x >= the costliest head): the number of
// groups, and with `first` their first heads (first[groups] = B * Hkv).  The
// Hkv heads of a sequence have one length, so a sequence is placed in O(1)
// steps plus one per group.
int pack_groups(const SplitKParams& p, int64_t x, int64_t ovh, uint16_t* first) {
    int groups = 0;
    int64_t sum = 0;
    for (int b = 0; b < p.B; ++b) {
        const int64_t c = (p.arg_pref[b + 1] - p.arg_pref[b]) / p.Hkv + ovh;
        int h = b * p.Hkv, n = p.Hkv;
        while (n > 0) {
            if (groups == 0 || sum + c > x) {
                if (first) first[groups] = (uint16_t)h;
                ++groups;
                sum = 0;
            }
            const int k = (int)std::min<int64_t>(n, (x - sum) / c);
            sum += k * c;
            h += k;
            n -= k;
        }
    }
    if (first) first[groups] = (uint16_t)(p.B * p.Hkv);
    return groups;
}

// Whole-head packing against the flattened chunks.  Packed, every head is
// streamed by one workgroup (the heads grouped into at most `slots`
// workgroups, each group as cheap as the grouping allows), so the launch has
// no partial records, arrivals or merges, but a workgroup streams at one
// CU's rate and pays each of its heads' segment start and end: its time is
// the costliest group at that rate, or the whole launch at the device's.
// Chunked, every CU streams an equal share at the device's rate, and the
// heads cut by the chunk boundaries pay the hand-off.  Rates and costs
// measured on MI355X with this kernel:
constexpr double kCuBytesPerUs = 37e3;     // one workgroup streaming its own heads (37 GB/s)
constexpr double kDevBytesPerUs = 6.9e6;   // the device on equal chunks (6.9 TB/s)
constexpr double kSegmentUs = 2.5;         // a segment's first loads and its merge and store
constexpr double kSplitUs = 9.0;           // chunked over packed, past the stream: records,
                                           // arrivals, merges and more segments per CU
                                           // (config 5b: 29.3 us chunked, 25.0 us packed)

// At most two whole heads per workgroup, in any order: the longest heads
// alone and the rest paired longest with shortest (the largest-first
// assignment, when there are at most twice as many heads as slots).  Returns
// the costliest workgroup (INT64_MAX when there are more heads than that),
// with `pairs` the two heads of each workgroup (0xFFFF: none) and *n_wg.
int64_t pair_heads(const SplitKParams& p, int slots, int64_t ovh, uint16_t* pairs, int* n_wg) {
    std::vector<std::pair<int64_t, int>> h;   // (cost, head) of the heads with keys
    for (int b = 0; b < p.B; ++b) {
        const int64_t L = (p.arg_pref[b + 1] - p.arg_pref[b]) / p.Hkv;
        if (L > 0)
            for (int k = 0; k < p.Hkv; ++k) h.emplace_back(L + ovh, b * p.Hkv + k);
    }
    const int n = (int)h.size();
    if (n == 0 || n > 2 * slots || slots > kMaxCutWg) return INT64_MAX;
    std::stable_sort(h.begin(), h.end(),
                     [](const std::pair<int64_t, int>& a, const std::pair<int64_t, int>& b) {
                         return a.first > b.first;
                     });
    const int singles = n <= slots ? n : 2 * slots - n;
    int64_t worst = 0;
    int w = 0;
    for (int i = 0; i < singles; ++i, ++w) {
        worst = std::max(worst, h[i].first);
        if (pairs) { pairs[2 * w] = (uint16_t)h[i].second; pairs[2 * w + 1] = 0xFFFF; }
    }
    for (int i = singles, j = n - 1; i < j; ++i, --j, ++w) {
        worst = std::max(worst, h[i].first + h[j].first);
        if (pairs) { pairs[2 * w] = (uint16_t)h[i].second; pairs[2 * w + 1] = (uint16_t)h[j].second; }
    }
    *n_wg = w;
    return worst;
}

bool plan_packing(SplitKParams& p, int slots, int64_t total_keys) {
    const int n_heads = p.B * p.Hkv;
    if (!p.arg_pref_valid || !p.fused || slots > kMaxPackWg || n_heads == 0 || n_heads > 65535 ||
        total_keys == 0)
        return false;
    const double key_bytes = 8.0 * p.d;   // one K row and one V row
    const int64_t ovh = (int64_t)(kSegmentUs * kCuBytesPerUs / key_bytes + 0.5);
    int64_t longest = 0;
    for (int b = 0; b < p.B; ++b)
        longest = std::max<int64_t>(longest, (p.arg_pref[b + 1] - p.arg_pref[b]) / p.Hkv);
    // smallest bottleneck x >= the costliest head whose grouping fits the slots
    int64_t lo = std::max<int64_t>(longest + ovh, (total_keys + n_heads * ovh + slots - 1) / slots);
    int64_t hi = lo;
    while (pack_groups(p, hi, ovh, nullptr) > slots) hi *= 2;
    while (lo < hi) {
        const int64_t mid = (lo + hi) / 2;
        if (pack_groups(p, mid, ovh, nullptr) <= slots) hi = mid; else lo = mid + 1;
    }
    int pair_wg = 0;
    const int64_t pair_x = pair_heads(p, slots, ovh, nullptr, &pair_wg);
    const int64_t x = std::min(lo, pair_x);
    const double stream_us = (double)total_keys * key_bytes / kDevBytesPerUs;
    const double packed_us = std::max((double)x * key_bytes / kCuBytesPerUs, stream_us);
    if (packed_us > stream_us + kSplitUs) return false;
    if (pair_x < lo) {
        pair_heads(p, slots, ovh, p.pack_head, &p.n_wg);
        p.packed = 2;
    } else {
        p.n_wg = pack_groups(p, lo, ovh, p.pack_head);
        p.packed = 1;
    }
    return true;
}

// Cut chunks.  With equal chunks, every segment of a workgroup after its
// first costs it that segment's hand-off and the latency of its first loads
// (6-8 us at the loaded latency of a device-wide stream: a workgroup's first
// two blocks of a segment arrive ~7.8 us after it starts), so workgroups with
// more segments end later (config-3 decode on MI355X, equal chunks: 84, 93
// and 97 us for 1, 2 and 3 segments).  Cut, a workgroup's budget x counts
// that cost: in flattened order, each workgroup takes keys until its keys plus
// ovh per segment after its first reach x (ovh: the cost in keys at one
// workgroup's share of the device's rate).  Swept on MI355X from 0 to 16 us:
// config-3 decode 112.4 us at 0 and ~108.5 from 3 to 10; the G = 8 decode
// (16-row tile) 103.6 at 0, 100.5 at 3, 97.1 at 8 and 96.7 at 10, 98.7 at 13.
constexpr double kCutSegmentUs = 8.0;
constexpr double kCutWgBytesPerUs = 26e3;   // 6.7 TB/s over 256 workgroups

int64_t cut_segment_keys(int d) { return (int64_t)(kCutSegmentUs * kCutWgBytesPerUs / (8.0 * d) + 0.5); }

// The number of workgroups of the cut with budget x (with `ends`, their chunk
// ends), or max_wg + 1 if it takes more than max_wg workgroups or gives a head
// more than max_parts of them.
int cut_chunks(const SplitKParams& p, int64_t x, int64_t ovh, int max_wg, int* ends) {
    int count = 0;
    int64_t cost = 0;
    bool open = false;
    for (int b = 0; b < p.B; ++b) {
        const int64_t L = (p.arg_pref[b + 1] - p.arg_pref[b]) / p.Hkv;
        for (int kvh = 0; kvh < p.Hkv && L > 0; ++kvh) {
            const int64_t h0 = p.arg_pref[b] + kvh * L;
            int64_t pos = 0;
            int parts = 0;
            while (pos < L) {
                if (open && cost + ovh + kKeyBlock > x) {   // no room for another segment
                    if (ends) ends[count - 1] = (int)(h0 + pos);
                    open = false;
                }
                if (open) {
                    cost += ovh;
                } else {
                    if (++count > max_wg) return max_wg + 1;
                    cost = 0;
                    open = true;
                }
                const int64_t take = std::min(L - pos, x - cost);
                cost += take;
                pos += take;
                if (++parts > p.max_parts) return max_wg + 1;
                if (cost >= x) {
                    if (ends) ends[count - 1] = (int)(h0 + pos);
                    open = false;
                }
            }
        }
    }
    if (open && ends) ends[count - 1] = p.arg_pref[p.B];
    return count;
}

// The smallest budget whose cut fits `slots` workgroups (and at least 4
// blocks and an eighth of the longest head, as for equal chunks).
bool plan_cut(SplitKParams& p, int slots, int64_t total_keys, int max_len) {
    slots = std::min(slots, kMaxCutWg);
    if (!p.arg_pref_valid || !p.fused || total_keys == 0 || total_keys > INT32_MAX || slots < 1)
        return false;
    const int64_t ovh = cut_segment_keys(p.d);
    int64_t lo = std::max<int64_t>((total_keys + slots - 1) / slots,
                                   std::max<int64_t>(4 * kKeyBlock, (max_len + 7) / 8));
    int64_t hi = lo;
    while (cut_chunks(p, hi, ovh, slots, nullptr) > slots) {
        if (hi > total_keys) return false;
        hi *= 2;
    }
    while (lo < hi) {
        const int64_t mid = (lo + hi) / 2;
        if (cut_chunks(p, mid, ovh, slots, nullptr) <= slots) hi = mid; else lo = mid + 1;
    }
    p.n_wg = cut_chunks(p, lo, ovh, slots, p.chunk_end);
    p.chunk = (int)std::min<int64_t>(lo, INT32_MAX);
    p.cut = 1;
    return true;
}

// Equal flattened chunks, whole 16-key blocks, and at most max_parts
// workgroups sharing any one head (a chunk boundary can add two).
void plan_equal(SplitKParams& p, int slots, int64_t total_keys, int max_len) {
    int64_t chunk = (total_keys + slots - 1) / (slots > 0 ? slots : 1);
    int64_t min_chunk = (max_len + (p.max_parts - 2) - 1) / (p.max_parts - 2);
    if (min_chunk < 4 * kKeyBlock) min_chunk = 4 * kKeyBlock;   // a block for each of the 4 waves
    // At most ~8 workgroups per head: a small problem (few, short heads)
    // otherwise splits into many short chunks whose records cost the merging
    // workgroup more round trips than the extra keys per chunk cost to stream.
    if (min_chunk < (max_len + 7) / 8) min_chunk = (max_len + 7) / 8;
    if (chunk < min_chunk) chunk = min_chunk;
    chunk = (chunk + kKeyBlock - 1) / kKeyBlock * kKeyBlock;
    if (chunk < kKeyBlock) chunk = kKeyBlock;
    p.chunk = (int)chunk;
    int64_t n_wg = (total_keys + chunk - 1) / chunk;
    p.n_wg = (int)(n_wg < 1 ? 1 : n_wg);
}

void plan_split_layout(SplitKParams& p, int slots, int64_t total_keys, int max_len) {
    p.packed = 0;
    p.cut = 0;
    if (plan_packing(p, slots, total_keys)) return;
    if (plan_cut(p, slots, total_keys, max_len)) return;
    plan_equal(p, slots, total_keys, max_len);
}

}  // namespace nne
