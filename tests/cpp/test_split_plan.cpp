// Invariants of the split-K launch planner (csrc/splitk_plan.cpp), on the
// CPU: for named decode / cross-attention shapes and a seeded sweep of ragged
// batches, the layout that plan_split_layout picks must
//   * cover every flattened key exactly once (ranges in order, the last
//     ending at the total), with at most `slots` workgroups; only a packed
//     group of empty heads may have an empty range;
//   * packed: whole heads in flattened runs, no empty group, each group's
//     keys plus the per-head cost within the planned bottleneck; or paired:
//     every head with keys in exactly one workgroup, at most two per
//     workgroup, no empty head, the costliest pair cheaper than the
//     flattened runs' bottleneck;
//   * cut: every workgroup's keys plus the per-segment cost within the
//     budget, no workgroup closed with room for another segment (except the
//     last), no head shared by more than max_parts workgroups, the budget the
//     smallest that fits the slots, and partial-record slots (workgroup +
//     head) unique and inside the workspace;
//   * equal: whole 16-key blocks, the fewest chunks that cover the keys.
// Prints "<failed> of <checks> checks failed" and exits non-zero on failure.
#include <algorithm>
#include <cstdio>
#include <random>
#include <set>
#include <string>
#include <vector>

#include "splitk_plan.hpp"

using namespace nne;

static int g_checks = 0, g_failed = 0;
static std::string g_case;

#define CHECK(cond, ...)                                        \
    do {                                                        \
        ++g_checks;                                             \
        if (!(cond)) {                                          \
            ++g_failed;                                         \
            std::printf("FAIL [%s] ", g_case.c_str());          \
            std::printf(__VA_ARGS__);                           \
            std::printf("\n");                                  \
        }                                                       \
    } while (0)

struct Shape {
    int B, Hkv, d, R;
    std::vector<int> lens;   // keys per sequence (the new row included)
    int slots;
};

static void setup(SplitKParams& p, const Shape& s) {
    p = SplitKParams{};
    p.B = s.B;
    p.Hkv = s.Hkv;
    p.d = s.d;
    p.R = s.R;
    p.fused = 1;
    p.arg_pref_valid = s.B <= kArgSeqs ? 1 : 0;
    p.max_parts = std::min(512, 1024 / s.R);
    if (p.arg_pref_valid) {
        p.arg_pref[0] = 0;
        for (int b = 0; b < s.B; ++b) p.arg_pref[b + 1] = p.arg_pref[b] + s.Hkv * s.lens[b];
    }
}

// Flattened [start, end) of every head (b * Hkv + kvh).
static std::vector<std::pair<int64_t, int64_t>> head_ranges(const Shape& s) {
    std::vector<std::pair<int64_t, int64_t>> h;
    int64_t pos = 0;
    for (int b = 0; b < s.B; ++b)
        for (int k = 0; k < s.Hkv; ++k) {
            h.emplace_back(pos, pos + s.lens[b]);
            pos += s.lens[b];
        }
    return h;
}

// Returns the mode the planner chose: 'p' packed, 'c' cut, 'e' equal.
static char check_layout(const Shape& s) {
    SplitKParams p;
    setup(p, s);
    const auto heads = head_ranges(s);
    int64_t total = 0, max_len = 0;
    for (int L : s.lens) {
        total += (int64_t)s.Hkv * L;
        max_len = std::max<int64_t>(max_len, L);
    }
    plan_split_layout(p, s.slots, total, (int)max_len);
    CHECK(p.n_wg >= 1, "n_wg %d", p.n_wg);

    // Workgroup ranges [start[w], start[w+1]).
    std::vector<int64_t> start;
    char mode;
    if (p.packed == 2) {
        CHECK(p.n_wg <= s.slots && p.n_wg <= kMaxCutWg, "paired n_wg %d > slots %d", p.n_wg, s.slots);
        const int64_t ovh = (int64_t)(2.5 * 37e3 / (8.0 * s.d) + 0.5);
        std::vector<int> seen(heads.size(), 0);
        int64_t worst = 0;
        for (int w = 0; w < p.n_wg; ++w) {
            int64_t cost = 0;
            for (int j = 0; j < 2; ++j) {
                const int h = p.pack_head[2 * w + j];
                if (j == 1 && h == 0xFFFF) continue;
                CHECK(h < (int)heads.size(), "workgroup %d head %d out of range", w, h);
                if (h >= (int)heads.size()) continue;
                CHECK(heads[h].second > heads[h].first, "workgroup %d streams empty head %d", w, h);
                ++seen[h];
                cost += heads[h].second - heads[h].first + ovh;
            }
            worst = std::max(worst, cost);
        }
        for (size_t h = 0; h < heads.size(); ++h)
            CHECK(seen[h] == (heads[h].second > heads[h].first ? 1 : 0), "head %zu streamed %d times", h,
                  seen[h]);
        // chosen only when cheaper than the flattened runs' bottleneck
        int64_t longest = 0, total_cost = 0;
        for (const auto& h : heads) {
            longest = std::max<int64_t>(longest, h.second - h.first + ovh);
            total_cost += h.second - h.first + ovh;
        }
        int64_t lo = std::max<int64_t>(longest, (total_cost + s.slots - 1) / s.slots), hi = lo;
        while (pack_groups(p, hi, ovh, nullptr) > s.slots) hi *= 2;
        while (lo < hi) {
            const int64_t mid = (lo + hi) / 2;
            if (pack_groups(p, mid, ovh, nullptr) <= s.slots) hi = mid; else lo = mid + 1;
        }
        const int64_t x = lo;
        CHECK(worst < x, "paired bottleneck %lld not below the runs' %lld", (long long)worst, (long long)x);
        return 'p';
    }
    if (p.packed) {
        mode = 'p';
        CHECK(p.n_wg <= s.slots, "packed n_wg %d > slots %d", p.n_wg, s.slots);
        CHECK(p.pack_head[0] == 0, "first group starts at head %d", p.pack_head[0]);
        CHECK(p.pack_head[p.n_wg] == s.B * s.Hkv, "groups end at head %d of %d", p.pack_head[p.n_wg],
              s.B * s.Hkv);
        for (int w = 0; w < p.n_wg; ++w) {
            CHECK(p.pack_head[w] < p.pack_head[w + 1], "group %d empty", w);
            start.push_back(heads[p.pack_head[w]].first);
        }
        start.push_back(total);
    } else if (p.cut) {
        mode = 'c';
        CHECK(p.n_wg <= std::min(s.slots, kMaxCutWg), "cut n_wg %d", p.n_wg);
        start.push_back(0);
        for (int w = 0; w < p.n_wg; ++w) start.push_back(p.chunk_end[w]);
    } else {
        mode = 'e';
        CHECK(p.chunk % kKeyBlock == 0 && p.chunk >= kKeyBlock, "chunk %d", p.chunk);
        CHECK((int64_t)p.n_wg * p.chunk >= total && (int64_t)(p.n_wg - 1) * p.chunk < total,
              "n_wg %d x chunk %d vs %lld keys", p.n_wg, p.chunk, (long long)total);
        for (int w = 0; w < p.n_wg; ++w) start.push_back((int64_t)w * p.chunk);
        start.push_back(total);
    }
    // Cover: in order, ending at the total; a range is empty only for a
    // packed group of empty heads (the kernel returns at once for it).
    for (size_t w = 0; w + 1 < start.size(); ++w) {
        bool may_be_empty = false;
        if (mode == 'p') {
            may_be_empty = true;
            for (int h = p.pack_head[w]; h < p.pack_head[w + 1]; ++h)
                may_be_empty = may_be_empty && heads[h].first == heads[h].second;
        }
        CHECK(start[w] < start[w + 1] || (may_be_empty && start[w] == start[w + 1]),
              "range %zu [%lld, %lld) empty or reversed", w, (long long)start[w], (long long)start[w + 1]);
    }
    CHECK(start.back() == total, "ranges end at %lld, keys %lld", (long long)start.back(), (long long)total);
    if (mode == 'p') {   // packed groups end at head boundaries
        std::set<int64_t> ends;
        for (const auto& h : heads) ends.insert(h.second);
        for (size_t w = 1; w < start.size(); ++w)
            CHECK(ends.count(start[w]) == 1 || start[w] == total, "group %zu ends inside a head", w - 1);
    }
    if (mode == 'c') {
        const int64_t ovh = cut_segment_keys(s.d), x = p.chunk;
        std::vector<int> parts(heads.size(), 0);
        std::set<int64_t> slots_used;
        const int64_t slot_limit = (int64_t)s.slots + s.B * s.Hkv;
        for (int w = 0; w < p.n_wg; ++w) {
            int64_t keys = start[w + 1] - start[w];
            int segs = 0;
            for (size_t h = 0; h < heads.size(); ++h) {
                if (heads[h].first == heads[h].second) continue;
                if (heads[h].first < start[w + 1] && heads[h].second > start[w]) {
                    ++segs;
                    ++parts[h];
                    const bool whole = heads[h].first >= start[w] && heads[h].second <= start[w + 1];
                    if (!whole) {   // a partial record in slot w + head
                        const int64_t slot = w + (int64_t)h;
                        CHECK(slots_used.insert(slot).second, "slot %lld used twice", (long long)slot);
                        CHECK(slot < slot_limit, "slot %lld past the workspace (%lld)", (long long)slot,
                              (long long)slot_limit);
                    }
                }
            }
            const int64_t cost = keys + ovh * (segs - 1);
            CHECK(cost <= x, "workgroup %d cost %lld > budget %lld", w, (long long)cost, (long long)x);
            if (w + 1 < p.n_wg)
                CHECK(cost + ovh + kKeyBlock > x, "workgroup %d closed with room (cost %lld, budget %lld)", w,
                      (long long)cost, (long long)x);
        }
        for (size_t h = 0; h < heads.size(); ++h)
            CHECK(parts[h] <= p.max_parts, "head %zu in %d workgroups > %d", h, parts[h], p.max_parts);
        // The smallest budget: one key less needs more workgroups (or breaks
        // the floor of 4 blocks / an eighth of the longest head).
        const int64_t floor_x = std::max<int64_t>((total + s.slots - 1) / s.slots,
                                                  std::max<int64_t>(4 * kKeyBlock, (max_len + 7) / 8));
        if (x > floor_x)
            CHECK(cut_chunks(p, x - 1, ovh, std::min(s.slots, kMaxCutWg), nullptr) > std::min(s.slots, kMaxCutWg),
                  "budget %lld not minimal", (long long)x);
    }
    return mode;
}

int main() {
    // Named shapes: the mode the measurements chose for each.
    struct Named {
        const char* name;
        Shape s;
        char mode;
    };
    std::vector<Named> named;
    {
        std::mt19937 rng(3);
        Shape c3{32, 8, 128, 4, {}, 256};   // config 3 decode: L ~ U[512, 4096] + 1
        for (int b = 0; b < 32; ++b) c3.lens.push_back(512 + (int)(rng() % 3585) + 1);
        named.push_back({"config3", c3, 'c'});
        Shape g8 = c3;
        g8.R = 16;
        named.push_back({"g8", g8, 'c'});
        Shape c5b{8, 20, 64, 16, std::vector<int>(8, 1500), 256};   // cross-attention, 160 heads
        named.push_back({"config5b", c5b, 'p'});
        Shape gpt2{32, 12, 64, 4, {}, 256};   // GPT-2-small decode attend
        for (int b = 0; b < 32; ++b) gpt2.lens.push_back(128 + (int)(rng() % 897) + 1);
        named.push_back({"gpt2", gpt2, 'p'});   // paired (checked below)
        Shape big{150, 2, 128, 4, {}, 256};   // prefix not in the arguments: equal chunks
        for (int b = 0; b < 150; ++b) big.lens.push_back((int)(rng() % 3000));
        named.push_back({"b150", big, 'e'});
    }
    for (const auto& n : named) {
        g_case = n.name;
        const char mode = check_layout(n.s);
        CHECK(mode == n.mode, "mode %c, expected %c", mode, n.mode);
        SplitKParams p;
        setup(p, n.s);
        int64_t total = 0, max_len = 0;
        for (int L : n.s.lens) {
            total += (int64_t)n.s.Hkv * L;
            max_len = std::max<int64_t>(max_len, L);
        }
        plan_split_layout(p, n.s.slots, total, (int)max_len);
        if (std::string(n.name) == "gpt2") CHECK(p.packed == 2, "gpt2 packed %d, expected pairs", p.packed);
        if (std::string(n.name) == "config5b") CHECK(p.packed == 1, "5b packed %d, expected runs", p.packed);
    }

    // Seeded sweep: ragged batches with empty sequences, one long head among
    // short ones, equal lengths, few and many sequences, several slot counts.
    std::mt19937 rng(0x5EED);
    int counts[3] = {0, 0, 0};
    for (int it = 0; it < 400; ++it) {
        Shape s;
        s.B = 1 + (int)(rng() % 160);   // past 128: no prefix in the arguments
        const int hkv_choices[] = {1, 2, 4, 8};
        s.Hkv = hkv_choices[rng() % 4];
        s.d = rng() % 2 ? 64 : 128;
        const int r_choices[] = {1, 4, 8, 16, 32, 64};
        s.R = r_choices[rng() % 6];
        const int slot_choices[] = {8, 64, 200, 256};
        s.slots = slot_choices[rng() % 4];
        const int kind = (int)(rng() % 4);
        int64_t sum = 0;
        for (int b = 0; b < s.B; ++b) {
            int L;
            if (kind == 0) L = (int)(rng() % 5000);                                   // ragged
            else if (kind == 1) L = rng() % 8 == 0 ? 0 : 1 + (int)(rng() % 200);       // short, some empty
            else if (kind == 2) L = 1000;                                             // equal
            else L = b == 0 ? 20000 + (int)(rng() % 20000) : 1 + (int)(rng() % 300);  // one long head
            s.lens.push_back(L);
            sum += L;
        }
        if (sum == 0) s.lens[0] = 17;
        g_case = "sweep " + std::to_string(it);
        const char mode = check_layout(s);
        ++counts[mode == 'p' ? 0 : (mode == 'c' ? 1 : 2)];
    }
    std::printf("sweep layouts: %d packed, %d cut, %d equal\n", counts[0], counts[1], counts[2]);
    std::printf("%d of %d checks failed\n", g_failed, g_checks);
    return g_failed == 0 ? 0 : 1;
}
