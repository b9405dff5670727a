// Invariants of the deep kernel's key-split plans (csrc/deep_plan.cpp), on
// the CPU.
//   * ragged (decode over ragged lengths): every call returns (also with more
//     (sequence, KV head) pairs than CUs, where no split fits the one round);
//     a plan gives each pair ceil(tiles / target) parts (one for an empty or
//     short pair), at most kDeepMaxSplit, all pairs of a sequence alike, all
//     parts within the CUs, part_prefix rising from 0 to the part count; the
//     target is the smallest from max(4, ceil(total / CUs), ceil(longest / 8))
//     whose parts fit the CUs (against a linear scan or a bisection), the split is
//     taken only when 4 * longest >= 5 * target, and its records fit
//     max_bytes;
//   * equal split: none unless at most half as many workgroups as CUs and
//     8+ tiles; at most kDeepMaxSplit parts of at least 4 tiles covering the
//     longest unit, all parts in one round, records within max_bytes.
// Prints "<failed> of <checks> checks failed" and exits non-zero on failure.
#include <algorithm>
#include <cstdio>
#include <random>
#include <string>
#include <vector>

#include "deep_plan.hpp"

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

static int64_t tiles_of(int32_t keys) { return ((int64_t)(keys > 0 ? keys : 0) + 31) / 32; }

static int g_ragged_taken = 0, g_ragged_declined = 0, g_split_taken = 0;

static void check_ragged(int B, int Hkv, int G, int d, const std::vector<int32_t>& lens, int cus,
                         uint64_t max_bytes) {
    char buf[160];
    std::snprintf(buf, sizeof buf, "ragged B=%d Hkv=%d G=%d d=%d cus=%d max_bytes=%llu", B, Hkv, G, d,
                  cus, (unsigned long long)max_bytes);
    g_case = buf;
    DeepParams p{};
    p.B = B; p.Hkv = Hkv; p.G = G; p.Tq = 1; p.Hq = Hkv * G; p.d = d;
    const uint64_t bytes = deep_ragged_plan(p, lens.data(), cus, max_bytes);
    const int64_t heads = (int64_t)B * Hkv;
    int64_t total = 0, longest = 0;
    for (int b = 0; b < B; ++b) {
        total += tiles_of(lens[b]) * Hkv;
        longest = std::max(longest, tiles_of(lens[b]));
    }
    auto parts = [](int64_t t, int64_t target) { return t > target ? (t + target - 1) / target : 1; };
    auto parts_of = [&](int64_t target) {
        int64_t n = 0;
        for (int b = 0; b < B; ++b) n += parts(tiles_of(lens[b]), target) * Hkv;
        return n;
    };
    const bool eligible = G <= 32 && d <= kDeepChunk && heads > 0 && heads <= kDeepMaxHeads && heads <= cus;
    // The smallest target from the lower bound whose parts fit the CUs: a
    // linear scan where that is short, else bisection (the part count falls as
    // the target grows; at target >= longest every pair is one part).
    int64_t target = -1;
    if (eligible) {
        const int64_t t0 = std::max<int64_t>({4, (total + cus - 1) / cus, (longest + kDeepMaxSplit - 1) / kDeepMaxSplit});
        if (longest - t0 <= 20000) {
            target = t0;
            while (parts_of(target) > cus) ++target;
        } else {
            int64_t lo = t0 - 1, hi = std::max(longest, t0);
            while (hi - lo > 1) {
                const int64_t mid = (lo + hi) / 2;
                (parts_of(mid) > cus ? lo : hi) = mid;
            }
            target = hi;
        }
        CHECK(parts_of(target) <= cus && (target == t0 || parts_of(target - 1) > cus), "reference target");
    }
    const uint64_t want_bytes =
        eligible ? (uint64_t)parts_of(target) * (uint64_t)G * (kDeepChunk + 2) * 4u : 0;
    const bool want = eligible && 4 * longest >= 5 * target && want_bytes <= max_bytes && parts_of(target) <= 65535;
    if (!want) {
        ++g_ragged_declined;
        CHECK(bytes == 0 && p.ragged == 0, "expected no ragged split, got %llu bytes ragged=%d",
              (unsigned long long)bytes, p.ragged);
        return;
    }
    ++g_ragged_taken;
    CHECK(bytes == want_bytes && p.ragged == 1, "bytes %llu want %llu ragged=%d", (unsigned long long)bytes,
          (unsigned long long)want_bytes, p.ragged);
    if (p.ragged != 1) return;
    CHECK(p.split_tiles == target, "target %d want %lld", p.split_tiles, (long long)target);
    CHECK(p.n_split == kDeepMaxSplit && p.rpu == G, "n_split %d rpu %d", p.n_split, p.rpu);
    CHECK(p.part_prefix[0] == 0, "part_prefix[0] = %d", p.part_prefix[0]);
    int64_t n = 0;
    for (int b = 0; b < B; ++b) {
        const int64_t t = tiles_of(lens[b]);
        for (int k = 0; k < Hkv; ++k) {
            const int h = b * Hkv + k;
            const int np = (int)p.part_prefix[h + 1] - (int)p.part_prefix[h];
            CHECK(np == parts(t, p.split_tiles), "pair %d: %d parts for %lld tiles at target %d", h, np,
                  (long long)t, p.split_tiles);
            CHECK(np >= 1 && np <= kDeepMaxSplit, "pair %d: %d parts", h, np);
            CHECK((int64_t)np * p.split_tiles >= t, "pair %d: parts do not cover its tiles", h);
            n += np;
        }
    }
    CHECK(n == p.part_prefix[heads] && n <= cus, "parts %lld prefix %d cus %d", (long long)n,
          p.part_prefix[heads], cus);
    CHECK(bytes <= max_bytes, "records exceed max_bytes");
}

static void check_split(int B, int Hkv, int G, int Tq, int d, int max_tiles, int cus, uint64_t max_bytes) {
    char buf[160];
    std::snprintf(buf, sizeof buf, "split B=%d Hkv=%d G=%d Tq=%d d=%d tiles=%d cus=%d", B, Hkv, G, Tq, d,
                  max_tiles, cus);
    g_case = buf;
    DeepParams p{};
    p.B = B; p.Hkv = Hkv; p.G = G; p.Tq = Tq; p.Hq = Hkv * G; p.d = d;
    const uint64_t bytes = deep_split_plan(p, max_tiles, cus, max_bytes);
    const int64_t rows = (int64_t)G * Tq;
    const int64_t wg = (int64_t)B * Hkv * ((rows + 31) / 32) * ((d + kDeepChunk - 1) / kDeepChunk);
    CHECK(p.rpu == (int)std::min<int64_t>(rows, 32), "rpu %d", p.rpu);
    if (bytes == 0) {
        CHECK(p.n_split == 1, "no split but n_split %d", p.n_split);
        // Declined only where a split cannot run or pay.
        const bool could = wg > 0 && 2 * wg <= cus && max_tiles >= 8 &&
                           (uint64_t)wg * (uint64_t)p.rpu * (kDeepChunk + 2) * 4u * 2u <= max_bytes;
        CHECK(!could, "declined a split that fits (wg %lld)", (long long)wg);
        return;
    }
    ++g_split_taken;
    CHECK(wg > 0 && 2 * wg <= cus && max_tiles >= 8, "split of %lld workgroups over %d CUs", (long long)wg, cus);
    CHECK(p.n_split >= 2 && p.n_split <= kDeepMaxSplit, "n_split %d", p.n_split);
    CHECK(p.n_split * wg <= cus, "parts do not fit one round");
    CHECK(p.split_tiles >= 4, "parts of %d tiles", p.split_tiles);
    CHECK((int64_t)p.split_tiles * p.n_split >= max_tiles, "parts do not cover the longest unit");
    CHECK(bytes == (uint64_t)wg * p.rpu * (kDeepChunk + 2) * 4u * p.n_split && bytes <= max_bytes,
          "bytes %llu", (unsigned long long)bytes);
    // Parts as many as the CUs, the tiles (4 each) and the records allow.
    const int64_t cap = std::min<int64_t>({kDeepMaxSplit, cus / wg, max_tiles / 4});
    if (p.n_split < cap)
        CHECK(bytes / p.n_split * (p.n_split + 1) > max_bytes, "fewer parts (%d) than fit (%lld)", p.n_split,
              (long long)cap);
}

int main() {
    // Named cases: the benchmark-like decode batches, and more pairs than CUs
    // (B = 64, Hkv = 8 on 256 CUs: 512 pairs), which must return at once.
    std::mt19937 rng(7);
    auto uniform_lens = [&](int B, int lo, int hi) {
        std::vector<int32_t> v(B);
        std::uniform_int_distribution<int> u(lo, hi);
        for (auto& x : v) x = u(rng);
        return v;
    };
    check_ragged(8, 8, 4, 512, uniform_lens(8, 512, 4096), 256, UINT64_MAX);
    check_ragged(32, 8, 4, 512, uniform_lens(32, 512, 4096), 256, UINT64_MAX);
    check_ragged(64, 8, 4, 512, uniform_lens(64, 512, 4096), 256, UINT64_MAX);
    check_ragged(40, 8, 4, 320, uniform_lens(40, 1, 100000), 256, UINT64_MAX);
    check_ragged(128, 4, 8, 512, uniform_lens(128, 1, 1 << 20), 256, UINT64_MAX);
    check_ragged(1, 1, 1, 512, std::vector<int32_t>{1 << 30}, 256, UINT64_MAX);
    check_ragged(255, 1, 1, 512, uniform_lens(255, 1 << 20, 1 << 24), 256, UINT64_MAX);
    check_ragged(4, 8, 4, 512, std::vector<int32_t>(4, 0), 256, UINT64_MAX);
    check_ragged(8, 8, 4, 512, uniform_lens(8, 512, 4096), 256, 4096);   // records do not fit

    // Seeded sweep.
    std::uniform_int_distribution<int> ub(1, 160), uh(1, 16), ug(1, 40), ud(65, 160), uc(0, 4), ul(0, 5);
    const int cus_list[] = {8, 32, 80, 256, 304};
    for (int it = 0; it < 4000; ++it) {
        const int B = ub(rng), Hkv = uh(rng), G = ug(rng), d = 4 * ud(rng);
        const int cus = cus_list[uc(rng)];
        std::vector<int32_t> lens(B);
        const int kind = ul(rng);
        std::uniform_int_distribution<int> ushort(0, 200), ulong(512, 1 << 16), uhuge(1 << 16, 1 << 26);
        for (auto& x : lens)
            x = kind == 0 ? ushort(rng) : kind == 5 ? uhuge(rng) : ulong(rng);
        if (kind == 1 && B > 1) lens[0] = 1 << 20;   // one long sequence among short ones
        const uint64_t mb = (it % 7 == 0) ? (uint64_t)(it % 5) * 300000u : UINT64_MAX;
        check_ragged(B, Hkv, G, d, lens, cus, mb);
        const int Tq = 1 + (it % 3 == 0 ? ub(rng) : 0);
        std::uniform_int_distribution<int> ut(0, 5000);
        check_split(1 + B % 4, 1 + Hkv % 4, 1 + G % 8, Tq, d, ut(rng), cus, mb);
    }
    std::printf("ragged plans: %d taken, %d declined; equal splits taken: %d\n", g_ragged_taken,
                g_ragged_declined, g_split_taken);
    std::printf("%d of %d checks failed\n", g_failed, g_checks);
    return g_failed == 0 && g_ragged_taken > 0 && g_ragged_declined > 0 && g_split_taken > 0 ? 0 : 1;
}
