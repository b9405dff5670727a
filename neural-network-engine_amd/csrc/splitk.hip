// Few-query attention for decode and cross-attention, plus the KV-cache append.
//
// Semantics: every query row attends to all keys of its sequence with no mask
// -- the reference's single-token decode (src/models/llama.rs:239-296 with
// t = 1: append first, then attend to all L rows including the new one) and
// its cross-attention (src/nn/attention.rs:193-203) -- or, for a few causal
// rows (masked), query t sees keys c <= q_off + t: a multi-token step over a
// cache (the bottom-right mask of llama.rs:277-292 and attention.rs:101-108).  Sequences may have
// different lengths (lens[b]); the reference handles ragged batches as
// separate B = 1 calls.
//
// MI355X mapping.  The work is HBM-bound (about 2 FLOP per byte of K/V), so the
// kernel is organised around streaming each KV head's cache exactly once and
// keeping everything else off the critical path:
//   * the (sequence, KV head, key) rows of the whole batch are flattened and
//     cut into equal chunks, one per workgroup and one workgroup per CU:
//     every CU streams the same number of bytes whatever the ragged lengths
//     (per-head splits leave a long tail);
//   * a workgroup serves all R = G * T_q <= 16 query rows that read a KV head,
//     so grouped-query sharing costs no extra HBM traffic;
//   * its 4 waves run independently over interleaved 16-key blocks (no
//     workgroup barrier until the final merge).  Per block, on
//     v_mfma_f32_16x16x4_f32:
//       S^T = K Q^T  (keys x query rows; Q^T lives in registers, K is staged
//                     through a wave-private LDS slice to reach MFMA layout),
//       online softmax in registers: a query row's 16 scores sit in 4
//       registers of 4 lanes, so its max / sum are 3 in-lane ops plus two
//       lane swaps (v_permlane16_swap, v_permlane32_swap),
//       O^T += V^T P^T (P^T register r is the B operand of step r; V is loaded
//                     straight from HBM in operand layout, one 16-byte load
//                     feeding four MFMAs);
//     the next block's K and V loads are in flight while a block computes;
//   * the 4 waves' (max, sum, O) are merged through LDS; a head covered by
//     one workgroup is written directly, otherwise each workgroup leaves a
//     partial record (agent-scope stores, then a wait until they are
//     performed) and counts itself in on the head's arrival counter; the last
//     of the head's workgroups merges its records inside the same launch.
//     Without counters, or with too many sequences for the prefix to travel in
//     the kernel arguments, the per-head combine kernel merges them instead;
//   * in a decode step the new K/V row is read straight from the caller's
//     k_new / v_new and written into the cache by the workgroup whose split
//     holds it; lens[b] is advanced inside the launch (or by the combine
//     kernel).
// The hand-off uses per-access coherence rather than fences: on gfx950 an
// agent-scope fence is a whole-L2 writeback and invalidate.
#include <atomic>
#include <algorithm>
#include <climits>
#include <cstddef>
#include <utility>

#include "nne_common.hpp"
#include "nne_launch.hpp"
#include "splitk_plan.hpp"

namespace nne {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int KB = kKeyBlock;     // keys per block (one 16x16x4 MFMA tile of keys)
constexpr int MAX_SEQS = 2048;    // sequences per launch (prefix array in LDS)
constexpr int MAX_PARTS = 512;    // workgroups sharing one head
constexpr int COMBINE_ML = 8192;  // (record, row) pairs the combine kernel holds in LDS
constexpr int MAX_WG = 2048;      // workgroups of one split launch

__device__ __forceinline__ int clamp_len(int L, int max_keys) {
    return L < 0 ? 0 : (L > max_keys ? max_keys : L);
}

// Reduce over the 4 lanes {l, l^16, l^32, l^48} (rows of 16 lanes).
__device__ __forceinline__ float quad_rows_max(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float quad_rows_sum(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Reductions over a row of 16 lanes (DPP row_ror 8, 4, 2, 1); every lane of
// the row ends with the result.
template <int CTRL>
__device__ __forceinline__ float dpp_row(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_row<0x128>(x));
    x = fmaxf(x, dpp_row<0x124>(x));
    x = fmaxf(x, dpp_row<0x122>(x));
    return fmaxf(x, dpp_row<0x121>(x));
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_row<0x128>(x);
    x += dpp_row<0x124>(x);
    x += dpp_row<0x122>(x);
    return x + dpp_row<0x121>(x);
}

// f(std::integral_constant<int, 0>) ... f(std::integral_constant<int, N-1>):
// MFMA broadcast selectors must be compile-time constants.
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// v_mfma_f32_4x4x1_16b_f32: 16 blocks of 4 lanes; lane 4b + i supplies A_b[i]
// and B_b[i], and register r of lane 4b + j receives D_b[r][j].  With CB > 0,
// each group of 2^CB blocks takes A from its block AB.
template <int CB, int AB>
__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, CB, AB, 0);
}


// 16-byte load, non-temporal when each byte is read by one wave only.
template <bool NT>
__device__ __forceinline__ vf4 load4(const float* p) {
    if constexpr (NT) return __builtin_nontemporal_load(reinterpret_cast<const vf4*>(p));
    else return *reinterpret_cast<const vf4*>(p);
}

// Orders this wave's LDS accesses on both sides of a cross-lane exchange.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Flattened key space: head h = b*Hkv + kvh owns keys [pref[b] + kvh*L_b,
// pref[b] + (kvh+1)*L_b) where pref[b] = Hkv * sum_{b' < b} L_b'.  Workgroup w
// takes [w*chunk, (w+1)*chunk): every workgroup streams the same number of
// K/V rows, whatever the ragged lengths, and a range may span several heads.

// Key count of sequence b in this launch (the cached rows, plus the new row
// in a decode step), clamped to what the host validated.
template <bool APPEND>
__device__ __forceinline__ int seq_len(const SplitKParams& p, int b) {
    if (!p.lens) return p.tk;
    const int L_old = clamp_len(p.lens[b], p.max_keys);
    return APPEND ? clamp_len(L_old + 1, p.max_keys) : L_old;
}

// Builds pref[0..B] in LDS: copied from the kernel arguments when the host
// computed it, else scanned from lens by wave 0 (a wave-wide scan per 64
// sequences).
template <bool APPEND>
__device__ __forceinline__ void build_prefix(const SplitKParams& p, int* pref, int tid, int lane,
                                             int wave, int arg_pref_tid) {
    if (p.arg_pref_valid) {
        if (tid <= p.B) pref[tid] = arg_pref_tid;   // p.arg_pref[tid]; B <= kArgSeqs < 256
    } else if (wave == 0) {
        int carry = 0;
        if (lane == 0) pref[0] = 0;
        for (int base = 0; base < p.B; base += 64) {
            const int b = base + lane;
            int x = b < p.B ? p.Hkv * seq_len<APPEND>(p, b) : 0;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int y = __shfl_up(x, off);
                if (lane >= off) x += y;
            }
            if (b < p.B) pref[b + 1] = carry + x;
            carry += __shfl(x, 63);
        }
    }
}

// Merges the n partial records (slots s0 .. s0+n-1) of one head into its
// output, then clears the head's arrival counter.  Thread t owns the 4-float
// groups t, t + 256, ... of the R x D output rows: it reads its row's
// (max, sum) and its 4 floats of O from every record and combines them in
// record order -- M = max_c m_c, w_c = 2^(m_c - M), O = sum_c w_c O_c /
// sum_c w_c l_c -- so the result has the same bits whichever workgroup
// merges, and nothing goes through LDS or a barrier.  The records are read
// with 16-byte (O) and 8-byte ((max, sum)) coherent loads through a range
// that ends with the head's last record, NREC records per round trip, every
// load of a round issued before the first use (loads past the last record
// read zeros without a memory access).
template <int D, int ROWS>
__device__ __forceinline__ void merge_head_records(const SplitKParams& p, int b, int kvh, int head,
                                                   int64_t s0, int n, int tid) {
    constexpr int VPT = (ROWS * D / 4 + 255) / 256;   // 4-float groups per thread
    constexpr int NREC = VPT >= 8 ? 2 : 16 / VPT;     // records per round trip
    const int R = p.R, n4 = R * D / 4;
    const __amdgpu_buffer_rsrc_t orange =
        coherent_range(p.ws_o + s0 * R * D, (uint32_t)n * (uint32_t)(R * D) * 4u);
    const __amdgpu_buffer_rsrc_t mrange =
        coherent_range(p.ws_ml + s0 * R * 2, (uint32_t)n * (uint32_t)R * 8u);
#pragma unroll
    for (int v = 0; v < VPT; ++v) {
        const int g = tid + 256 * v;
        if (g >= n4) break;
        const int rr = 4 * g / D, dd = 4 * g % D;
        // Row maximum over every record (a separate round only when the
        // records do not fit one).
        float M = kNegInf;
        if (n > NREC) {
            for (int c0 = 0; c0 < n; c0 += 16) {
                float m[16];
#pragma unroll
                for (int c = 0; c < 16; ++c)
                    m[c] = load_coherent2(mrange, (uint32_t)(((c0 + c) * R + rr) * 8)).x;
#pragma unroll
                for (int c = 0; c < 16; ++c)
                    if (c0 + c < n) M = fmaxf(M, m[c]);
            }
        }
        float den = 0.f;
        vf4 acc = vf4{0.f, 0.f, 0.f, 0.f};
        for (int c0 = 0; c0 < n; c0 += NREC) {
            float2 ml[NREC];
            vf4 o[NREC];
#pragma unroll
            for (int c = 0; c < NREC; ++c) {
                ml[c] = load_coherent2(mrange, (uint32_t)(((c0 + c) * R + rr) * 8));
                o[c] = load_coherent4(orange, (uint32_t)(((c0 + c) * R * D + 4 * g) * 4));
            }
            if (n <= NREC) {
#pragma unroll
                for (int c = 0; c < NREC; ++c)
                    if (c < n) M = fmaxf(M, ml[c].x);
            }
            const float M_use = M == kNegInf ? 0.f : M;
#pragma unroll
            for (int c = 0; c < NREC; ++c) {
                if (c0 + c < n) {
                    const float w = fast_exp2(ml[c].x - M_use);
                    den += w * ml[c].y;
                    acc += w * o[c];
                }
            }
        }
        const int gr = p.row0 + rr, hq = kvh * p.G + gr / p.Tq, t = gr % p.Tq;
        float* orow = p.o.p + b * p.o.sb + hq * p.o.sh + t * p.o.st;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (dd + i < p.d) orow[dd + i] = den > 0.f ? acc[i] / den : 0.f;
    }
    if (tid == 0)
        __hip_atomic_store(p.ws_cnt + head, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ROWS = 16: R <= 16 query rows per KV head on v_mfma_f32_16x16x4_f32 (above).
// ROWS = 32 / 64: 2 / 4 row groups of 16 rows; the waves split into the row
// groups (2 / 1 waves each), and the waves of a group interleave the blocks,
// so every K/V byte of the chunk is read from HBM once for all the rows (the
// row groups' loads of one block meet in L1 / L2, so they use ordinary loads).
// ROWS = 4: R <= 4 rows (single-token decode with G <= 4) on
// v_mfma_f32_4x4x1_16b_f32, which wastes no MFMA work on padding rows:
//   S = Q K^T: lane l scores key l % 16 over dim group l / 16 (D/4 dims); Q is
//     the broadcast A operand (8 dims of 4 rows per register), K comes from
//     the LDS slice; the 4 dim groups are summed with two lane swaps;
//   O += P V: V keeps the coalesced row layout of its load (LPR lanes per key
//     row, 64 / LPR keys per load), P is the broadcast A operand (one register
//     holds the 16 keys' probabilities, regrouped through LDS); each key group
//     accumulates its own partial O, summed once per segment.
// MASK: causal rows (p.masked), compiled only into the variants that serve them.
// A split launch places at most one workgroup on a CU (its chunks are cut
// for that), so the 16-row tiles at d >= 128 may take the whole register
// file (AGPRs included) instead of spilling.
template <int D, bool APPEND, int ROWS, bool MASK = false>
__global__ __launch_bounds__(256, (D >= 128 && ROWS >= 16) ? 1 : 2) void splitk_kernel(const SplitKParams p) {
    constexpr bool NARROW = ROWS == 4;
    constexpr int RG = NARROW ? 1 : ROWS / 16;   // row groups of 16 rows
    constexpr int WPR = 4 / RG;                  // waves per row group
    constexpr bool NT = RG == 1;                 // each block read by one wave only
    constexpr int KS = D + 4;            // LDS row stride (16-byte reads conflict-free)
    constexpr int LPR = D / 4;           // lanes per K row in the coalesced load
    constexpr int RPI = 64 / LPR;        // K rows per load instruction
    constexpr int NK = KB / RPI;         // K float4 loads per lane per block
    constexpr int NH = D / 64;           // V float4 loads per key step
    constexpr int NQ = D / 4;            // Q^T registers per lane
    constexpr int NB = D / 16;           // 16-dim output blocks
    constexpr int OS = D + 4;            // merge-buffer row stride (rows start 4 banks apart)
    constexpr int NQN = D / 16;          // narrow: Q registers per lane
    constexpr int CBV = D == 128 ? 3 : 2;  // narrow: PV broadcast group (LPR / 4 blocks)
    // K/V blocks held in registers per wave.  At d = 256 one 16-key block is
    // 32 KB of K and V per wave, and the other waves cover its latency.  The
    // 4-row tile at d = 128 also keeps one: 256 workgroups with 2 blocks per
    // wave in flight hold ~32 MB of loads, and that queue sets the loaded
    // latency (a segment's first blocks arrived 7.8 us after its start, 3.7
    // us with one), while the other waves' blocks keep the stream busy
    // (config-3 decode 108.8 -> 107.5 us on MI355X; the 16-row tile, with 4x
    // the MFMA work per block, loses 5 us with one).
    constexpr int DEPTH = (D >= 256 || (D >= 128 && NARROW)) ? 1 : 2;
    static_assert(ROWS == 4 || ROWS == 16 || ROWS == 32 || ROWS == 64, "row tile");
    static_assert(!NARROW || D <= 128, "4-row tile up to d = 128");
    static_assert(4 * (NARROW ? 4 : 16) * OS <= 4 * KB * KS, "merge buffer must fit in the K slices");
    static_assert(NK == 4 * NH, "K and V loads per block");

    __shared__ __attribute__((aligned(16))) float lds[4 * KB * KS];
    __shared__ float ml_s[4][16][2];
    __shared__ vf4 p_s[4][16];           // narrow: P of a wave's 16 keys
    __shared__ int pend_s[2][4];         // fused combine: heads this workgroup merges
    __shared__ int n_pend_s;
    __shared__ int pref[MAX_SEQS + 1];
    __shared__ int cut_s[kMaxCutWg + 1]; // cut chunks: workgroup w streams [cut_s[w], cut_s[w+1])

    const int tid = threadIdx.x, lane = tid & 63;
    // Wave index as a scalar: keeps the per-wave block loop uniform, so the
    // compiler neither masks it nor drains the prefetched loads at its head.
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;
    // row group of this wave and its place among the group's waves
    const int rgw = wave / WPR, kw = wave % WPR;
    const int my_row = 16 * rgw + col;    // 16-row tiles: this lane's query row
    // narrow lane roles: QK broadcast block within the dim group, A row, and
    // the P element supplied to PV (key RPI * block + key group, row).
    const int na = (lane >> 2) & 3, ni = lane & 3;
    const int p_idx = 4 * (RPI * ((lane % LPR) >> 2) + lane / LPR) + ni;
    const int wg = blockIdx.x;
    // Kernel arguments: the loads of the tables go out first, then the scalar
    // fields' cache lines together, so the prologue waits one round trip for
    // all of them.  (Left to the compiler, each first use paid its own, in a
    // chain: 1-2 us per launch before the first K/V load.)
    const int arg_pref_tid = p.arg_pref[min(tid, kArgSeqs)];
    const int ph0 = p.pack_head[min(wg, kMaxPackWg - 1)];
    const int ph1 = p.pack_head[min(wg + 1, kMaxPackWg)];
    const int pa = p.pack_head[min(2 * wg, kMaxPackWg - 1)];
    const int pb = p.pack_head[min(2 * wg + 1, kMaxPackWg - 1)];
    const int cut_tid = p.chunk_end[min(tid, kMaxCutWg - 1)];
    warm_kernargs<0, offsetof(SplitKParams, arg_pref), offsetof(SplitKParams, fused),
                  offsetof(SplitKParams, pack_head)>();
    asm volatile("" ::"v"(arg_pref_tid), "v"(ph0), "v"(ph1), "v"(pa), "v"(pb), "v"(cut_tid));   // one wait

    build_prefix<APPEND>(p, pref, tid, lane, wave, arg_pref_tid);
    if (p.cut) {
        if (tid == 0) cut_s[0] = 0;
        if (tid < p.n_wg) cut_s[tid + 1] = cut_tid;
    }
    __syncthreads();
    if (wg == 0 && !p.arg_pref_valid)   // snapshot for the combine kernel (lens may advance meanwhile)
        for (int b = tid; b <= p.B; b += 256) p.ws_pref[b] = pref[b];

    const int total = pref[p.B];
    if (tid == 0) n_pend_s = 0;
    if (p.fused && wg == 0) {            // sequences with no keys: zero output
        for (int bb = 0; bb < p.B; ++bb) {
            if (pref[bb + 1] != pref[bb]) continue;
            for (int e = tid; e < p.Hkv * p.R * p.d; e += 256) {
                const int dd = e % p.d, rest = e / p.d, rr = rest % p.R, kv = rest / p.R;
                const int gr = p.row0 + rr, hq = kv * p.G + gr / p.Tq, t = gr % p.Tq;
                p.o.p[bb * p.o.sb + hq * p.o.sh + t * p.o.st + dd] = 0.f;
            }
        }
    }
    int g, g_end, g2 = 0, g2_end = 0;
    // Flattened start of head h (h = B * Hkv: the end of the last head).
    auto head_key = [&](int h) {
        const int bb = h / p.Hkv, kk = h % p.Hkv;
        return bb >= p.B ? total : pref[bb] + kk * ((pref[bb + 1] - pref[bb]) / p.Hkv);
    };
    if (p.packed == 2) {                 // paired: head pa, then head pb
        g = head_key(pa);
        g_end = head_key(pa + 1);
        if (pb != 0xFFFF) {
            g2 = head_key(pb);
            g2_end = head_key(pb + 1);
        }
    } else if (p.packed) {
        g = head_key(ph0);
        g_end = head_key(ph1);
    } else if (p.cut) {
        g = cut_s[wg];
        g_end = cut_s[wg + 1];
    } else {
        g = wg * p.chunk;
        g_end = min(total, g + p.chunk);
    }
    // Workgroup whose chunk holds flattened key `key`.
    auto owner = [&](int key) {
        if (!p.cut) return key / p.chunk;
        int lo = 0, hi = p.n_wg - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (cut_s[mid] <= key) lo = mid; else hi = mid - 1;
        }
        return lo;
    };
    if (g >= g_end) return;
    // first sequence whose keys reach past flattened key k
    auto seq_of = [&](int k) {
        int lo = 0, hi = p.B - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (pref[mid] <= k) lo = mid; else hi = mid - 1;
        }
        return lo;
    };
    int b = seq_of(g);

    float* Kw = lds + wave * KB * KS;    // this wave's K slice
    int v_col[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) v_col[h] = min(64 * h + 4 * col, p.d - 4);
    const int kc_col = min(4 * (lane % LPR), p.d - 4);
    // Row strides in 32 bits: the host guarantees rows * stride < 2^31 per head.
    const int kst = (int)p.kst, vst = (int)p.vst;

    while (g < g_end) {
        const int Lb = (pref[b + 1] - pref[b]) / p.Hkv;
        if (Lb == 0 || g >= pref[b + 1]) { ++b; continue; }
        const int kvh = (g - pref[b]) / Lb;
        const int h_start = pref[b] + kvh * Lb;
        const int key_begin = g - h_start;
        const int key_end = min(g_end, h_start + Lb) - h_start;
        const int head = b * p.Hkv + kvh;
        const bool whole = key_begin == 0 && key_end == Lb;

        const float* kb = p.k + b * p.ksb + kvh * p.ksh;
        const float* vb = p.v + b * p.vsb + kvh * p.vsh;

        // Decode step, segment holding the new row (key Lb - 1).  4-row tile:
        // the row is prefetched into registers here, patched into the last
        // block's operands, and stored into the cache after the block loop, so
        // no load waits on it.  16-row tile: stored into the cache first and
        // read back like any cached row.
        const bool has_new = APPEND && key_end == Lb;
        if (p.fused && has_new && p.lens_w && kvh == 0 && tid == 0) p.lens_w[b] = Lb;
        vf4 nk = vf4{0.f, 0.f, 0.f, 0.f}, nv = nk;
        if (NARROW && has_new) {
            nk = *reinterpret_cast<const vf4*>(p.k_new + b * p.kn_sb + kvh * p.kn_sh + kc_col);
            nv = *reinterpret_cast<const vf4*>(p.v_new + b * p.vn_sb + kvh * p.vn_sh + kc_col);
        }
        if (!NARROW && has_new) {
            const int row = Lb - 1;
            if (tid < D / 4 && 4 * tid < p.d) {
                const float* knb = p.k_new + b * p.kn_sb + kvh * p.kn_sh;
                const float* vnb = p.v_new + b * p.vn_sb + kvh * p.vn_sh;
                *reinterpret_cast<vf4*>(const_cast<float*>(kb) + (int64_t)row * p.kst + 4 * tid) =
                    *reinterpret_cast<const vf4*>(knb + 4 * tid);
                *reinterpret_cast<vf4*>(const_cast<float*>(vb) + (int64_t)row * p.vst + 4 * tid) =
                    *reinterpret_cast<const vf4*>(vnb + 4 * tid);
            }
            __syncthreads();
        }

        // Q^T fragment: lane holds query row `col`, dims grp*D/4 .. +D/4, pre-scaled.
        // Narrow: lane 16g + 4a + i holds row i, dims g*D/4 + 4t + a (t < D/16).
        float qf[NARROW ? NQN : NQ];
        if constexpr (NARROW) {
            const bool rok = ni < p.R;
            const int gr = p.row0 + (rok ? ni : 0);
            const int hq = kvh * p.G + gr / p.Tq, t = gr % p.Tq;
            const float* qp = p.q.p + b * p.q.sb + hq * p.q.sh + t * p.q.st;
#pragma unroll
            for (int t4 = 0; t4 < NQN; ++t4) {   // clamped loads, then select: no waits between them
                const int c = grp * (D / 4) + 4 * t4 + na;
                const float x = qp[min(c, p.d - 1)];
                qf[t4] = (rok && c < p.d) ? x * p.qscale : 0.f;
            }
        } else {
            const bool rok = my_row < p.R;
            const int gr = p.row0 + (rok ? my_row : 0);
            const int hq = kvh * p.G + gr / p.Tq, t = gr % p.Tq;
            const float* qp = p.q.p + b * p.q.sb + hq * p.q.sh + t * p.q.st;
#pragma unroll
            for (int s4 = 0; s4 < NQ / 4; ++s4) {   // clamped loads, then select
                const int c = grp * NQ + 4 * s4;
                const vf4 x = *reinterpret_cast<const vf4*>(qp + min(c, p.d - 4));
                const bool ok = rok && c < p.d;
                qf[4 * s4 + 0] = ok ? x.x * p.qscale : 0.f;
                qf[4 * s4 + 1] = ok ? x.y * p.qscale : 0.f;
                qf[4 * s4 + 2] = ok ? x.z * p.qscale : 0.f;
                qf[4 * s4 + 3] = ok ? x.w * p.qscale : 0.f;
            }
        }

        // K and V rows of the segment are read through buffer ranges that
        // end with its last key: loads of keys past it (the tail of the last
        // block, and the ring's loads beyond the segment) return zeros without
        // a memory access, and zero rows get weight 0 (their scores are masked
        // to -inf).  Columns past d read the row's last 4 floats (their Q
        // columns are zero, their O columns are never stored).  Loads are
        // branch-free, so the next block stays in flight while the current
        // one computes.  They are non-temporal where one wave reads a block:
        // each K/V byte is read once per launch, and keeping the stream out of
        // the caches' normal allocation lifts a chunked read of the cache from
        // ~6.0 to ~6.9 TB/s on MI355X.  (The host keeps a head under 2^30
        // floats, so the byte offsets fit in 32 bits.)
        const __amdgpu_buffer_rsrc_t krange = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(kb), 0, (uint32_t)key_end * (uint32_t)kst * 4u, 0x00020000);
        const __amdgpu_buffer_rsrc_t vrange = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(vb), 0, (uint32_t)key_end * (uint32_t)vst * 4u, 0x00020000);
        // Byte offset = a lane constant + a wave-uniform part per load (one
        // VALU add each; no per-load address registers live across blocks).
        const uint32_t k_lane = ((uint32_t)(lane / LPR) * (uint32_t)kst + (uint32_t)kc_col) * 4u;
        const uint32_t vn_lane = ((uint32_t)(lane / LPR) * (uint32_t)vst + (uint32_t)kc_col) * 4u;
        uint32_t vw_lane[NH];
#pragma unroll
        for (int h = 0; h < NH; ++h) vw_lane[h] = ((uint32_t)(4 * grp) * (uint32_t)vst + (uint32_t)v_col[h]) * 4u;
        auto ld = [&](__amdgpu_buffer_rsrc_t range, uint32_t lane_off, int key0, int st) __attribute__((always_inline)) {
            const uint32_t uni = (uint32_t)__builtin_amdgcn_readfirstlane(key0) * (uint32_t)st * 4u;
            return __builtin_bit_cast(vf4, __builtin_amdgcn_raw_buffer_load_b128(range, lane_off + uni, 0,
                                                                                 NT ? 2 : 0));
        };
        auto load_block = [&](vf4 (&kr)[NK], vf4 (&vr)[4 * NH], int kb0) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < NK; ++i) kr[i] = ld(krange, k_lane, kb0 + RPI * i, kst);
            if constexpr (NARROW) {
#pragma unroll
                for (int i = 0; i < NK; ++i) vr[i] = ld(vrange, vn_lane, kb0 + RPI * i, vst);
            } else {
#pragma unroll
                for (int st = 0; st < 4; ++st)
#pragma unroll
                    for (int h = 0; h < NH; ++h) vr[st * NH + h] = ld(vrange, vw_lane[h], kb0 + st, vst);
            }
        };

        floatx4 o[NARROW ? 4 : NB];
#pragma unroll
        for (int bb = 0; bb < (NARROW ? 4 : NB); ++bb) o[bb] = floatx4{0.f, 0.f, 0.f, 0.f};
        float m_run = kNegInf, l_run = 0.f;
        floatx4 m4 = floatx4{kNegInf, kNegInf, kNegInf, kNegInf};   // narrow: per row
        floatx4 l4 = floatx4{0.f, 0.f, 0.f, 0.f};                   // narrow: per row, this lane's key

        // One 16-key block: stage K, S^T = K Q^T, online softmax, O^T += V^T P^T.
        auto block = [&](vf4 (&kr)[NK], vf4 (&vr)[4 * NH], int kb0) __attribute__((always_inline)) {
            if (NARROW && has_new && kb0 + KB >= key_end) {
                // Rows at or past the new one (clamped loads) take the new row.
#pragma unroll
                for (int i = 0; i < NK; ++i) {
                    const bool fresh = kb0 + lane / LPR + RPI * i >= key_end - 1;
                    kr[i] = fresh ? nk : kr[i];
                    vr[i] = fresh ? nv : vr[i];
                }
            }
            wave_lds_sync();
#pragma unroll
            for (int i = 0; i < NK; ++i)
                *reinterpret_cast<vf4*>(Kw + (lane / LPR + RPI * i) * KS + 4 * (lane % LPR)) = kr[i];
            wave_lds_sync();

          if constexpr (NARROW) {
            floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
            const float* krow = Kw + col * KS + grp * (D / 4);
#pragma unroll
            for (int t = 0; t < NQN; ++t) {
                const vf4 kq = *reinterpret_cast<const vf4*>(krow + 4 * t);
                s = mfma4<2, 0>(qf[t], kq.x, s);
                s = mfma4<2, 1>(qf[t], kq.y, s);
                s = mfma4<2, 2>(qf[t], kq.z, s);
                s = mfma4<2, 3>(qf[t], kq.w, s);
            }
            // s[r] = score of query row r for key kb0 + col (summed over dim groups).
#pragma unroll
            for (int r = 0; r < 4; ++r) s[r] = quad_rows_sum(s[r]);
            if (kb0 + KB > key_end) {
                const bool ok = kb0 + col < key_end;
#pragma unroll
                for (int r = 0; r < 4; ++r) s[r] = ok ? s[r] : kNegInf;
            }
            if (MASK && kb0 + KB - 1 > p.q_off) {   // causal rows: key <= q_off + t
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    s[r] = kb0 + col <= p.q_off + (p.row0 + r) % p.Tq ? s[r] : kNegInf;
            }
            // Lazy rescale: keep each row's reference max until a score exceeds
            // it by 8 (a factor 256 in exp2), so most blocks skip the row max.
            bool grow = false;
#pragma unroll
            for (int r = 0; r < 4; ++r) grow |= s[r] > m4[r] + 8.f;
            if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float m_new = fmaxf(m4[r], row16_max(s[r]));
                    const float alpha = fast_exp2(m4[r] - (m_new == kNegInf ? 0.f : m_new));
                    l4[r] *= alpha;
#pragma unroll
                    for (int c = 0; c < 4; ++c) o[c][r] *= alpha;
                    m4[r] = m_new;
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[r] = fast_exp2(s[r] - (m4[r] == kNegInf ? 0.f : m4[r]));
                l4[r] += s[r];
            }
            // Regroup P for the PV broadcast: lane supplies P[row ni][key p_idx / 4].
            if (lane < 16) p_s[wave][lane] = vf4{s[0], s[1], s[2], s[3]};
            wave_lds_sync();
            const float pa = reinterpret_cast<const float*>(p_s[wave])[p_idx];
            static_for<NK>([&](auto vi) __attribute__((always_inline)) {
                constexpr int V = decltype(vi)::value;
                const vf4 vv = vr[V];
                o[0] = mfma4<CBV, V>(pa, vv.x, o[0]);
                o[1] = mfma4<CBV, V>(pa, vv.y, o[1]);
                o[2] = mfma4<CBV, V>(pa, vv.z, o[2]);
                o[3] = mfma4<CBV, V>(pa, vv.w, o[3]);
            });
          } else {
            floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
            const float* krow = Kw + col * KS + grp * NQ;
#pragma unroll
            for (int t = 0; t < NQ / 4; ++t) {
                const vf4 kq = *reinterpret_cast<const vf4*>(krow + 4 * t);
                s = __builtin_amdgcn_mfma_f32_16x16x4f32(kq.x, qf[4 * t + 0], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_16x16x4f32(kq.y, qf[4 * t + 1], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_16x16x4f32(kq.z, qf[4 * t + 2], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_16x16x4f32(kq.w, qf[4 * t + 3], s, 0, 0, 0);
            }
            // s[r] = score of key kb0 + 4*grp + r for query row `col`.
            if (kb0 + KB > key_end) {
#pragma unroll
                for (int r = 0; r < 4; ++r) s[r] = (kb0 + 4 * grp + r < key_end) ? s[r] : kNegInf;
            }
            if (MASK && kb0 + KB - 1 > p.q_off) {   // causal rows: key <= q_off + t
                const int last = p.q_off + (p.row0 + my_row) % p.Tq;
#pragma unroll
                for (int r = 0; r < 4; ++r) s[r] = (kb0 + 4 * grp + r <= last) ? s[r] : kNegInf;
            }
            float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
            mt = quad_rows_max(mt);
            const float m_new = fmaxf(m_run, mt);
            const float m_use = (m_new == kNegInf) ? 0.f : m_new;
            const float alpha = fast_exp2(m_run - m_use);
            float ls = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s[r] = fast_exp2(s[r] - m_use);
                ls += s[r];
            }
            l_run = alpha * l_run + ls;     // this lane's 4 keys; summed over lanes below
            m_run = m_new;
#pragma unroll
            for (int bb = 0; bb < NB; ++bb) o[bb] *= alpha;

            // O^T += V^T P^T.  Step st pairs key kb0 + 4*grp + st (= register st
            // of P^T); dim block 4h + c covers dims 64h + 4*i + c, i = lane % 16.
#pragma unroll
            for (int st = 0; st < 4; ++st)
#pragma unroll
                for (int h = 0; h < NH; ++h) {
                    const vf4 vv = vr[st * NH + h];
                    o[4 * h + 0] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, s[st], o[4 * h + 0], 0, 0, 0);
                    o[4 * h + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, s[st], o[4 * h + 1], 0, 0, 0);
                    o[4 * h + 2] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, s[st], o[4 * h + 2], 0, 0, 0);
                    o[4 * h + 3] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, s[st], o[4 * h + 3], 0, 0, 0);
                }
          }
        };

        // Ring of DEPTH register buffers over this wave's blocks (kw,
        // kw+WPR, ...): while one block computes, the next DEPTH-1 blocks'
        // loads are in flight.  The loop has a single exit at its end, which
        // lets the next blocks' loads issue before the wait for the current
        // block's data.  At d = 64 (8 KB of K/V per 16-key block) 3 and 4
        // buffers measured slower than 2: cross-attention over 1500 frames
        // 29.6 and 30.5 against 28.9 us, GPT-2 decode attend 35.0 and 35.3
        // against 32.5 us.
        const int n_blocks = (key_end - key_begin + KB - 1) / KB;
        const int n_mine = kw < n_blocks ? (n_blocks - kw + WPR - 1) / WPR : 0;
        vf4 kq[DEPTH][NK], vq[DEPTH][4 * NH];
        int kb0 = key_begin + kw * KB;
#pragma unroll
        for (int s = 0; s + 1 < DEPTH; ++s) load_block(kq[s], vq[s], kb0 + WPR * KB * s);
        int done = 0;
        for (; done + DEPTH <= n_mine; done += DEPTH, kb0 += WPR * KB * DEPTH) {
#pragma unroll
            for (int s = 0; s < DEPTH; ++s) {
                load_block(kq[(s + DEPTH - 1) % DEPTH], vq[(s + DEPTH - 1) % DEPTH],
                           kb0 + WPR * KB * (s + DEPTH - 1));
                block(kq[s], vq[s], kb0 + WPR * KB * s);
            }
        }
#pragma unroll
        for (int s = 0; s + 1 < DEPTH; ++s)
            if (done + s < n_mine) block(kq[s], vq[s], kb0 + WPR * KB * s);
        if (NARROW && has_new && wave == 0 && lane < LPR && 4 * lane < p.d) {
            const int row = Lb - 1;
            *reinterpret_cast<vf4*>(const_cast<float*>(kb) + row * kst + 4 * lane) = nk;
            *reinterpret_cast<vf4*>(const_cast<float*>(vb) + row * vst + 4 * lane) = nv;
        }
        float* ob = lds;                  // [4 waves][ROWS rows][OS]
        if constexpr (NARROW) {
            // Sum the key groups' partial O: o[c][r] = O[row r][dim 4 (lane % LPR) + c].
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    o[c][r] = RPI == 2 ? pair_sum(o[c][r]) : quad_rows_sum(o[c][r]);
            float l_tot[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) l_tot[r] = row16_sum(l4[r]);
            __syncthreads();              // every wave is done with its K slice
            if (lane < LPR) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    *reinterpret_cast<vf4*>(ob + (wave * 4 + r) * OS + 4 * lane) =
                        vf4{o[0][r], o[1][r], o[2][r], o[3][r]};
            }
            if (lane == 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) { ml_s[wave][r][0] = m4[r]; ml_s[wave][r][1] = l_tot[r]; }
            }
        } else {
            const float l_tot = quad_rows_sum(l_run);
            // Merge the 4 waves through LDS: O[row col][dim] with
            // dim = 64h + 16*grp + 4*reg + c  for  o[4h + c][reg].
            __syncthreads();              // every wave is done with its K slice
#pragma unroll
            for (int h = 0; h < NH; ++h)
#pragma unroll
                for (int reg = 0; reg < 4; ++reg)
                    *reinterpret_cast<vf4*>(ob + (wave * 16 + col) * OS + 64 * h + 16 * grp + 4 * reg) =
                        vf4{o[4 * h + 0][reg], o[4 * h + 1][reg], o[4 * h + 2][reg], o[4 * h + 3][reg]};
            if (grp == 0) { ml_s[wave][col][0] = m_run; ml_s[wave][col][1] = l_tot; }
        }
        __syncthreads();

        // Rows of the 16-row tiles sit at ob[(wave * 16 + row % 16) * OS];
        // row rr is the row group rr / 16, whose WPR waves are merged.
        constexpr int RPW = NARROW ? 4 : 16;
        const int64_t slot = (int64_t)wg + head;    // unique per (workgroup, head)
        for (int e = tid; e < p.R * D; e += 256) {
            const int rr = e / D, dd = e % D;
            const int w0 = (rr / RPW) * WPR, lr = rr % RPW;
            float M = kNegInf;
#pragma unroll
            for (int j = 0; j < WPR; ++j) M = fmaxf(M, ml_s[w0 + j][lr][0]);
            const float M_use = M == kNegInf ? 0.f : M;
            float l = 0.f, acc = 0.f;
#pragma unroll
            for (int j = 0; j < WPR; ++j) {
                const float f = fast_exp2(ml_s[w0 + j][lr][0] - M_use);
                l += f * ml_s[w0 + j][lr][1];
                acc += f * ob[((w0 + j) * RPW + lr) * OS + dd];
            }
            if (whole) {
                if (dd < p.d) {
                    const int gr = p.row0 + rr, hq = kvh * p.G + gr / p.Tq, t = gr % p.Tq;
                    p.o.p[b * p.o.sb + hq * p.o.sh + t * p.o.st + dd] = l > 0.f ? acc / l : 0.f;
                }
            } else {
                store_coherent(p.ws_o + (slot * p.R + rr) * D + dd, acc);
                if (dd == 0) {
                    store_coherent(p.ws_ml + (slot * p.R + rr) * 2, M);
                    store_coherent(p.ws_ml + (slot * p.R + rr) * 2 + 1, l);
                }
            }
        }
        if (p.fused && !whole) {
            // Count this workgroup in.  The last of the head's n workgroups
            // merges it after its own segments (a workgroup has at most two
            // split heads: its first and its last segment).
            const int w_first = key_begin == 0 ? wg : owner(h_start);
            const int w_last = key_end == Lb ? wg : owner(h_start + Lb - 1);
            wait_stores_performed();
            __syncthreads();
            if (tid == 0) {
                const unsigned old = __hip_atomic_fetch_add(p.ws_cnt + head, 1u, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
                if (old == (unsigned)(w_last - w_first) && n_pend_s < 2) {
                    pend_s[n_pend_s][0] = b;
                    pend_s[n_pend_s][1] = kvh;
                    pend_s[n_pend_s][2] = w_first;
                    pend_s[n_pend_s][3] = w_last - w_first + 1;
                    ++n_pend_s;
                }
            }
        }
        __syncthreads();                  // LDS is reused by the next segment
        g = h_start + key_end;
        if (g >= g_end && g2 < g2_end) {  // paired packing: the second head
            g = g2;
            g_end = g2_end;
            g2 = g2_end;
            b = seq_of(g);
        }
    }
    const int n_pend = n_pend_s;
    for (int i = 0; i < n_pend; ++i) {
        const int bb = pend_s[i][0], kv = pend_s[i][1], w_first = pend_s[i][2], n = pend_s[i][3];
        merge_head_records<D, ROWS>(p, bb, kv, bb * p.Hkv + kv, (int64_t)w_first + bb * p.Hkv + kv, n,
                                    tid);
    }
}

// Per (sequence, KV head): zero output for an empty sequence, merge the
// partial records of the workgroups that shared the head, and in a decode step
// publish the sequence's new length.  Every global load is issued before the
// first barrier (partial O rows into registers, (max, sum) pairs into LDS), so
// the kernel costs one memory round trip.
template <int D, int ROWS>
__global__ __launch_bounds__(256) void splitk_combine_kernel(const SplitKParams p) {
    constexpr int EPT = ROWS * D / 256;   // output elements per thread (R <= ROWS)
    constexpr int NPRE = EPT >= 16 ? 2 : 4;   // partials per element held in registers
    __shared__ float2 ml_s[COMBINE_ML];   // [n records][R rows], n * R <= COMBINE_ML
    const int head = blockIdx.x;
    const int b = head / p.Hkv, kvh = head % p.Hkv;
    const int tid = threadIdx.x;
    const int* pr = p.arg_pref_valid ? p.arg_pref : p.ws_pref;
    const int p0 = pr[b], p1 = pr[b + 1];
    const int Lb = (p1 - p0) / p.Hkv;
    if (p.lens_w && kvh == 0 && tid == 0) p.lens_w[b] = Lb;
    auto out_ptr = [&](int rr) {
        const int gr = p.row0 + rr, hq = kvh * p.G + gr / p.Tq, t = gr % p.Tq;
        return p.o.p + b * p.o.sb + hq * p.o.sh + t * p.o.st;
    };
    if (Lb == 0) {
        for (int e = tid; e < p.R * p.d; e += 256) out_ptr(e / p.d)[e % p.d] = 0.f;
        return;
    }
    const int h_start = p0 + kvh * Lb;
    const int w_first = h_start / p.chunk, w_last = (h_start + Lb - 1) / p.chunk;
    const int n = w_last - w_first + 1;
    if (n <= 1) return;                   // written directly by the split kernel
    const int64_t s0 = (int64_t)w_first + head;   // slots s0 .. s0 + n - 1
    const int RD = p.R * D;
    const float* o_src = p.ws_o + s0 * RD;

    float pre[EPT][NPRE];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int e = tid + 256 * j;
#pragma unroll
        for (int c = 0; c < NPRE; ++c)
            pre[j][c] = (e < RD && c < n) ? o_src[(int64_t)c * RD + e] : 0.f;
    }
    for (int e = tid; e < n * p.R; e += 256)
        ml_s[e] = *reinterpret_cast<const float2*>(p.ws_ml + ((s0 + e / p.R) * p.R + e % p.R) * 2);
    __syncthreads();
    if (tid < p.R) {                      // weights: exp2(m_c - M) / sum_c exp2(m_c - M) l_c
        float M = kNegInf;
        for (int c = 0; c < n; ++c) M = fmaxf(M, ml_s[c * p.R + tid].x);
        const float M_use = M == kNegInf ? 0.f : M;
        float den = 0.f;
        for (int c = 0; c < n; ++c) den += fast_exp2(ml_s[c * p.R + tid].x - M_use) * ml_s[c * p.R + tid].y;
        const float inv = den > 0.f ? 1.f / den : 0.f;
        for (int c = 0; c < n; ++c) ml_s[c * p.R + tid].x = fast_exp2(ml_s[c * p.R + tid].x - M_use) * inv;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int e = tid + 256 * j;
        if (e >= RD) break;
        const int rr = e / D, dd = e % D;
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < NPRE; ++c)
            if (c < n) acc += ml_s[c * p.R + rr].x * pre[j][c];
        for (int c = NPRE; c < n; ++c) acc += ml_s[c * p.R + rr].x * o_src[(int64_t)c * RD + e];
        if (dd < p.d) out_ptr(rr)[dd] = acc;
    }
}

template <int D, int ROWS>
hipError_t launch_rows(const SplitKParams& p, hipStream_t stream) {
    if (p.n_wg > 0) {
        // Causal rows come only from few-query prefill steps (<= 16 rows).
        bool masked = false;
        if constexpr (ROWS <= 16) masked = p.masked != 0;
        if (p.k_new)
            hipLaunchKernelGGL((splitk_kernel<D, true, ROWS>), dim3(p.n_wg), dim3(256), 0, stream, p);
        else if (masked)
            hipLaunchKernelGGL((splitk_kernel<D, false, ROWS <= 16 ? ROWS : 16, true>), dim3(p.n_wg),
                               dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL((splitk_kernel<D, false, ROWS>), dim3(p.n_wg), dim3(256), 0, stream, p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (p.fused) return hipSuccess;
    hipLaunchKernelGGL((splitk_combine_kernel<D, ROWS>), dim3(p.B * p.Hkv), dim3(256), 0, stream, p);
    return hipGetLastError();
}

// Row tile of a launch: 4 rows (single-token decode with G <= 4, d <= 128),
// else the smallest of 16 / 32 / 64 that holds the launch's rows.
template <int D>
hipError_t launch_splitk_d(const SplitKParams& p, hipStream_t stream) {
    if (D <= 128 && p.R <= 4) {
        if constexpr (D <= 128) return launch_rows<D, 4>(p, stream);
    }
    if (p.R <= 16) return launch_rows<D, 16>(p, stream);
    if (p.R <= 32) return launch_rows<D, 32>(p, stream);
    if constexpr (D <= 128) return launch_rows<D, 64>(p, stream);
    return hipErrorInvalidValue;
}

// ---- KV append (prefill-style, many rows) ---------------------------------

// Writes new rows [B, Hkv, t_new, d] at row lens[b] + t of each (b, kv head).
__global__ void kv_append_kernel(float* kc, float* vc, const int32_t* lens, View4 kn, View4 vn,
                                 int B, int Hkv, int cap, int d, int t_new) {
    const int64_t n = (int64_t)B * Hkv * t_new * d;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int dd = e % d;
        int64_t r = e / d;
        const int t = r % t_new; r /= t_new;
        const int h = r % Hkv;
        const int b = r / Hkv;
        const int row = lens[b] + t;
        if (row < 0 || row >= cap) continue;   // host validated; never taken when consistent
        const int64_t dst = (((int64_t)b * Hkv + h) * cap + row) * d + dd;
        kc[dst] = kn.p[b * kn.sb + h * kn.sh + t * kn.st + dd * kn.sd];
        vc[dst] = vn.p[b * vn.sb + h * vn.sh + t * vn.st + dd * vn.sd];
    }
}

__global__ void zero_u32_kernel(uint32_t* x, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        x[i] = 0u;
}

__global__ void lens_bump_kernel(int32_t* lens, int B, int t_new) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) lens[b] += t_new;
}

}  // namespace

namespace {

// Workgroups of a split launch: one per CU.  Measured on MI355X against one
// per resident slot (2-3 per CU): the same at config-3 decode, and 4-13 %
// faster where more than one fits (config-5b cross-attention 28.2 against
// 32.6 us, d = 64 decode 59.5 against 61.8 us, B = 8 decode 40.1 against
// 42.5 us): a CU serves the loads of its first workgroup ahead of the others,
// so co-resident workgroups with equal chunks finish at different times,
// and fewer chunks also mean fewer partial records to merge.
int split_workgroups() {
    static std::atomic<int> cached[64];   // callers on several threads may fill it at once
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
            cus = 256;
        n = cus < MAX_WG ? cus : MAX_WG;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

}  // namespace

int splitk_padded_dim(int d) {
    if (d <= 64) return 64;
    if (d <= 128) return 128;
    if (d <= 256) return 256;
    return 0;
}

int splitk_max_rows() { return 16; }
int splitk_rows_per_launch(int d) { return splitk_padded_dim(d) >= 256 ? 32 : 64; }
int splitk_max_seqs() { return MAX_SEQS; }
int splitk_max_workgroups() { return MAX_WG; }

SplitKWorkspace splitk_workspace_layout(int B, int Hkv, int R, int d) {
    SplitKWorkspace w;
    const int D = splitk_padded_dim(d);
    // Record slot = workgroup + head: a launch has at most split_workgroups()
    // workgroups on this device (its chunks are at least total / that many keys).
    const uint64_t slots = (uint64_t)split_workgroups() + (uint64_t)B * Hkv;
    w.ml_offset = ((uint64_t)(B + 1) * 4 + 255) / 256 * 256;
    w.o_offset = w.ml_offset + (slots * R * 2 * 4 + 255) / 256 * 256;
    w.total_bytes = w.o_offset + slots * R * D * 4;
    return w;
}

namespace {

template <int D>
hipError_t launch_flat(SplitKParams p, int64_t total_keys, int max_len, hipStream_t stream) {
    plan_split_layout(p, split_workgroups(), total_keys, max_len);
    return launch_splitk_d<D>(p, stream);
}

}  // namespace

namespace {

// One launch (plus, without the fused merge, its combine kernel) over at most
// MAX_SEQS sequences and one tile of rows.
hipError_t launch_one(SplitKParams p, int64_t total_keys, int max_len, void* workspace,
                      hipStream_t stream, const int32_t* seq_lens, uint32_t* counters) {
    // Small batches carry the flattened prefix in the arguments, which saves
    // every workgroup the scan over lens.
    p.arg_pref_valid = p.B <= kArgSeqs ? 1 : 0;
    if (p.arg_pref_valid) {
        p.arg_pref[0] = 0;
        for (int b = 0; b < p.B; ++b)
            p.arg_pref[b + 1] = p.arg_pref[b] + p.Hkv * (seq_lens ? seq_lens[b] : p.tk);
    }
    // Fused combine needs the prefix in the arguments (no workgroup reads
    // lens, so the lens bump can happen inside the launch) and n * R <= 1024.
    p.fused = p.arg_pref_valid && counters != nullptr;
    p.max_parts = std::min(MAX_PARTS, (p.fused ? 1024 : COMBINE_ML) / p.R);
    const SplitKWorkspace w = splitk_workspace_layout(p.B, p.Hkv, p.R, p.d);
    char* base = static_cast<char*>(workspace);
    p.ws_pref = reinterpret_cast<int32_t*>(base);
    p.ws_cnt = counters;
    p.ws_ml = reinterpret_cast<float*>(base + w.ml_offset);
    p.ws_o = reinterpret_cast<float*>(base + w.o_offset);
    switch (splitk_padded_dim(p.d)) {
        case 64: return launch_flat<64>(p, total_keys, max_len, stream);
        case 128: return launch_flat<128>(p, total_keys, max_len, stream);
        case 256: return launch_flat<256>(p, total_keys, max_len, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_splitk(SplitKParams p, int64_t total_keys, int max_len, void* workspace,
                         hipStream_t stream, const int32_t* seq_lens, uint32_t* counters,
                         int row_begin, int row_count) {
    p.G = p.Hq / p.Hkv;
    // Batches beyond MAX_SEQS sequences: one launch per block of sequences,
    // in stream order, sharing the workspace and counters.
    if (p.B > MAX_SEQS) {
        for (int b0 = 0; b0 < p.B; b0 += MAX_SEQS) {
            SplitKParams c = p;
            c.B = std::min(MAX_SEQS, p.B - b0);
            c.q.p += b0 * p.q.sb;
            c.o.p += b0 * p.o.sb;
            c.k += b0 * p.ksb;
            c.v += b0 * p.vsb;
            if (c.lens) c.lens += b0;
            if (c.lens_w) c.lens_w += b0;
            if (c.k_new) {
                c.k_new += b0 * p.kn_sb;
                c.v_new += b0 * p.vn_sb;
            }
            int64_t keys = 0;
            for (int b = 0; b < c.B; ++b) keys += (int64_t)p.Hkv * (seq_lens ? seq_lens[b0 + b] : p.tk);
            const hipError_t e = launch_splitk(c, keys, max_len, workspace, stream,
                                               seq_lens ? seq_lens + b0 : nullptr, counters,
                                               row_begin, row_count);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // More query rows per KV head than one tile holds: one launch per range
    // of rows.  A decode step appends in the first; the later launches read
    // the stored row from the cache (lens has advanced by then).
    const int rows_end = row_count < 0 ? p.G * p.Tq : row_begin + row_count;
    const int rpl = splitk_rows_per_launch(p.d);
    for (int r0 = row_begin; r0 < rows_end; r0 += rpl) {
        SplitKParams c = p;
        c.row0 = r0;
        c.R = std::min(rpl, rows_end - r0);
        if (r0 > row_begin && p.k_new) {
            c.k_new = nullptr;
            c.v_new = nullptr;
            c.lens_w = nullptr;
        }
        const hipError_t e = launch_one(c, total_keys, max_len, workspace, stream, seq_lens, counters);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t zero_counters(uint32_t* counters, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, counters, n);
    return hipGetLastError();
}

hipError_t launch_kv_append(float* kc, float* vc, int32_t* lens_dev, View4 kn, View4 vn, int B,
                            int Hkv, int cap, int d, int t_new, hipStream_t stream) {
    const int64_t n = (int64_t)B * Hkv * t_new * d;
    if (n > 0) {
        int64_t blocks = (n + 255) / 256;
        if (blocks > 65536) blocks = 65536;
        hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, kc, vc,
                           lens_dev, kn, vn, B, Hkv, cap, d, t_new);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (B > 0 && t_new > 0)
        hipLaunchKernelGGL(lens_bump_kernel, dim3((B + 255) / 256), dim3(256), 0, stream, lens_dev,
                           B, t_new);
    return hipGetLastError();
}

}  // namespace nne
