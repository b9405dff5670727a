// FlashAttention forward for gfx950 on full-fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
// Algorithm: the tiled online softmax of the reference's
// flash_attention_forward (src/nn/flash_attention.rs:91-195) -- per query row a
// running max m and sum l, P = exp(S - m), O = alpha*O + P V, O /= l at the end
// with rows that saw no key left at zero (:186-194), fully masked key tiles
// skipped (:101-104) -- generalised to grouped-query heads (KV head hq / G) and
// a causal offset.
//
// MI355X mapping.  One wave owns 32 query rows and computes the score tile
// transposed, S^T = K Q^T, on 32x32x2 MFMAs:
//   A = K tile  (lane l supplies key l%32, reduction index l/32)
//   B = Q^T     (lane l supplies query row l%32; held in registers, pre-scaled
//                by scale*log2(e) so the softmax is a bare exp2)
// The reduction (head-dim) order is permuted so that lane half h covers dims
// [h*D/2, h*D/2 + D/2): each lane then reads its K operands as contiguous
// 16-byte LDS vectors.  The accumulator layout of S^T puts query row l%32 in
// lane l and keys 8*(r/4) + 4*(l/32) + r%4 in register r, so
//   * the row max / row sum are 16 in-lane ops plus one lane-pair exchange
//     (v_permlane32_swap),
//   * P^T register r is already the B operand of step r of O^T = V^T P^T
//     (the key order of that reduction is chosen to match), so P never
//     leaves registers,
//   * every O^T accumulator of a lane belongs to that lane's query row, so the
//     online-softmax rescale is a lane-local multiply -- done lazily, only
//     when a row max grows by more than 2^8.
// K and V tiles (32 keys) are staged through LDS, double buffered, with the
// next tile's global loads in flight while the current tile is computed.  The
// G query heads that share a KV head run as waves of one workgroup and read
// the same staged tiles.  Workgroups are numbered so that each XCD works on a
// contiguous range of KV heads (its own L2) and, within a head, the longest
// causal row blocks start first.
//
// Problems with fewer work items than CUs instead cut each item's key tiles
// into chunks, one workgroup per (item, chunk); the last chunk of an item to
// finish folds the partial (max, sum, O) records in chunk order (the same
// combine as the online softmax, so the result is independent of arrival
// order) and writes O.
#include <atomic>
#include <utility>
#include <vector>

#include "nne_common.hpp"
#include "nne_launch.hpp"

namespace nne {

namespace {

template <int D, bool VEC, int THREADS = 256>
struct TileLoader {
    // K/V tile of 32 keys x D dims = 8*D float4; 256 threads -> D/32 each.
    static constexpr int NV = 8 * D / THREADS;
    static constexpr int C4 = D / 4;    // float4 columns per row
    static_assert(NV * THREADS == 8 * D, "whole tile per pass");
    float4 kr[NV], vr[NV];

    __device__ __forceinline__ void load(const PrefillParams& p, const float* kb, const float* vb,
                                         int key0, int tid) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int idx = tid + THREADS * i;
            const int row = idx / C4, c = (idx % C4) * 4;
            const int key = key0 + row;
            if (VEC) {
                const bool ok = key < p.Tk && c < p.d;
                kr[i] = ok ? *reinterpret_cast<const float4*>(kb + key * p.k.st + c)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
                vr[i] = ok ? *reinterpret_cast<const float4*>(vb + key * p.v.st + c)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float kx[4], vx[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bool ok = key < p.Tk && c + j < p.d;
                    kx[j] = ok ? kb[key * p.k.st + (c + j) * p.k.sd] : 0.f;
                    vx[j] = ok ? vb[key * p.v.st + (c + j) * p.v.sd] : 0.f;
                }
                kr[i] = make_float4(kx[0], kx[1], kx[2], kx[3]);
                vr[i] = make_float4(vx[0], vx[1], vx[2], vx[3]);
            }
        }
    }

    __device__ __forceinline__ void store(float* ks, float* vs, int tid) const {
        constexpr int KS = D + 4, VS = D + 8;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int idx = tid + THREADS * i;
            const int row = idx / C4, c = (idx % C4) * 4;
            *reinterpret_cast<float4*>(ks + row * KS + c) = kr[i];
            *reinterpret_cast<float4*>(vs + row * VS + c) = vr[i];
        }
    }
};

// Last key index visible to any row of row block rb (or -1).
__device__ __forceinline__ int last_visible_key(const PrefillParams& p, int rb, bool causal) {
    if (!causal) return p.Tk - 1;
    int last_row = rb * 32 + 31;
    if (last_row > p.Tq - 1) last_row = p.Tq - 1;
    int lk = last_row + p.q_offset;
    return lk < p.Tk - 1 ? lk : p.Tk - 1;
}

// The j-th work item of the workgroup in slot q of XCD x (S slots per XCD):
// super-items x*per_xcd + q + k*S, k = 0, 1, ..., each one item (rank pr) or,
// with pairing, two (ranks pr and n_wg-1-pr).  Rank r is wgi = n_wg-1-r, so
// rank 0 holds the longest causal rows.  Returns 0 past the end, 2 for the
// missing partner of an odd middle rank, 1 with (head, wgi) otherwise.
__device__ __forceinline__ int item_at(const PrefillParams& p, int j, int x, int q, int S, int& head,
                                       int& wgi) {
    if (p.order_cu) {
        // Position pos in the XCD's items sorted longest first (rank-major over
        // its heads).  The hardware places workgroup q of an XCD on CU q % h
        // (h CUs, q < h first): with n <= 2h items the CUs that get a second
        // workgroup take a longer and a shorter item whose lengths add up to
        // about the same, and the CUs with one take the longest items.
        if (j > 0) return 0;
        const int h = p.order_cu, n = p.per_xcd;
        int pos = q;
        if (n <= 2 * h && n > h) {
            if (q >= h) pos = n - 1 - (q - h);
            else if (q >= n - h) pos = q - (n - h);
            else pos = (2 * h - n) + q;
        }
        head = x * p.order_hpx + pos % p.order_hpx;
        wgi = p.n_wg - 1 - pos / p.order_hpx;
        return 1;
    }
    const int k = p.pairing ? j >> 1 : j;
    const int s = x * p.per_xcd + q + k * S;
    int s_end = (x + 1) * p.per_xcd;
    if (s_end > p.n_super) s_end = p.n_super;
    if (s >= s_end) return 0;
    head = s / p.n_pairs;
    const int pr = s % p.n_pairs;
    int rank = pr;
    if (p.pairing && (j & 1)) {
        rank = p.n_wg - 1 - pr;
        if (rank == pr) return 2;
    }
    wgi = p.n_wg - 1 - rank;
    return 1;
}

// Two workgroups per CU for the persistent schedule.  At d = 128 the
// key-split variant (small problems, one short chunk per workgroup) and the
// scalar-load variant (views that are not 16-byte vectors) take the whole
// register file instead of spilling.
template <int D, bool CAUSAL, bool VEC, bool SPLIT>
__global__ __launch_bounds__(256, (D >= 128 && (SPLIT || !VEC)) ? 1 : 2) void prefill_mfma_kernel(const PrefillParams p) {
    constexpr int KS = D + 4;          // K row stride in LDS (16-byte reads conflict-free)
    constexpr int VS = D + 8;          // V row stride in LDS (lane halves on disjoint banks)
    constexpr int STAGE = 32 * KS + 32 * VS;
    constexpr int NB = D / 32;         // 32-wide output column blocks
    __shared__ __attribute__((aligned(16))) float lds[2 * STAGE];

    // ---- persistent workgroup: slot q of XCD x -------------------------------
    // Hardware dispatches consecutive workgroup ids round-robin over the 8
    // XCDs, so x = id & 7; each XCD owns a contiguous range of super-items
    // (whole KV heads, its own L2).  The workgroup runs its items one after the
    // other: no dispatch gaps, and the static schedule is balanced.
    const int x = blockIdx.x & 7, q = blockIdx.x >> 3, S = gridDim.x >> 3;

#pragma nounroll
    for (int j = 0;; ++j) {
    int head = 0, wgi = 0, chunk = 0, pair = 0;
    int n_parts = 1;
    if constexpr (SPLIT) {
        // Key split, one step only.  The (item, chunk) pairs are numbered
        // contiguously per head; XCD x (= workgroup id % 8, the hardware's
        // dealing order) takes the x-th eighth of that list, so the chunks of
        // an item share one L2 (they all read the item's Q).
        if (j > 0) break;
        const int per_head = p.part_prefix[p.n_wg];
        const int pairs = p.B * p.Hkv * per_head;
        const int ppx = (pairs + 7) >> 3;
        pair = (blockIdx.x & 7) * ppx + (blockIdx.x >> 3);
        if (pair >= pairs) break;
        head = pair / per_head;
        const int r = pair % per_head;
        int lo = 0, hi = p.n_wg - 1;     // last item with part_prefix <= r
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (p.part_prefix[mid] <= r) lo = mid; else hi = mid - 1;
        }
        wgi = lo;
        chunk = r - p.part_prefix[lo];
        n_parts = p.part_prefix[lo + 1] - p.part_prefix[lo];
    } else {
        const int st = item_at(p, j, x, q, S, head, wgi);
        if (st == 0) break;
        if (st == 2) continue;
    }
    // Lane-derived addressing is recomputed for every item rather than held
    // live across the whole persistent loop.
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int bi = head / p.Hkv, kvh = head % p.Hkv;

    const int unit = wgi * 4 + wave;
    const bool active = unit < p.n_units;
    const int rb = active ? unit / p.G : 0;
    const int g = active ? unit % p.G : 0;
    const int hq = kvh * p.G + g;
    const int row0 = rb * 32;
    const int qrow = row0 + l32;

    // ---- key-tile range ------------------------------------------------------
    const int n_kt = (p.Tk + 31) >> 5;
    int last_unit = wgi * 4 + 3;
    if (last_unit > p.n_units - 1) last_unit = p.n_units - 1;
    const int wg_last_key = last_visible_key(p, last_unit / p.G, CAUSAL);
    int n_tiles = wg_last_key < 0 ? 0 : (wg_last_key >> 5) + 1;
    if (n_tiles > n_kt) n_tiles = n_kt;
    const int wave_last_key = last_visible_key(p, rb, CAUSAL);
    const int wave_tiles = active ? (wave_last_key < 0 ? 0 : (wave_last_key >> 5) + 1) : 0;

    // Key tiles [t0, t1) of this workgroup: all of them, or one chunk (an
    // empty chunk still leaves its record).
    int t0 = 0, t1 = n_tiles;
    if constexpr (SPLIT) {
        t0 = min(n_tiles, chunk * p.chunk_tiles);
        t1 = min(n_tiles, t0 + p.chunk_tiles);
    }

    // ---- Q^T fragment: qf[s] = Q[qrow][half*D/2 + s] * scale*log2(e) ----------
    float qf[D / 2];
    {
        const float* qp = p.q.p + bi * p.q.sb + hq * p.q.sh + (int64_t)qrow * p.q.st;
        const bool rok = active && qrow < p.Tq;
#pragma unroll
        for (int s4 = 0; s4 < D / 8; ++s4) {
            const int c = half * (D / 2) + 4 * s4;
            float x[4];
            if (VEC) {
                float4 t = (rok && c < p.d) ? *reinterpret_cast<const float4*>(qp + c)
                                            : make_float4(0.f, 0.f, 0.f, 0.f);
                x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) x[j] = (rok && c + j < p.d) ? qp[(c + j) * p.q.sd] : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) qf[4 * s4 + j] = x[j] * p.qscale;
        }
    }

    const float* kb = p.k.p + bi * p.k.sb + kvh * p.k.sh;
    const float* vb = p.v.p + bi * p.v.sb + kvh * p.v.sh;

    floatx16 o[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[b][r] = 0.f;
    float m_run = kNegInf, l_run = 0.f;

    // The second item of a causal pair walks its key tiles backwards.  The
    // workgroups of an XCD then stand at only two key positions at any time
    // -- t on their first (long) items, total - t on their second (short)
    // ones, whatever their ranks -- so the head's K/V tiles they read stay in
    // the XCD's L2.  Walked forwards, every second item restarts at key 0 at
    // its own time and the walks spread over the whole head: config 4 read
    // 284 MB from HBM, 249 MB backwards (201 MB algorithmic); same time.
    const bool rev = !SPLIT && p.pairing && (j & 1);
    const int kstep = rev ? -1 : 1;
    const int kfirst = rev ? t1 - 1 : t0;
    const int n_it = t1 - t0;
    TileLoader<D, VEC> ld;
    if (n_it > 0) {
        ld.load(p, kb, vb, kfirst * 32, tid);
        ld.store(lds, lds + 32 * KS, tid);
    }
    __syncthreads();

    for (int it = 0; it < n_it; ++it) {
        const int kt = kfirst + kstep * it;
        const bool has_next = it + 1 < n_it;
        const bool mine = kt < wave_tiles;
        const float* Ks = lds + (it & 1) * STAGE;
        const float* Vs = Ks + 32 * KS;
        floatx16 s;
        if (mine) {
            // S^T = K Q^T  (32 keys x 32 rows), log2 domain.
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 0.f;
            const float* krow = Ks + l32 * KS + half * (D / 2);
            // Raised issue priority while this wave feeds the MFMA pipe, so the
            // two waves sharing a SIMD alternate MFMA and softmax phases.
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int t = 0; t < D / 8; ++t) {
                const float4 kq = *reinterpret_cast<const float4*>(krow + 4 * t);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq.x, qf[4 * t + 0], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq.y, qf[4 * t + 1], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq.z, qf[4 * t + 2], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq.w, qf[4 * t + 3], s, 0, 0, 0);
            }
            // Schedule: the first 4 K reads, then one read per 4 MFMAs, so
            // reads run 4 chunks (16 MFMAs) ahead of their use.
#pragma unroll
            for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
            for (int i = 0; i < D / 8 - 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);

            __builtin_amdgcn_s_setprio(0);
        }
        // The next tile's loads are issued after the QK^T MFMAs, so their
        // registers and the K operands are never live at the same time.
        if (has_next) ld.load(p, kb, vb, (kt + kstep) * 32, tid);
        if (mine) {
            // Mask keys past T_k and (causal) keys after row + q_offset.
            const int key0 = kt * 32;
            const bool need_mask = (key0 + 32 > p.Tk) || (CAUSAL && key0 + 31 > row0 + p.q_offset);
            if (need_mask) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = key0 + 8 * (r >> 2) + 4 * half + (r & 3);
                    const bool vis = key < p.Tk && (!CAUSAL || key <= qrow + p.q_offset);
                    s[r] = vis ? s[r] : kNegInf;
                }
            }

            // Online softmax for this lane's row (keys split over the lane pair).
            // m_run is the reference max the exponentials use.  It is raised,
            // and O and l rescaled, only when some row's tile max exceeds it by
            // more than 8 (log2 units): P values stay <= 2^8, the ratio O/l is
            // unchanged, and most tiles skip the 4*NB*4 multiplies.
            float mt = s[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
            mt = pair_max(mt);
            if (__builtin_amdgcn_ballot_w64(mt > m_run + 8.f) != 0) {
                const float m_new = fmaxf(m_run, mt);
                const float alpha = fast_exp2(m_run - ((m_new == kNegInf) ? 0.f : m_new));
                l_run *= alpha;
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[b][r] *= alpha;
                m_run = m_new;
            }
            const float m_use = (m_run == kNegInf) ? 0.f : m_run;
            float ls = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[r] = fast_exp2(s[r] - m_use);
                ls += s[r];
            }
            l_run += ls;

            // O^T += V^T P^T ; reduction step r pairs key 8*(r/4)+4*half+r%4.
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float* vrow = Vs + (8 * (r >> 2) + 4 * half + (r & 3)) * VS + l32;
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * b], s[r], o[b], 0, 0, 0);
            }
            // Schedule: V operands are read (two per ds_read2) 4 reads ahead of
            // the MFMAs that use them.
            constexpr int NVR = 16 * NB / 2;       // ds_read2_b32 per tile
#pragma unroll
            for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
            for (int i = 0; i < NVR - 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            __builtin_amdgcn_s_setprio(0);
        }

        if (has_next) {
            float* ks = lds + ((it + 1) & 1) * STAGE;
            ld.store(ks, ks + 32 * KS, tid);
        }
        __syncthreads();
    }

    float l_tot = pair_sum(l_run);
    if constexpr (SPLIT) {
        if (n_parts > 1) {
            // Partial record of this chunk, lane-major so that every store and
            // load is one coalesced wave access: O^T registers at
            // ws[grid*512 + ((slot*4 + wave)*(D/2) + i)*64 + lane] and
            // (max, sum) at ws[((slot*4 + wave)*64 + lane)*2], slot = pair.
            const int item = head * p.n_wg + wgi;
            const int64_t o_base = (int64_t)gridDim.x * 512;
            {
                float* wo = p.ws + o_base + ((int64_t)pair * 4 + wave) * (D / 2) * 64 + lane;
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r) store_coherent(wo + (b * 16 + r) * 64, o[b][r]);
                float* wml = p.ws + (((int64_t)pair * 4 + wave) * 64 + lane) * 2;
                store_coherent(wml, m_run);
                store_coherent(wml + 1, l_tot);
            }
            wait_stores_performed();
            __shared__ unsigned arrival_s;
            __syncthreads();
            if (tid == 0)
                arrival_s = __hip_atomic_fetch_add(p.cnt + item, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            if (arrival_s != (unsigned)(n_parts - 1)) break;   // not the last chunk (uniform)
            if (tid == 0) __hip_atomic_store(p.cnt + item, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

            // Last chunk: fold the item's records, this one's included, in
            // chunk order (online-softmax combine, GRP records per round
            // trip), so the result does not depend on which chunk came last.
            constexpr int GRP = D >= 128 ? 2 : 4;
            float M = kNegInf;
            l_tot = 0.f;
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[b][r] = 0.f;
            const int slot0 = pair - chunk;
            for (int i = 0; i < n_parts; i += GRP) {
                float mc[GRP], lc[GRP], oc[GRP][D / 2];
#pragma unroll
                for (int u = 0; u < GRP; ++u) {
                    // A missing last record of a group reads this chunk's own
                    // (finite) record with weight exp2(-inf) = 0.
                    const bool ok = i + u < n_parts;
                    const int64_t sl = ((int64_t)(slot0 + (ok ? i + u : chunk)) * 4 + wave);
                    const float* ro = p.ws + o_base + sl * (D / 2) * 64 + lane;
                    const float* rml = p.ws + (sl * 64 + lane) * 2;
                    const float m_ld = load_coherent(rml), l_ld = load_coherent(rml + 1);
                    mc[u] = ok ? m_ld : kNegInf;
                    lc[u] = ok ? l_ld : 0.f;
#pragma unroll
                    for (int e = 0; e < D / 2; ++e) oc[u][e] = load_coherent(ro + e * 64);
                }
#pragma unroll
                for (int u = 0; u < GRP; ++u) {
                    const float m_new = fmaxf(M, mc[u]);
                    const float mu = m_new == kNegInf ? 0.f : m_new;
                    const float a = fast_exp2(M - mu), bw = fast_exp2(mc[u] - mu);
                    l_tot = l_tot * a + lc[u] * bw;
#pragma unroll
                    for (int b = 0; b < NB; ++b)
#pragma unroll
                        for (int r = 0; r < 16; ++r) o[b][r] = o[b][r] * a + oc[u][b * 16 + r] * bw;
                    M = m_new;
                }
            }
        }
    }

    // ---- normalise and write O[qrow][dim], dim = 32b + 8(r/4) + 4*half + r%4 --
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (active && qrow < p.Tq) {
        float* op = p.o.p + bi * p.o.sb + hq * p.o.sh + (int64_t)qrow * p.o.st;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const int c = 32 * b + 8 * qq + 4 * half;
                if (VEC) {
                    if (c < p.d)
                        *reinterpret_cast<float4*>(op + c) =
                            make_float4(o[b][4 * qq] * inv, o[b][4 * qq + 1] * inv,
                                        o[b][4 * qq + 2] * inv, o[b][4 * qq + 3] * inv);
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (c + j < p.d) op[(c + j) * p.o.sd] = o[b][4 * qq + j] * inv;
                }
            }
        }
    }
    __syncthreads();   // the next item's first tile reuses the LDS stages
    }
}

// Head dims 129..256, padded to 256.  Q^T and O^T of 256 dims do not fit one
// wave's registers beside its K/V operands, so every 32-row unit is served
// by two waves, one per half of the head dim: wave (unit u, half h) holds
// Q^T and O^T of dims [128h, 128h + 128).  Per 32-key tile each wave computes
// the partial S^T over its dims (the d = 128 kernel's 64 MFMAs), the two swap
// their partials through the K/V stage that is idle during the tile, and
// both add them -- a + b == b + a, so the pair holds the same S bit for bit
// and runs the same online softmax -- then each accumulates its half of
// O^T = V^T P^T.  8 waves (4 units, the 4 (row block, query head) units of
// the d = 128 kernel) per workgroup and one workgroup per CU: two stages of
// 32 keys x 256 dims of K and V take 134 KB of LDS.  K/V come from HBM once
// per KV head and workgroup step, as at d <= 128.
template <bool CAUSAL>
__global__ __launch_bounds__(512, 1) void prefill_wide_kernel(const PrefillParams p) {
    constexpr int D = 256, DH = D / 2;
    constexpr int KS = D + 4, VS = D + 8;
    constexpr int STAGE = 32 * KS + 32 * VS;
    constexpr int NB = DH / 32;          // 32-wide output column blocks per wave
    constexpr int XW = 16 * 64;          // floats of one wave's partial S^T
    static_assert(8 * XW <= STAGE, "the partials fit the idle stage");
    __shared__ __attribute__((aligned(16))) float lds[2 * STAGE];

    const int x = blockIdx.x & 7, q = blockIdx.x >> 3, S = gridDim.x >> 3;

#pragma nounroll
    for (int j = 0;; ++j) {
    int head = 0, wgi = 0;
    const int st = item_at(p, j, x, q, S, head, wgi);
    if (st == 0) break;
    if (st == 2) continue;
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, half = lane >> 5;
    const int dh = wave >> 2;            // head-dim half of this wave
    const int bi = head / p.Hkv, kvh = head % p.Hkv;

    const int unit = wgi * 4 + (wave & 3);
    const bool active = unit < p.n_units;
    const int rb = active ? unit / p.G : 0;
    const int g = active ? unit % p.G : 0;
    const int hq = kvh * p.G + g;
    const int row0 = rb * 32;
    const int qrow = row0 + l32;

    const int n_kt = (p.Tk + 31) >> 5;
    int last_unit = wgi * 4 + 3;
    if (last_unit > p.n_units - 1) last_unit = p.n_units - 1;
    const int wg_last_key = last_visible_key(p, last_unit / p.G, CAUSAL);
    int n_tiles = wg_last_key < 0 ? 0 : (wg_last_key >> 5) + 1;
    if (n_tiles > n_kt) n_tiles = n_kt;
    const int wave_last_key = last_visible_key(p, rb, CAUSAL);
    const int wave_tiles = active ? (wave_last_key < 0 ? 0 : (wave_last_key >> 5) + 1) : 0;

    // Q^T fragment: qf[s] = Q[qrow][dh*128 + half*64 + s] * scale*log2(e)
    float qf[DH / 2];
    {
        const float* qp = p.q.p + bi * p.q.sb + hq * p.q.sh + (int64_t)qrow * p.q.st;
        const bool rok = active && qrow < p.Tq;
#pragma unroll
        for (int s4 = 0; s4 < DH / 8; ++s4) {
            const int c = dh * DH + half * (DH / 2) + 4 * s4;
            const float4 t = (rok && c < p.d) ? *reinterpret_cast<const float4*>(qp + c)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
            qf[4 * s4 + 0] = t.x * p.qscale;
            qf[4 * s4 + 1] = t.y * p.qscale;
            qf[4 * s4 + 2] = t.z * p.qscale;
            qf[4 * s4 + 3] = t.w * p.qscale;
        }
    }

    const float* kb = p.k.p + bi * p.k.sb + kvh * p.k.sh;
    const float* vb = p.v.p + bi * p.v.sb + kvh * p.v.sh;

    floatx16 o[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[b][r] = 0.f;
    float m_run = kNegInf, l_run = 0.f;

    // Second items of causal pairs walk their key tiles backwards, as in the
    // d <= 128 kernel (a head's K/V tiles stay in the XCD's L2: 688 -> 260 MB
    // read at B = 1, H = 16, T = 4096).
    const bool rev = p.pairing && (j & 1);
    const int kstep = rev ? -1 : 1;
    const int kfirst = rev ? n_tiles - 1 : 0;
    TileLoader<D, true, 512> ld;
    if (n_tiles > 0) {
        ld.load(p, kb, vb, kfirst * 32, tid);
        ld.store(lds, lds + 32 * KS, tid);
    }
    __syncthreads();

    for (int it = 0; it < n_tiles; ++it) {
        const int kt = kfirst + kstep * it;
        const bool has_next = it + 1 < n_tiles;
        const bool mine = kt < wave_tiles;
        const float* Ks = lds + (it & 1) * STAGE;
        const float* Vs = Ks + 32 * KS;
        float* other = lds + ((it + 1) & 1) * STAGE;   // idle until the next tile's store
        floatx16 s;
        if (mine) {
            // Partial S^T = K Q^T over this wave's 128 dims, log2 domain.
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = 0.f;
            const float* krow = Ks + l32 * KS + dh * DH + half * (DH / 2);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int t = 0; t < DH / 8; ++t) {
                const float4 kq = *reinterpret_cast<const float4*>(krow + 4 * t);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq.x, qf[4 * t + 0], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq.y, qf[4 * t + 1], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq.z, qf[4 * t + 2], s, 0, 0, 0);
                s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq.w, qf[4 * t + 3], s, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
            for (int i = 0; i < DH / 8 - 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
            __builtin_amdgcn_s_setprio(0);
            // This wave's partial, register-group major (each store one
            // contiguous, conflict-free 1 KB wave access).
            float* xo = other + wave * XW + 4 * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<float4*>(xo + 256 * i) =
                    make_float4(s[4 * i], s[4 * i + 1], s[4 * i + 2], s[4 * i + 3]);
        }
        if (has_next) ld.load(p, kb, vb, (kt + kstep) * 32, tid);
        __syncthreads();   // partials visible
        if (mine) {
            // Add the partner's partial: wave w pairs with wave w ^ 4.
            const float* xi = other + (wave ^ 4) * XW + 4 * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 t = *reinterpret_cast<const float4*>(xi + 256 * i);
                s[4 * i] += t.x;
                s[4 * i + 1] += t.y;
                s[4 * i + 2] += t.z;
                s[4 * i + 3] += t.w;
            }
            const int key0 = kt * 32;
            const bool need_mask = (key0 + 32 > p.Tk) || (CAUSAL && key0 + 31 > row0 + p.q_offset);
            if (need_mask) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = key0 + 8 * (r >> 2) + 4 * half + (r & 3);
                    const bool vis = key < p.Tk && (!CAUSAL || key <= qrow + p.q_offset);
                    s[r] = vis ? s[r] : kNegInf;
                }
            }
            // Online softmax with the lazy rescale of the d <= 128 kernel; both
            // waves of the pair take the same decisions on the same values.
            float mt = s[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[r]);
            mt = pair_max(mt);
            if (__builtin_amdgcn_ballot_w64(mt > m_run + 8.f) != 0) {
                const float m_new = fmaxf(m_run, mt);
                const float alpha = fast_exp2(m_run - ((m_new == kNegInf) ? 0.f : m_new));
                l_run *= alpha;
#pragma unroll
                for (int b = 0; b < NB; ++b)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[b][r] *= alpha;
                m_run = m_new;
            }
            const float m_use = (m_run == kNegInf) ? 0.f : m_run;
            float ls = 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[r] = fast_exp2(s[r] - m_use);
                ls += s[r];
            }
            l_run += ls;

            // O^T += V^T P^T over this wave's 128 output dims.
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float* vrow = Vs + (8 * (r >> 2) + 4 * half + (r & 3)) * VS + dh * DH + l32;
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[32 * b], s[r], o[b], 0, 0, 0);
            }
            constexpr int NVR = 16 * NB / 2;
#pragma unroll
            for (int i = 0; i < 4; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
#pragma unroll
            for (int i = 0; i < NVR - 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
            __builtin_amdgcn_s_setprio(0);
        }
        if (has_next) {
            __syncthreads();   // every partial read before the stage is refilled
            ld.store(other, other + 32 * KS, tid);
        }
        __syncthreads();
    }

    const float l_tot = pair_sum(l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (active && qrow < p.Tq) {
        float* op = p.o.p + bi * p.o.sb + hq * p.o.sh + (int64_t)qrow * p.o.st;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const int c = dh * DH + 32 * b + 8 * qq + 4 * half;
                if (c < p.d)
                    *reinterpret_cast<float4*>(op + c) =
                        make_float4(o[b][4 * qq] * inv, o[b][4 * qq + 1] * inv,
                                    o[b][4 * qq + 2] * inv, o[b][4 * qq + 3] * inv);
            }
        }
    }
    __syncthreads();   // the next item's first tile reuses the LDS stages
    }
}

// CUs and resident workgroups per CU of the kernel on the current device.
template <int D, bool CAUSAL, bool VEC>
void residency(int& cus, int& per_cu) {
    constexpr auto kernel = prefill_mfma_kernel<D, CAUSAL, VEC, false>;
    // Atomic: callers on several threads may fill the cache at once.
    static std::atomic<int> cached_cus[64], cached_per[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int c = cached_cus[dev].load(std::memory_order_acquire);
    int k = cached_per[dev].load(std::memory_order_relaxed);
    if (c == 0 || k == 0) {
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c < 8) c = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, kernel, 256, 0) !=
                hipSuccess || k < 1)
            k = 1;
        cached_per[dev].store(k, std::memory_order_relaxed);
        cached_cus[dev].store(c, std::memory_order_release);
    }
    cus = c;
    per_cu = k;
}

// One resident wave of persistent workgroups: k per CU on every CU (an
// uneven count would leave the CUs that hold more workgroups behind), 8*S in
// all with S = k * CUs / 8 per XCD, each XCD's super-items dealt round-robin.
// k minimises rounds * k (the time of a round grows with the workgroups that
// share a CU; one workgroup per CU leaves its SIMDs a single wave, taken as
// 30 % slower).  Causal problems with enough work pair ranks r and n_wg-1-r
// so that every super-item costs the same.  Fills p's schedule fields and
// returns S.
int persistent_slots(PrefillParams& p, bool causal, int cus, int k_max) {
    const int cu_per_xcd = cus / 8;
    const int64_t heads = (int64_t)p.B * p.Hkv;
    p.pairing = (causal && p.n_wg > 1 && heads * ((p.n_wg + 1) / 2) >= (int64_t)cus * k_max) ? 1 : 0;
    p.n_pairs = p.pairing ? (p.n_wg + 1) / 2 : p.n_wg;
    p.n_super = (int)(heads * p.n_pairs);
    p.per_xcd = (p.n_super + 7) / 8;
    int S = 1, best_rounds = 1;
    double best = 1e300;
    for (int k = 1; k <= k_max; ++k) {
        const int s = k * cu_per_xcd;
        const int rounds = (p.per_xcd + s - 1) / s;
        const double cost = (double)rounds * k * (k == 1 ? 1.3 : 1.0);
        if (cost < best) { best = cost; S = s; best_rounds = rounds; }
    }
    // A partly empty last round costs more than the hardware's own dispatch of
    // one super-item per workgroup (which also covers small problems).
    if (S >= p.per_xcd || (double)p.per_xcd / ((double)best_rounds * S) < 0.97) S = p.per_xcd;
    // Hardware dispatch of unpaired causal items: in head-major rank order the
    // two workgroups placed on a CU take items of the same rank from two heads
    // (both long or both short).  Longest first across the XCD's heads, with
    // complementary lengths per CU, took B = 1, H = 16, T = 4096, d = 128 from
    // 1016 to 592 us and B = 1, Hq = 32, Hkv = 8, T = 2048 from 401 to 296 us.
    p.order_cu = 0;
    p.order_hpx = 0;
    if (causal && !p.pairing && S == p.per_xcd && heads % 8 == 0 && cu_per_xcd > 0 &&
        (int64_t)p.per_xcd * 8 == heads * p.n_wg) {
        p.order_cu = cu_per_xcd;
        p.order_hpx = (int)(heads / 8);
    }
    return S;
}

template <int D, bool CAUSAL, bool VEC>
hipError_t launch_t(PrefillParams p, hipStream_t stream) {
    if (p.n_chunks > 1 && p.ws && p.cnt) {
        hipLaunchKernelGGL((prefill_mfma_kernel<D, CAUSAL, VEC, true>),
                           dim3(8 * ((p.B * p.Hkv * p.part_prefix[p.n_wg] + 7) / 8)), dim3(256), 0, stream, p);
        return hipGetLastError();
    }
    int cus = 0, k_max = 0;
    residency<D, CAUSAL, VEC>(cus, k_max);
    const int S = persistent_slots(p, CAUSAL, cus, k_max);
    hipLaunchKernelGGL((prefill_mfma_kernel<D, CAUSAL, VEC, false>), dim3(8 * S), dim3(256), 0, stream, p);
    return hipGetLastError();
}

// Head dims 129..256: the wave-pair kernel, one workgroup of 8 waves per CU.
template <bool CAUSAL>
hipError_t launch_wide_t(PrefillParams p, hipStream_t stream) {
    constexpr auto kernel = prefill_wide_kernel<CAUSAL>;
    static std::atomic<int> cached_cus[64], cached_per[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int cus = cached_cus[dev].load(std::memory_order_acquire);
    int k_max = cached_per[dev].load(std::memory_order_relaxed);
    if (cus == 0 || k_max == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus < 8)
            cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k_max, kernel, 512, 0) != hipSuccess ||
            k_max < 1)
            k_max = 1;
        cached_per[dev].store(k_max, std::memory_order_relaxed);
        cached_cus[dev].store(cus, std::memory_order_release);
    }
    const int S = persistent_slots(p, CAUSAL, cus, k_max);
    hipLaunchKernelGGL(kernel, dim3(8 * S), dim3(512), 0, stream, p);
    return hipGetLastError();
}

template <int D>
hipError_t launch_d(const PrefillParams& p, bool causal, bool vec, hipStream_t stream) {
    if (causal) return vec ? launch_t<D, true, true>(p, stream) : launch_t<D, true, false>(p, stream);
    return vec ? launch_t<D, false, true>(p, stream) : launch_t<D, false, false>(p, stream);
}

}  // namespace

int prefill_padded_dim(int d) {
    if (d <= 32) return 32;
    if (d <= 64) return 64;
    if (d <= 128) return 128;
    return 0;
}

namespace {

void derive_schedule(PrefillParams& p) {
    p.G = p.Hq / p.Hkv;
    p.n_rb = (p.Tq + 31) / 32;
    p.n_units = p.G * p.n_rb;
    p.n_wg = (p.n_units + 3) / 4;
    p.total = p.B * p.Hkv * p.n_wg;
}

int device_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    int c = cached[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c < 8)
            c = 256;
        cached[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

}  // namespace

// A problem with fewer work items than CUs leaves most SIMDs idle, and its
// time is the longest item's chain of key tiles.  Cutting every item's tiles
// into chunks, sized so that the chunks fill the CUs once (at most 16 chunks
// per item), shortens that chain to one chunk plus the merge of the item's
// records.
PrefillSplit prefill_split_plan(PrefillParams& p, bool causal, bool vec) {
    (void)vec;
    PrefillSplit r{0, 0};
    p.n_chunks = 0;
    p.chunk_tiles = 0;
    derive_schedule(p);
    const int D = prefill_padded_dim(p.d);
    const int cus = device_cus();
    if (p.total == 0 || D == 0 || p.total >= cus || p.n_wg > kMaxSplitItems) return r;
    // Key tiles of each work item, as the kernel counts them.
    const int n_kt = (p.Tk + 31) / 32;
    std::vector<int> tiles(p.n_wg);
    int max_t = 0;
    for (int w = 0; w < p.n_wg; ++w) {
        const int last_unit = std::min(w * 4 + 3, p.n_units - 1);
        int lk = p.Tk - 1;
        if (causal) {
            const int last_row = std::min(last_unit / p.G * 32 + 31, p.Tq - 1);
            lk = std::min(last_row + p.q_offset, p.Tk - 1);
        }
        tiles[w] = lk < 0 ? 0 : std::min(lk / 32 + 1, n_kt);
        max_t = std::max(max_t, tiles[w]);
    }
    if (max_t < 4) return r;
    // One workgroup per CU: measured against two per CU where they fit (d = 64),
    // the longer chunks with half the records and prologues are faster
    // (GPT-2 prompt, T = 1024: 33.9 against 31.0 us).
    const int64_t slots = cus;
    // Smallest chunk (<= 16 chunks per item) whose non-empty chunks fill the
    // CUs at most once.  One-tile chunks, where they fit, beat two-tile ones
    // (config 1: 12.4 against 13.0 us): the chain of tiles halves, the merge
    // grows by one round trip.
    int ch = std::max(1, (max_t + 15) / 16);
    for (;; ++ch) {
        int64_t n = 0;
        for (int w = 0; w < p.n_wg; ++w) n += std::max(1, (tiles[w] + ch - 1) / ch);
        if (n * p.B * p.Hkv <= slots || ch >= max_t) break;
    }
    const int nc = (max_t + ch - 1) / ch;
    if (nc < 2) return r;
    p.n_chunks = nc;
    p.chunk_tiles = ch;
    p.part_prefix[0] = 0;
    for (int w = 0; w < p.n_wg; ++w)
        p.part_prefix[w + 1] = (uint16_t)(p.part_prefix[w] + std::max(1, (tiles[w] + ch - 1) / ch));
    // Per workgroup: (max, sum) of 4 waves x 64 lanes, and 4 x D/2 x 64 O values.
    const uint64_t grid = ((uint64_t)p.B * p.Hkv * p.part_prefix[p.n_wg] + 7) / 8 * 8;
    r.ws_bytes = grid * (512 + 128 * (uint64_t)D) * 4;
    r.n_counters = p.total;
    return r;
}

hipError_t launch_prefill_wide(PrefillParams p, bool causal, hipStream_t stream) {
    derive_schedule(p);
    if (p.total == 0) return hipSuccess;
    if (p.d <= 128 || p.d > 256) return hipErrorInvalidValue;
    return causal ? launch_wide_t<true>(p, stream) : launch_wide_t<false>(p, stream);
}

hipError_t launch_prefill(PrefillParams p, bool causal, bool vec, hipStream_t stream) {
    derive_schedule(p);
    if (p.total == 0) return hipSuccess;
    switch (prefill_padded_dim(p.d)) {
        case 32: return launch_d<32>(p, causal, vec, stream);
        case 64: return launch_d<64>(p, causal, vec, stream);
        case 128: return launch_d<128>(p, causal, vec, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace nne
