// Attention at head dims above 256: prefill, cross-attention and decode over a
// KV cache, on v_mfma_f32_32x32x2_f32; and prefill at 129-256 dims that the
// wave-pair kernel does not take (dims other than 256, small problems).
//
// Algorithm: the online softmax of the reference's flash_attention_forward
// (src/nn/flash_attention.rs:91-195) over 32-key tiles, rows that see no key
// left at zero (:186-194); with a KV cache, the cached attention of
// src/models/llama.rs:239-296 and src/nn/attention.rs:139-210 (every cached
// key visible to the new row).  The reference takes any head dim:
// flash_attention.rs:39-50 checks only that the shapes agree.
//
// MI355X mapping.  At d <= 256 one wave (or a wave pair) keeps Q^T and O^T of
// its 32 rows in registers and the workgroup stages 32-key K/V tiles in LDS,
// two at a time.  Above 256 dims neither fits: a 32-key K/V tile of 512 dims
// is 128 KB.  Here a workgroup of 8 waves serves one 32-row unit and reads
// K and V straight from global memory into MFMA operand layout (every byte of
// a K/V row once per unit and output chunk, the unit's waves splitting the
// row between them):
//  * S^T = K Q^T is split over the waves by dims.  Wave w takes the 8-dim
//    chunks j = w, w + 8, w + 16, ...; lane half h holds dims 8j + 4h ..
//    8j + 4h + 3 of its row (one 16-byte load), and MFMA c of a chunk pairs
//    dims 8j + c and 8j + 4 + c.  Q^T of a wave's first 16 chunks (128 dims)
//    stays in registers; further chunks (d > 1024) are read again each tile.
//  * The 8 partial S^T (4 KB each) meet in LDS: wave w adds elements
//    [128w, 128w + 128) of all 8 in wave order and stores the sum, and every
//    wave then reads the whole S, so all 8 hold the same S bit for bit and
//    take the same online-softmax decisions.  (Every wave adding all 8
//    partials itself read 8x the LDS bytes: d = 512 prefill 2.92 -> 2.75 ms
//    with the split sum.)  Both buffers are double-buffered: two barriers
//    per tile.
//  * O^T += V^T P^T is split over the waves by 32-dim output blocks: wave w
//    owns blocks w and w + 8 of the workgroup's 512-dim output chunk (32
//    accumulator registers).  Each V operand load is one 128-byte row segment
//    per half-wave.
//  * The next tile's K (up to 8 chunks) is loaded during the current tile's
//    exchange, softmax and P V, and a tile's V at its start, under its S.
//  Prefill problems with more workgroups than CUs use a 4-wave form
//  instead, two workgroups per CU: each wave takes twice the chunks and
//  output blocks (S from 4 partials, Q^T of its last 8 chunks in LDS), so a
//  tile's MFMAs per wave double against the same exchange and softmax, and
//  one workgroup's exchange overlaps the other's MFMAs.  At 129-256 dims a
//  2-wave form does the same over a 256-dim output chunk, four workgroups
//  per CU.
//  Above 512 dims an unsplit unit takes one 8-wave workgroup per 1024-dim
//  output chunk (4 output blocks and 16 S chunks per wave, half of its Q^T in
//  LDS), each chunk recomputing S; key splits keep 512-dim chunks, whose
//  records the combine kernel merges.  Workgroup ids go
//  to the 8 XCDs in turn; XCD x takes the x-th eighth of the (sequence, KV
//  head, unit, chunk) list, so the units of a KV head, which read the same
//  K/V rows, share an L2, and causal units are taken longest first (on the
//  8-wave form across the XCD's KV heads when each XCD holds whole heads).
//  Problems with too few units to fill the device (decode steps of small
//  batches, few-query cross-attention) cut each unit's keys into parts, one
//  workgroup each, equal parts or (ragged decode) parts by length; every part
//  leaves a partial record -- the online softmax's (max, sum) and unnormalised
//  O -- and deep_combine_kernel merges them.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "nne_common.hpp"
#include "nne_launch.hpp"

namespace nne {

namespace {

constexpr int XW = 16 * 64;                     // floats of one wave's partial S^T

__device__ __forceinline__ vf4 load4(const float* p) { return *reinterpret_cast<const vf4*>(p); }

__device__ __forceinline__ int clamp_keys(int64_t x, int tk) {
    return x < 0 ? 0 : (x > tk ? tk : (int)x);
}

// DW waves per workgroup.  Per wave: QC chunks of S (STREAMQ: further chunks
// read again each tile) and OB output blocks (the workgroup's output chunk is
// 32 * DW * OB dims).  Q^T of the chunks stays in registers, except that the
// forms with 4 output blocks per wave keep their last 8 chunks in LDS.  KP
// chunks of the next tile's K are loaded during the current tile, and VP key
// steps of a tile's V at its start; the rest is loaded in groups of 4 inside
// its phase.  8 waves: one workgroup per CU (2 output blocks per wave, or 4 on
// a 1024-dim chunk above 512 dims); 4 waves: two per CU; 2 waves (head dims
// up to 256): four per CU.  Co-resident workgroups' exchanges and softmaxes
// interleave with each other's MFMAs.
template <bool CAUSAL, int DW, int QC, int OB, bool STREAMQ, bool SPLIT>
__global__ __launch_bounds__(64 * DW, DW == 8 ? 1 : 2) void deep_attention_kernel(const DeepParams p) {
    static_assert((DW == 8 && OB == 2) || (QC == 16 && OB == 4 && !SPLIT && (DW == 8 || !STREAMQ)),
                  "the workgroup forms");
    constexpr bool OB4 = OB == 4;
    constexpr int KP = OB4 ? 4 : (QC < 8 ? QC : 8);
    constexpr int VP = OB <= 2 ? 16 : 4;
    constexpr int QL = OB4 ? 8 : 0;  // Q^T chunks in LDS (the last QL of QC)
    constexpr int CB = 32 * DW;          // dims between a wave's output blocks
    __shared__ __attribute__((aligned(16))) float xs[2 * DW * XW];
    __shared__ __attribute__((aligned(16))) float red[2 * XW];
    __shared__ __attribute__((aligned(16))) float qs[QL > 0 ? DW * QL * 256 : 4];

    // Output chunk of one workgroup: kDeepChunk dims, or (unsplit forms) 256
    // on 2 waves and 1024 on 8 waves with 4 blocks each.
    static_assert(32 * DW * OB == kDeepChunk || !SPLIT, "output chunk of one workgroup");
    // Key-split launches (few units, no K/V sharing between them worth an
    // L2) deal the workgroups round-robin over the XCDs instead, so that the
    // parts of ragged sequences spread over the whole device.
    const int idx = SPLIT ? (int)blockIdx.x : (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
    if (idx >= p.total) return;   // whole workgroup: no barrier is skipped
    int split = SPLIT ? idx % p.n_split : 0;
    int oc = (SPLIT ? idx / p.n_split : idx) % p.n_oc;
    int hu = (SPLIT ? idx / p.n_split : idx) / p.n_oc;
    if (!SPLIT && p.order_hpx) {
        // Causal units of the XCD's order_hpx whole KV heads, longest first
        // across those heads (rank-major).
        const int pos = blockIdx.x >> 3, cols = p.order_hpx * p.n_oc;
        oc = (pos % cols) % p.n_oc;
        hu = ((blockIdx.x & 7) * p.order_hpx + (pos % cols) / p.n_oc) * p.n_units + pos / cols;
    }
    if (SPLIT && p.ragged) {
        // Pair of workgroup idx: the pairs whose first part is at most idx,
        // counted over the workgroup (part_prefix rises strictly).
        const int nh = p.B * p.Hkv;
        const int t = threadIdx.x;
        hu = __syncthreads_count(t < nh && (int)p.part_prefix[t < nh ? t : 0] <= idx) - 1;
        split = idx - (int)p.part_prefix[hu];
        oc = 0;
    }
    const int ui = hu % p.n_units, head = hu / p.n_units;
    // Causal units by rank ui, longest first: by their last query position,
    // the G query heads of one position block in turn when units do not
    // straddle heads.
    const int ntb = p.Tq >> 5;
    const int unit = !CAUSAL ? ui
                   : (p.G > 1 && (p.Tq & 31) == 0) ? (ui % p.G) * ntb + (ntb - 1 - ui / p.G)
                                                  : p.n_units - 1 - ui;
    const int bi = head / p.Hkv, kvh = head % p.Hkv;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, half = lane >> 5;

    // Row l32 of the unit: flattened row r of the KV head.
    const int rows = p.G * p.Tq;
    const int r0 = unit * 32;
    const int r_last = r0 + 31 < rows ? r0 + 31 : rows - 1;
    const int r = r0 + l32;
    const bool active = r < rows;
    const int g = active ? r / p.Tq : 0;
    const int t = active ? r % p.Tq : 0;
    const int hq = kvh * p.G + g;

    const int tk = p.lens ? p.lens[bi] : p.Tk;
    int kend = tk;   // keys some row of the unit sees
    int kall = tk;   // keys every row of the unit sees
    // keys this lane's row sees
    const int klim = CAUSAL ? clamp_keys((int64_t)t + p.q_offset + 1, tk) : tk;
    if (CAUSAL) {
        const bool one = r0 / p.Tq == r_last / p.Tq;
        const int t_max = one ? r_last % p.Tq : p.Tq - 1;
        const int t_min = one ? r0 % p.Tq : 0;
        kend = clamp_keys((int64_t)t_max + p.q_offset + 1, tk);
        kall = clamp_keys((int64_t)t_min + p.q_offset + 1, tk);
    }
    const int n_tiles = (kend + 31) >> 5;
    // This workgroup's key tiles (all of the unit's without a key split).
    const int t_begin = SPLIT ? split * p.split_tiles : 0;
    int t_end = SPLIT ? t_begin + p.split_tiles : n_tiles;
    if (t_end > n_tiles) t_end = n_tiles;

    // This wave's chunks of S (8 dims each) and output blocks (32 dims each).
    const int nj = (p.d + 7) >> 3;
    const int nq = wave < nj ? (nj - 1 - wave) / DW + 1 : 0;
    const int nbt = (p.d + 31) >> 5;
    const int gb0 = oc * (CB * OB / 32) + wave;
    const int nob = gb0 < nbt ? min(OB, (nbt - 1 - gb0) / DW + 1) : 0;

    const float* qp = p.q.p + bi * p.q.sb + hq * p.q.sh + (int64_t)t * p.q.st;
    vf4 qf[QC - QL];
#pragma unroll
    for (int i = 0; i < QC; ++i) {
        const int c = 8 * (wave + DW * i) + 4 * half;
        const vf4 x = (active && c < p.d) ? load4(qp + c) * p.qscale : vf4{0.f, 0.f, 0.f, 0.f};
        if (i < QC - QL) qf[i < QC - QL ? i : 0] = x;
        else *reinterpret_cast<vf4*>(qs + ((wave * QL + i - (QC - QL)) * 64 + lane) * 4) = x;
    }
    if (QL > 0) __syncthreads();

    const float* kb = p.k.p + bi * p.k.sb + kvh * p.k.sh;
    const float* vb = p.v.p + bi * p.v.sb + kvh * p.v.sh;
    const int od = oc * CB * OB + 32 * wave + l32;   // this lane's dim of output block 0

    // K and V of a tile are read through buffer ranges that start at the
    // tile's first key and end with the last key of the unit (rows past it
    // read as zero without a memory access), so no load needs a predicate
    // and the byte offsets are a lane constant plus a small uniform part.
    // K columns past d (the odd half of a last 8-dim chunk when d % 8 == 4)
    // are read from memory next to the row and zeroed; V columns past d read
    // the row's last float and only reach O columns never stored.
    auto range = [&](const float* base, int64_t st, int key0) {
        const int nk = kend - key0 < 32 ? kend - key0 : 32;
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base + key0 * st), 0,
                                                 (uint32_t)nk * (uint32_t)st * 4u, 0x00020000);
    };
    const uint32_t k_lane = ((uint32_t)l32 * (uint32_t)p.k.st + 8 * wave + 4 * half) * 4u;
    auto load_k = [&](__amdgpu_buffer_rsrc_t rk, int i) -> vf4 {
        if (i >= nq) return vf4{0.f, 0.f, 0.f, 0.f};   // wave-uniform: past the wave's chunks
        vf4 x = __builtin_bit_cast(
            vf4, __builtin_amdgcn_raw_buffer_load_b128(rk, k_lane + (uint32_t)(32 * DW * i), 0, 0));
        if (p.d & 4) {
            const int c = 8 * (wave + DW * i) + 4 * half;
            if (c >= p.d) x = vf4{0.f, 0.f, 0.f, 0.f};
        }
        return x;
    };
    uint32_t v_lane[OB];
#pragma unroll
    for (int b = 0; b < OB; ++b) {
        const int c = od + CB * b < p.d ? od + CB * b : p.d - 1;
        v_lane[b] = ((uint32_t)(4 * half) * (uint32_t)p.v.st + (uint32_t)c) * 4u;
    }
    // (Blocks past the wave's last valid one read clamped columns too: the
    // loads stay branch-free, and those operands are never used.)
    auto load_v = [&](__amdgpu_buffer_rsrc_t rv, int j, float (&dst)[OB]) {
        const uint32_t uni = (uint32_t)(8 * (j >> 2) + (j & 3)) * (uint32_t)p.v.st * 4u;
#pragma unroll
        for (int b = 0; b < OB; ++b)
            dst[b] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rv, v_lane[b], uni, 0));
    };

    floatx16 o[OB];
#pragma unroll
    for (int b = 0; b < OB; ++b)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) o[b][rr] = 0.f;
    float m_run = kNegInf, l_run = 0.f;

    // Key-split launches (decode steps and few-query problems) stream K/V from
    // HBM, not from an L2 shared with other units: V is loaded a whole tile
    // ahead there (the first tile's here), where at the tile's start it would
    // wait at P V for the HBM latency.
    constexpr bool VAHEAD = SPLIT && QC <= 8;   // (above 512 dims the registers do not hold it)
    static_assert(!VAHEAD || VP == 16, "V a tile ahead needs all key steps in registers");
    float vn[VAHEAD ? VP : 1][OB];
    if (VAHEAD && t_begin < t_end) {
        const __amdgpu_buffer_rsrc_t rv0 = range(vb, p.v.st, 32 * t_begin);
#pragma unroll
        for (int j = 0; j < VP; ++j) load_v(rv0, j, vn[j]);
    }
    vf4 kq[KP];
    if (t_begin < t_end) {
        const __amdgpu_buffer_rsrc_t rk = range(kb, p.k.st, 32 * t_begin);
#pragma unroll
        for (int i = 0; i < KP; ++i)
            kq[i] = load_k(rk, i);
    }

    for (int it = t_begin; it < t_end; ++it) {
        const int key0 = it * 32;
        float* xb = xs + (it & 1) * (DW * XW);

        // V of the tile's first VP key steps: in flight under the S MFMAs,
        // the exchange and the softmax.
        const __amdgpu_buffer_rsrc_t rk = range(kb, p.k.st, key0);
        const __amdgpu_buffer_rsrc_t rv = range(vb, p.v.st, key0);
        float vp[VP][OB];
        if (VAHEAD) {
#pragma unroll
            for (int j = 0; j < VP; ++j)
#pragma unroll
                for (int b = 0; b < OB; ++b) vp[j][b] = vn[j][b];
            if (it + 1 < t_end) {
                const __amdgpu_buffer_rsrc_t rv1 = range(vb, p.v.st, key0 + 32);
#pragma unroll
                for (int j = 0; j < VP; ++j) load_v(rv1, j, vn[j]);
            }
        } else {
#pragma unroll
            for (int j = 0; j < VP; ++j) load_v(rv, j, vp[j]);
        }
        __builtin_amdgcn_sched_barrier(0);

        // Partial S^T = K Q^T over this wave's chunks, log2 domain.
        floatx16 s;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) s[rr] = 0.f;
        {
            vf4 kg[2][4];
            if (QC > KP) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    kg[0][i] = load_k(rk, KP + i);
            }
            // Chunks in pairs behind one wave-uniform branch each (a branch
            // around every accumulating MFMA would copy s each time); chunks
            // past the wave's count have zero K and Q^T.
#pragma unroll
            for (int g2 = 0; g2 < KP; g2 += 2) {
                if (g2 < nq) {
#pragma unroll
                    for (int i = g2; i < g2 + 2 && i < KP; ++i) {
                        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq[i][0], qf[i][0], s, 0, 0, 0);
                        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq[i][1], qf[i][1], s, 0, 0, 0);
                        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq[i][2], qf[i][2], s, 0, 0, 0);
                        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kq[i][3], qf[i][3], s, 0, 0, 0);
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            // Chunks KP.. in groups of 4, the next group's loads issued first.
#pragma unroll
            for (int gi = 0; gi < (QC - KP) / 4; ++gi) {
                if (KP + 4 * gi < nq) {
                    if (gi + 1 < (QC - KP) / 4) {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            kg[(gi + 1) & 1][i] = load_k(rk, KP + 4 * (gi + 1) + i);
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const vf4 kk = kg[gi & 1][i];
                        const int ci = KP + 4 * gi + i;
                        const vf4 qq = ci >= QC - QL ? load4(qs + ((wave * QL + ci - (QC - QL)) * 64 + lane) * 4)
                                                     : qf[ci < QC - QL ? ci : 0];
                        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[0], qq[0], s, 0, 0, 0);
                        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[1], qq[1], s, 0, 0, 0);
                        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[2], qq[2], s, 0, 0, 0);
                        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[3], qq[3], s, 0, 0, 0);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (STREAMQ) {
                for (int i = QC; i < nq; ++i) {
                    const int c = 8 * (wave + DW * i) + 4 * half;
                    const vf4 qq = (active && c < p.d) ? load4(qp + c) * p.qscale
                                                       : vf4{0.f, 0.f, 0.f, 0.f};
                    const vf4 kk = load_k(rk, i);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[0], qq[0], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[1], qq[1], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[2], qq[2], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[3], qq[3], s, 0, 0, 0);
                }
            }
        }
        // The next tile's first KP chunks of K: in flight under the exchange,
        // the softmax and P V.
        if (it + 1 < t_end) {
            const __amdgpu_buffer_rsrc_t rk1 = range(kb, p.k.st, key0 + 32);
#pragma unroll
            for (int i = 0; i < KP; ++i)
                kq[i] = load_k(rk1, i);
        }
        __builtin_amdgcn_sched_barrier(0);
        // Register-group major (each store one contiguous 1 KB wave access).
        {
            float* xo = xb + wave * XW + 4 * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<vf4*>(xo + 256 * i) =
                    vf4{s[4 * i], s[4 * i + 1], s[4 * i + 2], s[4 * i + 3]};
        }
        __syncthreads();   // the tile's partials visible
        // Wave w adds elements [XW/DW w, XW/DW (w + 1)) of the DW partials in
        // wave order, then every wave reads the whole sum.
        {
            float* rb = red + (it & 1) * XW;
            if (DW == 8) {
                const int e = 128 * wave + 2 * lane;
                float2 a = *reinterpret_cast<const float2*>(xb + e);
#pragma unroll
                for (int w = 1; w < DW; ++w) {
                    const float2 x = *reinterpret_cast<const float2*>(xb + w * XW + e);
                    a.x += x.x;
                    a.y += x.y;
                }
                *reinterpret_cast<float2*>(rb + e) = a;
            } else {
#pragma unroll
                for (int e4 = 0; e4 < XW / DW / 256; ++e4) {
                    const int e = (XW / DW) * wave + 4 * lane + 256 * e4;
                    vf4 a = load4(xb + e);
#pragma unroll
                    for (int w = 1; w < DW; ++w) a += load4(xb + w * XW + e);
                    *reinterpret_cast<vf4*>(rb + e) = a;
                }
            }
            __syncthreads();
            if (nob == 0) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const vf4 t4 = load4(rb + 4 * lane + 256 * i);
                s[4 * i] = t4[0];
                s[4 * i + 1] = t4[1];
                s[4 * i + 2] = t4[2];
                s[4 * i + 3] = t4[3];
            }
        }
        if (key0 + 32 > kall) {
#pragma unroll
            for (int rr = 0; rr < 16; ++rr) {
                const int key = key0 + 8 * (rr >> 2) + 4 * half + (rr & 3);
                s[rr] = key < klim ? s[rr] : kNegInf;
            }
        }
        // Online softmax with a lazy rescale: the running max moves only when
        // a tile's max exceeds it by more than 2^8 (log2 domain); the sums and
        // O then stay below 2^8 times their final size.
        float mt = s[0];
#pragma unroll
        for (int rr = 1; rr < 16; ++rr) mt = fmaxf(mt, s[rr]);
        mt = pair_max(mt);
        if (__builtin_amdgcn_ballot_w64(mt > m_run + 8.f) != 0) {
            const float m_new = fmaxf(m_run, mt);
            const float alpha = fast_exp2(m_run - ((m_new == kNegInf) ? 0.f : m_new));
            l_run *= alpha;
#pragma unroll
            for (int b = 0; b < OB; ++b)
#pragma unroll
                for (int rr = 0; rr < 16; ++rr) o[b][rr] *= alpha;
            m_run = m_new;
        }
        const float m_use = (m_run == kNegInf) ? 0.f : m_run;
        float ls = 0.f;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) {
            s[rr] = fast_exp2(s[rr] - m_use);
            ls += s[rr];
        }
        l_run += ls;

        // O^T += V^T P^T over this wave's output blocks: the first VP key
        // steps from registers, the rest in groups of 4 loaded one group ahead.
        // One copy of the loop per count of valid blocks, so the MFMAs carry
        // no per-block branch (a branch around an accumulating MFMA costs a
        // copy of its 16 accumulator registers).
        auto pv = [&](auto nbk) {
            constexpr int NBK = decltype(nbk)::value;
            float vg[2][4][OB];
            if (VP < 16) {
#pragma unroll
                for (int j = 0; j < 4; ++j) load_v(rv, VP + j, vg[0][j]);
            }
#pragma unroll
            for (int j = 0; j < VP; ++j)
#pragma unroll
                for (int b = 0; b < NBK; ++b)
                    o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vp[j][b], s[j], o[b], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int gi = 0; gi < (16 - VP) / 4; ++gi) {
                if (gi + 1 < (16 - VP) / 4) {
#pragma unroll
                    for (int j = 0; j < 4; ++j) load_v(rv, VP + 4 * (gi + 1) + j, vg[(gi + 1) & 1][j]);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int b = 0; b < NBK; ++b)
                        o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vg[gi & 1][j][b],
                                                                    s[VP + 4 * gi + j], o[b], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        if (nob >= OB) pv(std::integral_constant<int, OB>{});
        else if (OB > 1 && nob == 1) pv(std::integral_constant<int, 1>{});
        else if (OB > 2 && nob == 2) pv(std::integral_constant<int, (OB > 2 ? 2 : 1)>{});
        else if (OB > 3 && nob == 3) pv(std::integral_constant<int, (OB > 3 ? 3 : 1)>{});
    }

    // ---- write O[row][dim], dim = 32 gb + 8 (rr/4) + 4 half + rr%4: normalised,
    // or with a key split the partial record -- (max, sum) of the rows, then
    // their unnormalised O over this chunk ----
    const float l_tot = pair_sum(l_run);
    float* op;
    float mul;
    bool wr;
    if (SPLIT) {
        const int64_t rec = p.ragged ? (int64_t)idx
                                     : ((int64_t)(head * p.n_units + unit) * p.n_oc + oc) * p.n_split + split;
        float* rb = p.ws + rec * p.rpu * (kDeepChunk + 2);
        wr = l32 < p.rpu;
        if (wr && wave == 0 && half == 0) {
            rb[2 * l32] = m_run;
            rb[2 * l32 + 1] = l_tot;
        }
        op = rb + 2 * p.rpu + (int64_t)l32 * kDeepChunk - oc * kDeepChunk;
        mul = 1.f;
    } else {
        op = p.o.p + bi * p.o.sb + hq * p.o.sh + (int64_t)t * p.o.st;
        mul = l_tot > 0.f ? 1.f / l_tot : 0.f;
        wr = active;
    }
    if (wr) {
#pragma unroll
        for (int b = 0; b < OB; ++b) {
            if (b < nob) {
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const int c = od - l32 + CB * b + 8 * qq + 4 * half;
                    if (c < p.d)
                        *reinterpret_cast<vf4*>(op + c) =
                            vf4{o[b][4 * qq] * mul, o[b][4 * qq + 1] * mul,
                                o[b][4 * qq + 2] * mul, o[b][4 * qq + 3] * mul};
                }
            }
        }
    }
}

// Merges the n_split partial records of one (unit, chunk) of a key-split
// launch: O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s (M the largest
// m_s; rows with no visible key stay zero), the records added in split order.
__global__ __launch_bounds__(256) void deep_combine_kernel(const DeepParams p) {
    __shared__ float w_s[kDeepMaxSplit][32];   // weight of part s for row r
    __shared__ float inv_s[32];
    const int c = blockIdx.x;      // (head * n_units + unit) * n_oc + chunk
    const int oc = c % p.n_oc, hu = c / p.n_oc;
    const int unit = hu % p.n_units, head = hu / p.n_units;
    const int bi = head / p.Hkv, kvh = head % p.Hkv;
    const int tid = threadIdx.x;
    const int64_t rstride = (int64_t)p.rpu * (kDeepChunk + 2);
    // ragged: pair c's records part_prefix[c] .. part_prefix[c + 1] - 1
    const int n_parts = p.ragged ? (int)p.part_prefix[c + 1] - (int)p.part_prefix[c] : p.n_split;
    const float* rb = p.ws + (p.ragged ? (int64_t)p.part_prefix[c] : (int64_t)c * p.n_split) * rstride;
    if (tid < p.rpu) {
        float M = kNegInf;
        for (int sp = 0; sp < n_parts; ++sp) M = fmaxf(M, rb[sp * rstride + 2 * tid]);
        const float M_use = M == kNegInf ? 0.f : M;
        float l = 0.f;
        for (int sp = 0; sp < n_parts; ++sp) {
            const float w = fast_exp2(rb[sp * rstride + 2 * tid] - M_use);
            w_s[sp][tid] = w;
            l += w * rb[sp * rstride + 2 * tid + 1];
        }
        inv_s[tid] = l > 0.f ? 1.f / l : 0.f;
    }
    __syncthreads();
    const int rows = p.G * p.Tq;
    const int ndim = p.d - oc * kDeepChunk < kDeepChunk ? p.d - oc * kDeepChunk : kDeepChunk;
    for (int e = tid; e < p.rpu * (kDeepChunk / 4); e += 256) {
        const int rr = e / (kDeepChunk / 4), c4 = 4 * (e % (kDeepChunk / 4));
        const int r = unit * 32 + rr;
        if (r >= rows || c4 >= ndim) continue;
        vf4 acc = vf4{0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < n_parts; ++sp)
            acc += w_s[sp][rr] * *reinterpret_cast<const vf4*>(rb + sp * rstride + 2 * p.rpu +
                                                               (int64_t)rr * kDeepChunk + c4);
        const int g = r / p.Tq, t = r % p.Tq;
        float* op = p.o.p + bi * p.o.sb + (kvh * p.G + g) * p.o.sh + (int64_t)t * p.o.st;
        *reinterpret_cast<vf4*>(op + oc * kDeepChunk + c4) = acc * inv_s[rr];
    }
}

template <bool CAUSAL, int DW, int QC, int OB, bool STREAMQ>
hipError_t launch_deep_v(DeepParams p, hipStream_t stream) {
    // (The split is a template parameter: its tile range and record path cost
    // the unsplit kernel 35 VGPRs and 7 % at d = 512 when shared.)
    const int64_t rows = (int64_t)p.G * p.Tq;
    const int64_t units = (rows + 31) / 32;
    const int64_t n_oc = (p.d + 32 * DW * OB - 1) / (32 * DW * OB);
    if (p.n_split < 1 || (p.n_split > 1 && (!p.ws || p.n_split > kDeepMaxSplit || p.split_tiles < 1 ||
                                            p.rpu != (int)(rows < 32 ? rows : 32))))
        return hipErrorInvalidValue;
    const int64_t base = (int64_t)p.B * p.Hkv * units * n_oc;
    if (p.ragged && (p.n_split < 2 || units != 1 || n_oc != 1 || base > kDeepMaxHeads))
        return hipErrorInvalidValue;
    const int64_t total = p.ragged ? (int64_t)p.part_prefix[base] : base * p.n_split;
    if (total == 0) return hipSuccess;
    if (total > INT32_MAX - 8) return hipErrorInvalidValue;
    p.n_units = (int)units;
    p.n_oc = (int)n_oc;
    p.total = (int)total;
    p.per_xcd = (int)((total + 7) / 8);
    // Causal units longest first across the XCD's KV heads on the 8-wave form
    // (its one or two rounds then end together: B = 1, H = 16, T = 1024, d =
    // 512 185 -> 176 us).  The 4-wave form runs many rounds and keeps a KV
    // head's units together in the XCD's L2: across heads it read 2.4x the
    // bytes from beyond the L2 (d = 512 line 3.9 against 1.6 GB) for 0.7 %.
    p.order_hpx = DW == 8 && CAUSAL && p.n_split == 1 && ((int64_t)p.B * p.Hkv) % 8 == 0 ? p.B * p.Hkv / 8 : 0;
    if (p.n_split == 1) {
        hipLaunchKernelGGL((deep_attention_kernel<CAUSAL, DW, QC, OB, STREAMQ, false>),
                           dim3(8 * p.per_xcd), dim3(64 * DW), 0, stream, p);
        return hipGetLastError();
    }
    if constexpr (DW == 8 && OB == 2) {
        hipLaunchKernelGGL((deep_attention_kernel<CAUSAL, DW, QC, OB, STREAMQ, true>), dim3(8 * p.per_xcd),
                           dim3(64 * DW), 0, stream, p);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(deep_combine_kernel, dim3((unsigned)base), dim3(256), 0, stream, p);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;   // (the forms with 4 output blocks serve unsplit launches only)
}

// Up to 512 dims, problems of full 32-row units with more workgroups than
// CUs (causal: more than two per CU) run the 4-wave form.  Fewer workgroups
// keep 8 waves busy on a CU to the end (a causal launch of 2 workgroups per
// CU ran 10 % slower on the 4-wave form: once a CU's short unit ends, its
// long one runs alone with one wave per SIMD), and so do decode steps (a few
// rows per unit, streaming their caches: B = 32, d = 512 634 us with 8
// waves, 781 us with 4).
// Head dims 129-256 (prefill the wave-pair kernel does not take) run the
// 2-wave form unsplit, and the 8-wave form's key split.
template <bool CAUSAL>
hipError_t launch_deep_t(const DeepParams& p, int cus, hipStream_t stream) {
    if (p.d <= 256 && p.n_split == 1) return launch_deep_v<CAUSAL, 2, 16, 4, false>(p, stream);
    const int64_t rows = (int64_t)p.G * p.Tq, units = (rows + 31) / 32;
    const int64_t wg = (int64_t)p.B * p.Hkv * units * ((p.d + kDeepChunk - 1) / kDeepChunk);
    if (p.d <= 512 && p.n_split == 1 && rows >= 32 && wg > (CAUSAL ? 2 : 1) * (int64_t)cus)
        return launch_deep_v<CAUSAL, 4, 16, 4, false>(p, stream);
    if (p.d <= 512) return launch_deep_v<CAUSAL, 8, 8, 2, false>(p, stream);
    // Above 512 dims unsplit launches take 1024-dim output chunks (S computed
    // once per 1024 dims instead of per 512: d = 1024 non-causal B = 1, H = 8,
    // T = 2048 2.03 -> 1.17 ms, d = 2048 causal B = 1, H = 4, T = 2048 3.80 ->
    // 2.16 ms); key splits keep 512-dim records.
    if (p.n_split == 1) {
        if (p.d <= 1024) return launch_deep_v<CAUSAL, 8, 16, 4, false>(p, stream);
        return launch_deep_v<CAUSAL, 8, 16, 4, true>(p, stream);
    }
    if (p.d <= 1024) return launch_deep_v<CAUSAL, 8, 16, 2, false>(p, stream);
    return launch_deep_v<CAUSAL, 8, 16, 2, true>(p, stream);
}

}  // namespace

hipError_t launch_deep(DeepParams p, bool causal, int cus, hipStream_t stream) {
    if (p.d <= 128 || p.d % 4 != 0 || p.Hkv <= 0 || p.G <= 0) return hipErrorInvalidValue;
    return causal ? launch_deep_t<true>(p, cus, stream) : launch_deep_t<false>(p, cus, stream);
}

}  // namespace nne
