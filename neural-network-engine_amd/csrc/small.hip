// Prefill for problems too small to fill the device: one workgroup per
// (sequence, query head, block of 16 query rows) -- two, each with half of the
// output dims, while that leaves at most one per CU -- whose waves split the
// block's key tiles and merge through LDS.
//
// Algorithm: the online softmax of the reference's flash_attention_forward
// (src/nn/flash_attention.rs:91-195) over 16-key tiles, each wave keeping a
// running (max, sum, O) for the block's 16 rows, then the same combine across
// the waves: O = sum_w 2^(m_w - M) O_w / sum_w 2^(m_w - M) l_w, with rows
// that see no key left at zero (:186-194).  Keys visible to row r are
// c <= r + q_offset (causal) and c < T_k.
//
// MI355X mapping.  A small problem's time is a chain of latencies, not
// arithmetic: a launch, the first loads, the tiles one wave must run in
// sequence, and any hand-off between workgroups.  Here the waves of one
// workgroup take the tiles of one row block side by side (8 waves, at most
// two tiles each, loaded at once), and the partial results never leave the
// CU: no global records, no arrival counters, no second round trip.
// Per tile, on v_mfma_f32_16x16x4_f32 (the layout of the split-K kernel's
// 16-row tile):
//   S^T = K Q^T  (Q^T in registers, pre-scaled by scale * log2(e); K staged
//                 through a wave-private LDS slice into operand layout),
//   a row's 16 scores sit in 4 registers of 4 lanes: max / sum are 3 in-lane
//   ops and two lane swaps,
//   O^T += V^T P^T (P^T register r is the B operand of step r; V loaded
//                 straight from HBM in operand layout).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>

#include "nne_common.hpp"
#include "nne_launch.hpp"

namespace nne {

namespace {

constexpr int SKB = 16;   // keys per tile, query rows per block

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float rows4_max(float x) {   // over lanes {l, l^16, l^32, l^48}
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows4_sum(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Waves per workgroup; each takes at most two tiles, both loaded at once.
// Measured at config 1 (B=1, H=4, T=256, d=64, causal), queued calls on
// MI355X: 16 waves of one tile each 7.0 us, 8 waves of two tiles 6.5 us --
// the LDS merge of twice as many partial O cost more than the second tile.
// The heaviest causal block (16 tiles) keeps its CU's four MFMA pipes busy
// for ~1.7 us (~1.3 us with half of P V per workgroup); with the ~1.6 us
// launch and ~1.5 us first loads that is most of the call.  Config 1 with two
// workgroups per block: 6.3 -> 5.8 us; with four (a quarter of P V each,
// 4-byte V loads) 6.15 us.
constexpr int SMALL_WAVES = 8;
constexpr int SMALL_TILES_PER_WAVE = 2;
template <int D>
constexpr int small_waves() { return SMALL_WAVES; }

// DP = 2: the 4 components of each V vector (dims 4i + c) are split over two
// workgroups per row block, c in {0, 1} and {2, 3}.  Both compute the block's
// whole S = Q K^T and softmax (the same bits), each its half of O = P V, so
// the heaviest block's MFMA work per CU drops from 32 to 24 instructions per
// tile and its V loads by half, with no hand-off between them.
template <int D, bool CAUSAL, int DP>
__global__ __launch_bounds__(64 * small_waves<D>(), 1) void small_prefill_kernel(const PrefillParams p) {
    constexpr int NW = small_waves<D>();
    constexpr int KS = D + 4;            // LDS row stride (16-byte reads conflict-free)
    constexpr int LPR = D / 4;           // lanes per K row in the coalesced load
    constexpr int RPI = 64 / LPR;        // K rows per load instruction
    constexpr int NK = SKB / RPI;        // K float4 loads per lane per tile
    constexpr int NH = D / 64;           // V float4 loads per key step
    constexpr int NQ = D / 4;            // Q^T registers per lane
    static_assert(NK == 4 * NH, "K and V loads per tile");

    // K slices of the waves during the tile loop, then the waves' partial O.
    __shared__ __attribute__((aligned(16))) float lds[NW * SKB * KS];
    __shared__ __attribute__((aligned(16))) float q_s[SKB * KS];   // the block's Q rows
    __shared__ float ml_s[NW][SKB][2];
    __shared__ float wgt_s[NW][SKB];     // merge weight of wave w for row r

    // Every scalar argument's cache line in one round trip (left to the
    // compiler, the first uses chain three of them before the first load).
    warm_kernargs<0, offsetof(PrefillParams, part_prefix)>();
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;

    // Workgroup -> (sequence, query head, row block).  The hardware deals
    // consecutive workgroup ids to the 8 XCDs in turn; XCD x takes the x-th
    // eighth of the block list, so the blocks of one head -- which read the
    // same K/V tiles -- share an L2.  In causal problems the blocks with the
    // most keys come first.
    const int n_rb = (p.Tq + SKB - 1) / SKB;
    const int n_items = p.B * p.Hq * n_rb;
    const int per_xcd = (n_items * DP + 7) >> 3;
    const int idx_p = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (idx_p >= n_items * DP) return;   // whole workgroup: no barrier is skipped
    const int idx = idx_p / DP, part = idx_p % DP;
    const int rb_i = idx % n_rb, bh = idx / n_rb;
    const int rb = CAUSAL ? n_rb - 1 - rb_i : rb_i;
    const int bi = bh / p.Hq, hq = bh % p.Hq, kvh = hq / p.G;
    const int r0 = rb * SKB;
    const int row = r0 + col;            // this lane's query row

    int n_keys = p.Tk;
    if (CAUSAL) n_keys = min(p.Tk, min(p.Tq - 1, r0 + SKB - 1) + p.q_offset + 1);
    const int n_tiles = n_keys > 0 ? (n_keys + SKB - 1) / SKB : 0;

    const float* kb = p.k.p + bi * p.k.sb + kvh * p.k.sh;
    const float* vb = p.v.p + bi * p.v.sb + kvh * p.v.sh;
    const int kst = (int)p.k.st, vst = (int)p.v.st;
    const int kc_col = min(4 * (lane % LPR), p.d - 4);
    int v_col[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) v_col[h] = min(64 * h + 4 * col, p.d - 4) + (4 / DP) * part;
    float* Kw = lds + wave * SKB * KS;

    // The block's 16 Q rows, loaded once for all waves (scaled by
    // scale * log2(e); rows past T_q and columns past d are zero).  Their
    // loads go first, so staging them waits for nothing else.
    static_assert(SKB * (D / 4) <= 64 * NW, "one Q vector per thread");
    const int qe = tid, q_r = qe / (D / 4), q_c = 4 * (qe % (D / 4));
    const bool q_ok = qe < SKB * (D / 4) && r0 + q_r < p.Tq && q_c < p.d;
    vf4 qx = vf4{0.f, 0.f, 0.f, 0.f};
    if (q_ok)
        qx = *reinterpret_cast<const vf4*>(p.q.p + bi * p.q.sb + hq * p.q.sh +
                                          (int64_t)(r0 + q_r) * p.q.st + q_c);
    // Both tiles of this wave (wave and wave + NW) in flight at once.  Loads
    // clamp to the last key (masked below) and to the row's last 4 floats
    // past d (their Q columns are zero), so none is out of bounds.
    typedef float vfp __attribute__((ext_vector_type(4 / DP)));   // this part's V components
    vf4 kr[SMALL_TILES_PER_WAVE][NK];
    vfp vr[SMALL_TILES_PER_WAVE][4 * NH];
    auto load_tile = [&](vf4 (&kt)[NK], vfp (&vt)[4 * NH], int kb0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NK; ++i) {
            const int key = min(kb0 + lane / LPR + RPI * i, n_keys - 1);
            kt[i] = *reinterpret_cast<const vf4*>(kb + key * kst + kc_col);
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int key = min(kb0 + 4 * grp + st, n_keys - 1);
#pragma unroll
            for (int h = 0; h < NH; ++h)
                vt[st * NH + h] = *reinterpret_cast<const vfp*>(vb + key * vst + v_col[h]);
        }
    };
#pragma unroll
    for (int j = 0; j < SMALL_TILES_PER_WAVE; ++j)
        if (wave + j * NW < n_tiles) load_tile(kr[j], vr[j], (wave + j * NW) * SKB);
    if (qe < SKB * (D / 4)) *reinterpret_cast<vf4*>(q_s + q_r * KS + q_c) = qx * p.qscale;
    __syncthreads();
    float qf[NQ];
#pragma unroll
    for (int s4 = 0; s4 < NQ / 4; ++s4) {
        const vf4 x = *reinterpret_cast<const vf4*>(q_s + col * KS + grp * NQ + 4 * s4);
        qf[4 * s4 + 0] = x.x;
        qf[4 * s4 + 1] = x.y;
        qf[4 * s4 + 2] = x.z;
        qf[4 * s4 + 3] = x.w;
    }

    constexpr int NC = 4 / DP;           // V components (dim blocks per h) of this part
    floatx4 o[NH * NC];
#pragma unroll
    for (int b = 0; b < NH * NC; ++b) o[b] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = kNegInf, l_run = 0.f;
    // last key this lane's row may see (tile masks only where a tile reaches past it)
    const int row_last = CAUSAL ? row + p.q_offset : p.Tk - 1;

#pragma unroll
    for (int j = 0; j < SMALL_TILES_PER_WAVE; ++j) {
        const int t = wave + j * NW;
        if (t >= n_tiles) break;         // wave-uniform
        const int kb0 = t * SKB;
        wave_lds_fence();
#pragma unroll
        for (int i = 0; i < NK; ++i)
            *reinterpret_cast<vf4*>(Kw + (lane / LPR + RPI * i) * KS + 4 * (lane % LPR)) = kr[j][i];
        wave_lds_fence();

        // S^T = K Q^T: s[r] = score of key kb0 + 4*grp + r for row `col`.
        floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
        const float* krow = Kw + col * KS + grp * NQ;
#pragma unroll
        for (int i = 0; i < NQ / 4; ++i) {
            const vf4 kq = *reinterpret_cast<const vf4*>(krow + 4 * i);
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(kq.x, qf[4 * i + 0], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(kq.y, qf[4 * i + 1], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(kq.z, qf[4 * i + 2], s, 0, 0, 0);
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(kq.w, qf[4 * i + 3], s, 0, 0, 0);
        }
        if (kb0 + SKB > n_keys || (CAUSAL && kb0 + SKB - 1 > r0 + p.q_offset)) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = kb0 + 4 * grp + r;
                s[r] = (key < n_keys && key <= row_last) ? s[r] : kNegInf;
            }
        }
        float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        mt = rows4_max(mt);
        const float m_new = fmaxf(m_run, mt);
        const float m_use = m_new == kNegInf ? 0.f : m_new;
        const float alpha = fast_exp2(m_run - m_use);
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[r] = fast_exp2(s[r] - m_use);
            ls += s[r];
        }
        l_run = alpha * l_run + ls;       // this lane's 4 keys; summed over lanes below
        m_run = m_new;
#pragma unroll
        for (int b = 0; b < NH * NC; ++b) o[b] *= alpha;
        // O^T += V^T P^T: step st pairs key kb0 + 4*grp + st (register st of
        // P^T); dim block NC*h + c covers dims 64h + 4*i + NC*part + c,
        // i = lane % 16.
#pragma unroll
        for (int st = 0; st < 4; ++st)
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const vfp vv = vr[j][st * NH + h];
#pragma unroll
                for (int c = 0; c < NC; ++c)
                    o[NC * h + c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[c], s[st], o[NC * h + c], 0, 0, 0);
            }
    }

    // Merge the waves' (max, sum, O) through LDS: O[row col][dim] with
    // dim = 64h + 16*grp + 4*reg + NC*part + c  for  o[NC*h + c][reg].
    const float l_tot = rows4_sum(l_run);
    __syncthreads();                      // every wave is done with its K slice
    float* ob = lds;                      // [NW waves][16 rows][KS]
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int reg = 0; reg < 4; ++reg) {
            vfp ov;
#pragma unroll
            for (int c = 0; c < NC; ++c) ov[c] = o[NC * h + c][reg];
            *reinterpret_cast<vfp*>(ob + (wave * SKB + col) * KS + 64 * h + 16 * grp + 4 * reg + NC * part) = ov;
        }
    if (grp == 0) {
        ml_s[wave][col][0] = m_run;
        ml_s[wave][col][1] = l_tot;
    }
    __syncthreads();
    // Weight of wave w for row r: 2^(m_w - M) / sum_w' 2^(m_w' - M) l_w'
    // (0 for waves without a tile, and for rows that saw no key), computed
    // once per (row, wave) by NW-lane groups, in a fixed order.
    const int n_active = min(NW, n_tiles);   // waves that ran a tile
    if (tid < SKB * NW) {
        const int rr = tid / NW, w = tid % NW;
        const float m = w < n_active ? ml_s[w][rr][0] : kNegInf;
        float M = m;
#pragma unroll
        for (int off = 1; off < NW; off <<= 1) M = fmaxf(M, __shfl_xor(M, off, NW));
        const float f = w < n_active ? fast_exp2(m - (M == kNegInf ? 0.f : M)) : 0.f;
        float L = f * (w < n_active ? ml_s[w][rr][1] : 0.f);
#pragma unroll
        for (int off = 1; off < NW; off <<= 1) L += __shfl_xor(L, off, NW);
        wgt_s[w][rr] = L > 0.f ? f / L : 0.f;
    }
    __syncthreads();
    // 16-byte output vectors (8-byte with DP = 2: this part's 2 of every 4
    // dims; d % 4 == 0 and 16-byte views on this path).
    for (int e = tid; e < SKB * (D / 4); e += 64 * NW) {
        const int rr = e / (D / 4), c = 4 * (e % (D / 4)) + NC * part;
        vfp acc = vfp(0.f);
#pragma unroll
        for (int w = 0; w < NW; ++w)
            acc += wgt_s[w][rr] * *reinterpret_cast<const vfp*>(ob + (w * SKB + rr) * KS + c);
        if (r0 + rr < p.Tq && c < p.d)
            *reinterpret_cast<vfp*>(p.o.p + bi * p.o.sb + hq * p.o.sh + (int64_t)(r0 + rr) * p.o.st + c) = acc;
    }
}

template <int D, int DP>
hipError_t launch_small_dp(const PrefillParams& p, bool causal, int n_items, hipStream_t stream) {
    const dim3 grid((unsigned)(8 * ((n_items * DP + 7) / 8))), block(64 * small_waves<D>());
    if (causal)
        hipLaunchKernelGGL((small_prefill_kernel<D, true, DP>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((small_prefill_kernel<D, false, DP>), grid, block, 0, stream, p);
    return hipGetLastError();
}

// Two workgroups per row block (each half of P V) while that still leaves
// at most one per CU.
template <int D>
hipError_t launch_small_d(const PrefillParams& p, bool causal, int cus, hipStream_t stream) {
    const int n_rb = (p.Tq + SKB - 1) / SKB;
    const int n_items = p.B * p.Hq * n_rb;
    if (2 * n_items <= cus) return launch_small_dp<D, 2>(p, causal, n_items, stream);
    return launch_small_dp<D, 1>(p, causal, n_items, stream);
}

}  // namespace

bool small_prefill_fits(const PrefillParams& p, bool vec, int cus) {
    if (!vec || p.d % 4 != 0 || p.d > 128 || p.Hkv == 0) return false;
    // key offsets are 32-bit in the kernel
    if ((int64_t)p.Tk * p.k.st >= INT32_MAX || (int64_t)p.Tk * p.v.st >= INT32_MAX) return false;
    const int64_t wgs = (int64_t)p.B * p.Hq * ((p.Tq + SKB - 1) / SKB);
    // Tiles of the heaviest row block: at most two per wave.
    const int64_t tiles = ((int64_t)p.Tk + SKB - 1) / SKB;
    return wgs > 0 && wgs <= cus && tiles <= SMALL_TILES_PER_WAVE * SMALL_WAVES;
}

hipError_t launch_small_prefill(PrefillParams p, bool causal, int cus, hipStream_t stream) {
    p.G = p.Hq / p.Hkv;
    if ((int64_t)p.B * p.Hq * p.Tq == 0) return hipSuccess;
    return p.d <= 64 ? launch_small_d<64>(p, causal, cus, stream) : launch_small_d<128>(p, causal, cus, stream);
}

}  // namespace nne
