// Prefill for problems too small to fill the device: one workgroup per
// (sequence, query head, block of 16 query rows), whose waves split the
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
// workgroup take the tiles of one row block side by side (up to 16 waves,
// 4 per SIMD, at d <= 64; 8 at d = 128), so the heaviest causal block of a
// T = 256 head runs one tile per wave, and the partial results never leave
// the CU: no global records, no arrival counters, no second round trip.
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

// Waves per workgroup: 4 per SIMD at d <= 64 (<= 128 registers each), 2 at
// d = 128.
template <int D>
constexpr int small_waves() { return D <= 64 ? 16 : 8; }

template <int D, bool CAUSAL>
__global__ __launch_bounds__(64 * small_waves<D>(), 1) void small_prefill_kernel(const PrefillParams p) {
    constexpr int NW = small_waves<D>();
    constexpr int KS = D + 4;            // LDS row stride (16-byte reads conflict-free)
    constexpr int LPR = D / 4;           // lanes per K row in the coalesced load
    constexpr int RPI = 64 / LPR;        // K rows per load instruction
    constexpr int NK = SKB / RPI;        // K float4 loads per lane per tile
    constexpr int NH = D / 64;           // V float4 loads per key step
    constexpr int NQ = D / 4;            // Q^T registers per lane
    constexpr int NB = D / 16;           // 16-dim output blocks
    static_assert(NK == 4 * NH, "K and V loads per tile");

    // K slices of the waves during the tile loop, then the waves' partial O.
    __shared__ __attribute__((aligned(16))) float lds[NW * SKB * KS];
    __shared__ float ml_s[NW][SKB][2];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;

    // Workgroup -> (sequence, query head, row block); in causal problems the
    // blocks with the most keys go first.
    const int n_rb = (p.Tq + SKB - 1) / SKB;
    const int idx = blockIdx.x;
    const int rb_i = idx % n_rb, bh = idx / n_rb;
    const int rb = CAUSAL ? n_rb - 1 - rb_i : rb_i;
    const int bi = bh / p.Hq, hq = bh % p.Hq, kvh = hq / p.G;
    const int r0 = rb * SKB;
    const int row = r0 + col;            // this lane's query row

    int n_keys = p.Tk;
    if (CAUSAL) n_keys = min(p.Tk, min(p.Tq - 1, r0 + SKB - 1) + p.q_offset + 1);
    const int n_tiles = n_keys > 0 ? (n_keys + SKB - 1) / SKB : 0;

    // Q^T fragment: lane holds row `col`, dims grp*NQ .. +NQ, pre-scaled.
    float qf[NQ];
    {
        const bool rok = row < p.Tq;
        const float* qp = p.q.p + bi * p.q.sb + hq * p.q.sh + (int64_t)(rok ? row : 0) * p.q.st;
#pragma unroll
        for (int s4 = 0; s4 < NQ / 4; ++s4) {
            const int c = grp * NQ + 4 * s4;
            const vf4 x = *reinterpret_cast<const vf4*>(qp + min(c, p.d - 4));
            const bool ok = rok && c < p.d;
            qf[4 * s4 + 0] = ok ? x.x * p.qscale : 0.f;
            qf[4 * s4 + 1] = ok ? x.y * p.qscale : 0.f;
            qf[4 * s4 + 2] = ok ? x.z * p.qscale : 0.f;
            qf[4 * s4 + 3] = ok ? x.w * p.qscale : 0.f;
        }
    }
    const float* kb = p.k.p + bi * p.k.sb + kvh * p.k.sh;
    const float* vb = p.v.p + bi * p.v.sb + kvh * p.v.sh;
    const int kst = (int)p.k.st, vst = (int)p.v.st;
    const int kc_col = min(4 * (lane % LPR), p.d - 4);
    int v_col[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) v_col[h] = min(64 * h + 4 * col, p.d - 4);
    float* Kw = lds + wave * SKB * KS;

    floatx4 o[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) o[b] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = kNegInf, l_run = 0.f;
    // last key this lane's row may see (tile masks only where a tile reaches past it)
    const int row_last = CAUSAL ? row + p.q_offset : p.Tk - 1;

    for (int t = wave; t < n_tiles; t += NW) {
        const int kb0 = t * SKB;
        vf4 kr[NK], vr[4 * NH];
        // Loads clamp to the last key (masked below) and to the row's last 4
        // floats past d (their Q columns are zero), so none is out of bounds.
#pragma unroll
        for (int i = 0; i < NK; ++i) {
            const int key = min(kb0 + lane / LPR + RPI * i, n_keys - 1);
            kr[i] = *reinterpret_cast<const vf4*>(kb + key * kst + kc_col);
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int key = min(kb0 + 4 * grp + st, n_keys - 1);
#pragma unroll
            for (int h = 0; h < NH; ++h)
                vr[st * NH + h] = *reinterpret_cast<const vf4*>(vb + key * vst + v_col[h]);
        }
        wave_lds_fence();
#pragma unroll
        for (int i = 0; i < NK; ++i)
            *reinterpret_cast<vf4*>(Kw + (lane / LPR + RPI * i) * KS + 4 * (lane % LPR)) = kr[i];
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
        for (int b = 0; b < NB; ++b) o[b] *= alpha;
        // O^T += V^T P^T: step st pairs key kb0 + 4*grp + st (register st of
        // P^T); dim block 4h + c covers dims 64h + 4*i + c, i = lane % 16.
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

    // Merge the waves' (max, sum, O) through LDS: O[row col][dim] with
    // dim = 64h + 16*grp + 4*reg + c  for  o[4h + c][reg].
    const float l_tot = rows4_sum(l_run);
    __syncthreads();                      // every wave is done with its K slice
    float* ob = lds;                      // [NW waves][16 rows][KS]
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
        for (int reg = 0; reg < 4; ++reg)
            *reinterpret_cast<vf4*>(ob + (wave * SKB + col) * KS + 64 * h + 16 * grp + 4 * reg) =
                vf4{o[4 * h + 0][reg], o[4 * h + 1][reg], o[4 * h + 2][reg], o[4 * h + 3][reg]};
    if (grp == 0) {
        ml_s[wave][col][0] = m_run;
        ml_s[wave][col][1] = l_tot;
    }
    __syncthreads();
    const int n_active = min(NW, n_tiles);   // waves that ran a tile
    for (int e = tid; e < SKB * D; e += 64 * NW) {
        const int rr = e / D, dd = e % D;
        if (r0 + rr >= p.Tq || dd >= p.d) continue;
        float M = kNegInf;
        for (int w = 0; w < n_active; ++w) M = fmaxf(M, ml_s[w][rr][0]);
        const float M_use = M == kNegInf ? 0.f : M;
        float l = 0.f, acc = 0.f;
        for (int w = 0; w < n_active; ++w) {
            const float f = fast_exp2(ml_s[w][rr][0] - M_use);
            l += f * ml_s[w][rr][1];
            acc += f * ob[(w * SKB + rr) * KS + dd];
        }
        p.o.p[bi * p.o.sb + hq * p.o.sh + (int64_t)(r0 + rr) * p.o.st + dd] = l > 0.f ? acc / l : 0.f;
    }
}

template <int D>
hipError_t launch_small_d(const PrefillParams& p, bool causal, hipStream_t stream) {
    const int n_rb = (p.Tq + SKB - 1) / SKB;
    const dim3 grid((unsigned)(p.B * p.Hq * n_rb)), block(64 * small_waves<D>());
    if (causal)
        hipLaunchKernelGGL((small_prefill_kernel<D, true>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((small_prefill_kernel<D, false>), grid, block, 0, stream, p);
    return hipGetLastError();
}

}  // namespace

bool small_prefill_fits(const PrefillParams& p, bool vec, int cus) {
    if (!vec || p.d % 4 != 0 || p.d > 128 || p.Hkv == 0) return false;
    // key offsets are 32-bit in the kernel
    if ((int64_t)p.Tk * p.k.st >= INT32_MAX || (int64_t)p.Tk * p.v.st >= INT32_MAX) return false;
    const int64_t wgs = (int64_t)p.B * p.Hq * ((p.Tq + SKB - 1) / SKB);
    // Tiles of the heaviest row block: at most two per wave.
    const int64_t tiles = ((int64_t)p.Tk + SKB - 1) / SKB;
    const int nw = p.d <= 64 ? small_waves<64>() : small_waves<128>();
    return wgs > 0 && wgs <= cus && tiles <= 2 * nw;
}

hipError_t launch_small_prefill(PrefillParams p, bool causal, hipStream_t stream) {
    p.G = p.Hq / p.Hkv;
    if ((int64_t)p.B * p.Hq * p.Tq == 0) return hipSuccess;
    return p.d <= 64 ? launch_small_d<64>(p, causal, stream) : launch_small_d<128>(p, causal, stream);
}

}  // namespace nne
