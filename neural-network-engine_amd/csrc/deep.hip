// Attention at head dims above 256: prefill, cross-attention and decode over a
// KV cache, on v_mfma_f32_32x32x2_f32.
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
// a K/V row once per unit, the unit's waves splitting the row between them):
//  * S^T = K Q^T is split over the waves by dims.  Wave w takes the 8-dim
//    chunks j = w, w + 8, w + 16, ...; lane half h holds dims 8j + 4h ..
//    8j + 4h + 3 of its row (one 16-byte load), and MFMA c of a chunk pairs
//    dims 8j + c and 8j + 4 + c.  Q^T of a wave's first 16 chunks stays in
//    registers; further chunks (d > 1024) are read again each tile.
//  * The 8 partial S^T (4 KB each) meet in LDS, double-buffered so one barrier
//    per tile suffices; every wave adds them in wave order, so all 8 hold the
//    same S bit for bit and take the same online-softmax decisions.
//  * O^T += V^T P^T is split over the waves by 32-dim output blocks: wave w
//    owns blocks w, w + 8, w + 16, w + 24 of the workgroup's 1024-dim output
//    chunk (64 accumulator registers).  Each V operand load is one 128-byte
//    row segment per half-wave.
//  A unit of more than 1024 dims takes one workgroup per output chunk, each
//  recomputing S.  Workgroup ids go to the 8 XCDs in turn; XCD x takes the
//  x-th eighth of the (sequence, KV head, unit, chunk) list, so the units of
//  a KV head, which read the same K/V rows, share an L2, and causal units
//  are taken longest first.
#include <hip/hip_runtime.h>

#include "nne_common.hpp"
#include "nne_launch.hpp"

namespace nne {

namespace {

constexpr int DW = 8;                           // waves per workgroup
constexpr int OB = kDeepChunk / 32 / DW;        // output blocks per wave
constexpr int XW = 16 * 64;                     // floats of one wave's partial S^T

__device__ __forceinline__ vf4 load4(const float* p) { return *reinterpret_cast<const vf4*>(p); }

__device__ __forceinline__ int clamp_keys(int64_t x, int tk) {
    return x < 0 ? 0 : (x > tk ? tk : (int)x);
}

// QC: chunks per wave whose Q^T stays in registers (8 up to d = 512, 16 up
// to d = 1024); STREAMQ: further chunks read again each tile.
template <bool CAUSAL, int QC, bool STREAMQ>
__global__ __launch_bounds__(64 * DW, 1) void deep_attention_kernel(const DeepParams p) {
    __shared__ __attribute__((aligned(16))) float xs[2 * DW * XW];

    const int idx = (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
    if (idx >= p.total) return;   // whole workgroup: no barrier is skipped
    const int oc = idx % p.n_oc;
    const int hu = idx / p.n_oc;
    const int ui = hu % p.n_units, head = hu / p.n_units;
    const int unit = CAUSAL ? p.n_units - 1 - ui : ui;
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

    // This wave's chunks of S (8 dims each) and output blocks (32 dims each).
    const int nj = (p.d + 7) >> 3;
    const int nq = wave < nj ? ((nj - 1 - wave) >> 3) + 1 : 0;
    const int nbt = (p.d + 31) >> 5;
    const int gb0 = oc * (kDeepChunk / 32) + wave;
    const int nob = gb0 < nbt ? min(OB, ((nbt - 1 - gb0) >> 3) + 1) : 0;

    const float* qp = p.q.p + bi * p.q.sb + hq * p.q.sh + (int64_t)t * p.q.st;
    vf4 qf[QC];
#pragma unroll
    for (int i = 0; i < QC; ++i) {
        const int c = 8 * (wave + DW * i) + 4 * half;
        qf[i] = (active && c < p.d) ? load4(qp + c) * p.qscale : vf4{0.f, 0.f, 0.f, 0.f};
    }

    const float* kb = p.k.p + bi * p.k.sb + kvh * p.k.sh;
    const float* vb = p.v.p + bi * p.v.sb + kvh * p.v.sh;
    const int od = oc * kDeepChunk + 32 * wave + l32;   // this lane's dim of output block 0

    floatx16 o[OB];
#pragma unroll
    for (int b = 0; b < OB; ++b)
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) o[b][rr] = 0.f;
    float m_run = kNegInf, l_run = 0.f;

    for (int it = 0; it < n_tiles; ++it) {
        const int key0 = it * 32;
        float* xb = xs + (it & 1) * (DW * XW);

        // Partial S^T = K Q^T over this wave's chunks, log2 domain.
        floatx16 s;
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) s[rr] = 0.f;
        {
            // Chunks in groups of 4 (16 registers of K each), the next group's
            // loads issued before the current group's MFMAs; the scheduling
            // barriers keep the compiler from hoisting every load of the tile.
            const bool kok = key0 + l32 < kend;
            const float* krow = kb + (int64_t)(key0 + l32) * p.k.st;
            vf4 kq[2][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = 8 * (wave + DW * i) + 4 * half;
                kq[0][i] = (kok && i < nq && c < p.d) ? load4(krow + c) : vf4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int gi = 0; gi < QC / 4; ++gi) {
                if (4 * gi < nq) {
                    if (gi + 1 < QC / 4) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int ii = 4 * (gi + 1) + i;
                            const int c = 8 * (wave + DW * ii) + 4 * half;
                            kq[(gi + 1) & 1][i] = (kok && ii < nq && c < p.d)
                                                      ? load4(krow + c)
                                                      : vf4{0.f, 0.f, 0.f, 0.f};
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const vf4 kk = kq[gi & 1][i];
                        const vf4 qq = qf[4 * gi + i];
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
                    const vf4 kk = (kok && c < p.d) ? load4(krow + c) : vf4{0.f, 0.f, 0.f, 0.f};
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[0], qq[0], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[1], qq[1], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[2], qq[2], s, 0, 0, 0);
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk[3], qq[3], s, 0, 0, 0);
                }
            }
        }
        // Register-group major (each store one contiguous 1 KB wave access).
        {
            float* xo = xb + wave * XW + 4 * lane;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<vf4*>(xo + 256 * i) =
                    vf4{s[4 * i], s[4 * i + 1], s[4 * i + 2], s[4 * i + 3]};
        }
        __syncthreads();   // the tile's partials visible
        if (nob == 0) continue;   // no output dims here; the wave still adds its partial

        // S = the partials added in wave order (the same bits in every wave).
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vf4 a = load4(xb + 4 * lane + 256 * i);
#pragma unroll
            for (int w = 1; w < DW; ++w) a += load4(xb + w * XW + 4 * lane + 256 * i);
            s[4 * i] = a[0];
            s[4 * i + 1] = a[1];
            s[4 * i + 2] = a[2];
            s[4 * i + 3] = a[3];
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

        // O^T += V^T P^T over this wave's output blocks, keys in groups of 4
        // register steps (16 V operands), the next group's loads issued first.
        {
            float vq[2][4][OB];
            auto load_v = [&](int rg, float (&dst)[4][OB]) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int rr = 4 * rg + j;
                    const int key = key0 + 8 * (rr >> 2) + 4 * half + (rr & 3);
                    const bool vok = key < kend;
                    const float* vrow = vb + (int64_t)key * p.v.st + od;
#pragma unroll
                    for (int b = 0; b < OB; ++b)
                        dst[j][b] = (vok && b < nob && od + 256 * b < p.d) ? vrow[256 * b] : 0.f;
                }
            };
            load_v(0, vq[0]);
#pragma unroll
            for (int rg = 0; rg < 4; ++rg) {
                if (rg + 1 < 4) load_v(rg + 1, vq[(rg + 1) & 1]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int b = 0; b < OB; ++b)
                        if (b < nob)
                            o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vq[rg & 1][j][b],
                                                                        s[4 * rg + j], o[b], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }

    // ---- normalise and write O[row][dim], dim = 32 gb + 8 (rr/4) + 4 half + rr%4 ----
    const float l_tot = pair_sum(l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (active) {
        float* op = p.o.p + bi * p.o.sb + hq * p.o.sh + (int64_t)t * p.o.st;
#pragma unroll
        for (int b = 0; b < OB; ++b) {
            if (b < nob) {
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const int c = od - l32 + 256 * b + 8 * qq + 4 * half;
                    if (c < p.d)
                        *reinterpret_cast<vf4*>(op + c) =
                            vf4{o[b][4 * qq] * inv, o[b][4 * qq + 1] * inv,
                                o[b][4 * qq + 2] * inv, o[b][4 * qq + 3] * inv};
                }
            }
        }
    }
}

template <bool CAUSAL>
hipError_t launch_deep_t(const DeepParams& p, hipStream_t stream) {
    const dim3 grid(8 * p.per_xcd), block(64 * DW);
    if (p.d <= 8 * DW * 8)
        hipLaunchKernelGGL((deep_attention_kernel<CAUSAL, 8, false>), grid, block, 0, stream, p);
    else if (p.d <= 8 * DW * 16)
        hipLaunchKernelGGL((deep_attention_kernel<CAUSAL, 16, false>), grid, block, 0, stream, p);
    else
        hipLaunchKernelGGL((deep_attention_kernel<CAUSAL, 16, true>), grid, block, 0, stream, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_deep(DeepParams p, bool causal, hipStream_t stream) {
    if (p.d <= 256 || p.d % 4 != 0 || p.Hkv <= 0 || p.G <= 0) return hipErrorInvalidValue;
    const int64_t rows = (int64_t)p.G * p.Tq;
    const int64_t units = (rows + 31) / 32;
    const int64_t n_oc = (p.d + kDeepChunk - 1) / kDeepChunk;
    const int64_t total = (int64_t)p.B * p.Hkv * units * n_oc;
    if (total == 0) return hipSuccess;
    if (total > INT32_MAX - 8) return hipErrorInvalidValue;
    p.n_units = (int)units;
    p.n_oc = (int)n_oc;
    p.total = (int)total;
    p.per_xcd = (int)((total + 7) / 8);
    return causal ? launch_deep_t<true>(p, stream) : launch_deep_t<false>(p, stream);
}

}  // namespace nne
