// Few-query attention for decode and cross-attention, plus the KV-cache append.
//
// Semantics: every query row attends to all keys of its sequence with no mask
// -- the reference's single-token decode (src/models/llama.rs:239-296 with
// t = 1: append first, then attend to all L rows including the new one) and
// its cross-attention (src/nn/attention.rs:193-203).  Sequences may have
// different lengths (lens[b]); the reference handles ragged batches as
// separate B = 1 calls.
//
// MI355X mapping.  The work is HBM-bound (about 2 FLOP per byte of K/V), so the
// kernel is organised around streaming each KV head's cache exactly once:
//   * a workgroup owns one split (a run of 64-key tiles) of one
//     (sequence, KV head) and serves all R = G * T_q query rows that read that
//     KV head, so grouped-query sharing costs no extra HBM traffic;
//   * K and V tiles are read with fully coalesced 16-byte loads (32 lanes per
//     512-byte row at d = 128) and staged in LDS; the next tile's loads are
//     issued before the current tile is computed;
//   * per tile: scores on VALU from LDS (query rows broadcast from LDS), a
//     one-wave-per-row online softmax, then P V accumulated in registers;
//   * splits of one sequence are merged by a small combine kernel from
//     partial (max, sum, O) records; single-split sequences write their output
//     directly.
#include "nne_common.hpp"
#include "nne_launch.hpp"

namespace nne {

namespace {

constexpr int KT = 64;   // keys per tile

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
    return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

template <int D, int RMAX>
__global__ __launch_bounds__(256, 2) void splitk_kernel(const SplitKParams p, int keys_per_split) {
    constexpr int KS = D + 4;                 // LDS row stride
    constexpr int C4 = D / 4;                 // float4 per row
    constexpr int NV = KT * C4 / 256;         // float4 per thread per tile
    constexpr int NG = 256 / C4;              // key groups in the P V layout
    constexpr int KPG = KT / NG;              // keys per group per tile
    static_assert(4 * RMAX * D <= KT * KS, "reduction buffer must fit in the K tile");

    __shared__ __attribute__((aligned(16))) float Ks[KT * KS];
    __shared__ __attribute__((aligned(16))) float Vs[KT * KS];
    __shared__ __attribute__((aligned(16))) float qs[RMAX * D];
    __shared__ float sc[RMAX * KT];
    __shared__ float m_run[RMAX], l_run[RMAX], alph[RMAX];

    const int head = blockIdx.x / p.n_chunks;
    const int split = blockIdx.x % p.n_chunks;
    const int bi = head / p.Hkv, kvh = head % p.Hkv;
    const int L = p.lens ? p.lens[bi] : p.tk;
    const int key_begin = split * keys_per_split;
    if (key_begin >= L) return;
    const int key_end = min(L, key_begin + keys_per_split);
    const int n_splits = (L + keys_per_split - 1) / keys_per_split;
    const int n_tiles = (key_end - key_begin + KT - 1) / KT;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // Query rows -> LDS, pre-scaled by scale*log2(e).
    for (int e = tid; e < RMAX * D; e += 256) {
        const int rr = e / D, dd = e % D;
        float x = 0.f;
        if (rr < p.R && dd < p.d) {
            const int hq = kvh * p.G + rr / p.Tq, t = rr % p.Tq;
            x = p.q.p[bi * p.q.sb + hq * p.q.sh + t * p.q.st + dd] * p.qscale;
        }
        qs[e] = x;
    }
    if (tid < RMAX) { m_run[tid] = kNegInf; l_run[tid] = 0.f; }

    const float* kb = p.k + bi * p.ksb + kvh * p.ksh;
    const float* vb = p.v + bi * p.vsb + kvh * p.vsh;

    // Tile loads: float4 index tid + 256*i -> (row, col4).
    float4 kr[NV], vr[NV];
    auto load_tile = [&](int key0) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int idx = tid + 256 * i;
            const int row = idx / C4, c = (idx % C4) * 4;
            const int key = key0 + row;
            const bool ok = key < key_end && c < p.d;
            kr[i] = ok ? *reinterpret_cast<const float4*>(kb + key * p.kst + c)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
            vr[i] = ok ? *reinterpret_cast<const float4*>(vb + key * p.vst + c)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };

    const int c4 = tid % C4, kg = tid / C4;   // P V layout
    float4 o[RMAX];
#pragma unroll
    for (int rr = 0; rr < RMAX; ++rr) o[rr] = make_float4(0.f, 0.f, 0.f, 0.f);

    load_tile(key_begin);
    for (int it = 0; it < n_tiles; ++it) {
        const int key0 = key_begin + it * KT;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int idx = tid + 256 * i;
            const int row = idx / C4, c = (idx % C4) * 4;
            *reinterpret_cast<float4*>(Ks + row * KS + c) = kr[i];
            *reinterpret_cast<float4*>(Vs + row * KS + c) = vr[i];
        }
        __syncthreads();
        if (it + 1 < n_tiles) load_tile(key0 + KT);

        // Scores: thread -> key kk, rows wave + 4j.
        {
            const int kk = tid % KT;
            const int rg = tid / KT;
            float acc[RMAX / 4];
#pragma unroll
            for (int j = 0; j < RMAX / 4; ++j) acc[j] = 0.f;
            const float* krow = Ks + kk * KS;
#pragma unroll 8
            for (int c = 0; c < D; c += 4) {
                const float4 kv = *reinterpret_cast<const float4*>(krow + c);
#pragma unroll
                for (int j = 0; j < RMAX / 4; ++j) {
                    const float4 qv = *reinterpret_cast<const float4*>(qs + (rg + 4 * j) * D + c);
                    acc[j] += kv.x * qv.x + kv.y * qv.y + kv.z * qv.z + kv.w * qv.w;
                }
            }
            const bool kvis = key0 + kk < key_end;
#pragma unroll
            for (int j = 0; j < RMAX / 4; ++j) {
                const int rr = rg + 4 * j;
                if (rr < p.R) sc[rr * KT + kk] = kvis ? acc[j] : kNegInf;
            }
        }
        __syncthreads();

        // Online softmax, one wave per row (64 keys = 64 lanes).
        for (int rr = wave; rr < p.R; rr += 4) {
            const float x = sc[rr * KT + lane];
            const float mt = wave_max(x);
            const float m_old = m_run[rr];
            const float m_new = fmaxf(m_old, mt);
            const float m_use = (m_new == kNegInf) ? 0.f : m_new;
            const float pv = fast_exp2(x - m_use);
            sc[rr * KT + lane] = pv;
            const float ls = wave_sum(pv);
            if (lane == 0) {
                const float alpha = fast_exp2(m_old - m_use);
                alph[rr] = alpha;
                l_run[rr] = alpha * l_run[rr] + ls;
                m_run[rr] = m_new;
            }
        }
        __syncthreads();

        // O += P V for this thread's 4 dims over its key group.
#pragma unroll
        for (int rr = 0; rr < RMAX; ++rr) {
            if (rr < p.R) {
                const float a = alph[rr];
                o[rr].x *= a; o[rr].y *= a; o[rr].z *= a; o[rr].w *= a;
            }
        }
#pragma unroll
        for (int i = 0; i < KPG; ++i) {
            const int key = kg + NG * i;
            const float4 v4 = *reinterpret_cast<const float4*>(Vs + key * KS + 4 * c4);
#pragma unroll
            for (int rr = 0; rr < RMAX; ++rr) {
                if (rr < p.R) {
                    const float pv = sc[rr * KT + key];
                    o[rr].x += pv * v4.x; o[rr].y += pv * v4.y;
                    o[rr].z += pv * v4.z; o[rr].w += pv * v4.w;
                }
            }
        }
        __syncthreads();
    }

    // Reduce O over key groups: first inside the wave (lanes differing in the
    // bits above log2(C4)), then across the 4 waves through LDS.
#pragma unroll
    for (int off = C4; off < 64; off <<= 1) {
#pragma unroll
        for (int rr = 0; rr < RMAX; ++rr) {
            o[rr].x += __shfl_xor(o[rr].x, off);
            o[rr].y += __shfl_xor(o[rr].y, off);
            o[rr].z += __shfl_xor(o[rr].z, off);
            o[rr].w += __shfl_xor(o[rr].w, off);
        }
    }
    float* red = Ks;   // [4 waves][RMAX][D]
    if (lane < C4) {
#pragma unroll
        for (int rr = 0; rr < RMAX; ++rr)
            *reinterpret_cast<float4*>(red + (wave * RMAX + rr) * D + 4 * c4) = o[rr];
    }
    __syncthreads();

    const bool direct = n_splits == 1;
    for (int e = tid; e < p.R * D; e += 256) {
        const int rr = e / D, dd = e % D;
        const float acc = red[(0 * RMAX + rr) * D + dd] + red[(1 * RMAX + rr) * D + dd] +
                          red[(2 * RMAX + rr) * D + dd] + red[(3 * RMAX + rr) * D + dd];
        if (direct) {
            if (dd < p.d) {
                const int hq = kvh * p.G + rr / p.Tq, t = rr % p.Tq;
                const float l = l_run[rr];
                p.o.p[bi * p.o.sb + hq * p.o.sh + t * p.o.st + dd] = l > 0.f ? acc / l : 0.f;
            }
        } else {
            p.ws_o[((int64_t)(head * p.n_chunks + split) * p.R + rr) * D + dd] = acc;
        }
    }
    if (!direct && tid < p.R) {
        float* ml = p.ws_ml + ((int64_t)(head * p.n_chunks + split) * p.R + tid) * 2;
        ml[0] = m_run[tid];
        ml[1] = l_run[tid];
    }
}

// Merges the per-split partials of one (sequence, KV head, row).
template <int D>
__global__ __launch_bounds__(64) void splitk_combine_kernel(const SplitKParams p, int keys_per_split) {
    const int item = blockIdx.x;             // (head, rr)
    const int head = item / p.R, rr = item % p.R;
    const int bi = head / p.Hkv, kvh = head % p.Hkv;
    const int L = p.lens ? p.lens[bi] : p.tk;
    const int n = (L + keys_per_split - 1) / keys_per_split;
    if (n == 1) return;                      // written directly by the split kernel
    const int hq = kvh * p.G + rr / p.Tq, t = rr % p.Tq;
    float* op = p.o.p + bi * p.o.sb + hq * p.o.sh + t * p.o.st;
    if (n == 0) {                            // empty sequence: output stays zero
        for (int dd = threadIdx.x; dd < p.d; dd += 64) op[dd] = 0.f;
        return;
    }
    const float* ml = p.ws_ml + ((int64_t)head * p.n_chunks * p.R + rr) * 2;
    float M = kNegInf;
    for (int c = 0; c < n; ++c) M = fmaxf(M, ml[(int64_t)c * p.R * 2]);
    const float M_use = M == kNegInf ? 0.f : M;
    float den = 0.f;
    for (int c = 0; c < n; ++c)
        den += fast_exp2(ml[(int64_t)c * p.R * 2] - M_use) * ml[(int64_t)c * p.R * 2 + 1];
    const float inv = den > 0.f ? 1.f / den : 0.f;
    const float* wo = p.ws_o + ((int64_t)head * p.n_chunks * p.R + rr) * D;
    for (int dd = threadIdx.x; dd < p.d; dd += 64) {
        float acc = 0.f;
        for (int c = 0; c < n; ++c)
            acc += fast_exp2(ml[(int64_t)c * p.R * 2] - M_use) * wo[(int64_t)c * p.R * D + dd];
        op[dd] = acc * inv;
    }
}

template <int D, int RMAX>
hipError_t launch_splitk_t(const SplitKParams& p, int keys_per_split, hipStream_t stream) {
    const int grid = p.B * p.Hkv * p.n_chunks;
    if (grid > 0)
        hipLaunchKernelGGL((splitk_kernel<D, RMAX>), dim3(grid), dim3(256), 0, stream, p,
                           keys_per_split);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int cgrid = p.B * p.Hkv * p.R;
    if (cgrid > 0)
        hipLaunchKernelGGL((splitk_combine_kernel<D>), dim3(cgrid), dim3(64), 0, stream, p,
                           keys_per_split);
    return hipGetLastError();
}

template <int D>
hipError_t launch_splitk_d(const SplitKParams& p, int kps, hipStream_t stream) {
    if (p.R <= 4) return launch_splitk_t<D, 4>(p, kps, stream);
    if (p.R <= 8) return launch_splitk_t<D, 8>(p, kps, stream);
    return launch_splitk_t<D, 16>(p, kps, stream);
}

// ---- KV append --------------------------------------------------------------

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
        const int64_t dst = (((int64_t)b * Hkv + h) * cap + lens[b] + t) * d + dd;
        kc[dst] = kn.p[b * kn.sb + h * kn.sh + t * kn.st + dd * kn.sd];
        vc[dst] = vn.p[b * vn.sb + h * vn.sh + t * vn.st + dd * vn.sd];
    }
}

__global__ void lens_bump_kernel(int32_t* lens, int B, int t_new) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) lens[b] += t_new;
}

}  // namespace

int splitk_padded_dim(int d) {
    if (d <= 32) return 32;
    if (d <= 64) return 64;
    if (d <= 128) return 128;
    return 0;
}

int splitk_max_rows() { return 16; }

int splitk_keys_per_split(int max_len, int n_heads) {
    // Enough splits to give each of the 256 CUs several workgroups, in whole
    // 64-key tiles; at least 4 tiles per split so partials stay a small
    // fraction of the K/V bytes.
    int tiles = (max_len + KT - 1) / KT;
    int want_splits = (4 * 256 + n_heads - 1) / (n_heads > 0 ? n_heads : 1);
    int tps = (tiles + want_splits - 1) / (want_splits > 0 ? want_splits : 1);
    if (tps < 4) tps = 4;
    return tps * KT;
}

uint64_t splitk_workspace_bytes(int B, int Hkv, int R, int d, int max_len, int keys_per_split) {
    const int D = splitk_padded_dim(d);
    const int n_chunks = (max_len + keys_per_split - 1) / keys_per_split;
    return (uint64_t)B * Hkv * (n_chunks > 0 ? n_chunks : 1) * R * (D + 2) * sizeof(float);
}

hipError_t launch_splitk(SplitKParams p, int max_len, int keys_per_split, void* workspace,
                         hipStream_t stream) {
    p.G = p.Hq / p.Hkv;
    p.R = p.G * p.Tq;
    p.n_chunks = (max_len + keys_per_split - 1) / keys_per_split;
    if (p.n_chunks < 1) p.n_chunks = 1;
    const int D = splitk_padded_dim(p.d);
    p.ws_o = static_cast<float*>(workspace);
    p.ws_ml = p.ws_o + (int64_t)p.B * p.Hkv * p.n_chunks * p.R * D;
    switch (D) {
        case 32: return launch_splitk_d<32>(p, keys_per_split, stream);
        case 64: return launch_splitk_d<64>(p, keys_per_split, stream);
        case 128: return launch_splitk_d<128>(p, keys_per_split, stream);
        default: return hipErrorInvalidValue;
    }
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
