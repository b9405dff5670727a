// Decode prologue: the q/k/v projections of a decode step with bias and
// rotary position embedding fused into one launch, and RoPE on strided views.
//
// Reference: GroupedQueryAttention::forward_gqa_cached, steps 1-2
// (src/models/llama.rs:226-235): q = x Wq^T, k = x Wk^T, v = x Wv^T
// (Linear::forward, src/nn/linear.rs:47-57, bias added after the product),
// split into heads, then RotaryEmbedding::apply (llama.rs:110-157) on q and k
// at positions start_pos + t with the tables of RotaryEmbedding::new
// (llama.rs:74-107).
//
// MI355X mapping of the fused projection.  A decode step multiplies M = B
// rows (a few to a few dozen) by N = (Hq + 2 Hkv) d weight rows of length C
// (100 MB at LLaMA-7B shapes), so the launch is bound by streaming the
// weights once, with fp32 MFMA keeping the arithmetic (16 FLOP per weight
// byte at M = 32) under that stream:
//   * The weights are packed once (qkv_pack_kernel) into the order the
//     kernel's lanes consume them: every load instruction reads 1 KB of
//     contiguous memory and a workgroup's slice is one contiguous run.
//   * A tile is 64 output columns of one head: 32 RoPE pairs (dims
//     32u .. 32u+31 and their partners d/2 + 32u ..), so rotation happens
//     inside the tile.  Its 4 waves own 16 columns each and run
//     v_mfma_f32_16x16x4_f32 with the weight rows as A and up to 64 x rows
//     (MT tiles of 16) as B.
//   * The reduction dim C is split into S slices (one workgroup per (tile,
//     slice)) so the launch fills the GPU.  x is staged per 64-wide chunk in
//     LDS (double-buffered, one barrier per chunk) and shared by the 4 waves;
//     the next chunk's weights and x are loaded while a chunk computes.
//   * Slices write partial tiles with coherent stores; the last workgroup of
//     a tile (arrival counter) adds them in slice order, adds the bias,
//     rotates q/k with the reference's roundings and writes the rows to
//     [B, H, 1, d] outputs (the q, k_new and v_new of the decode step).
#include <algorithm>
#include <cmath>
#include <type_traits>

#include "nne_common.hpp"
#include "nne_launch.hpp"

namespace nne {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int QKV_KC = 64;           // k per chunk
constexpr int QKV_MAX_MT = 4;        // x rows per launch: 16 * QKV_MAX_MT
constexpr int QKV_XS = QKV_KC + 4;   // LDS row stride of an x chunk (16-byte reads conflict-free)
constexpr int QKV_MAX_S = 8;         // slices of C per tile

// x * cos + rot * sin with each product and the sum rounded to f32, as the
// reference's three tensor ops round them (llama.rs:154-156).
__device__ __forceinline__ float rope_rotate(float x, float c, float rot, float s) {
#pragma clang fp contract(off)
    const float term1 = x * c;
    const float term2 = rot * s;
    return term1 + term2;
}

// Column tr (0..63) of tile u of a head: the pair-first dims 32u .. 32u+31,
// then their partners d/2 + 32u .. d/2 + 32u + 31.
__device__ __forceinline__ int tile_dim(int tr, int u, int half) {
    return tr < 32 ? 32 * u + tr : half + 32 * u + (tr - 32);
}

// Packed weights: float4 number ((((t * n_chunks + j) * 4 + w) * 4 + i) * 64 + l)
// holds the weight row of tile t's column 16 w + (l % 16) at
// k = 64 j + 4 (l / 16) + 16 i .. + 3 -- the A operand of lane l for chunk j,
// load i of wave w.
__global__ void qkv_pack_kernel(const float* wq, const float* wk, const float* wv, float* packed,
                                int C, int Hq, int Hkv, int d) {
    const int n_chunks = C / QKV_KC;
    const int tiles_per_head = d / 64, half = d / 2;
    const int64_t n4 = (int64_t)(Hq + 2 * Hkv) * d * C / 4;
    for (int64_t f = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; f < n4;
         f += (int64_t)gridDim.x * blockDim.x) {
        const int l = f % 64;
        int64_t rest = f / 64;
        const int i = rest % 4; rest /= 4;
        const int w = rest % 4; rest /= 4;
        const int j = rest % n_chunks;
        const int t = rest / n_chunks;
        const int hh = t / tiles_per_head, u = t % tiles_per_head;
        const int dim = tile_dim(16 * w + (l & 15), u, half);
        const float* src;
        if (hh < Hq) src = wq + (int64_t)(hh * d + dim) * C;
        else if (hh < Hq + Hkv) src = wk + (int64_t)((hh - Hq) * d + dim) * C;
        else src = wv + (int64_t)((hh - Hq - Hkv) * d + dim) * C;
        const int k = QKV_KC * j + 4 * (l >> 4) + 16 * i;
        *reinterpret_cast<vf4*>(packed + 4 * f) = *reinterpret_cast<const vf4*>(src + k);
    }
}

template <int MT>
__global__ __launch_bounds__(256, 2) void qkv_rope_kernel(const QkvParams p) {
    __shared__ __attribute__((aligned(16))) float xs[2][16 * MT][QKV_XS];   // x chunk [row][k]
    __shared__ float fin[64][65];                                          // tile [column][row]
    __shared__ int is_last;

    warm_kernargs<0, sizeof(QkvParams)>();   // every argument's line in one round trip
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, q4 = lane >> 4;
    const int tile = blockIdx.x / p.S, slice = blockIdx.x % p.S;
    const int n_chunks = p.C / QKV_KC;
    const int j0 = slice * p.kc_per_slice;
    const int j1 = min(n_chunks, j0 + p.kc_per_slice);
    const int nj = j1 - j0;

    // The tile belongs to one head of q, k or v.  Thread tid finishes column
    // tid % 64 of rows tid / 64 + 4 k if its workgroup adds the tile up; the
    // positions and biases it needs are loaded behind the first chunks, off
    // the launch's tail.
    const int tiles_per_head = p.d / 64, half = p.d / 2;
    const int hh = tile / tiles_per_head, u = tile % tiles_per_head;
    const int which = hh < p.Hq ? 0 : (hh < p.Hq + p.Hkv ? 1 : 2);
    const int head = which == 0 ? hh : (which == 1 ? hh - p.Hq : hh - p.Hq - p.Hkv);
    const float* bias = p.bias[which];
    const int ocol = tid & 63, orow = tid >> 6;
    const int dim = tile_dim(ocol, u, half);
    const int pcol = ocol ^ 32;   // columns c and c ^ 32 hold dims i and i + d/2 of one pair
    const bool rotate = which < 2 && p.cos;
    float b_own = 0.f, b_partner = 0.f;
    constexpr int ROWS = 4 * MT;   // rows per thread
    int pos[ROWS];

    // The workgroup's packed weights, 16 KB per chunk (4 KB per wave, 1 KB per
    // load instruction), read through a buffer range that ends with its slice:
    // the pipeline's loads past the last chunk return zeros without a memory
    // access.  (As clamped re-reads of the last chunk they fetched 32 KB per
    // workgroup from HBM again -- non-temporal lines are gone from L2 by then
    // -- 15 MB, 15 % of a config-3 launch.)
    const __amdgpu_buffer_rsrc_t wrange = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(p.wp) + (int64_t)(tile * n_chunks + j0) * 4096, 0,
        (uint32_t)max(nj, 0) * 16384u, 0x00020000);
    const uint32_t wlane = (uint32_t)(wave * 256 + lane) * 16;
    // x chunk staging: thread tid moves float4 number tid + 256 q of the
    // 16 MT rows x 16 float4 chunk (rows past M repeat row M - 1; their output
    // columns are never stored).
    auto load_x = [&](vf4 (&xr)[MT], int j) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < MT; ++q) {
            const int f = tid + 256 * q;
            const int m = min(f >> 4, p.M - 1);
            xr[q] = *reinterpret_cast<const vf4*>(p.x + (int64_t)m * p.x_rs + QKV_KC * j + 4 * (f & 15));
        }
    };
    auto store_x = [&](const vf4 (&xr)[MT], int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < MT; ++q) {
            const int f = tid + 256 * q;
            *reinterpret_cast<vf4*>(&xs[buf][f >> 4][4 * (f & 15)]) = xr[q];
        }
    };
    auto load_w = [&](vf4 (&w)[4], int jj) __attribute__((always_inline)) {   // non-temporal
#pragma unroll
        for (int i = 0; i < 4; ++i)
            w[i] = __builtin_bit_cast(vf4, __builtin_amdgcn_raw_buffer_load_b128(
                                               wrange, wlane + (uint32_t)(jj * 1024 + 64 * i) * 16, 0, 2));
    };

    floatx4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](const vf4 (&w)[4], int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vf4 xv[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t)
                xv[t] = *reinterpret_cast<const vf4*>(&xs[buf][16 * t + r][4 * q4 + 16 * i]);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[i][c], xv[t][c], acc[t], 0, 0, 0);
        }
    };

    // Chunk pipeline: step j computes chunk j (weights in register buffer
    // j % 3, x in LDS buffer j % 2) while the weights of chunk j + 2 and the x
    // of chunk j + 3 are loaded into registers and chunk j + 1's x (loaded
    // two steps earlier) is moved into LDS; one barrier per step, so neither
    // the HBM weight stream nor the L2 reads of x wait at a barrier.  Weight
    // loads past the last chunk read zeros (above) and x loads reread the last
    // chunk (an L2 hit); neither is used.  Unrolled by 6 so every buffer index
    // is a compile-time constant.
    vf4 wbuf[3][4], xr[3][MT];
    auto cl = [&](int jj) { return min(jj, nj - 1); };
    if (nj > 0) {
        load_x(xr[0], j0);
        load_w(wbuf[0], 0);
        load_w(wbuf[1], 1);
        load_x(xr[1], j0 + cl(1));
        load_x(xr[2], j0 + cl(2));
        store_x(xr[0], 0);
    }
#pragma unroll
    for (int k = 0; k < ROWS; ++k) pos[k] = rotate && orow + 4 * k < p.M ? p.pos[orow + 4 * k] : 0;
    if (bias) {
        b_own = bias[head * p.d + dim];
        b_partner = bias[head * p.d + tile_dim(pcol, u, half)];
    }
    __syncthreads();
    auto step = [&](int jj, auto ji) __attribute__((always_inline)) {
        constexpr int J = decltype(ji)::value;   // jj % 6
        load_w(wbuf[(J + 2) % 3], jj + 2);
        load_x(xr[J % 3], j0 + cl(jj + 3));
        __builtin_amdgcn_sched_barrier(0);
        // Raised wave priority over the MFMAs: the other workgroup on the CU
        // issues its loads and LDS traffic under them (at most ~1 % on MI355X:
        // B = 32 25.2 -> 25.0 us in one A/B, level in another).
        __builtin_amdgcn_s_setprio(1);
        compute(wbuf[J % 3], J % 2);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
        store_x(xr[(J + 1) % 3], (J + 1) % 2);
        __syncthreads();
    };
    for (int jj = 0; jj < nj; jj += 6) {
        step(jj, std::integral_constant<int, 0>{});
        if (jj + 1 >= nj) break;
        step(jj + 1, std::integral_constant<int, 1>{});
        if (jj + 2 >= nj) break;
        step(jj + 2, std::integral_constant<int, 2>{});
        if (jj + 3 >= nj) break;
        step(jj + 3, std::integral_constant<int, 3>{});
        if (jj + 4 >= nj) break;
        step(jj + 4, std::integral_constant<int, 4>{});
        if (jj + 5 >= nj) break;
        step(jj + 5, std::integral_constant<int, 5>{});
    }

    // acc[t][rr] = partial y[tile column 16 wave + 4 q4 + rr][x row 16 t + r].
    const int col0 = 16 * wave + 4 * q4;
    if (p.S > 1) {
        float* part = p.ws + ((int64_t)tile * p.S + slice) * 64 * 64;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) store_coherent(part + (col0 + rr) * 64 + 16 * t + r, acc[t][rr]);
        wait_stores_performed();
        __syncthreads();
        if (tid == 0) {
            const unsigned old = __hip_atomic_fetch_add(p.cnt + tile, 1u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            is_last = old == (unsigned)(p.S - 1);
        }
        __syncthreads();
        if (!is_last) return;
    }

    // RoPE table entries of this thread's outputs, loaded before the partial
    // tiles so both round trips overlap.
    float* out = p.out[which];
    const int64_t osb = p.o_sb[which], osh = p.o_sh[which];
    float cs[ROWS], sn[ROWS];
    if (rotate) {
#pragma unroll
        for (int k = 0; k < ROWS; ++k) {
            if (orow + 4 * k < p.M) {
                const int64_t tb = (int64_t)pos[k] * p.d + dim;
                cs[k] = p.cos[tb];
                sn[k] = p.sin[tb];
            }
        }
    }

    if (p.S > 1) {
        // Last slice of the tile: add the partials in slice order.  A thread
        // adds 4 rows of a column with 16-byte loads, every slice's loads of a
        // round issued before the first add.
        const float* base = p.ws + (int64_t)tile * p.S * 64 * 64;
        const __amdgpu_buffer_rsrc_t range = coherent_range(base, (uint32_t)p.S * 64 * 64 * 4);
        const int rg = (p.M + 3) >> 2, n_g = 64 * rg;
        for (int g0 = 0; g0 < n_g; g0 += 2 * 256) {
            vf4 v[2][QKV_MAX_S];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int g = g0 + tid + 256 * q;
                const int col = g / rg, rq = g % rg;
#pragma unroll
                for (int sl = 0; sl < QKV_MAX_S; ++sl)
                    v[q][sl] = (g < n_g && sl < p.S)
                                   ? load_coherent4(range, (uint32_t)(((sl * 64 + col) * 64 + 4 * rq) * 4))
                                   : vf4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int g = g0 + tid + 256 * q;
                if (g >= n_g) continue;
                vf4 sum = v[q][0];
#pragma unroll
                for (int sl = 1; sl < QKV_MAX_S; ++sl)
                    if (sl < p.S) sum = sum + v[q][sl];
                const int col = g / rg, rq = g % rg;
#pragma unroll
                for (int i = 0; i < 4; ++i) fin[col][4 * rq + i] = sum[i];
            }
        }
        if (tid == 0)
            __hip_atomic_store(p.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) fin[col0 + rr][16 * t + r] = acc[t][rr];
    }
    __syncthreads();

    // Bias, RoPE (rotate_half(x) = [-x2, x1], llama.rs:149-152), store.
#pragma unroll
    for (int k = 0; k < ROWS; ++k) {
        const int m = orow + 4 * k;
        if (m >= p.M) break;
        float val = fin[ocol][m];
        if (bias) val = val + b_own;
        if (rotate) {
            float partner = fin[pcol][m];
            if (bias) partner = partner + b_partner;
            const float rot = ocol < 32 ? -partner : partner;
            val = rope_rotate(val, cs[k], rot, sn[k]);
        }
        out[m * osb + head * osh + dim] = val;
    }
}

// RotaryEmbedding::apply on a strided [B, H, T, d] view: one thread per
// (i, i + d/2) pair; row t of sequence b takes table row pos[b] + t.  Reads
// both elements before writing, so out may alias x with the same strides.
__global__ void rope_apply_kernel(View4 x, OutView4 o, int B, int H, int T, int d,
                                  const float* cos_t, const float* sin_t, const int32_t* pos) {
    const int half = d / 2;
    const int64_t n = (int64_t)B * H * T * half;
    for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < n;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int i = e % half;
        int64_t rest = e / half;
        const int t = rest % T; rest /= T;
        const int h = rest % H;
        const int b = rest / H;
        const float* xr = x.p + b * x.sb + h * x.sh + t * x.st;
        float* orow = o.p + b * o.sb + h * o.sh + t * o.st;
        const float x1 = xr[i * x.sd], x2 = xr[(i + half) * x.sd];
        const int64_t tb = ((int64_t)pos[b] + t) * d;
        const float y1 = rope_rotate(x1, cos_t[tb + i], -x2, sin_t[tb + i]);
        const float y2 = rope_rotate(x2, cos_t[tb + i + half], x1, sin_t[tb + i + half]);
        orow[i * o.sd] = y1;
        orow[(i + half) * o.sd] = y2;
    }
}

template <int MT>
hipError_t launch_qkv_mt(const QkvParams& p, hipStream_t stream) {
    hipLaunchKernelGGL(qkv_rope_kernel<MT>, dim3(p.n_tiles * p.S), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace

void rope_tables_host(float* cos_out, float* sin_out, int64_t max_seq_len, int64_t d, float theta) {
    // RotaryEmbedding::new (llama.rs:74-107), in f32 like the reference.
    const int64_t half = d / 2;
    for (int64_t i = 0; i < half; ++i) {
        const float exponent = (float)(2 * i) / (float)d;
        const float inv_freq = 1.0f / powf(theta, exponent);
        for (int64_t pos = 0; pos < max_seq_len; ++pos) {
            const float freq = (float)pos * inv_freq;
            const float c = cosf(freq), s = sinf(freq);
            cos_out[pos * d + i] = c;
            cos_out[pos * d + i + half] = c;
            sin_out[pos * d + i] = s;
            sin_out[pos * d + i + half] = s;
        }
    }
}

int qkv_max_rows_per_launch() { return 16 * QKV_MAX_MT; }

uint64_t qkv_packed_floats(int C, int Hq, int Hkv, int d) {
    return (uint64_t)(Hq + 2 * Hkv) * d * C;
}

hipError_t launch_qkv_pack(const float* wq, const float* wk, const float* wv, float* packed, int C,
                           int Hq, int Hkv, int d, hipStream_t stream) {
    const int64_t n4 = (int64_t)qkv_packed_floats(C, Hq, Hkv, d) / 4;
    if (n4 <= 0) return hipSuccess;
    int64_t blocks = (n4 + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(qkv_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, wq, wk, wv,
                       packed, C, Hq, Hkv, d);
    return hipGetLastError();
}

QkvWorkspace qkv_workspace(int C, int Hq, int Hkv, int d, int cus) {
    // K slices: enough workgroups for about two per CU, each slice at least 2
    // chunks long (GPT-2-small's d_model 768, 12 chunks: 6 slices, 8.8 -> 8.3 us
    // at B = 32 against 3 slices of 4).
    QkvWorkspace w;
    w.n_tiles = (Hq + 2 * Hkv) * d / 64;
    const int n_chunks = C / QKV_KC;
    int S = std::max(1, (2 * cus + w.n_tiles / 2) / std::max(w.n_tiles, 1));
    S = std::max(1, std::min(std::min(S, QKV_MAX_S), n_chunks / 2));
    w.kc_per_slice = (n_chunks + S - 1) / S;
    w.S = (n_chunks + w.kc_per_slice - 1) / w.kc_per_slice;
    w.floats = w.S > 1 ? (uint64_t)w.n_tiles * w.S * 64 * 64 : 0;
    return w;
}

hipError_t launch_qkv_rope(QkvParams p, hipStream_t stream) {
    // Rows beyond 64 go in further launches of up to 64 rows each.
    const int M = p.M;
    for (int m0 = 0; m0 < M; m0 += 16 * QKV_MAX_MT) {
        QkvParams q = p;
        q.M = std::min(16 * QKV_MAX_MT, M - m0);
        q.x = p.x + (int64_t)m0 * p.x_rs;
        q.pos = p.pos ? p.pos + m0 : nullptr;
        for (int j = 0; j < 3; ++j) q.out[j] = p.out[j] + (int64_t)m0 * p.o_sb[j];
        const int mt = (q.M + 15) / 16;
        hipError_t e = mt == 1 ? launch_qkv_mt<1>(q, stream)
                     : mt == 2 ? launch_qkv_mt<2>(q, stream)
                               : launch_qkv_mt<4>(q, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_rope_apply(View4 x, OutView4 o, int B, int H, int T, int d, const float* cos_t,
                             const float* sin_t, const int32_t* pos, hipStream_t stream) {
    const int64_t n = (int64_t)B * H * T * (d / 2);
    if (n <= 0) return hipSuccess;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(rope_apply_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, o, B, H,
                       T, d, cos_t, sin_t, pos);
    return hipGetLastError();
}

}  // namespace nne
