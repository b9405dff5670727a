/*
 * rayon_path.c -- timing restatement of the reference engine's CPU path for
 * standard (non-flash) attention, as the reference runs it on x86_64 with
 * AVX2 + FMA: the batched GEMM / GEMV kernels of src/tensor/matmul.rs, the
 * fused row softmax of src/tensor/reduce.rs, the repeat-KV broadcast of
 * src/models/llama.rs, the additive causal mask, the strided gathers of
 * `to_contiguous` and the per-step `Tensor::cat` of the KV cache.
 *
 * TEST INFRASTRUCTURE ONLY.  bench.py's cpu_baseline legs time it beside the
 * GPU; tests/test_rayon_path.py checks its outputs against oracle.c (the
 * parity oracle) within the parity bar.  The product library never links,
 * loads or calls it.
 *
 * oracle.c restates the reference's arithmetic in a fixed order and is what
 * parity is pinned on.  This file restates the reference's *cost structure*
 * for the same computation: which buffers it materialises, which loops are
 * AVX2 / FMA and how they tile, which loops are element by element with a
 * heap-allocated index vector per element, and how Rayon splits the work.
 * Its sums run in the reference's order (8-lane FMA partial sums, the same
 * horizontal reductions), so it differs from oracle.c by rounding only.
 *
 * Rayon -> OpenMP.  The reference nests `par_chunks_mut` loops: the batched
 * matmul (matmul.rs:1167-1215, :1278-1314) splits the output over its B*H
 * matrices and each matrix's GEMM splits it again over row or column chunks
 * (matmul.rs:95-97, :360-361, :750-751, :891-893).  Rayon's work stealing
 * lets idle threads take inner chunks; here every (matrix, inner chunk) pair
 * is one item of a single dynamically scheduled loop, with the reference's
 * chunk sizes.  Elementwise `par_iter_mut` loops become static OpenMP loops.
 * Serial reference loops (Tensor::cat, to_contiguous, the mask build,
 * Storage::zeros) stay serial.
 *
 * Built with -O3 -mavx2 -mfma -ffp-contract=off (oracle/Makefile): the
 * reference's kernels are AVX2/FMA intrinsics (`#[target_feature(enable =
 * "avx2,fma")]`), and Rust never contracts a*b+c into an FMA by itself.  The
 * reference builds with target-cpu=native (.cargo/config.toml:1-2), which may
 * let LLVM use wider vectors in its plain loops (the mul_scalar pass, the
 * softmax exp loop is scalar either way: `f32::exp` is a libm call).
 */
#define _POSIX_C_SOURCE 199309L
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ---------------------------------------------------------------------- */
/* Strided views (src/tensor/mod.rs:20-27; shape.rs:6-31, 80-145)          */
/* ---------------------------------------------------------------------- */

#define RP_MAXD 6

typedef struct {
    const float *p;
    int nd;
    size_t sh[RP_MAXD];
    size_t st[RP_MAXD];
    size_t off;
} view_t;

static size_t v_numel(const view_t *v) {
    size_t n = 1;
    for (int i = 0; i < v->nd; ++i) n *= v->sh[i];
    return n;
}

static void c_strides(const size_t *sh, int nd, size_t *st) {
    size_t s = 1;
    for (int i = nd - 1; i >= 0; --i) {
        st[i] = s;
        s *= sh[i];
    }
}

/* RawTensor::is_contiguous (mod.rs:179-181, shape.rs:20-31): offset 0 and
 * C strides on every dimension longer than 1. */
static int v_contig(const view_t *v) {
    size_t ex[RP_MAXD];
    if (v->off != 0) return 0;
    c_strides(v->sh, v->nd, ex);
    for (int i = 0; i < v->nd; ++i)
        if (v->sh[i] > 1 && v->st[i] != ex[i]) return 0;
    return 1;
}

static view_t v_contig_view(const float *p, int nd, const size_t *sh) {
    view_t v;
    memset(&v, 0, sizeof v);
    v.p = p;
    v.nd = nd;
    for (int i = 0; i < nd; ++i) v.sh[i] = sh[i];
    c_strides(v.sh, nd, v.st);
    return v;
}

/* shape.rs:124-135 */
static void flat_to_multi(size_t flat, const size_t *sh, int nd, size_t *multi) {
    size_t rem = flat;
    for (int i = nd - 1; i >= 0; --i) {
        if (sh[i] == 0) {
            multi[i] = 0;
        } else {
            multi[i] = rem % sh[i];
            rem /= sh[i];
        }
    }
}

/* shape.rs:139-145 */
static size_t multi_to_off(const size_t *multi, const size_t *st, int nd, size_t base) {
    size_t off = base;
    for (int i = 0; i < nd; ++i) off += multi[i] * st[i];
    return off;
}

/* `vec![0; ndim]` for the per-element index vector the reference allocates
 * (mod.rs:302, ops.rs:31, 72, 263): a zeroed heap allocation freed at the end
 * of the element.  Kept on purpose: it is part of what those loops cost. */
static size_t *index_vec(int nd) { return (size_t *)calloc((size_t)(nd > 0 ? nd : 1), sizeof(size_t)); }

static float *alloc_f32(size_t n) { return (float *)malloc((n ? n : 1) * sizeof(float)); }

/* `vec![0.0; n]`: the zero-initialised output buffers of the ops. */
static float *zeros_f32(size_t n) { return (float *)calloc(n ? n : 1, sizeof(float)); }

/* RawTensor::to_contiguous (mod.rs:184-197): the same storage when already
 * contiguous, else a serial gather through get_by_flat_index (mod.rs:301-306),
 * one index vector per element.  *copied says whether a buffer was made. */
static float *to_contiguous(const view_t *v, int *copied) {
    if (v_contig(v)) {
        *copied = 0;
        return (float *)v->p;
    }
    size_t n = v_numel(v);
    float *out = alloc_f32(n);
    for (size_t i = 0; i < n; ++i) {
        size_t *multi = index_vec(v->nd);
        flat_to_multi(i, v->sh, v->nd, multi);
        out[i] = v->p[multi_to_off(multi, v->st, v->nd, v->off)];
        free(multi);
    }
    *copied = 1;
    return out;
}

/* broadcast_shapes + broadcast_strides (shape.rs:45-120): align right; a
 * dimension of length 1 gets stride 0. */
static void bcast_strides(const view_t *v, int nd_out, const size_t *sh_out, size_t *st) {
    int lead = nd_out - v->nd;
    for (int i = 0; i < nd_out; ++i) {
        if (i < lead) {
            st[i] = 0;
        } else {
            size_t d = v->sh[i - lead];
            st[i] = (d == 1 && sh_out[i] != 1) ? 0 : v->st[i - lead];
        }
    }
}

enum { OP_ADD = 0, OP_MUL = 1 };

/* RawTensor::binary_op (ops.rs:43-84).  Fast path: equal shapes, both
 * contiguous, one parallel pass.  Otherwise the general path: per output
 * element (in parallel) an index vector, the multi-index, two offsets. */
static float *binary_op(const view_t *a, const view_t *b, int op, int *nd_out, size_t *sh_out) {
    int same = a->nd == b->nd;
    for (int i = 0; same && i < a->nd; ++i) same = a->sh[i] == b->sh[i];
    if (same && v_contig(a) && v_contig(b)) {
        size_t n = v_numel(a);
        float *out = zeros_f32(n);
        const float *x = a->p, *y = b->p;
#pragma omp parallel for schedule(static)
        for (size_t i = 0; i < n; ++i) out[i] = op == OP_ADD ? x[i] + y[i] : x[i] * y[i];
        *nd_out = a->nd;
        memcpy(sh_out, a->sh, sizeof(size_t) * (size_t)a->nd);
        return out;
    }
    int nd = a->nd > b->nd ? a->nd : b->nd;
    for (int i = 0; i < nd; ++i) {
        int ia = i - (nd - a->nd), ib = i - (nd - b->nd);
        size_t da = ia >= 0 ? a->sh[ia] : 1, db = ib >= 0 ? b->sh[ib] : 1;
        sh_out[i] = da > db ? da : db;
    }
    size_t sa[RP_MAXD], sb[RP_MAXD];
    bcast_strides(a, nd, sh_out, sa);
    bcast_strides(b, nd, sh_out, sb);
    size_t n = 1;
    for (int i = 0; i < nd; ++i) n *= sh_out[i];
    float *out = zeros_f32(n);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        size_t *multi = index_vec(nd);
        flat_to_multi(i, sh_out, nd, multi);
        float x = a->p[multi_to_off(multi, sa, nd, a->off)];
        float y = b->p[multi_to_off(multi, sb, nd, b->off)];
        out[i] = op == OP_ADD ? x + y : x * y;
        free(multi);
    }
    *nd_out = nd;
    return out;
}

/* RawTensor::unary_op, contiguous fast path (ops.rs:13-24), for mul_scalar
 * (ops.rs:118-120). */
static float *mul_scalar(const float *x, size_t n, float s) {
    float *out = zeros_f32(n);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) out[i] = x[i] * s;
    return out;
}

/* Storage::zeros (storage.rs:92-99): a pooled buffer resized and filled. */
static float *storage_zeros(size_t n) {
    float *z = alloc_f32(n);
    memset(z, 0, n * sizeof(float));
    return z;
}

/* RawTensor::cat along one axis (ops.rs:215-275): serial; per input element
 * an index vector, the multi-index, a bounds-checked get (mod.rs:241-259) and
 * the output offset. */
static float *cat2(const view_t *a, const view_t *b, int axis, size_t *sh_out) {
    int nd = a->nd;
    for (int i = 0; i < nd; ++i) sh_out[i] = a->sh[i];
    sh_out[axis] = a->sh[axis] + b->sh[axis];
    size_t st_out[RP_MAXD];
    c_strides(sh_out, nd, st_out);
    size_t n = 1;
    for (int i = 0; i < nd; ++i) n *= sh_out[i];
    float *out = zeros_f32(n);
    const view_t *ts[2] = {a, b};
    size_t cur = 0;
    for (int t = 0; t < 2; ++t) {
        const view_t *v = ts[t];
        size_t tn = v_numel(v);
        for (size_t idx = 0; idx < tn; ++idx) {
            size_t *multi = index_vec(nd);
            flat_to_multi(idx, v->sh, nd, multi);
            int ok = 1;
            for (int i = 0; i < nd; ++i) ok &= multi[i] < v->sh[i];
            float val = ok ? v->p[multi_to_off(multi, v->st, nd, v->off)] : 0.0f;
            multi[axis] += cur;
            out[multi_to_off(multi, st_out, nd, 0)] = val;
            free(multi);
        }
        cur += v->sh[axis];
    }
    return out;
}

/* ---------------------------------------------------------------------- */
/* Softmax over the last axis (reduce.rs:234-271, 274-330)                 */
/* ---------------------------------------------------------------------- */

__attribute__((target("avx2"))) static float row_max_avx2(const float *row, size_t n) {
    __m256 mv = _mm256_set1_ps(-INFINITY);
    size_t i = 0;
    for (; i + 8 <= n; i += 8) mv = _mm256_max_ps(mv, _mm256_loadu_ps(row + i));
    __m128 m = _mm_max_ps(_mm256_castps256_ps128(mv), _mm256_extractf128_ps(mv, 1));
    m = _mm_max_ps(m, _mm_movehl_ps(m, m));
    m = _mm_max_ss(m, _mm_shuffle_ps(m, m, 1));
    float r = _mm_cvtss_f32(m);
    for (; i < n; ++i)
        if (row[i] > r) r = row[i];
    return r;
}

__attribute__((target("avx2"))) static void scale_row_avx2(float *row, size_t n, float f) {
    __m256 vf = _mm256_set1_ps(f);
    size_t i = 0;
    for (; i + 8 <= n; i += 8) _mm256_storeu_ps(row + i, _mm256_mul_ps(_mm256_loadu_ps(row + i), vf));
    for (; i < n; ++i) row[i] *= f;
}

static float *softmax_last(const float *x, size_t rows, size_t d) {
    float *out = zeros_f32(rows * d);
#pragma omp parallel for schedule(static)
    for (size_t r = 0; r < rows; ++r) {
        const float *in = x + r * d;
        float *o = out + r * d;
        float mx = row_max_avx2(in, d);
        float sum = 0.0f;
        for (size_t j = 0; j < d; ++j) {
            float e = expf(in[j] - mx);
            o[j] = e;
            sum += e;
        }
        scale_row_avx2(o, d, sum > 0.0f ? 1.0f / sum : 0.0f);
    }
    return out;
}

/* ---------------------------------------------------------------------- */
/* GEMM / GEMV (matmul.rs)                                                 */
/* ---------------------------------------------------------------------- */

#define BLOCK_M 96
#define BLOCK_N 256
#define MR 6
#define NR 16

static size_t cdiv(size_t a, size_t b) { return (a + b - 1) / b; }
static size_t maxz(size_t a, size_t b) { return a > b ? a : b; }
static size_t minz(size_t a, size_t b) { return a < b ? a : b; }

__attribute__((target("avx2"))) static inline float hsum256(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

/* Chunking of one matrix's GEMM, as its own par_chunks_mut would split it. */
typedef struct {
    size_t chunk;   /* rows (GEMM) or output columns (GEMV) per chunk */
    size_t n_chunks;
} split_t;

static split_t split_nn(size_t m, size_t n, size_t threads) {
    split_t s;
    if (m == 1) {                                 /* gemv_m1_parallel, :749-751 */
        s.chunk = maxz(cdiv(n, threads), 64);
        s.n_chunks = cdiv(n, s.chunk);
    } else {                                      /* :95-97 */
        s.chunk = maxz(cdiv(cdiv(m, threads), MR) * MR, BLOCK_M);
        s.n_chunks = cdiv(m, s.chunk);
    }
    return s;
}

static split_t split_nt(size_t m, size_t n, size_t threads) {
    split_t s;
    if (m == 1) {                                 /* :891-893 */
        s.chunk = maxz(cdiv(cdiv(n, threads), 8) * 8, 16);
        s.n_chunks = cdiv(n, s.chunk);
    } else {                                      /* :360-361 */
        s.chunk = maxz(cdiv(m, threads), 16);
        s.n_chunks = cdiv(m, s.chunk);
    }
    return s;
}

/* gemm_2d_avx2_fma_parallel (matmul.rs:87-336), one row chunk: C = A B,
 * 6x16 register tiles over 256-column blocks, k unrolled by two. */
__attribute__((target("avx2,fma"))) static void gemm_nn_chunk(size_t m, size_t k, size_t n,
                                                              const float *a, const float *b,
                                                              float *c, size_t m_start,
                                                              size_t m_len) {
    (void)m;
    const float *ac = a + m_start * k;
    float *cc = c + m_start * n;
    for (size_t nb = 0; nb < n; nb += BLOCK_N) {
        size_t n_end = minz(nb + BLOCK_N, n);
        size_t i = 0;
        for (; i + MR <= m_len; i += MR) {
            const float *ar[MR];
            for (int r = 0; r < MR; ++r) ar[r] = ac + (i + r) * k;
            size_t j = nb;
            for (; j + NR <= n_end; j += NR) {
                __m256 acc[MR][2];
                for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = _mm256_setzero_ps();
                size_t p = 0;
                for (; p + 2 <= k; p += 2) {
                    for (int u = 0; u < 2; ++u) {
                        const float *bp = b + (p + u) * n + j;
                        __m256 b0 = _mm256_loadu_ps(bp), b1 = _mm256_loadu_ps(bp + 8);
                        for (int r = 0; r < MR; ++r) {
                            __m256 av = _mm256_set1_ps(ar[r][p + u]);
                            acc[r][0] = _mm256_fmadd_ps(av, b0, acc[r][0]);
                            acc[r][1] = _mm256_fmadd_ps(av, b1, acc[r][1]);
                        }
                    }
                }
                for (; p < k; ++p) {
                    const float *bp = b + p * n + j;
                    __m256 b0 = _mm256_loadu_ps(bp), b1 = _mm256_loadu_ps(bp + 8);
                    for (int r = 0; r < MR; ++r) {
                        __m256 av = _mm256_set1_ps(ar[r][p]);
                        acc[r][0] = _mm256_fmadd_ps(av, b0, acc[r][0]);
                        acc[r][1] = _mm256_fmadd_ps(av, b1, acc[r][1]);
                    }
                }
                for (int r = 0; r < MR; ++r) {
                    _mm256_storeu_ps(cc + (i + r) * n + j, acc[r][0]);
                    _mm256_storeu_ps(cc + (i + r) * n + j + 8, acc[r][1]);
                }
            }
            for (; j + 8 <= n_end; j += 8) {
                __m256 acc[MR];
                for (int r = 0; r < MR; ++r) acc[r] = _mm256_setzero_ps();
                for (size_t p = 0; p < k; ++p) {
                    __m256 bv = _mm256_loadu_ps(b + p * n + j);
                    for (int r = 0; r < MR; ++r)
                        acc[r] = _mm256_fmadd_ps(_mm256_set1_ps(ar[r][p]), bv, acc[r]);
                }
                for (int r = 0; r < MR; ++r) _mm256_storeu_ps(cc + (i + r) * n + j, acc[r]);
            }
            for (; j < n_end; ++j) {
                float s[MR] = {0};
                for (size_t p = 0; p < k; ++p) {
                    float bv = b[p * n + j];
                    for (int r = 0; r < MR; ++r) s[r] += ar[r][p] * bv;
                }
                for (int r = 0; r < MR; ++r) cc[(i + r) * n + j] = s[r];
            }
        }
        for (; i < m_len; ++i) {
            const float *arow = ac + i * k;
            float *crow = cc + i * n;
            size_t j = nb;
            for (; j + 8 <= n_end; j += 8) {
                __m256 acc = _mm256_setzero_ps();
                for (size_t p = 0; p < k; ++p)
                    acc = _mm256_fmadd_ps(_mm256_set1_ps(arow[p]), _mm256_loadu_ps(b + p * n + j), acc);
                _mm256_storeu_ps(crow + j, acc);
            }
            for (; j < n_end; ++j) {
                float s = 0.0f;
                for (size_t p = 0; p < k; ++p) s += arow[p] * b[p * n + j];
                crow[j] = s;
            }
        }
    }
}

/* gemv_m1_avx2_fma (matmul.rs:806-870), one column chunk: c += a B, B [k, n]. */
__attribute__((target("avx2,fma"))) static void gemv_nn_chunk(size_t k, size_t n, const float *a,
                                                              const float *b, float *c,
                                                              size_t j_start, size_t j_len) {
    float *cs = c + j_start;
    for (size_t kk = 0; kk < k; ++kk) {
        __m256 av = _mm256_set1_ps(a[kk]);
        const float *bp = b + kk * n + j_start;
        size_t j = 0;
        for (; j + 32 <= j_len; j += 32)
            for (int u = 0; u < 4; ++u)
                _mm256_storeu_ps(cs + j + 8 * u,
                                 _mm256_fmadd_ps(av, _mm256_loadu_ps(bp + j + 8 * u),
                                                 _mm256_loadu_ps(cs + j + 8 * u)));
        for (; j + 8 <= j_len; j += 8)
            _mm256_storeu_ps(cs + j, _mm256_fmadd_ps(av, _mm256_loadu_ps(bp + j), _mm256_loadu_ps(cs + j)));
        for (; j < j_len; ++j) cs[j] += a[kk] * bp[j];
    }
}

/* gemm_2d_a_bt_avx2_fma_parallel (matmul.rs:352-560), one row chunk:
 * C += A B^T with B [n, k], 4x4 tiles of 8-lane dot products. */
__attribute__((target("avx2,fma"))) static void gemm_nt_chunk(size_t k, size_t n, const float *a,
                                                              const float *b, float *c,
                                                              size_t m_start, size_t m_len) {
    size_t i = 0;
    for (; i + 4 <= m_len; i += 4) {
        const float *ar[4];
        for (int r = 0; r < 4; ++r) ar[r] = a + (m_start + i + r) * k;
        size_t j = 0;
        for (; j + 4 <= n; j += 4) {
            const float *br[4];
            for (int q = 0; q < 4; ++q) br[q] = b + (j + q) * k;
            __m256 acc[4][4];
            for (int r = 0; r < 4; ++r)
                for (int q = 0; q < 4; ++q) acc[r][q] = _mm256_setzero_ps();
            size_t p = 0;
            for (; p + 8 <= k; p += 8) {
                __m256 va[4], vb[4];
                for (int r = 0; r < 4; ++r) va[r] = _mm256_loadu_ps(ar[r] + p);
                for (int q = 0; q < 4; ++q) vb[q] = _mm256_loadu_ps(br[q] + p);
                for (int r = 0; r < 4; ++r)
                    for (int q = 0; q < 4; ++q) acc[r][q] = _mm256_fmadd_ps(va[r], vb[q], acc[r][q]);
            }
            float s[4][4];
            for (int r = 0; r < 4; ++r)
                for (int q = 0; q < 4; ++q) s[r][q] = hsum256(acc[r][q]);
            for (; p < k; ++p)
                for (int r = 0; r < 4; ++r)
                    for (int q = 0; q < 4; ++q) s[r][q] += ar[r][p] * br[q][p];
            for (int r = 0; r < 4; ++r)
                for (int q = 0; q < 4; ++q) c[(m_start + i + r) * n + j + q] += s[r][q];
        }
        for (; j < n; ++j) {
            const float *brow = b + j * k;
            for (int r = 0; r < 4; ++r) {
                __m256 acc = _mm256_setzero_ps();
                size_t p = 0;
                for (; p + 8 <= k; p += 8)
                    acc = _mm256_fmadd_ps(_mm256_loadu_ps(ar[r] + p), _mm256_loadu_ps(brow + p), acc);
                float s = hsum256(acc);
                for (; p < k; ++p) s += ar[r][p] * brow[p];
                c[(m_start + i + r) * n + j] += s;
            }
        }
    }
    for (; i < m_len; ++i) {
        const float *arow = a + (m_start + i) * k;
        for (size_t j = 0; j < n; ++j) {
            const float *brow = b + j * k;
            __m256 acc = _mm256_setzero_ps();
            size_t p = 0;
            for (; p + 8 <= k; p += 8)
                acc = _mm256_fmadd_ps(_mm256_loadu_ps(arow + p), _mm256_loadu_ps(brow + p), acc);
            float s = hsum256(acc);
            for (; p < k; ++p) s += arow[p] * brow[p];
            c[(m_start + i) * n + j] += s;
        }
    }
}

/* gemv_a_bt_m1_avx2_fma_parallel (matmul.rs:888-1056), one chunk of output
 * columns: c += a B^T with B [n, k]; 8-row, then 4-row, then 1-row dot
 * products. */
__attribute__((target("avx2,fma"))) static void gemv_nt_chunk(size_t k, const float *a,
                                                              const float *b, float *c,
                                                              size_t j_start, size_t j_len) {
    size_t j = 0;
#define RP_GEMV_ROWS(R)                                                                   \
    for (; j + (R) <= j_len; j += (R)) {                                                  \
        const float *br[R];                                                               \
        __m256 acc[R];                                                                    \
        for (int q = 0; q < (R); ++q) {                                                   \
            br[q] = b + (j_start + j + q) * k;                                            \
            acc[q] = _mm256_setzero_ps();                                                 \
        }                                                                                 \
        size_t p = 0;                                                                     \
        for (; p + 8 <= k; p += 8) {                                                      \
            __m256 va = _mm256_loadu_ps(a + p);                                           \
            for (int q = 0; q < (R); ++q)                                                 \
                acc[q] = _mm256_fmadd_ps(va, _mm256_loadu_ps(br[q] + p), acc[q]);         \
        }                                                                                 \
        float s[R];                                                                       \
        for (int q = 0; q < (R); ++q) s[q] = hsum256(acc[q]);                             \
        for (; p < k; ++p)                                                                \
            for (int q = 0; q < (R); ++q) s[q] += a[p] * br[q][p];                        \
        for (int q = 0; q < (R); ++q) c[j_start + j + q] += s[q];                         \
    }
    RP_GEMV_ROWS(8)
    RP_GEMV_ROWS(4)
    RP_GEMV_ROWS(1)
#undef RP_GEMV_ROWS
}

/* The batched matmul drivers (matmul.rs:1112-1221 `matmul`, :1224-1318
 * `matmul_transposed_b`) for same-shape batches: every matrix runs
 * gemm_2d_contiguous / gemm_2d_a_bt_contiguous (:30-80).  C must be zeroed
 * (`vec![0.0; ...]`): the transposed kernels accumulate. */
static void batched_matmul(int transposed_b, size_t nmat, size_t m, size_t k, size_t n,
                           const float *a, const float *b, float *c) {
    if (m == 0 || k == 0 || n == 0 || nmat == 0) return;
    size_t threads = (size_t)omp_get_max_threads();
    split_t s = transposed_b ? split_nt(m, n, threads) : split_nn(m, n, threads);
    long long items = (long long)(nmat * s.n_chunks);
#pragma omp parallel for schedule(dynamic, 1)
    for (long long it = 0; it < items; ++it) {
        size_t mat = (size_t)it / s.n_chunks, ch = (size_t)it % s.n_chunks;
        const float *am = a + mat * m * k, *bm = b + mat * k * n;
        float *cm = c + mat * m * n;
        size_t start = ch * s.chunk;
        if (m == 1) {
            size_t len = minz(s.chunk, n - start);
            if (transposed_b)
                gemv_nt_chunk(k, am, bm, cm, start, len);
            else
                gemv_nn_chunk(k, n, am, bm, cm, start, len);
        } else {
            size_t len = minz(s.chunk, m - start);
            if (transposed_b)
                gemm_nt_chunk(k, n, am, bm, cm, start, len);
            else
                gemm_nn_chunk(m, k, n, am, bm, cm, start, len);
        }
    }
}

/* ---------------------------------------------------------------------- */
/* Attention drivers                                                       */
/* ---------------------------------------------------------------------- */

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

/* Components of the wall time, in the order bench.py reports them. */
enum {
    T_REPEAT = 0,   /* repeat-KV: Storage::zeros + two broadcast adds */
    T_GATHER,       /* to_contiguous copies of strided operands */
    T_QK,           /* matmul_transposed_b */
    T_SCALE,        /* mul_scalar / broadcast mul by a scalar tensor */
    T_MASK,         /* mask build + broadcast add */
    T_SOFTMAX,      /* fused softmax */
    T_PV,           /* matmul */
    T_CAT,          /* Tensor::cat of the cache slot (decode) */
    T_FREE,         /* dropping the step's temporaries */
    T_LINEAR,       /* q/k/v projections (matmul_transposed_b + bias add) */
    T_ROPE,         /* RotaryEmbedding::apply on q and k */
    T_COUNT
};

enum { MODE_GQA = 0, MODE_MHA = 1, MODE_CROSS = 2 };

/* A [B, H, T, d] operand given either contiguous or as the reference's
 * transposed view of a [B, T, H, d] projection (reshape + transpose(1, 2)). */
static view_t bhtd_view(const float *p, size_t b, size_t h, size_t t, size_t d, int bthd) {
    size_t sh[4] = {b, h, t, d};
    view_t v = v_contig_view(p, 4, sh);
    if (bthd) {
        v.st[0] = t * h * d;
        v.st[1] = d;
        v.st[2] = h * d;
        v.st[3] = 1;
    }
    return v;
}

/* RawTensor::unsqueeze(2) of a 4-D view (mod.rs:435-460): a length-1 axis
 * inserted before the key axis. */
static view_t unsqueeze2(const view_t *src) {
    view_t u = *src;
    u.nd = 5;
    u.sh[0] = src->sh[0];
    u.sh[1] = src->sh[1];
    u.sh[2] = 1;
    u.sh[3] = src->sh[2];
    u.sh[4] = src->sh[3];
    u.st[2] = src->st[2] * src->sh[2];
    u.st[3] = src->st[2];
    u.st[4] = src->st[3];
    return u;
}

/*
 * The attention core of one call, from the projected (and rotated) q and the
 * slot's K/V to the context [B, Hq, Tq, d]:
 *   MODE_GQA   GroupedQueryAttention::forward_gqa_cached steps 4-7
 *              (llama.rs:253-296): repeat-KV when G > 1, mul_scalar, the
 *              -1e4 mask for t > 1 at start_pos, softmax, PV.
 *   MODE_MHA   MultiHeadAttention::forward_attention_cached steps 4-7
 *              (attention.rs:93-122): scale by a broadcast mul with a scalar
 *              tensor, the mask for t > 1 at start_pos = L - T (is_causal).
 *   MODE_CROSS forward_cross_attention_cached steps 3-5 (attention.rs:193-203).
 * Returns the context buffer (caller frees), times accumulated into t[].
 */
static float *attention_core(const view_t *q, const view_t *k_all, const view_t *v_all,
                             size_t b, size_t hq, size_t hkv, size_t tq, size_t tk, size_t d,
                             size_t start_pos, int mode, int causal, double *t) {
    size_t g = hq / hkv;
    double t0 = now_s(), t1;
    float *k_rep = NULL, *v_rep = NULL, *zeros = NULL;
    view_t kx = *k_all, vx = *v_all;
    if (mode == MODE_GQA && g > 1) {
        /* llama.rs:256-266: zeros [B, Hkv, G, L, d]; k.unsqueeze(2) + zeros */
        size_t zsh[5] = {b, hkv, g, tk, d};
        zeros = storage_zeros(b * hkv * g * tk * d);
        view_t z = v_contig_view(zeros, 5, zsh);
        view_t ku = unsqueeze2(k_all), vu = unsqueeze2(v_all);
        int nd;
        size_t sh[RP_MAXD];
        k_rep = binary_op(&ku, &z, OP_ADD, &nd, sh);
        v_rep = binary_op(&vu, &z, OP_ADD, &nd, sh);
        size_t rsh[4] = {b, hq, tk, d};
        kx = v_contig_view(k_rep, 4, rsh);
        vx = v_contig_view(v_rep, 4, rsh);
        t[T_REPEAT] += now_s() - t0;
    }

    /* matmul_transposed_b (matmul.rs:1260-1264): both operands made contiguous */
    int cq, ck, cv;
    t0 = now_s();
    float *qc = to_contiguous(q, &cq);
    float *kc = to_contiguous(&kx, &ck);
    t1 = now_s();
    t[T_GATHER] += t1 - t0;
    size_t nmat = b * hq;
    float *scores = zeros_f32(nmat * tq * tk);
    batched_matmul(1, nmat, tq, d, tk, qc, kc, scores);
    t0 = now_s();
    t[T_QK] += t0 - t1;

    float scale = 1.0f / sqrtf((float)d);
    float *scaled;
    if (mode == MODE_GQA) {
        scaled = mul_scalar(scores, nmat * tq * tk, scale);
    } else {
        size_t ssh[4] = {b, hq, tq, tk};
        view_t sv = v_contig_view(scores, 4, ssh);
        view_t sc;
        memset(&sc, 0, sizeof sc);
        sc.p = &scale;
        sc.nd = 0;
        int nd;
        size_t sh[RP_MAXD];
        scaled = binary_op(&sv, &sc, OP_MUL, &nd, sh);
    }
    t1 = now_s();
    t[T_SCALE] += t1 - t0;

    float *masked = NULL, *mask = NULL;
    int want_mask = tq > 1 && (mode == MODE_GQA || (mode == MODE_MHA && causal));
    if (want_mask) {
        /* llama.rs:277-292 / attention.rs:101-115: a [1, 1, T, L] tensor of 0
         * and -1e4 built serially, then added with broadcasting. */
        mask = zeros_f32(tq * tk);
        size_t sp = mode == MODE_GQA ? start_pos : (tk > tq ? tk - tq : 0);
        for (size_t r = 0; r < tq; ++r)
            for (size_t c = 0; c < tk; ++c)
                if (c > sp + r) mask[r * tk + c] = -1e4f;
        size_t msh[4] = {1, 1, tq, tk}, ssh[4] = {b, hq, tq, tk};
        view_t mv = v_contig_view(mask, 4, msh), sv = v_contig_view(scaled, 4, ssh);
        int nd;
        size_t sh[RP_MAXD];
        masked = binary_op(&sv, &mv, OP_ADD, &nd, sh);
        t[T_MASK] += now_s() - t1;
    }
    t0 = now_s();

    float *weights = softmax_last(masked ? masked : scaled, nmat * tq, tk);
    t1 = now_s();
    t[T_SOFTMAX] += t1 - t0;

    float *vc = to_contiguous(&vx, &cv);
    t0 = now_s();
    t[T_GATHER] += t0 - t1;
    float *ctx = zeros_f32(nmat * tq * d);
    batched_matmul(0, nmat, tq, tk, d, weights, vc, ctx);
    t1 = now_s();
    t[T_PV] += t1 - t0;

    if (cq) free(qc);
    if (ck) free(kc);
    if (cv) free(vc);
    free(scores);
    free(scaled);
    free(masked);
    free(mask);
    free(weights);
    free(k_rep);
    free(v_rep);
    free(zeros);
    t[T_FREE] += now_s() - t1;
    return ctx;
}

void rp_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
}

int rp_max_threads(void) { return omp_get_max_threads(); }

/*
 * One attention call.  q [B, Hq, Tq, d] and k, v [B, Hkv, Tk, d]; q_bthd /
 * kv_bthd say the operand is the reference's transposed view of a
 * [B, T, H, d] buffer (then non-contiguous, as the projections leave it).
 * out receives the context [B, Hq, Tq, d].  t[T_COUNT] accumulates seconds.
 */
int rp_attention(const float *q, const float *k, const float *v, float *out, int B, int Hq,
                 int Hkv, int Tq, int Tk, int d, int q_bthd, int kv_bthd, int start_pos,
                 int mode, int causal, double *t) {
    if (B < 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || Tq < 0 || Tk < 0 || d <= 0) return 1;
    if (mode != MODE_GQA && Hq != Hkv) return 1;
    view_t qv = bhtd_view(q, (size_t)B, (size_t)Hq, (size_t)Tq, (size_t)d, q_bthd);
    view_t kv = bhtd_view(k, (size_t)B, (size_t)Hkv, (size_t)Tk, (size_t)d, kv_bthd);
    view_t vv = bhtd_view(v, (size_t)B, (size_t)Hkv, (size_t)Tk, (size_t)d, kv_bthd);
    float *ctx = attention_core(&qv, &kv, &vv, (size_t)B, (size_t)Hq, (size_t)Hkv, (size_t)Tq,
                                (size_t)Tk, (size_t)d, (size_t)start_pos, mode, causal, t);
    memcpy(out, ctx, sizeof(float) * (size_t)B * (size_t)Hq * (size_t)Tq * (size_t)d);
    free(ctx);
    return 0;
}

/*
 * `steps` decode steps (t = 1) over a ragged batch, the way the reference
 * runs one: the slots need equal lengths across a batch, so every sequence is
 * its own B = 1 call (llama.rs:239-296 in MODE_GQA, attention.rs:79-122 in
 * MODE_MHA).  Per call: Tensor::cat of the slot's K and V with the new row
 * (a fresh [1, Hkv, L+1, d] buffer each, the old one dropped), then the
 * attention core over all L+1 rows with no mask.
 *   kc0, vc0  [B, Hkv, cap, d] head-major initial caches (lens0[b] rows used)
 *   q_all     [steps, B, Hq, d]; kn_all, vn_all [steps, B, Hkv, d]
 *   out_all   [steps, B, Hq, d] receives every step's context
 *   kc_end, vc_end (optional) [B, Hkv, cap, d] receive the final slots
 * Setting up the per-sequence slots is not timed; t[] covers the steps.
 */
int rp_decode_run(const float *q_all, const float *kc0, const float *vc0, const int32_t *lens0,
                  const float *kn_all, const float *vn_all, float *out_all, int B, int Hq,
                  int Hkv, int cap, int d, int steps, int mode, float *kc_end, float *vc_end,
                  double *t) {
    if (B <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv || d <= 0 || steps < 0 || cap < 0) return 1;
    if (mode != MODE_GQA && Hq != Hkv) return 1;
    for (int bi = 0; bi < B; ++bi)
        if (lens0[bi] < 0 || (int64_t)lens0[bi] + steps > (int64_t)cap) return 2;
    size_t hkv = (size_t)Hkv, hq = (size_t)Hq, dd = (size_t)d, capz = (size_t)cap;
    float **ks = (float **)calloc((size_t)B, sizeof(float *));
    float **vs = (float **)calloc((size_t)B, sizeof(float *));
    size_t *len = (size_t *)calloc((size_t)B, sizeof(size_t));
    for (int bi = 0; bi < B; ++bi) {
        len[bi] = (size_t)lens0[bi];
        ks[bi] = alloc_f32(hkv * len[bi] * dd);
        vs[bi] = alloc_f32(hkv * len[bi] * dd);
        for (size_t h = 0; h < hkv; ++h) {
            size_t src = (((size_t)bi * hkv + h) * capz) * dd, dst = h * len[bi] * dd;
            memcpy(ks[bi] + dst, kc0 + src, sizeof(float) * len[bi] * dd);
            memcpy(vs[bi] + dst, vc0 + src, sizeof(float) * len[bi] * dd);
        }
    }
    for (int s = 0; s < steps; ++s) {
        for (int bi = 0; bi < B; ++bi) {
            double t0 = now_s();
            size_t osh[4] = {1, hkv, len[bi], dd}, nsh[4] = {1, hkv, 1, dd}, sh[4];
            size_t row = ((size_t)s * (size_t)B + (size_t)bi) * hkv * dd;
            view_t ko = v_contig_view(ks[bi], 4, osh), vo = v_contig_view(vs[bi], 4, osh);
            view_t kn = v_contig_view(kn_all + row, 4, nsh), vn = v_contig_view(vn_all + row, 4, nsh);
            /* A slot that is still empty takes the new row as it is
             * (llama.rs:240-248; attention.rs:80-88). */
            float *kcat = len[bi] ? cat2(&ko, &kn, 2, sh) : NULL;
            float *vcat = len[bi] ? cat2(&vo, &vn, 2, sh) : NULL;
            if (!len[bi]) {
                kcat = alloc_f32(hkv * dd);
                vcat = alloc_f32(hkv * dd);
                memcpy(kcat, kn_all + row, sizeof(float) * hkv * dd);
                memcpy(vcat, vn_all + row, sizeof(float) * hkv * dd);
            }
            free(ks[bi]);
            free(vs[bi]);
            ks[bi] = kcat;
            vs[bi] = vcat;
            len[bi] += 1;
            t[T_CAT] += now_s() - t0;
            size_t ksh[4] = {1, hkv, len[bi], dd}, qsh[4] = {1, hq, 1, dd};
            view_t kv = v_contig_view(ks[bi], 4, ksh), vv = v_contig_view(vs[bi], 4, ksh);
            view_t qv = v_contig_view(q_all + ((size_t)s * (size_t)B + (size_t)bi) * hq * dd, 4, qsh);
            float *ctx = attention_core(&qv, &kv, &vv, 1, hq, hkv, 1, len[bi], dd, len[bi] - 1, mode,
                                        0, t);
            memcpy(out_all + ((size_t)s * (size_t)B + (size_t)bi) * hq * dd, ctx,
                   sizeof(float) * hq * dd);
            free(ctx);
        }
    }
    for (int bi = 0; bi < B; ++bi) {
        if (kc_end && vc_end)
            for (size_t h = 0; h < hkv; ++h) {
                size_t dst = (((size_t)bi * hkv + h) * capz) * dd, src = h * len[bi] * dd;
                memcpy(kc_end + dst, ks[bi] + src, sizeof(float) * len[bi] * dd);
                memcpy(vc_end + dst, vs[bi] + src, sizeof(float) * len[bi] * dd);
            }
        free(ks[bi]);
        free(vs[bi]);
    }
    free(ks);
    free(vs);
    free(len);
    return 0;
}

/* RawTensor::unary_op on a strided view (ops.rs:25-35), for neg (:102-104):
 * per element (in parallel) an index vector and the offset. */
static float *neg_strided(const view_t *v) {
    size_t n = v_numel(v);
    float *out = zeros_f32(n);
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) {
        size_t *multi = index_vec(v->nd);
        flat_to_multi(i, v->sh, v->nd, multi);
        out[i] = -v->p[multi_to_off(multi, v->st, v->nd, v->off)];
        free(multi);
    }
    return out;
}

/* RotaryEmbedding::apply (llama.rs:109-157) on a contiguous [1, H, 1, d]
 * row at position pos: slice views of the tables and of x, neg of the second
 * half, cat of [-x2, x1], x * cos and rotated * sin with broadcasting, then
 * the same-shape add.  Returns a new buffer. */
static float *rope_apply_row(const float *x, size_t h, size_t d, const float *cos_t,
                             const float *sin_t, size_t pos) {
    size_t half = d / 2, sh[4] = {1, h, 1, d}, tsh[4] = {1, 1, 1, d};
    view_t xv = v_contig_view(x, 4, sh);
    view_t cv = v_contig_view(cos_t + pos * d, 4, tsh), sv = v_contig_view(sin_t + pos * d, 4, tsh);
    view_t x1 = xv, x2 = xv;
    x1.sh[3] = half;
    x2.sh[3] = d - half;
    x2.off = half;
    x2.p = x;
    float *nx2 = neg_strided(&x2);
    size_t hsh[4] = {1, h, 1, d - half}, csh[4];
    view_t nv = v_contig_view(nx2, 4, hsh);
    float *rot = cat2(&nv, &x1, 3, csh);
    view_t rv = v_contig_view(rot, 4, sh);
    int nd;
    size_t osh[RP_MAXD];
    float *t1 = binary_op(&xv, &cv, OP_MUL, &nd, osh);
    float *t2 = binary_op(&rv, &sv, OP_MUL, &nd, osh);
    view_t a = v_contig_view(t1, 4, sh), b = v_contig_view(t2, 4, sh);
    float *out = binary_op(&a, &b, OP_ADD, &nd, osh);
    free(nx2);
    free(rot);
    free(t1);
    free(t2);
    return out;
}

/* Linear::forward (linear.rs:47-57) on one [1, 1, C] row: matmul_transposed_b
 * with the [N, C] weight (a single matrix: gemv_a_bt_m1_parallel), then the
 * broadcast bias add when there is a bias. */
static float *linear_row(const float *x, const float *w, const float *bias, size_t c, size_t n) {
    float *y = zeros_f32(n);
    batched_matmul(1, 1, 1, c, n, x, w, y);
    if (!bias) return y;
    size_t ysh[3] = {1, 1, n}, bsh[1] = {n};
    view_t yv = v_contig_view(y, 3, ysh), bv = v_contig_view(bias, 1, bsh);
    int nd;
    size_t osh[RP_MAXD];
    float *out = binary_op(&yv, &bv, OP_ADD, &nd, osh);
    free(y);
    return out;
}

/*
 * Steps 1-2 of a decode step (t = 1) for a ragged batch, one B = 1 call per
 * sequence as the reference runs it: the q/k/v projections
 * (llama.rs:226-229 / attention.rs:69-72), the head split (views only) and,
 * when tables are given, RoPE on q and k at the sequence's position
 * (llama.rs:234-235).
 *   x [B, C]; wq [Hq*d, C], wk/wv [Hkv*d, C]; bq/bk/bv optional biases;
 *   cos_t/sin_t [max_pos, d] or NULL; pos [B];
 *   q_out [B, Hq, d], k_out/v_out [B, Hkv, d].
 */
int rp_qkv_rope_run(const float *x, const float *wq, const float *wk, const float *wv,
                    const float *bq, const float *bk, const float *bv, const float *cos_t,
                    const float *sin_t, const int32_t *pos, int B, int C, int Hq, int Hkv, int d,
                    float *q_out, float *k_out, float *v_out, double *t) {
    if (B < 0 || C <= 0 || Hq <= 0 || Hkv <= 0 || d <= 0 || (cos_t && d % 2)) return 1;
    size_t c = (size_t)C, dd = (size_t)d, nq = (size_t)Hq * dd, nk = (size_t)Hkv * dd;
    for (int bi = 0; bi < B; ++bi) {
        const float *xr = x + (size_t)bi * c;
        double t0 = now_s();
        float *q = linear_row(xr, wq, bq, c, nq);
        float *k = linear_row(xr, wk, bk, c, nk);
        float *v = linear_row(xr, wv, bv, c, nk);
        double t1 = now_s();
        t[T_LINEAR] += t1 - t0;
        if (cos_t) {
            float *qr = rope_apply_row(q, (size_t)Hq, dd, cos_t, sin_t, (size_t)pos[bi]);
            float *kr = rope_apply_row(k, (size_t)Hkv, dd, cos_t, sin_t, (size_t)pos[bi]);
            free(q);
            free(k);
            q = qr;
            k = kr;
            t[T_ROPE] += now_s() - t1;
        }
        memcpy(q_out + (size_t)bi * nq, q, sizeof(float) * nq);
        memcpy(k_out + (size_t)bi * nk, k, sizeof(float) * nk);
        memcpy(v_out + (size_t)bi * nk, v, sizeof(float) * nk);
        free(q);
        free(k);
        free(v);
    }
    return 0;
}

int rp_components(void) { return T_COUNT; }
