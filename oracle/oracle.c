/*
 * oracle.c -- CPU restatement of the reference engine's attention algorithms.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP product path
 * is compared against, and the "port" CPU baseline that bench.py times beside
 * the GPU.  Nothing in the product library links, loads or calls it; only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may.
 *
 * Every routine restates one function of elvin-mark/neural-network-engine
 * (Rust, CPU, Rayon).  Citations are file:line into that repository.
 * All tensors here are row-major contiguous f32, which is what the reference
 * operates on after `to_contiguous()` (src/tensor/mod.rs:184-197).
 *
 * The Rayon fan-out of the reference (`par_chunks_mut` over the B*H head
 * matrices, src/nn/flash_attention.rs:69-71) is restated as a pthread pool
 * over the same (batch, head) work items; each item is computed with the
 * same sequential f32 arithmetic as the reference, so the thread count only
 * changes wall time, never results.
 *
 * Parity pinning (what checks each function, see tests/test_oracle.py):
 *   oracle_flash_forward      float64 closed form softmax(s*QK^T + M)V,
 *                             golden fixtures, block-size invariance,
 *                             causal row 0 == V[0], constant-V, uniform-score
 *                             mean, key permutation invariance, empty Tk.
 *   oracle_standard_attention float64 closed form with the -1e4 additive mask,
 *                             GQA == MHA on explicitly repeated K/V (brute
 *                             force), mask enumerated index by index, golden.
 *   oracle_kv_append          bit-exact read-back against concatenation.
 *   oracle_decode_step        equals the matching row of a causal prefill
 *                             (the cached-vs-full pattern of
 *                             tests/nn/kv_cache_tests.rs:30-103).
 *   oracle_rope_tables        float64 closed form cos/sin(p * theta^(-2i/d))
 *                             within f32 rounding, the [c, c] / [s, s] halves,
 *                             position 0 = (1, 0), the llama.rs:74-107 f32
 *                             steps recomputed in numpy bit for bit.
 *   oracle_rope_apply         float64 rotation of each (i, i + d/2) pair,
 *                             norm preservation, identity at position 0,
 *                             R(a) R(b) = R(a + b), q.k depending only on the
 *                             position difference.
 *   oracle_linear             float64 x W^T + b.
 *   oracle_qkv_rope           composition of the two above with the
 *                             [B, T, H, d] -> [B, H, T, d] head split.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

typedef void (*item_fn)(void *ctx, int64_t item);

typedef struct {
    item_fn fn;
    void *ctx;
    int64_t n_items;
    int64_t next;
    pthread_mutex_t lock;
} pool_t;

static void *pool_worker(void *arg) {
    pool_t *p = (pool_t *)arg;
    for (;;) {
        pthread_mutex_lock(&p->lock);
        int64_t it = p->next++;
        pthread_mutex_unlock(&p->lock);
        if (it >= p->n_items) break;
        p->fn(p->ctx, it);
    }
    return NULL;
}

/* Runs fn(ctx, i) for i in [0, n_items) on n_threads threads (dynamic
 * scheduling, like Rayon's work stealing over par_chunks_mut). */
static void parallel_for(item_fn fn, void *ctx, int64_t n_items, int n_threads) {
    if (n_threads <= 1 || n_items <= 1) {
        for (int64_t i = 0; i < n_items; ++i) fn(ctx, i);
        return;
    }
    if (n_threads > 256) n_threads = 256;
    pool_t p;
    p.fn = fn;
    p.ctx = ctx;
    p.n_items = n_items;
    p.next = 0;
    pthread_mutex_init(&p.lock, NULL);
    pthread_t th[256];
    int started = 0;
    for (int t = 0; t < n_threads; ++t) {
        if (pthread_create(&th[t], NULL, pool_worker, &p) != 0) break;
        ++started;
    }
    pool_worker(&p);
    for (int t = 0; t < started; ++t) pthread_join(th[t], NULL);
    pthread_mutex_destroy(&p.lock);
}

/* ------------------------------------------------------------------------- */
/* a1-a3: flash_attention_forward (src/nn/flash_attention.rs:19-199)          */
/* ------------------------------------------------------------------------- */

typedef struct {
    const float *q, *k, *v;
    float *out;
    int64_t tq, tk, d, br, bc;
    int causal;
    float sm_scale;
} flash_ctx;

/* One (batch, head) matrix: the body of the par_chunks_mut closure,
 * flash_attention.rs:71-195. */
static void flash_head(void *vctx, int64_t bh) {
    const flash_ctx *c = (const flash_ctx *)vctx;
    const int64_t tq = c->tq, tk = c->tk, d = c->d, br = c->br, bc = c->bc;
    const float *q_mat = c->q + bh * tq * d;          /* :72-76 */
    const float *k_mat = c->k + bh * tk * d;          /* :73-77 */
    const float *v_mat = c->v + bh * tk * d;          /* :74-78 */
    float *o_head = c->out + bh * tq * d;
    float *m = (float *)malloc(sizeof(float) * (size_t)(tq ? tq : 1));   /* :81 */
    float *l = (float *)malloc(sizeof(float) * (size_t)(tq ? tq : 1));   /* :82 */
    float *s_ij = (float *)malloc(sizeof(float) * (size_t)(br * bc));   /* :88 */
    float *p_ij = (float *)malloc(sizeof(float) * (size_t)(br * bc));   /* :89 */
    for (int64_t i = 0; i < tq; ++i) { m[i] = -INFINITY; l[i] = 0.0f; }
    memset(o_head, 0, sizeof(float) * (size_t)(tq * d));               /* :66 */

    const int64_t n_r = (tq + br - 1) / br;                            /* :84 */
    const int64_t n_c = (tk + bc - 1) / bc;                            /* :85 */
    for (int64_t i = 0; i < n_r; ++i) {
        const int64_t r_start = i * br;
        const int64_t r_end = (r_start + br < tq) ? r_start + br : tq;
        const int64_t m_r = r_end - r_start;
        for (int64_t j = 0; j < n_c; ++j) {
            const int64_t c_start = j * bc;
            const int64_t c_end = (c_start + bc < tk) ? c_start + bc : tk;
            const int64_t m_c = c_end - c_start;
            if (c->causal && c_start > r_end - 1) continue;            /* :102 */
            /* 1. S = (Q_i K_j^T) * scale, -inf above the diagonal  :107-124 */
            for (int64_t r = 0; r < m_r; ++r) {
                const int64_t rg = r_start + r;
                const float *q_row = q_mat + rg * d;
                for (int64_t cc = 0; cc < m_c; ++cc) {
                    const int64_t cg = c_start + cc;
                    if (c->causal && cg > rg) {
                        s_ij[r * bc + cc] = -INFINITY;
                    } else {
                        const float *k_row = k_mat + cg * d;
                        float dot = 0.0f;
                        for (int64_t x = 0; x < d; ++x) dot += q_row[x] * k_row[x];
                        s_ij[r * bc + cc] = dot * c->sm_scale;
                    }
                }
            }
            /* 2. online softmax per row                             :127-181 */
            for (int64_t r = 0; r < m_r; ++r) {
                const int64_t rg = r_start + r;
                float bmax = -INFINITY;
                for (int64_t cc = 0; cc < m_c; ++cc)
                    if (s_ij[r * bc + cc] > bmax) bmax = s_ij[r * bc + cc];
                if (bmax == -INFINITY) continue;                       /* :139 */
                const float old_m = m[rg];
                const float new_m = fmaxf(old_m, bmax);
                const float alpha = (old_m == -INFINITY) ? 0.0f : expf(old_m - new_m);
                float psum = 0.0f;
                for (int64_t cc = 0; cc < m_c; ++cc) {
                    const float sc = s_ij[r * bc + cc];
                    const float pv = (sc == -INFINITY) ? 0.0f : expf(sc - new_m);
                    p_ij[r * bc + cc] = pv;
                    psum += pv;
                }
                const float new_l = alpha * l[rg] + psum;              /* :165 */
                float *o_row = o_head + rg * d;
                for (int64_t x = 0; x < d; ++x) {                      /* :169-177 */
                    float pv = 0.0f;
                    for (int64_t cc = 0; cc < m_c; ++cc)
                        pv += p_ij[r * bc + cc] * v_mat[(c_start + cc) * d + x];
                    o_row[x] = alpha * o_row[x] + pv;
                }
                m[rg] = new_m;
                l[rg] = new_l;
            }
        }
    }
    /* 4. O /= l, rows with l == 0 stay zero                          :186-195 */
    for (int64_t rg = 0; rg < tq; ++rg) {
        const float row_sum = l[rg];
        if (row_sum > 0.0f) {
            const float inv_l = 1.0f / row_sum;
            for (int64_t x = 0; x < d; ++x) o_head[rg * d + x] *= inv_l;
        }
    }
    free(m); free(l); free(s_ij); free(p_ij);
}

/* has_scale == 0 reproduces `scale.unwrap_or(1.0 / (d as f32).sqrt())`
 * (flash_attention.rs:50); br/bc are clamped to >= 16 (:51-52). */
void oracle_flash_forward(const float *q, const float *k, const float *v, float *out,
                          int64_t b, int64_t h, int64_t tq, int64_t tk, int64_t d,
                          int is_causal, int has_scale, float scale,
                          int64_t block_r, int64_t block_c, int n_threads) {
    flash_ctx c;
    c.q = q; c.k = k; c.v = v; c.out = out;
    c.tq = tq; c.tk = tk; c.d = d;
    c.br = block_r < 16 ? 16 : block_r;
    c.bc = block_c < 16 ? 16 : block_c;
    c.causal = is_causal;
    c.sm_scale = has_scale ? scale : 1.0f / sqrtf((float)d);
    parallel_for(flash_head, &c, b * h, n_threads);
}

/* ------------------------------------------------------------------------- */
/* a5/a7/a8: standard (matmul -> mask -> softmax -> matmul) attention         */
/*   GQA:   GroupedQueryAttention::forward_gqa_cached, llama.rs:253-296       */
/*   MHA:   MultiHeadAttention::forward_attention_cached, attention.rs:93-122 */
/*   cross: forward_cross_attention_cached, attention.rs:193-203             */
/* ------------------------------------------------------------------------- */

typedef struct {
    const float *q, *k, *v;
    float *out;
    int64_t hq, hkv, tq, tk, d, g;
    int64_t start_pos;
    int masked;
    float scale;
} std_ctx;

/* One (batch, query head) matrix.  The repeat-KV broadcast of llama.rs:256-266
 * (k.unsqueeze(2) + zeros[B,Hkv,G,L,d] -> [B,Hq,L,d]) makes query head hq read
 * KV head hq / G; here that mapping is applied directly instead of
 * materialising the G copies (the values read are identical). */
static void std_head(void *vctx, int64_t bhq) {
    const std_ctx *c = (const std_ctx *)vctx;
    const int64_t bi = bhq / c->hq, hq = bhq % c->hq;
    const int64_t kvh = hq / c->g;                                         /* llama.rs:256-266 */
    const int64_t tq = c->tq, tk = c->tk, d = c->d;
    const float *q_mat = c->q + bhq * tq * d;
    const float *k_mat = c->k + (bi * c->hkv + kvh) * tk * d;
    const float *v_mat = c->v + (bi * c->hkv + kvh) * tk * d;
    float *o_mat = c->out + bhq * tq * d;
    float *row = (float *)malloc(sizeof(float) * (size_t)(tk ? tk : 1));
    for (int64_t r = 0; r < tq; ++r) {
        /* scores = q . k^T, then * scale                    llama.rs:272-274 */
        for (int64_t cc = 0; cc < tk; ++cc) {
            float dot = 0.0f;
            for (int64_t x = 0; x < d; ++x) dot += q_mat[r * d + x] * k_mat[cc * d + x];
            float s = dot * c->scale;
            /* additive -1e4 where c > start_pos + r        llama.rs:277-292,
             * attention.rs:102-116 (start_pos = Tk - Tq there) */
            if (c->masked && cc > c->start_pos + r) s += -1e4f;
            row[cc] = s;
        }
        /* softmax, last axis fast path                      reduce.rs:240-268 */
        if (tk > 0) {
            float mx = -INFINITY;
            for (int64_t cc = 0; cc < tk; ++cc) if (row[cc] > mx) mx = row[cc];
            float sum = 0.0f;
            for (int64_t cc = 0; cc < tk; ++cc) { row[cc] = expf(row[cc] - mx); sum += row[cc]; }
            const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
            for (int64_t cc = 0; cc < tk; ++cc) row[cc] *= inv;
        }
        /* context = weights . V                            llama.rs:296 */
        for (int64_t x = 0; x < d; ++x) {
            float acc = 0.0f;
            for (int64_t cc = 0; cc < tk; ++cc) acc += row[cc] * v_mat[cc * d + x];
            o_mat[r * d + x] = acc;
        }
    }
    free(row);
}

/* q [B,Hq,Tq,d], k/v [B,Hkv,Tk,d], out [B,Hq,Tq,d].
 * masked != 0 applies the -1e4 mask at c > start_pos + r; callers follow the
 * reference and pass masked = (Tq > 1) for GQA (llama.rs:277) and
 * masked = is_causal && Tq > 1 with start_pos = Tk - Tq for MHA
 * (attention.rs:102-104).  Cross-attention passes masked = 0. */
void oracle_standard_attention(const float *q, const float *k, const float *v, float *out,
                               int64_t b, int64_t hq, int64_t hkv, int64_t tq, int64_t tk,
                               int64_t d, int masked, int64_t start_pos, int has_scale,
                               float scale, int n_threads) {
    std_ctx c;
    c.q = q; c.k = k; c.v = v; c.out = out;
    c.hq = hq; c.hkv = hkv; c.tq = tq; c.tk = tk; c.d = d;
    c.g = hq / hkv;
    c.start_pos = start_pos;
    c.masked = masked;
    c.scale = has_scale ? scale : 1.0f / sqrtf((float)d);   /* llama.rs:273 */
    parallel_for(std_head, &c, b * hq, n_threads);
}

/* ------------------------------------------------------------------------- */
/* a6: KV cache append (kv_cache.rs:63-72, Tensor::cat along axis 2,          */
/* src/tensor/ops.rs:215-275), stated on the fixed-capacity head-major layout  */
/* cache[B][Hkv][cap][d] with per-sequence lengths.                           */
/* ------------------------------------------------------------------------- */

/* Appends k_new/v_new [B,Hkv,t_new,d] at row lens[b] of every (b, kvh) and
 * advances lens[b] by t_new.  Returns 0, or 3 if some sequence would exceed
 * cap (the cat-based reference has no capacity; the fixed layout does). */
int oracle_kv_append(float *k_cache, float *v_cache, int32_t *lens,
                     const float *k_new, const float *v_new,
                     int64_t b, int64_t hkv, int64_t cap, int64_t d, int64_t t_new) {
    for (int64_t bi = 0; bi < b; ++bi)
        if ((int64_t)lens[bi] + t_new > cap) return 3;
    for (int64_t bi = 0; bi < b; ++bi) {
        for (int64_t h = 0; h < hkv; ++h) {
            float *kd = k_cache + ((bi * hkv + h) * cap + lens[bi]) * d;
            float *vd = v_cache + ((bi * hkv + h) * cap + lens[bi]) * d;
            const float *ks = k_new + (bi * hkv + h) * t_new * d;
            const float *vs = v_new + (bi * hkv + h) * t_new * d;
            memcpy(kd, ks, sizeof(float) * (size_t)(t_new * d));
            memcpy(vd, vs, sizeof(float) * (size_t)(t_new * d));
        }
        lens[bi] += (int32_t)t_new;
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* a7: one decode step over ragged sequences: append, then attend with t = 1  */
/* and no mask to all L rows including the new one (llama.rs:239-296 with     */
/* t = 1).  The reference batch path needs equal L, so each sequence is its   */
/* own B = 1 call; that is what this loop does.                               */
/* ------------------------------------------------------------------------- */

typedef struct {
    const float *q;
    const float *k_cache, *v_cache;
    const int32_t *lens;
    float *out;
    int64_t hq, hkv, cap, d;
    float scale;
} dec_ctx;

static void dec_item(void *vctx, int64_t bhq) {
    const dec_ctx *c = (const dec_ctx *)vctx;
    const int64_t bi = bhq / c->hq, h = bhq % c->hq, d = c->d;
    const int64_t kvh = h / (c->hq / c->hkv);                 /* llama.rs:256-266 */
    const float *qv = c->q + bhq * d;
    const float *kk = c->k_cache + (bi * c->hkv + kvh) * c->cap * d;
    const float *vv = c->v_cache + (bi * c->hkv + kvh) * c->cap * d;
    float *o = c->out + bhq * d;
    const int64_t L = c->lens[bi];
    float *row = (float *)malloc(sizeof(float) * (size_t)(L ? L : 1));
    for (int64_t cc = 0; cc < L; ++cc) {                       /* llama.rs:272-274 */
        float dot = 0.0f;
        for (int64_t x = 0; x < d; ++x) dot += qv[x] * kk[cc * d + x];
        row[cc] = dot * c->scale;
    }
    if (L > 0) {                                               /* reduce.rs:256-267 */
        float mx = -INFINITY;
        for (int64_t cc = 0; cc < L; ++cc) if (row[cc] > mx) mx = row[cc];
        float sum = 0.0f;
        for (int64_t cc = 0; cc < L; ++cc) { row[cc] = expf(row[cc] - mx); sum += row[cc]; }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        for (int64_t cc = 0; cc < L; ++cc) row[cc] *= inv;
    }
    for (int64_t x = 0; x < d; ++x) {                          /* llama.rs:296 */
        float acc = 0.0f;
        for (int64_t cc = 0; cc < L; ++cc) acc += row[cc] * vv[cc * d + x];
        o[x] = acc;
    }
    free(row);
}

/* q [B,Hq,1,d]; caches [B][Hkv][cap][d]; lens[B] (updated); out [B,Hq,1,d].
 * k_new/v_new [B,Hkv,1,d] are appended first (llama.rs:239-251).
 * Returns 0, or 3 on capacity overflow (nothing is written then). */
int oracle_decode_step(const float *q, float *k_cache, float *v_cache, int32_t *lens,
                       const float *k_new, const float *v_new, float *out,
                       int64_t b, int64_t hq, int64_t hkv, int64_t cap, int64_t d,
                       int has_scale, float scale, int n_threads) {
    int rc = oracle_kv_append(k_cache, v_cache, lens, k_new, v_new, b, hkv, cap, d, 1);
    if (rc) return rc;
    dec_ctx c;
    c.q = q; c.k_cache = k_cache; c.v_cache = v_cache; c.lens = lens; c.out = out;
    c.hq = hq; c.hkv = hkv; c.cap = cap; c.d = d;
    c.scale = has_scale ? scale : 1.0f / sqrtf((float)d);
    parallel_for(dec_item, &c, b * hq, n_threads);
    return 0;
}

/* Same as oracle_decode_step without the append: attends q to the first
 * lens[b] rows of each sequence's cache. */
void oracle_decode_attend(const float *q, const float *k_cache, const float *v_cache,
                          const int32_t *lens, float *out, int64_t b, int64_t hq,
                          int64_t hkv, int64_t cap, int64_t d, int has_scale, float scale,
                          int n_threads) {
    dec_ctx c;
    c.q = q; c.k_cache = k_cache; c.v_cache = v_cache; c.lens = lens; c.out = out;
    c.hq = hq; c.hkv = hkv; c.cap = cap; c.d = d;
    c.scale = has_scale ? scale : 1.0f / sqrtf((float)d);
    parallel_for(dec_item, &c, b * hq, n_threads);
}

/* ------------------------------------------------------------------------- */
/* Decode prologue: Linear projections and rotary position embedding.        */
/* ------------------------------------------------------------------------- */

/* RotaryEmbedding::new (src/models/llama.rs:74-107): inv_freq[i] =
 * 1 / theta^((2i) / d) in f32; for every position p < max_seq_len and
 * i < d/2, cos[p][i] = cos[p][i + d/2] = cosf(p * inv_freq[i]) and the same
 * for sin.  Tables are [max_seq_len][d]. */
void oracle_rope_tables(float *cos_out, float *sin_out, int64_t max_seq_len, int64_t d,
                        float theta) {
    const int64_t half = d / 2;
    for (int64_t i = 0; i < half; ++i) {
        const float exponent = (float)(2 * i) / (float)d;
        const float inv_freq = 1.0f / powf(theta, exponent);
        for (int64_t p = 0; p < max_seq_len; ++p) {
            const float freq = (float)p * inv_freq;
            const float c = cosf(freq), s = sinf(freq);
            cos_out[p * d + i] = c;
            cos_out[p * d + i + half] = c;
            sin_out[p * d + i] = s;
            sin_out[p * d + i + half] = s;
        }
    }
}

/* RotaryEmbedding::apply (src/models/llama.rs:110-157) on x [B, H, T, d]:
 * out = x * cos + rotate_half(x) * sin with rotate_half(x) = [-x2, x1]
 * (:149-156), row t of sequence b taking table row start_pos[b] + t (the
 * reference slices rows [start_pos, start_pos + T), :141-142; ragged batches
 * give each sequence its own start).  Each product and the sum are rounded
 * to f32 separately, as the reference's three tensor ops are. */
void oracle_rope_apply(const float *x, float *out, const float *cos_t, const float *sin_t,
                       int64_t b, int64_t h, int64_t t, int64_t d, const int32_t *start_pos) {
    const int64_t half = d / 2;
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t hi = 0; hi < h; ++hi)
            for (int64_t ti = 0; ti < t; ++ti) {
                const int64_t pos = (int64_t)start_pos[bi] + ti;
                const float *c = cos_t + pos * d, *s = sin_t + pos * d;
                const float *xr = x + ((bi * h + hi) * t + ti) * d;
                float *o = out + ((bi * h + hi) * t + ti) * d;
                for (int64_t i = 0; i < d; ++i) {
                    const float rot = i < half ? -xr[i + half] : xr[i - half];
                    const float term1 = xr[i] * c[i];
                    const float term2 = rot * s[i];
                    o[i] = term1 + term2;
                }
            }
}

/* Linear::forward (src/nn/linear.rs:47-57): y = x W^T (+ b) with x [M, K],
 * W [N, K] (weight [out_features, in_features]), b [N] or NULL, y [M, N];
 * each dot product summed in k order in f32, then the bias added. */
void oracle_linear(const float *x, const float *w, const float *bias, float *y, int64_t m,
                   int64_t k, int64_t n) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (int64_t kk = 0; kk < k; ++kk) acc += x[i * k + kk] * w[j * k + kk];
            y[i * n + j] = bias ? acc + bias[j] : acc;
        }
}

/* Steps 1-2 of GroupedQueryAttention::forward_gqa_cached
 * (src/models/llama.rs:226-235) for x [B, T, C]: q = x Wq^T (+ bq) reshaped
 * [B, T, Hq, d] -> [B, Hq, T, d], the same for k and v with Hkv heads, then
 * RoPE on q and k at positions start_pos[b] + t.  Outputs are contiguous
 * [B, Hq, T, d] and [B, Hkv, T, d]. */
void oracle_qkv_rope(const float *x, const float *wq, const float *wk, const float *wv,
                     const float *bq, const float *bk, const float *bv, const float *cos_t,
                     const float *sin_t, const int32_t *start_pos, float *q_out, float *k_out,
                     float *v_out, int64_t b, int64_t t, int64_t c, int64_t hq, int64_t hkv,
                     int64_t d) {
    const int64_t m = b * t;
    float *yq = (float *)malloc(sizeof(float) * (size_t)(m * hq * d));
    float *yk = (float *)malloc(sizeof(float) * (size_t)(m * hkv * d));
    float *yv = (float *)malloc(sizeof(float) * (size_t)(m * hkv * d));
    float *tq = (float *)malloc(sizeof(float) * (size_t)(m * hq * d));
    float *tk = (float *)malloc(sizeof(float) * (size_t)(m * hkv * d));
    oracle_linear(x, wq, bq, yq, m, c, hq * d);
    oracle_linear(x, wk, bk, yk, m, c, hkv * d);
    oracle_linear(x, wv, bv, yv, m, c, hkv * d);
    /* [B, T, H, d] -> [B, H, T, d] (llama.rs:231-233) */
    for (int64_t bi = 0; bi < b; ++bi)
        for (int64_t ti = 0; ti < t; ++ti) {
            for (int64_t hi = 0; hi < hq; ++hi)
                memcpy(tq + ((bi * hq + hi) * t + ti) * d, yq + ((bi * t + ti) * hq + hi) * d,
                       sizeof(float) * (size_t)d);
            for (int64_t hi = 0; hi < hkv; ++hi) {
                memcpy(tk + ((bi * hkv + hi) * t + ti) * d, yk + ((bi * t + ti) * hkv + hi) * d,
                       sizeof(float) * (size_t)d);
                memcpy(v_out + ((bi * hkv + hi) * t + ti) * d, yv + ((bi * t + ti) * hkv + hi) * d,
                       sizeof(float) * (size_t)d);
            }
        }
    oracle_rope_apply(tq, q_out, cos_t, sin_t, b, hq, t, d, start_pos);
    oracle_rope_apply(tk, k_out, cos_t, sin_t, b, hkv, t, d, start_pos);
    free(yq); free(yk); free(yv); free(tq); free(tk);
}
