/*
 * nne_attn.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Drop-in boundary for elvin-mark/neural-network-engine's attention forward:
 * the Rust side keeps its Tensor / FlashAttention / KVCache API and calls these
 * functions through a thin `extern "C"` crate.  Plain pointers and sizes only:
 * every tensor argument is a DEVICE pointer to f32 data plus a 4-D shape and
 * element strides ([batch, head, row, dim]); a NULL strides pointer means
 * row-major contiguous.  `stream` is a hipStream_t (NULL = default stream).
 * Calls enqueue work and return without synchronising.
 *
 * Return value: NNE_OK or an error code that maps onto the reference's
 * EngineError (src/error.rs:6-58); nne_last_error() returns the message of the
 * calling thread's last failure.  No call aborts the process.
 *
 * Threads: any entry point may be called from several threads at once, as the
 * reference's functions may (Module: Send + Sync, src/nn/module.rs:7).  Calls
 * on one stream, from one thread or several (the NULL stream is shared by
 * all threads), run in that stream's order and share the workspace and
 * counters the library keeps for it when the caller passes none.  The caller
 * orders calls that write the same output or the same KV cache, and calls
 * nne_stream_release only when no other call uses that stream.
 *
 * Ownership: every device buffer a call touches can be the caller's.  Inputs,
 * outputs and KV caches always are; the scratch of split computations is the
 * caller's nne_workspace_t when one is passed (see below), and only a NULL
 * workspace makes the library use memory of its own.
 */
#ifndef NNE_ATTN_H
#define NNE_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    NNE_OK = 0,
    NNE_EINVAL = 1,    /* EngineError::InvalidArgument   (src/error.rs:42) */
    NNE_ESHAPE = 2,    /* EngineError::ShapeMismatch     (src/error.rs:12) */
    NNE_ECAPACITY = 3, /* KV cache append past capacity -> EngineError::GpuError */
    NNE_EHIP = 4       /* HIP runtime failure            -> EngineError::GpuError (src/error.rs:48) */
};

#define NNE_ABI_VERSION 4

int nne_abi_version(void);

/* Message for the calling thread's last non-OK return (empty if none). */
const char *nne_last_error(void);

/* ---- device memory owned by the caller (the Rust side) -------------------
 * The reference keeps tensors in host Vec<f32> storage (src/tensor/storage.rs:84-163);
 * on the GPU path the caller allocates and frees device buffers with these. */
int nne_dev_alloc(void **ptr, uint64_t bytes);
int nne_dev_free(void *ptr);
int nne_memcpy_h2d(void *dst, const void *src, uint64_t bytes, void *stream);
int nne_memcpy_d2h(void *dst, const void *src, uint64_t bytes, void *stream);
int nne_memcpy_d2d(void *dst, const void *src, uint64_t bytes, void *stream);
int nne_stream_sync(void *stream);
/* Frees the workspace and arrival counters the library keeps for `stream` on
 * the current device (used by nne_attention_forward and
 * nne_flash_attention_forward on small or few-query problems, by the decode
 * entry points with a NULL workspace and by nne_qkv_rope), after waiting for
 * the stream.  Call it before destroying a stream the library has used; a
 * later call on the stream allocates them again.  No counterpart in the
 * reference, whose CPU path allocates per call: it is for long-running
 * callers that create and destroy streams. */
int nne_stream_release(void *stream);

/* Bytes of device memory the library holds for `stream` on the current
 * device (its per-stream workspace and counters, retired ones included); 0
 * when every call on the stream brought its own workspace.  No counterpart
 * in the reference: a check for callers that own all buffers. */
uint64_t nne_stream_resource_bytes(void *stream);

/* ---- caller-owned workspace ----------------------------------------------
 * Split computations hand partial results between the workgroups of one
 * launch: split-K decode and few-query attention, the key split of prefill
 * problems too small to fill the device, and the fused decode prologue.
 * They need
 *   records   device memory for the partial records (no initialisation), and
 *   counters  uint32 arrival counters that are zero when the call starts;
 *             every call leaves the counters it used at zero, so an array
 *             zeroed once with nne_counters_init serves any number of calls
 *             of any entry point.
 * Alignment: records at least 16-byte aligned (the kernels move them with
 * 16-byte loads and stores; allocations from hipMalloc are 256-byte aligned),
 * counters 4-byte aligned -- NNE_EINVAL otherwise.
 * The *_workspace_size queries give what a call needs; one workspace sized
 * for the largest of them serves every call.  Calls that share a workspace
 * must not overlap in time (calls on one stream never do).  A NULL
 * workspace makes the call use the library's per-stream one (allocated in
 * stream order on first use, kept until nne_stream_release or the end of the
 * process). */
typedef struct nne_workspace {
    void *records;          /* device memory, records_bytes long */
    uint64_t records_bytes;
    uint32_t *counters;     /* device array of n_counters zeroed counters */
    uint64_t n_counters;
} nne_workspace_t;

typedef struct nne_workspace_size {
    uint64_t records_bytes;
    uint64_t n_counters;
} nne_workspace_size_t;

/* Zeroes n counters on the stream with a fill kernel (no memset node, so the
 * call can be captured in a HIP graph). */
int nne_counters_init(uint32_t *counters, uint64_t n, void *stream);

/* ---- prefill -------------------------------------------------------------
 * Replaces `flash_attention_forward(q, k, v, is_causal, scale, block_size_r,
 * block_size_c) -> Result<RawTensor>` (src/nn/flash_attention.rs:19-199).
 * Same checks and error classes as the reference: K and V must match Q in
 * batch, heads and head dim and each other in length (:43-48, NNE_ESHAPE);
 * has_scale = 0 means scale = 1/sqrt(d) (:50); block sizes are accepted and
 * only validated (they change the reference's rounding order, not the result).
 * Causal masking is top-left: key c is visible to query row r iff c <= r
 * (:113).  Rows that see no key are zero (:186-194).  `o` has Q's shape.
 * Any head dim; above 128 the tensors must be 16-byte vector views
 * (d % 4 == 0, unit dim stride, other strides multiples of 4, 16-byte
 * aligned) -- NNE_EINVAL otherwise.  Above 256 dims a separate kernel runs
 * (MFMA, K/V read straight into operand layout), and so do 129-255 dims and
 * d = 256 problems too small to fill the device on the 256-dim kernel;
 * problems with too few query rows to fill the device split their keys over
 * several workgroups, with records in the workspace. */
int nne_flash_attention_forward(const float *q, const int64_t q_shape[4], const int64_t q_strides[4],
                                const float *k, const int64_t k_shape[4], const int64_t k_strides[4],
                                const float *v, const int64_t v_shape[4], const int64_t v_strides[4],
                                float *o, const int64_t o_strides[4], int is_causal, int has_scale,
                                float scale, int64_t block_size_r, int64_t block_size_c, void *stream);

/* Grouped-query / offset generalisation of the same forward, for the
 * reference's standard attention paths: GroupedQueryAttention::forward_gqa_cached
 * (src/models/llama.rs:253-296), MultiHeadAttention::forward_attention_cached
 * (src/nn/attention.rs:93-122) and forward_cross_attention_cached
 * (src/nn/attention.rs:193-203).  k_shape[1] must divide q_shape[1]; query
 * head hq reads KV head hq / (Hq / Hkv) (llama.rs:256-266).  With is_causal,
 * key c is visible to row r iff c <= r + q_offset (llama.rs uses
 * q_offset = start_pos, attention.rs uses Tk - Tq).  The reference's additive
 * -1e4 mask and this exact exclusion give identical f32 results whenever
 * |scores| < ~4e3.  Few-query problems (Hq/Hkv * Tq <= 16 rows per KV head,
 * causal or not) run on the split-K kernel; problems with fewer work items
 * than the device has CUs split their key range across workgroups.  Both use
 * the library's per-stream workspace and counters here; nne_attention_forward_ws
 * takes the caller's. */
int nne_attention_forward(const float *q, const int64_t q_shape[4], const int64_t q_strides[4],
                          const float *k, const int64_t k_shape[4], const int64_t k_strides[4],
                          const float *v, const int64_t v_shape[4], const int64_t v_strides[4],
                          float *o, const int64_t o_strides[4], int is_causal, int64_t q_offset,
                          int has_scale, float scale, void *stream);

/* Workspace a prefill call of this geometry may need (an upper bound over
 * every layout of the same shapes); {0, 0} for problems that need none.
 * NNE_ESHAPE / NNE_EINVAL as the call itself would return. */
int nne_attention_workspace_size(const int64_t q_shape[4], const int64_t k_shape[4], int is_causal,
                                 int64_t q_offset, nne_workspace_size_t *out);

/* nne_flash_attention_forward and nne_attention_forward with the caller's
 * workspace (NULL: the library's per-stream one). */
int nne_flash_attention_forward_ws(const float *q, const int64_t q_shape[4],
                                   const int64_t q_strides[4], const float *k,
                                   const int64_t k_shape[4], const int64_t k_strides[4],
                                   const float *v, const int64_t v_shape[4],
                                   const int64_t v_strides[4], float *o, const int64_t o_strides[4],
                                   int is_causal, int has_scale, float scale, int64_t block_size_r,
                                   int64_t block_size_c, const nne_workspace_t *ws, void *stream);
int nne_attention_forward_ws(const float *q, const int64_t q_shape[4], const int64_t q_strides[4],
                             const float *k, const int64_t k_shape[4], const int64_t k_strides[4],
                             const float *v, const int64_t v_shape[4], const int64_t v_strides[4],
                             float *o, const int64_t o_strides[4], int is_causal, int64_t q_offset,
                             int has_scale, float scale, const nne_workspace_t *ws, void *stream);

/* ---- KV cache ------------------------------------------------------------
 * Replaces KVCache (src/nn/kv_cache.rs:11-74) and the per-layer
 * (Tensor, Tensor) slots models append to with Tensor::cat (llama.rs:239-251,
 * attention.rs:79-91).  Storage per layer: K and V device buffers laid out
 * [B][Hkv][capacity][d] (head-major, contiguous, d % 4 == 0), plus the
 * sequence lengths kept twice: lens_dev (int32[B], device, read by kernels)
 * and lens_host (int32[B], host, used for validation and launch sizing).
 * Functions that append update both. */

/* Appends k_new / v_new ([B, Hkv, t_new, d], any strides) at row lens[b] of
 * every (b, kv head) in place -- the KVCache::update of kv_cache.rs:49-74
 * without the O(L) copy.  NNE_ECAPACITY (nothing written) if some
 * lens_host[b] + t_new > capacity. */
int nne_kv_append(float *k_cache, float *v_cache, int32_t *lens_dev, int32_t *lens_host,
                  const float *k_new, const int64_t k_new_strides[4], const float *v_new,
                  const int64_t v_new_strides[4], int64_t B, int64_t Hkv, int64_t capacity,
                  int64_t d, int64_t t_new, void *stream);

/* Records bytes a decode call of this geometry needs (any cache length, or
 * cache lengths up to max_len when max_len > 0 above 256 dims; 0 for
 * geometry no decode kernel takes).  Above 256 dims the records serve the
 * deep kernel's key split, used when the batch has too few (sequence, KV
 * head) pairs to fill the device: a smaller caller workspace gives fewer key
 * parts, never an error, and no counters are needed.  Up to 256 dims decode
 * calls also need B * Hkv counters: nne_decode_workspace_size gives both
 * (NNE_EINVAL for geometry no decode call takes). */
uint64_t nne_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t d, int64_t max_len);
int nne_decode_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t d,
                              nne_workspace_size_t *out);

/* Single-token decode attention over the cache: q [B, Hq, 1, d] attends to
 * the first lens[b] rows of its sequence, no mask (llama.rs:239-296 with
 * t = 1).  Ragged lengths, any Hq / Hkv, any batch, any head dim that is a
 * multiple of 4.  With more than 4 query heads per KV head or d > 128, q
 * must be a 16-byte vector view (strides multiples of 4, 16-byte aligned;
 * above 256 dims o too).  Up to 256 dims NNE_EINVAL if capacity * d >= 2^30
 * (a head's rows are addressed with 32-bit byte offsets).  ws: the caller's
 * workspace of at least nne_decode_workspace_size, or NULL for the library's
 * per-stream one. */
int nne_decode_attention(const float *q, const int64_t q_strides[4], const float *k_cache,
                         const float *v_cache, const int32_t *lens_dev, const int32_t *lens_host,
                         float *o, const int64_t o_strides[4], int64_t B, int64_t Hq, int64_t Hkv,
                         int64_t capacity, int64_t d, int has_scale, float scale,
                         const nne_workspace_t *ws, void *stream);

/* One decode step with the semantics of nne_kv_append of one row followed by
 * nne_decode_attention -- the append-then-attend order of llama.rs:239-296
 * and attention.rs:79-122 -- fused: the new row is attended from k_new /
 * v_new directly and stored into the cache by the attention kernel, and
 * lens_dev / lens_host advance by one (above 256 dims: the append kernel,
 * then the attention kernel, in stream order).  ws as for nne_decode_attention.
 * NNE_ECAPACITY (nothing written) if a sequence is full. */
int nne_decode_step(const float *q, const int64_t q_strides[4], float *k_cache, float *v_cache,
                    int32_t *lens_dev, int32_t *lens_host, const float *k_new,
                    const int64_t k_new_strides[4], const float *v_new,
                    const int64_t v_new_strides[4], float *o, const int64_t o_strides[4],
                    int64_t B, int64_t Hq, int64_t Hkv, int64_t capacity, int64_t d,
                    int has_scale, float scale, const nne_workspace_t *ws, void *stream);

/* Bytes of device scratch behind nne_decode_step_noalloc, one copy per GPU. */
#define NNE_NOALLOC_SCRATCH_BYTES (16u << 20)

/* No counterpart in the reference: a variant of nne_decode_step for callers
 * that cannot allocate device memory during the call (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, semantics and errors as nne_decode_step without the workspace:
 * its split-K partial records and arrival counters live in a static device
 * array of NNE_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds
 * until the process ends, and the call makes no device allocation (no
 * hipMalloc or hipFree; it clears its counters with a fill kernel, not a
 * memset).  Like nne_decode_step, the call plans the step on the host from
 * lens_host (split layout, append row) and advances lens_host itself; a HIP
 * graph captured from one call therefore replays that same step, for the same
 * lengths, and does not advance to later steps.  NNE_EINVAL if the step needs
 * more scratch than that (at
 * d = 128 it holds about 7800 (sequence, KV head) pairs with up to 4 query
 * heads per KV head, about 1700 with up to 16); above 256 dims the scratch
 * holds the key split's records, and a step whose records do not fit takes
 * fewer key parts instead.  Every
 * call on a GPU shares that GPU's array: calls that overlap in time on one
 * GPU (any stream, any thread) race, and the caller must serialise them. */
int nne_decode_step_noalloc(const float *q, const int64_t q_strides[4], float *k_cache,
                            float *v_cache, int32_t *lens_dev, int32_t *lens_host,
                            const float *k_new, const int64_t k_new_strides[4], const float *v_new,
                            const int64_t v_new_strides[4], float *o, const int64_t o_strides[4],
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t capacity, int64_t d,
                            int has_scale, float scale, void *stream);

/* ---- decode prologue -----------------------------------------------------
 * The steps of GroupedQueryAttention::forward_gqa_cached before attention
 * (src/models/llama.rs:226-235): q/k/v projections (Linear::forward,
 * src/nn/linear.rs:47-57) and rotary position embedding (RotaryEmbedding,
 * llama.rs:64-158).  Positions are per sequence: the reference's start_pos
 * (the cache length before the step, llama.rs:525) for each b. */

/* RotaryEmbedding::new (llama.rs:74-107): fills HOST arrays cos_out and
 * sin_out of max_seq_len * head_dim floats, in f32 exactly as the reference
 * (inv_freq[i] = 1 / theta^(2i / head_dim); both halves of a row hold
 * cos / sin(pos * inv_freq[i])).  Copy them to the device once
 * (nne_memcpy_h2d).  NNE_EINVAL for an odd head_dim (the reference asserts). */
int nne_rope_tables(float *cos_out, float *sin_out, int64_t max_seq_len, int64_t head_dim,
                    float theta);

/* RotaryEmbedding::apply (llama.rs:110-157) on a [B, H, T, d] view: row t of
 * sequence b is rotated with table row start[b] + t (start_dev on the device,
 * start_host the same values on the host, for validation).  out may be x with
 * the same strides.  Products and the sum are rounded like the reference's
 * x * cos + rotate_half(x) * sin, so results are bit-identical to it.
 * NNE_ESHAPE if d != table_head_dim (:119-124); NNE_EINVAL if a range
 * [start, start + T) exceeds max_seq_len (:131-139). */
int nne_rope_apply(const float *x, const int64_t x_shape[4], const int64_t x_strides[4], float *out,
                   const int64_t out_strides[4], const float *cos_table, const float *sin_table,
                   int64_t max_seq_len, int64_t table_head_dim, const int32_t *start_dev,
                   const int32_t *start_host, void *stream);

/* Bytes of the packed q/k/v weights of nne_qkv_pack (0 for unsupported
 * geometry: d and C must be multiples of 64). */
uint64_t nne_qkv_packed_bytes(int64_t C, int64_t Hq, int64_t Hkv, int64_t d);

/* Packs the three Linear weights of GroupedQueryAttention (q_proj, k_proj,
 * v_proj: [H * d, C] row-major, llama.rs:189-192) once, into the order the
 * fused projection streams them (tiles of 64 output columns holding 32 RoPE
 * pairs, 64-wide slices of C, MFMA lane order).  The weights are static, so
 * this runs once per layer; packed must hold nne_qkv_packed_bytes bytes. */
int nne_qkv_pack(const float *wq, const float *wk, const float *wv, float *packed, int64_t C,
                 int64_t Hq, int64_t Hkv, int64_t d, void *stream);

/* Fused decode prologue (t = 1): for every sequence b, with x row b at
 * x + b * x_row_stride ([B, C], d_model C),
 *   q = RoPE(x Wq^T + bq), k = RoPE(x Wk^T + bk), v = x Wv^T + bv
 * at position pos[b] (pos_dev on the device, pos_host for validation), split
 * into heads and written to contiguous q_out [B, Hq, 1, d], k_out and v_out
 * [B, Hkv, 1, d] -- the q, k_new and v_new of nne_decode_step, which appends
 * k/v in place and attends.  w_packed comes from nne_qkv_pack; biases are
 * [H * d] or NULL (llama.rs uses Linear::without_bias).  One launch streams
 * the weights once; the reduction over C is split across workgroups whose
 * partial sums are merged inside the launch, in a fixed order, with the
 * library's per-stream workspace and counters (nne_qkv_rope_ws takes the
 * caller's).
 * Requires d % 64 == 0, C % 64 == 0, x rows 16-byte aligned with
 * x_row_stride >= C and a multiple of 4.  NNE_ESHAPE if d != table_head_dim;
 * NNE_EINVAL if pos[b] >= max_seq_len.  With cos_table = sin_table = NULL
 * nothing is rotated and positions are not read: the q/k/v projections of
 * MultiHeadAttention::forward_attention_cached (src/nn/attention.rs:66-75,
 * with biases, as GPT-2 and Whisper use it). */
int nne_qkv_rope(const float *x, int64_t x_row_stride, const float *w_packed, const float *bq,
                 const float *bk, const float *bv, const float *cos_table, const float *sin_table,
                 int64_t max_seq_len, int64_t table_head_dim, const int32_t *pos_dev,
                 const int32_t *pos_host, float *q_out, float *k_out, float *v_out, int64_t B,
                 int64_t C, int64_t Hq, int64_t Hkv, int64_t d, void *stream);

/* Workspace of nne_qkv_rope_ws (any B). */
int nne_qkv_workspace_size(int64_t C, int64_t Hq, int64_t Hkv, int64_t d, nne_workspace_size_t *out);

/* nne_qkv_rope with the caller's workspace (NULL: the library's per-stream one). */
int nne_qkv_rope_ws(const float *x, int64_t x_row_stride, const float *w_packed, const float *bq,
                    const float *bk, const float *bv, const float *cos_table, const float *sin_table,
                    int64_t max_seq_len, int64_t table_head_dim, const int32_t *pos_dev,
                    const int32_t *pos_host, float *q_out, float *k_out, float *v_out, int64_t B,
                    int64_t C, int64_t Hq, int64_t Hkv, int64_t d, const nne_workspace_t *ws,
                    void *stream);

#ifdef __cplusplus
}
#endif

#endif /* NNE_ATTN_H */
