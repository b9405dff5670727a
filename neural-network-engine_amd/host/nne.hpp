// nne.hpp -- C++ host API of the MI355X attention path, mirroring the
// reference engine's Rust API for this path so that a caller (or a test) reads
// the same way as against the reference:
//
//   flash_attention_forward(q, k, v, is_causal, scale, block_size_r,
//                           block_size_c) -> Result<RawTensor>
//                                      src/nn/flash_attention.rs:19-199
//   FlashAttention{q_proj, k_proj, v_proj, out_proj, num_heads, d_model,
//                  head_dim, is_causal, block_size}, new / forward_flash /
//                  forward                src/nn/flash_attention.rs:202-292
//   Linear{weight, bias, in_features, out_features}, new / forward
//                                      src/nn/linear.rs:9-60
//   KVCache new / reset / num_layers / current_seq_len / update
//                                      src/nn/kv_cache.rs:11-74
//   EngineError / Result<T>            src/error.rs:6-58
//   RotaryEmbedding new / apply        src/models/llama.rs:64-158
//   GroupedQueryAttention new / forward_gqa_cached / forward_gqa
//                                      src/models/llama.rs:160-301
//   MultiHeadAttention new / forward_attention(_cached) /
//     forward_cross_attention(_cached) src/nn/attention.rs:9-210
//   WhisperKVCache                     src/models/whisper.rs:325-350
//
// Differences that come from the hardware, not from taste:
//   * RawTensor data live in device memory (HBM); to_vec() copies to the host.
//     Views (transpose, slice, reshape of contiguous data) share storage, as the
//     reference's strided RawTensor does (src/tensor/mod.rs:20-27).
//   * KVCache is device-resident with a capacity fixed at creation and rows
//     appended in place (the reference concatenates, kv_cache.rs:63-72); it
//     adds decode_step / attend for single-token decode (llama.rs:239-296,
//     t = 1) and accepts ragged per-sequence lengths.
//   * attention_forward is the grouped-query entry (Hkv divides Hq, query head
//     hq reads KV head hq / (Hq / Hkv), llama.rs:256-266; causal key c visible
//     to row r iff c <= r + q_offset) that the reference spreads over its
//     model code.
//   * randn / uniform draw from a seeded generator (manual_seed); the
//     reference's thread_rng is unseeded.
// Everything runs on the HIP default stream; every call that returns data to
// the host synchronises it.  All compute goes through include/nne_attn.h.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <variant>
#include <vector>

#include "nne_attn.h"

namespace nne {

// src/error.rs:8-52: the variants this path produces, with the same messages.
struct EngineError {
    enum class Kind { ShapeMismatch, IncompatibleShapes, InvalidArgument, GpuError, NonContiguousTensor };
    Kind kind = Kind::InvalidArgument;
    std::vector<size_t> expected, actual;        // ShapeMismatch
    std::string op;                              // IncompatibleShapes
    std::vector<std::vector<size_t>> shapes;     // IncompatibleShapes
    std::string message;                         // InvalidArgument / GpuError payload

    static EngineError shape_mismatch(std::vector<size_t> expected, std::vector<size_t> actual);
    static EngineError incompatible_shapes(std::string op, std::vector<std::vector<size_t>> shapes);
    static EngineError invalid_argument(std::string message);
    static EngineError gpu_error(std::string message);
    static EngineError non_contiguous_tensor();

    std::string to_string() const;               // the #[error(...)] text of the variant
    bool operator==(const EngineError& o) const;
};

// Result<T> = std::result::Result<T, EngineError> (src/error.rs:6).
template <class T>
class Result {
  public:
    Result(T value) : v_(std::move(value)) {}
    Result(EngineError error) : v_(std::move(error)) {}
    bool is_ok() const { return v_.index() == 0; }
    bool is_err() const { return v_.index() == 1; }
    const T& value() const { return check(), std::get<0>(v_); }
    T& value() { return check(), std::get<0>(v_); }
    const EngineError& error() const {
        if (is_ok()) throw std::logic_error("called error() on an Ok Result");
        return std::get<1>(v_);
    }
    // Rust's unwrap(): the value, or a std::runtime_error carrying the error text.
    T unwrap() { return check(), std::move(std::get<0>(v_)); }

  private:
    void check() const {
        if (is_err()) throw std::runtime_error(std::get<1>(v_).to_string());
    }
    std::variant<T, EngineError> v_;
};

// Seeds the generator behind RawTensor::randn / uniform and the layer inits.
void manual_seed(uint64_t seed);

// Strided f32 tensor in device memory (src/tensor/mod.rs:20-27).
class RawTensor {
  public:
    RawTensor() = default;                               // no storage, shape []

    // src/tensor/mod.rs:60-77; throws std::invalid_argument if data.size() != numel(shape).
    static RawTensor from_vec(const std::vector<float>& data, std::vector<size_t> shape);
    static RawTensor zeros(const std::vector<size_t>& shape);
    static RawTensor randn(const std::vector<size_t>& shape, float mean, float std);
    static RawTensor uniform(const std::vector<size_t>& shape, float low, float high);
    static RawTensor kaiming_uniform(const std::vector<size_t>& shape, size_t fan_in);

    const std::vector<size_t>& shape() const { return shape_; }
    const std::vector<size_t>& strides() const { return strides_; }  // in elements
    size_t ndim() const { return shape_.size(); }
    size_t numel() const;
    bool is_contiguous() const;

    float* data() const;                                 // device pointer of element 0
    std::vector<float> to_vec() const;                   // row-major copy on the host
    RawTensor to_contiguous() const;                     // device copy when strided

    Result<RawTensor> transpose(size_t a, size_t b) const;          // view
    Result<RawTensor> reshape(const std::vector<size_t>& shape) const;
    Result<RawTensor> slice(size_t axis, size_t start, size_t end) const;  // view

    // Wraps device memory owned elsewhere (kept alive by `owner`).
    static RawTensor view(std::shared_ptr<float> owner, size_t offset, std::vector<size_t> shape,
                          std::vector<size_t> strides);

  private:
    std::shared_ptr<float> storage_;
    size_t offset_ = 0;
    std::vector<size_t> shape_, strides_;
};

// src/nn/flash_attention.rs:19-199.  Output: a new contiguous [B, H, Tq, d].
Result<RawTensor> flash_attention_forward(const RawTensor& q, const RawTensor& k, const RawTensor& v,
                                          bool is_causal, std::optional<float> scale,
                                          size_t block_size_r, size_t block_size_c);

// Grouped-query attention core (llama.rs:253-296; attention.rs:93-122, 193-203):
// q [B, Hq, Tq, d], k/v [B, Hkv, Tk, d], Hkv | Hq.  Output: new contiguous [B, Hq, Tq, d].
Result<RawTensor> attention_forward(const RawTensor& q, const RawTensor& k, const RawTensor& v,
                                    bool is_causal, int64_t q_offset = 0,
                                    std::optional<float> scale = std::nullopt);

// src/nn/linear.rs:9-60: y = x W^T + b on the last axis (rocBLAS SGEMM).
class Linear {
  public:
    Linear(size_t in_features, size_t out_features);     // bias, Kaiming-uniform weight
    static Linear with_bias(size_t in_features, size_t out_features, bool has_bias);
    static Linear without_bias(size_t in_features, size_t out_features);
    Result<RawTensor> forward(const RawTensor& input) const;

    RawTensor weight;                                    // [out_features, in_features]
    std::optional<RawTensor> bias;                       // [out_features]
    size_t in_features = 0, out_features = 0;

  private:
    Linear() = default;
};

// src/nn/flash_attention.rs:202-292 (forward only: the reference's output is a leaf, :273).
class FlashAttention {
  public:
    // Throws std::invalid_argument unless num_heads divides d_model (the reference asserts).
    FlashAttention(size_t d_model, size_t num_heads, bool is_causal);
    // x [B, T, C] -> [B, T, C].  The projections are read as [B, H, T, d] views
    // and the attention output is written straight into [B, T, H, d], so the
    // reference's transpose/reshape copies (:259-275) disappear.
    Result<RawTensor> forward_flash(const RawTensor& x) const;
    Result<RawTensor> forward(const RawTensor& x) const { return forward_flash(x); }

    Linear q_proj, k_proj, v_proj, out_proj;
    size_t num_heads, d_model, head_dim;
    bool is_causal;
    size_t block_size = 64;
};

// src/nn/kv_cache.rs:11-74 on a device-resident, fixed-capacity layout:
// per layer K and V [B, Hkv, capacity, d] and per-sequence lengths.
class KVCache {
  public:
    KVCache(size_t num_layers, size_t batch, size_t num_kv_heads, size_t capacity, size_t head_dim);

    // One entry of the reference's `pub layers: Vec<Option<(Tensor, Tensor)>>`
    // (kv_cache.rs:13), as a handle on layer i of the device cache.  Reading
    // it materialises (K, V) views [B, Hkv, L, d] of the filled rows (L = the
    // longest sequence) -- no copy; assigning to it writes the device cache,
    // so the models' slot idioms keep their meaning:
    //   for (auto slot : cache.layers()) slot = {RawTensor::zeros({0}), RawTensor::zeros({0})};
    //                                  // llama.rs:501-503: an engaged, empty slot
    //   auto s = cache.layers().get_mut(i);   // llama.rs:464-468 (Option<&mut (K, V)>)
    //   slot = std::nullopt;                   // kv_cache.rs:25-29 (None)
    class Slot {
      public:
        bool has_value() const;                          // Some(..)
        explicit operator bool() const { return has_value(); }
        // The (K, V) views; throws std::bad_optional_access for None.
        std::pair<RawTensor, RawTensor> value() const;
        // *slot = None: the layer holds nothing (lengths 0).
        Slot& operator=(std::nullopt_t);
        // *slot = Some((k, v)): k, v [B, Hkv, L, d] (any strides, L <= capacity)
        // become the layer's rows 0..L; k of zero elements makes an empty,
        // engaged slot.  set() reports shape / capacity errors; operator=
        // throws them.
        Result<bool> set(const RawTensor& k, const RawTensor& v);
        Slot& operator=(const std::pair<RawTensor, RawTensor>& kv);
        // Option::take: contiguous copies of the rows, and the slot becomes None.
        std::optional<std::pair<RawTensor, RawTensor>> take();
        KVCache& cache() const { return *cache_; }
        size_t layer_idx() const { return layer_; }

      private:
        friend class KVCache;
        Slot(KVCache* c, size_t i) : cache_(c), layer_(i) {}
        KVCache* cache_;
        size_t layer_;
    };
    // The slots as a Vec-like range (size, operator[], get_mut, iteration).
    class Layers {
      public:
        class iterator {
          public:
            Slot operator*() const { return Slot(c_, i_); }
            iterator& operator++() { ++i_; return *this; }
            bool operator!=(const iterator& o) const { return i_ != o.i_; }

          private:
            friend class Layers;
            iterator(KVCache* c, size_t i) : c_(c), i_(i) {}
            KVCache* c_;
            size_t i_;
        };
        size_t size() const { return c_->num_layers(); }
        Slot operator[](size_t i) const;                 // throws std::out_of_range past the end
        std::optional<Slot> get_mut(size_t i) const;     // None past the end
        iterator begin() const { return iterator(c_, 0); }
        iterator end() const { return iterator(c_, size()); }

      private:
        friend class KVCache;
        explicit Layers(KVCache* c) : c_(c) {}
        KVCache* c_;
    };
    Layers layers() { return Layers(this); }

    void reset();                                        // kv_cache.rs:25-29
    size_t num_layers() const;                           // kv_cache.rs:32-34
    size_t current_seq_len(size_t layer_idx) const;      // kv_cache.rs:37-44 (longest sequence)

    // kv_cache.rs:49-74: appends k_new / v_new [B, Hkv, t, d] to every sequence
    // and returns views [B, Hkv, L, d] of the filled rows (L = longest sequence).
    Result<std::pair<RawTensor, RawTensor>> update(size_t layer_idx, const RawTensor& k_new,
                                                   const RawTensor& v_new);
    // Single-token decode: q [B, Hq, 1, d] attends to the cached rows of its sequence.
    Result<RawTensor> attend(size_t layer_idx, const RawTensor& q,
                             std::optional<float> scale = std::nullopt);
    // Append one row per sequence, then attend (llama.rs:239-296 with t = 1).
    Result<RawTensor> decode_step(size_t layer_idx, const RawTensor& q, const RawTensor& k_new,
                                  const RawTensor& v_new, std::optional<float> scale = std::nullopt);
    // Declares rows [0, lens[b]) of each sequence filled (ragged batches).
    Result<bool> set_lengths(size_t layer_idx, const std::vector<int32_t>& lens);

    RawTensor k(size_t layer_idx) const;                 // full [B, Hkv, capacity, d]
    RawTensor v(size_t layer_idx) const;
    const std::vector<int32_t>& lengths(size_t layer_idx) const;
    const int32_t* lengths_device(size_t layer_idx) const;   // the same lengths on the device

    size_t batch, num_kv_heads, capacity, head_dim;

  private:
    Result<bool> check_layer(size_t layer_idx) const;
    // The cache's own decode workspace (records + zeroed counters), grown to
    // what num_heads query heads need; the library allocates nothing.
    const ::nne_workspace_t* workspace(size_t num_heads);

    struct Layer {
        std::shared_ptr<float> k, v;
        std::shared_ptr<int32_t> lens_dev;
        std::vector<int32_t> lens_host;
        bool engaged = false;    // Some(..) in the reference's slot vector
    };
    std::vector<Layer> layers_;
    std::shared_ptr<void> ws_;
    std::shared_ptr<uint32_t> counters_;
    std::shared_ptr<::nne_workspace_t> ws_desc_;
};

// src/models/llama.rs:64-158.  Tables are built on the host in f32 exactly as
// the reference builds them and kept on the device.
class RotaryEmbedding {
  public:
    // Throws std::invalid_argument for an odd head_dim (the reference asserts, :75).
    RotaryEmbedding(size_t head_dim, size_t max_seq_len, float theta);
    // :110-157: x [B, H, T, D] (any strides) -> new contiguous tensor, row t of
    // every sequence rotated at position start_pos + t.
    Result<RawTensor> apply(const RawTensor& x, size_t start_pos) const;
    // Per-sequence start positions (ragged caches).
    Result<RawTensor> apply(const RawTensor& x, const std::vector<int32_t>& start_pos) const;

    RawTensor cos_cached, sin_cached;                    // [1, 1, max_seq_len, head_dim]
    size_t head_dim, max_seq_len;
};

// src/models/llama.rs:160-300, forward only.  Decode steps (t = 1 with a cache)
// run the fused projection + RoPE launch on weights packed at construction and
// the append + attend launch; other inputs project with GEMMs, rotate, append
// and run the attention kernel with q_offset = start_pos.
class GroupedQueryAttention {
  public:
    // Throws std::invalid_argument unless num_heads divides d_model and
    // num_kv_heads divides num_heads (the reference asserts, :174-183).
    GroupedQueryAttention(size_t d_model, size_t num_heads, size_t num_kv_heads, size_t max_seq_len,
                          float rope_theta = 10000.f);
    // :205-296.  x [B, T, C].  With a cache, start_pos must equal the cached
    // length of every sequence of the layer (the reference's start_pos is the
    // cache length, :525).
    Result<RawTensor> forward_gqa_cached(const RawTensor& x, size_t start_pos, KVCache* cache = nullptr,
                                         size_t layer_idx = 0);
    // The reference's call shape, forward_gqa_cached(x, start_pos, layer_slot)
    // (llama.rs:463-471): an empty optional or a None slot runs uncached.
    Result<RawTensor> forward_gqa_cached(const RawTensor& x, size_t start_pos,
                                         std::optional<KVCache::Slot> layer_cache);
    Result<RawTensor> forward_gqa(const RawTensor& x, size_t start_pos) {   // :298-301
        return forward_gqa_cached(x, start_pos, nullptr);
    }
    // Re-packs q/k/v_proj weights for the fused decode projection; call after
    // changing them.
    void repack();

    Linear q_proj, k_proj, v_proj, o_proj;
    RotaryEmbedding rope;
    size_t num_heads, num_kv_heads, head_dim, num_queries_per_kv;

  private:
    std::shared_ptr<float> w_packed_;                    // null when d or d_model is not a multiple of 64
};

// src/nn/attention.rs:9-210, forward only: biased projections (Linear::new),
// causal or full self-attention with an optional KV cache (bottom-right mask
// q_offset = L - T for multi-token steps, :101-108), and cross-attention whose
// projected memory K/V are computed once into a slot (:139-191).
class MultiHeadAttention {
  public:
    // Throws std::invalid_argument unless num_heads divides d_model (:23-30).
    MultiHeadAttention(size_t d_model, size_t num_heads, bool is_causal);
    Result<RawTensor> forward_attention(const RawTensor& x) { return forward_attention_cached(x, nullptr); }
    // :51-129.  x [B, T, C]; cache layer layer_idx holds this layer's rows.
    Result<RawTensor> forward_attention_cached(const RawTensor& x, KVCache* cache, size_t layer_idx = 0);
    // forward_attention_cached(x, layer_slot) as GPT-2 calls it (gpt2.rs:141).
    Result<RawTensor> forward_attention_cached(const RawTensor& x, std::optional<KVCache::Slot> layer_cache);
    // :132-210.  x [B, T_q, C], memory [B, T_kv, C]; slot (if given) caches the
    // projected memory K/V [B, H, T_kv, d] on its first use.
    Result<RawTensor> forward_cross_attention(const RawTensor& x, const RawTensor& memory) {
        return forward_cross_attention_cached(x, memory, nullptr);
    }
    Result<RawTensor> forward_cross_attention_cached(const RawTensor& x, const RawTensor& memory,
                                                     std::optional<std::pair<RawTensor, RawTensor>>* slot);
    void repack();   // after changing q/k/v_proj weights

    Linear q_proj, k_proj, v_proj, out_proj;
    size_t num_heads, d_model, head_dim;
    bool is_causal;

  private:
    std::shared_ptr<float> w_packed_;
};

// src/models/whisper.rs:325-350: per decoder layer a self-attention cache and a
// cross-attention slot (empty until the first decoding step projects memory).
struct WhisperKVCache {
    WhisperKVCache(size_t num_layers, size_t batch, size_t num_heads, size_t capacity, size_t head_dim)
        : self_attn(num_layers, batch, num_heads, capacity, head_dim), cross_attn(num_layers) {}
    void reset() {                                       // whisper.rs:342-350
        self_attn.reset();
        for (auto& s : cross_attn) s.reset();
    }
    KVCache self_attn;
    std::vector<std::optional<std::pair<RawTensor, RawTensor>>> cross_attn;
};

}  // namespace nne
