// C++ host API of the attention path (declared in nne.hpp): tensors in device
// memory, the reference's function / layer / cache API, and error mapping
// from the C ABI's status codes onto EngineError.  Attention itself always
// runs through include/nne_attn.h; the two small kernels here only gather a
// strided tensor and add a bias row.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <random>
#include <sstream>

#include "nne.hpp"
#include "nne_attn.h"

namespace nne {

namespace {

constexpr int kMaxDims = 8;

struct GatherArgs {
    const float* src;
    float* dst;
    int64_t n;
    int nd;
    int64_t shape[kMaxDims];
    int64_t stride[kMaxDims];
};

__global__ void gather_kernel(GatherArgs a) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < a.n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t idx = i, off = 0;
        for (int d = a.nd - 1; d >= 0; --d) {
            const int64_t c = idx % a.shape[d];
            idx /= a.shape[d];
            off += c * a.stride[d];
        }
        a.dst[i] = a.src[off];
    }
}

__global__ void bias_add_kernel(float* y, const float* bias, int64_t rows, int64_t cols) {
    const int64_t n = rows * cols;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        y[i] += bias[i % cols];
}

unsigned grid_for(int64_t n) {
    int64_t blocks = (n + 255) / 256;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(blocks, 4096));
}

std::string dims(const std::vector<size_t>& v) {      // Rust {:?} of a Vec<usize>
    std::ostringstream s;
    s << "[";
    for (size_t i = 0; i < v.size(); ++i) s << (i ? ", " : "") << v[i];
    s << "]";
    return s.str();
}

std::mutex g_rng_mu;
std::mt19937_64 g_rng(0x5EED);

std::vector<size_t> contiguous_strides(const std::vector<size_t>& shape) {
    std::vector<size_t> st(shape.size());
    size_t acc = 1;
    for (size_t i = shape.size(); i-- > 0;) {
        st[i] = acc;
        acc *= shape[i];
    }
    return st;
}

size_t count(const std::vector<size_t>& shape) {
    size_t n = 1;
    for (size_t s : shape) n *= s;
    return n;
}

// Strips the Display prefix the C ABI puts in front of its messages, so that
// EngineError::to_string() does not repeat it.
std::string payload(const char* msg, const char* prefix) {
    std::string m = msg ? msg : "";
    const size_t n = std::strlen(prefix);
    return m.compare(0, n, prefix) == 0 ? m.substr(n) : m;
}

EngineError from_status(int rc) {
    const char* msg = nne_last_error();
    if (rc == NNE_EINVAL) return EngineError::invalid_argument(payload(msg, "Invalid configuration or argument: "));
    return EngineError::gpu_error(payload(msg, "GPU compute error: "));
}

// Device allocation through the C ABI; zero bytes gives an empty pointer.
template <class T>
std::shared_ptr<T> device_alloc(size_t n) {
    void* p = nullptr;
    if (nne_dev_alloc(&p, (uint64_t)n * sizeof(T)) != NNE_OK)
        throw std::runtime_error(from_status(NNE_EHIP).to_string());
    return std::shared_ptr<T>(static_cast<T*>(p), [](T* q) { nne_dev_free(q); });
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess)
        throw std::runtime_error(EngineError::gpu_error(std::string(what) + ": " + hipGetErrorString(e)).to_string());
}

std::vector<int64_t> as_i64(const std::vector<size_t>& v) { return std::vector<int64_t>(v.begin(), v.end()); }

}  // namespace

// ---- EngineError ------------------------------------------------------------

EngineError EngineError::shape_mismatch(std::vector<size_t> expected, std::vector<size_t> actual) {
    EngineError e;
    e.kind = Kind::ShapeMismatch;
    e.expected = std::move(expected);
    e.actual = std::move(actual);
    return e;
}
EngineError EngineError::incompatible_shapes(std::string op, std::vector<std::vector<size_t>> shapes) {
    EngineError e;
    e.kind = Kind::IncompatibleShapes;
    e.op = std::move(op);
    e.shapes = std::move(shapes);
    return e;
}
EngineError EngineError::invalid_argument(std::string message) {
    EngineError e;
    e.kind = Kind::InvalidArgument;
    e.message = std::move(message);
    return e;
}
EngineError EngineError::gpu_error(std::string message) {
    EngineError e;
    e.kind = Kind::GpuError;
    e.message = std::move(message);
    return e;
}
EngineError EngineError::non_contiguous_tensor() {
    EngineError e;
    e.kind = Kind::NonContiguousTensor;
    return e;
}

std::string EngineError::to_string() const {
    switch (kind) {
        case Kind::ShapeMismatch:
            return "Shape mismatch error: expected shape " + dims(expected) + ", got " + dims(actual);
        case Kind::IncompatibleShapes: {
            std::string s = "Incompatible shapes for operation " + op + ": [";
            for (size_t i = 0; i < shapes.size(); ++i) s += (i ? ", " : "") + dims(shapes[i]);
            return s + "]";
        }
        case Kind::InvalidArgument: return "Invalid configuration or argument: " + message;
        case Kind::GpuError: return "GPU compute error: " + message;
        case Kind::NonContiguousTensor: return "Tensor is not contiguous in memory";
    }
    return "";
}

bool EngineError::operator==(const EngineError& o) const {
    return kind == o.kind && expected == o.expected && actual == o.actual && op == o.op &&
           shapes == o.shapes && message == o.message;
}

// ---- RawTensor ---------------------------------------------------------------

void manual_seed(uint64_t seed) {
    std::lock_guard<std::mutex> lock(g_rng_mu);
    g_rng.seed(seed);
}

RawTensor RawTensor::view(std::shared_ptr<float> owner, size_t offset, std::vector<size_t> shape,
                          std::vector<size_t> strides) {
    RawTensor t;
    t.storage_ = std::move(owner);
    t.offset_ = offset;
    t.shape_ = std::move(shape);
    t.strides_ = std::move(strides);
    return t;
}

RawTensor RawTensor::from_vec(const std::vector<float>& data, std::vector<size_t> shape) {
    const size_t n = count(shape);
    if (data.size() != n)
        throw std::invalid_argument("Data length " + std::to_string(data.size()) + " does not match shape " +
                                    dims(shape) + " (expected " + std::to_string(n) + ")");
    auto buf = device_alloc<float>(n);
    if (n && nne_memcpy_h2d(buf.get(), data.data(), n * 4, nullptr) != NNE_OK)
        throw std::runtime_error(from_status(NNE_EHIP).to_string());
    auto st = contiguous_strides(shape);
    return view(std::move(buf), 0, std::move(shape), std::move(st));
}

RawTensor RawTensor::zeros(const std::vector<size_t>& shape) {
    const size_t n = count(shape);
    auto buf = device_alloc<float>(n);
    if (n) hip_check(hipMemset(buf.get(), 0, n * 4), "hipMemset");
    return view(std::move(buf), 0, shape, contiguous_strides(shape));
}

RawTensor RawTensor::randn(const std::vector<size_t>& shape, float mean, float std) {
    std::vector<float> data(count(shape));
    {
        std::lock_guard<std::mutex> lock(g_rng_mu);
        std::normal_distribution<float> dist(mean, std);
        for (float& x : data) x = dist(g_rng);
    }
    return from_vec(data, shape);
}

RawTensor RawTensor::uniform(const std::vector<size_t>& shape, float low, float high) {
    std::vector<float> data(count(shape));
    {
        std::lock_guard<std::mutex> lock(g_rng_mu);
        std::uniform_real_distribution<float> dist(low, high);
        for (float& x : data) x = dist(g_rng);
    }
    return from_vec(data, shape);
}

RawTensor RawTensor::kaiming_uniform(const std::vector<size_t>& shape, size_t fan_in) {
    const float bound = std::sqrt(6.0f / (float)std::max<size_t>(fan_in, 1));   // tensor/mod.rs:128-131
    return uniform(shape, -bound, bound);
}

size_t RawTensor::numel() const { return count(shape_); }

bool RawTensor::is_contiguous() const { return strides_ == contiguous_strides(shape_); }

float* RawTensor::data() const { return storage_ ? storage_.get() + offset_ : nullptr; }

RawTensor RawTensor::to_contiguous() const {
    if (is_contiguous() || numel() == 0) return *this;
    if (ndim() > (size_t)kMaxDims) throw std::invalid_argument("to_contiguous: more than 8 dimensions");
    auto buf = device_alloc<float>(numel());
    GatherArgs a{};
    a.src = data();
    a.dst = buf.get();
    a.n = (int64_t)numel();
    a.nd = (int)ndim();
    for (size_t i = 0; i < ndim(); ++i) {
        a.shape[i] = (int64_t)shape_[i];
        a.stride[i] = (int64_t)strides_[i];
    }
    hipLaunchKernelGGL(gather_kernel, dim3(grid_for(a.n)), dim3(256), 0, nullptr, a);
    hip_check(hipGetLastError(), "gather_kernel");
    return view(std::move(buf), 0, shape_, contiguous_strides(shape_));
}

std::vector<float> RawTensor::to_vec() const {
    RawTensor c = to_contiguous();
    std::vector<float> out(c.numel());
    if (!out.empty() && nne_memcpy_d2h(out.data(), c.data(), out.size() * 4, nullptr) != NNE_OK)
        throw std::runtime_error(from_status(NNE_EHIP).to_string());
    return out;
}

Result<RawTensor> RawTensor::transpose(size_t a, size_t b) const {
    if (a >= ndim() || b >= ndim())
        return EngineError::invalid_argument("transpose axes (" + std::to_string(a) + ", " +
                                             std::to_string(b) + ") out of range for " + dims(shape_));
    RawTensor t = *this;
    std::swap(t.shape_[a], t.shape_[b]);
    std::swap(t.strides_[a], t.strides_[b]);
    return t;
}

Result<RawTensor> RawTensor::reshape(const std::vector<size_t>& shape) const {
    if (count(shape) != numel())
        return EngineError::shape_mismatch(shape, shape_);
    RawTensor c = to_contiguous();
    return view(c.storage_, c.offset_, shape, contiguous_strides(shape));
}

Result<RawTensor> RawTensor::slice(size_t axis, size_t start, size_t end) const {
    if (axis >= ndim() || start > end || end > shape_[axis])
        return EngineError::invalid_argument("slice [" + std::to_string(start) + ", " + std::to_string(end) +
                                             ") of axis " + std::to_string(axis) + " out of range for " +
                                             dims(shape_));
    RawTensor t = *this;
    t.offset_ += start * strides_[axis];
    t.shape_[axis] = end - start;
    return t;
}

// ---- attention -----------------------------------------------------------

Result<RawTensor> flash_attention_forward(const RawTensor& q, const RawTensor& k, const RawTensor& v,
                                          bool is_causal, std::optional<float> scale,
                                          size_t block_size_r, size_t block_size_c) {
    if (q.ndim() != 4 || k.ndim() != 4 || v.ndim() != 4)          // flash_attention.rs:32-37
        return EngineError::invalid_argument(
            "FlashAttention expects 4D tensors [Batch, Heads, SeqLen, Dim], got Q:" + dims(q.shape()) +
            ", K:" + dims(k.shape()) + ", V:" + dims(v.shape()));
    const auto &qs = q.shape(), &ks = k.shape(), &vs = v.shape();
    if (qs[0] != ks[0] || qs[0] != vs[0] || qs[1] != ks[1] || qs[1] != vs[1] || qs[3] != ks[3] ||
        qs[3] != vs[3] || ks[2] != vs[2])                         // flash_attention.rs:43-48
        return EngineError::shape_mismatch({qs[0], qs[1], ks[2], qs[3]}, {ks[0], ks[1], ks[2], ks[3]});
    RawTensor out = RawTensor::zeros(qs);
    const auto q_shape = as_i64(qs), k_shape = as_i64(ks), v_shape = as_i64(vs);
    const auto q_st = as_i64(q.strides()), k_st = as_i64(k.strides()), v_st = as_i64(v.strides());
    const auto o_st = as_i64(out.strides());
    const int rc = nne_flash_attention_forward(
        q.data(), q_shape.data(), q_st.data(), k.data(), k_shape.data(), k_st.data(), v.data(),
        v_shape.data(), v_st.data(), out.data(), o_st.data(), is_causal ? 1 : 0, scale ? 1 : 0,
        scale.value_or(0.f), (int64_t)block_size_r, (int64_t)block_size_c, nullptr);
    if (rc != NNE_OK) return from_status(rc);
    return out;
}

Result<RawTensor> attention_forward(const RawTensor& q, const RawTensor& k, const RawTensor& v,
                                    bool is_causal, int64_t q_offset, std::optional<float> scale) {
    if (q.ndim() != 4 || k.ndim() != 4 || v.ndim() != 4)
        return EngineError::invalid_argument("attention expects 4D tensors [Batch, Heads, SeqLen, Dim], got Q:" +
                                             dims(q.shape()) + ", K:" + dims(k.shape()) + ", V:" +
                                             dims(v.shape()));
    const auto &qs = q.shape(), &ks = k.shape(), &vs = v.shape();
    const size_t hkv = ks[1];
    if (qs[0] != ks[0] || qs[0] != vs[0] || hkv != vs[1] || qs[3] != ks[3] || qs[3] != vs[3] ||
        ks[2] != vs[2] || hkv == 0 || qs[1] % hkv != 0)
        return EngineError::shape_mismatch({qs[0], hkv > 0 && qs[1] % hkv == 0 ? hkv : qs[1], ks[2], qs[3]},
                                           {ks[0], hkv, ks[2], ks[3]});
    RawTensor out = RawTensor::zeros(qs);
    const auto q_shape = as_i64(qs), k_shape = as_i64(ks), v_shape = as_i64(vs);
    const auto q_st = as_i64(q.strides()), k_st = as_i64(k.strides()), v_st = as_i64(v.strides());
    const auto o_st = as_i64(out.strides());
    const int rc = nne_attention_forward(q.data(), q_shape.data(), q_st.data(), k.data(), k_shape.data(),
                                         k_st.data(), v.data(), v_shape.data(), v_st.data(), out.data(),
                                         o_st.data(), is_causal ? 1 : 0, q_offset, scale ? 1 : 0,
                                         scale.value_or(0.f), nullptr);
    if (rc != NNE_OK) return from_status(rc);
    return out;
}

// ---- Linear ------------------------------------------------------------------

namespace {

rocblas_handle blas() {
    thread_local rocblas_handle h = nullptr;
    if (!h && rocblas_create_handle(&h) != rocblas_status_success)
        throw std::runtime_error(EngineError::gpu_error("rocblas_create_handle failed").to_string());
    return h;
}

}  // namespace

Linear::Linear(size_t in, size_t out) { *this = with_bias(in, out, true); }

Linear Linear::with_bias(size_t in, size_t out, bool has_bias) {   // linear.rs:28-42
    Linear l;
    l.in_features = in;
    l.out_features = out;
    l.weight = RawTensor::kaiming_uniform({out, in}, in);
    if (has_bias) {
        const float bound = 1.0f / std::sqrt((float)in);
        l.bias = RawTensor::uniform({out}, -bound, bound);
    }
    return l;
}

Linear Linear::without_bias(size_t in, size_t out) { return with_bias(in, out, false); }

Result<RawTensor> Linear::forward(const RawTensor& input) const {   // linear.rs:45-56
    if (input.ndim() == 0 || input.shape().back() != in_features)
        return EngineError::incompatible_shapes("matmul_transposed_b", {input.shape(), weight.shape()});
    RawTensor x = input.to_contiguous();
    const size_t rows = x.numel() / std::max<size_t>(in_features, 1);
    std::vector<size_t> out_shape = x.shape();
    out_shape.back() = out_features;
    RawTensor y = RawTensor::zeros(out_shape);
    if (rows && out_features) {
        // Row-major Y[rows, out] = X[rows, in] W^T is column-major
        // Y^T[out, rows] = W[out, in] (stored as W^T, transposed) x X^T[in, rows].
        const float one = 1.f, zero = 0.f;
        if (rocblas_sgemm(blas(), rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)out_features,
                          (rocblas_int)rows, (rocblas_int)in_features, &one, weight.data(),
                          (rocblas_int)in_features, x.data(), (rocblas_int)in_features, &zero, y.data(),
                          (rocblas_int)out_features) != rocblas_status_success)
            return EngineError::gpu_error("rocblas_sgemm failed");
        if (bias) {
            hipLaunchKernelGGL(bias_add_kernel, dim3(grid_for((int64_t)(rows * out_features))), dim3(256), 0,
                               nullptr, y.data(), bias->data(), (int64_t)rows, (int64_t)out_features);
            if (hipGetLastError() != hipSuccess) return EngineError::gpu_error("bias_add_kernel launch failed");
        }
    }
    return y;
}

// ---- FlashAttention layer ----------------------------------------------------

namespace {

// flash_attention.rs:217-223, checked before any projection is allocated.
size_t divisible_d_model(size_t d_model, size_t num_heads) {
    if (num_heads == 0 || d_model % num_heads != 0)
        throw std::invalid_argument("d_model (" + std::to_string(d_model) + ") must be divisible by num_heads (" +
                                    std::to_string(num_heads) + ")");
    return d_model;
}

}  // namespace

FlashAttention::FlashAttention(size_t d_model_, size_t num_heads_, bool is_causal_)
    : q_proj(divisible_d_model(d_model_, num_heads_), d_model_), k_proj(d_model_, d_model_),
      v_proj(d_model_, d_model_), out_proj(d_model_, d_model_), num_heads(num_heads_), d_model(d_model_),
      head_dim(d_model_ / num_heads_), is_causal(is_causal_) {}

Result<RawTensor> FlashAttention::forward_flash(const RawTensor& x) const {
    if (x.ndim() != 3)                                               // flash_attention.rs:240-246
        return EngineError::incompatible_shapes("FlashAttention forward (expected 3D input [B, T, C])", {x.shape()});
    const size_t b = x.shape()[0], t = x.shape()[1], h = num_heads, d = head_dim;
    auto q = q_proj.forward(x);
    if (q.is_err()) return q.error();
    auto k = k_proj.forward(x);
    if (k.is_err()) return k.error();
    auto v = v_proj.forward(x);
    if (v.is_err()) return v.error();
    // [B, T, C] read as [B, H, T, d]: strides (T*C, d, C, 1); the output is written
    // the same way, i.e. directly in [B, T, C].
    const std::vector<size_t> hs{b, h, t, d}, st{t * d_model, d, d_model, 1};
    RawTensor merged = RawTensor::zeros({b, t, d_model});
    const auto shape = as_i64(hs), strides = as_i64(st);
    const int rc = nne_flash_attention_forward(
        q.value().data(), shape.data(), strides.data(), k.value().data(), shape.data(), strides.data(),
        v.value().data(), shape.data(), strides.data(), merged.data(), strides.data(), is_causal ? 1 : 0, 0, 0.f,
        (int64_t)block_size, (int64_t)block_size, nullptr);
    if (rc != NNE_OK) return from_status(rc);
    return out_proj.forward(merged);
}

// ---- KVCache -----------------------------------------------------------------

KVCache::KVCache(size_t num_layers, size_t batch_, size_t num_kv_heads_, size_t capacity_, size_t head_dim_)
    : batch(batch_), num_kv_heads(num_kv_heads_), capacity(capacity_), head_dim(head_dim_) {
    const size_t n = batch * num_kv_heads * capacity * head_dim;
    for (size_t i = 0; i < num_layers; ++i) {
        Layer l;
        l.k = device_alloc<float>(n);
        l.v = device_alloc<float>(n);
        l.lens_dev = device_alloc<int32_t>(batch);
        if (n) {
            hip_check(hipMemset(l.k.get(), 0, n * 4), "hipMemset");
            hip_check(hipMemset(l.v.get(), 0, n * 4), "hipMemset");
        }
        if (batch) hip_check(hipMemset(l.lens_dev.get(), 0, batch * 4), "hipMemset");
        l.lens_host.assign(batch, 0);
        layers_.push_back(std::move(l));
    }
}

void KVCache::reset() {                                             // kv_cache.rs:25-29
    for (auto& l : layers_) {
        std::fill(l.lens_host.begin(), l.lens_host.end(), 0);
        if (batch) hip_check(hipMemset(l.lens_dev.get(), 0, batch * 4), "hipMemset");
        l.engaged = false;
    }
}

// ---- KVCache slots (kv_cache.rs:13) --------------------------------------------

bool KVCache::Slot::has_value() const { return cache_->layers_.at(layer_).engaged; }

std::pair<RawTensor, RawTensor> KVCache::Slot::value() const {
    if (!has_value()) throw std::bad_optional_access();
    const size_t L = cache_->current_seq_len(layer_);
    return {cache_->k(layer_).slice(2, 0, L).value(), cache_->v(layer_).slice(2, 0, L).value()};
}

KVCache::Slot& KVCache::Slot::operator=(std::nullopt_t) {
    KVCache& c = *cache_;
    Layer& l = c.layers_.at(layer_);
    std::fill(l.lens_host.begin(), l.lens_host.end(), 0);
    if (c.batch) hip_check(hipMemset(l.lens_dev.get(), 0, c.batch * 4), "hipMemset");
    l.engaged = false;
    return *this;
}

Result<bool> KVCache::Slot::set(const RawTensor& k, const RawTensor& v) {
    KVCache& c = *cache_;
    if (k.numel() == 0 && v.numel() == 0) {          // Some((zeros[0], zeros[0])): engaged, empty
        *this = std::nullopt;
        c.layers_.at(layer_).engaged = true;
        return true;
    }
    const std::vector<size_t> want{c.batch, c.num_kv_heads, k.ndim() == 4 ? k.shape()[2] : 0, c.head_dim};
    if (k.shape() != want) return EngineError::shape_mismatch(want, k.shape());
    if (v.shape() != want) return EngineError::shape_mismatch(want, v.shape());
    if (want[2] > c.capacity)
        return EngineError::gpu_error("KV cache slot of " + std::to_string(want[2]) + " rows exceeds capacity " +
                                      std::to_string(c.capacity));
    // Rows 0..L of every sequence: lengths to zero, then the append kernel.
    *this = std::nullopt;
    auto r = c.update(layer_, k, v);
    if (r.is_err()) return r.error();
    return true;
}

KVCache::Slot& KVCache::Slot::operator=(const std::pair<RawTensor, RawTensor>& kv) {
    set(kv.first, kv.second).unwrap();
    return *this;
}

std::optional<std::pair<RawTensor, RawTensor>> KVCache::Slot::take() {
    if (!has_value()) return std::nullopt;
    auto kv = value();
    auto copy = [](const RawTensor& t) {
        if (!t.is_contiguous()) return t.to_contiguous();
        RawTensor out = RawTensor::zeros(t.shape());
        if (t.numel() && nne_memcpy_d2d(out.data(), t.data(), t.numel() * 4, nullptr) != NNE_OK)
            throw std::runtime_error(from_status(NNE_EHIP).to_string());
        return out;
    };
    std::pair<RawTensor, RawTensor> out{copy(kv.first), copy(kv.second)};
    if (nne_stream_sync(nullptr) != NNE_OK) throw std::runtime_error(from_status(NNE_EHIP).to_string());
    *this = std::nullopt;
    return out;
}

KVCache::Slot KVCache::Layers::operator[](size_t i) const {
    if (i >= size())
        throw std::out_of_range("KVCache layer index " + std::to_string(i) + " out of range (total layers: " +
                                std::to_string(size()) + ")");
    return Slot(c_, i);
}

std::optional<KVCache::Slot> KVCache::Layers::get_mut(size_t i) const {
    if (i >= size()) return std::nullopt;
    return Slot(c_, i);
}

size_t KVCache::num_layers() const { return layers_.size(); }

size_t KVCache::current_seq_len(size_t layer_idx) const {
    if (layer_idx >= layers_.size() || batch == 0) return 0;
    const auto& l = layers_[layer_idx].lens_host;
    return (size_t)*std::max_element(l.begin(), l.end());
}

Result<bool> KVCache::check_layer(size_t layer_idx) const {
    if (layer_idx >= layers_.size())                                 // kv_cache.rs:55-61
        return EngineError::invalid_argument("KVCache layer index " + std::to_string(layer_idx) +
                                             " out of range (total layers: " + std::to_string(layers_.size()) +
                                             ")");
    return true;
}

RawTensor KVCache::k(size_t layer_idx) const {
    const std::vector<size_t> s{batch, num_kv_heads, capacity, head_dim};
    return RawTensor::view(layers_.at(layer_idx).k, 0, s, contiguous_strides(s));
}

RawTensor KVCache::v(size_t layer_idx) const {
    const std::vector<size_t> s{batch, num_kv_heads, capacity, head_dim};
    return RawTensor::view(layers_.at(layer_idx).v, 0, s, contiguous_strides(s));
}

const std::vector<int32_t>& KVCache::lengths(size_t layer_idx) const { return layers_.at(layer_idx).lens_host; }

const int32_t* KVCache::lengths_device(size_t layer_idx) const { return layers_.at(layer_idx).lens_dev.get(); }

Result<std::pair<RawTensor, RawTensor>> KVCache::update(size_t layer_idx, const RawTensor& k_new,
                                                       const RawTensor& v_new) {
    auto ok = check_layer(layer_idx);
    if (ok.is_err()) return ok.error();
    const std::vector<size_t> want{batch, num_kv_heads, k_new.ndim() == 4 ? k_new.shape()[2] : 0, head_dim};
    if (k_new.shape() != want) return EngineError::shape_mismatch(want, k_new.shape());
    if (v_new.shape() != want) return EngineError::shape_mismatch(want, v_new.shape());
    Layer& l = layers_[layer_idx];
    const auto kst = as_i64(k_new.strides()), vst = as_i64(v_new.strides());
    const int rc = nne_kv_append(l.k.get(), l.v.get(), l.lens_dev.get(), l.lens_host.data(), k_new.data(), kst.data(),
                                 v_new.data(), vst.data(), (int64_t)batch, (int64_t)num_kv_heads,
                                 (int64_t)capacity, (int64_t)head_dim, (int64_t)want[2], nullptr);
    if (rc != NNE_OK) return from_status(rc);
    l.engaged = true;
    const size_t L = current_seq_len(layer_idx);
    auto kv = k(layer_idx).slice(2, 0, L), vv = v(layer_idx).slice(2, 0, L);
    return std::make_pair(kv.value(), vv.value());
}

const nne_workspace_t* KVCache::workspace(size_t num_heads) {
    nne_workspace_size_t need{0, 0};
    if (nne_decode_workspace_size((int64_t)batch, (int64_t)num_heads, (int64_t)num_kv_heads, (int64_t)head_dim,
                                  &need) != NNE_OK)
        return nullptr;   // the call itself reports the geometry error
    if (!ws_desc_) ws_desc_ = std::make_shared<nne_workspace_t>(nne_workspace_t{nullptr, 0, nullptr, 0});
    nne_workspace_t& w = *ws_desc_;
    if (need.records_bytes > w.records_bytes) {
        auto buf = device_alloc<char>(need.records_bytes);
        ws_ = std::shared_ptr<void>(buf, buf.get());
        w.records = ws_.get();
        w.records_bytes = need.records_bytes;
    }
    if (need.n_counters > w.n_counters) {
        counters_ = device_alloc<uint32_t>(need.n_counters);
        if (nne_counters_init(counters_.get(), need.n_counters, nullptr) != NNE_OK)
            throw std::runtime_error(from_status(NNE_EHIP).to_string());
        w.counters = counters_.get();
        w.n_counters = need.n_counters;
    }
    return ws_desc_.get();
}

Result<RawTensor> KVCache::attend(size_t layer_idx, const RawTensor& q, std::optional<float> scale) {
    auto ok = check_layer(layer_idx);
    if (ok.is_err()) return ok.error();
    if (q.ndim() != 4 || q.shape()[0] != batch || q.shape()[2] != 1 || q.shape()[3] != head_dim)
        return EngineError::shape_mismatch({batch, q.ndim() == 4 ? q.shape()[1] : 0, 1, head_dim}, q.shape());
    Layer& l = layers_[layer_idx];
    RawTensor out = RawTensor::zeros(q.shape());
    const auto qst = as_i64(q.strides()), ost = as_i64(out.strides());
    const nne_workspace_t* ws = workspace(q.shape()[1]);
    const int rc = nne_decode_attention(q.data(), qst.data(), l.k.get(), l.v.get(), l.lens_dev.get(),
                                        l.lens_host.data(), out.data(), ost.data(), (int64_t)batch,
                                        (int64_t)q.shape()[1], (int64_t)num_kv_heads, (int64_t)capacity,
                                        (int64_t)head_dim, scale ? 1 : 0, scale.value_or(0.f), ws, nullptr);
    if (rc != NNE_OK) return from_status(rc);
    return out;
}

Result<RawTensor> KVCache::decode_step(size_t layer_idx, const RawTensor& q, const RawTensor& k_new,
                                       const RawTensor& v_new, std::optional<float> scale) {
    auto ok = check_layer(layer_idx);
    if (ok.is_err()) return ok.error();
    if (q.ndim() != 4 || q.shape()[0] != batch || q.shape()[2] != 1 || q.shape()[3] != head_dim)
        return EngineError::shape_mismatch({batch, q.ndim() == 4 ? q.shape()[1] : 0, 1, head_dim}, q.shape());
    const std::vector<size_t> want{batch, num_kv_heads, 1, head_dim};
    if (k_new.shape() != want) return EngineError::shape_mismatch(want, k_new.shape());
    if (v_new.shape() != want) return EngineError::shape_mismatch(want, v_new.shape());
    Layer& l = layers_[layer_idx];
    RawTensor out = RawTensor::zeros(q.shape());
    const auto qst = as_i64(q.strides()), ost = as_i64(out.strides());
    const int64_t hq = (int64_t)q.shape()[1];
    nne_workspace_size_t fits{0, 0};
    if (nne_decode_workspace_size(std::max<int64_t>((int64_t)batch, 1), hq, (int64_t)num_kv_heads,
                                  (int64_t)head_dim, &fits) != NNE_OK) {
        // Geometry the decode step does not take (head dim not a multiple of
        // 4): append, then attend every sequence to its own first lens[b]
        // rows, no mask (llama.rs:239-296 with t = 1), on the general kernel.
        auto kv = update(layer_idx, k_new, v_new);
        if (kv.is_err()) return kv.error();
        for (size_t b = 0; b < batch; ++b) {
            const size_t L = (size_t)l.lens_host[b];
            RawTensor qb = q.slice(0, b, b + 1).value(), ob = out.slice(0, b, b + 1).value();
            RawTensor kb = k(layer_idx).slice(0, b, b + 1).value().slice(2, 0, L).value();
            RawTensor vb = v(layer_idx).slice(0, b, b + 1).value().slice(2, 0, L).value();
            const auto qs = as_i64(qb.shape()), qbs = as_i64(qb.strides()), obs = as_i64(ob.strides());
            const auto ks = as_i64(kb.shape()), kbs = as_i64(kb.strides()), vbs = as_i64(vb.strides());
            const int rc = nne_attention_forward(qb.data(), qs.data(), qbs.data(), kb.data(), ks.data(), kbs.data(),
                                                 vb.data(), ks.data(), vbs.data(), ob.data(), obs.data(), 0, 0,
                                                 scale ? 1 : 0, scale.value_or(0.f), nullptr);
            if (rc != NNE_OK) return from_status(rc);
        }
        return out;
    }
    const auto kst = as_i64(k_new.strides()), vst = as_i64(v_new.strides());
    const nne_workspace_t* ws = workspace(q.shape()[1]);
    const int rc = nne_decode_step(q.data(), qst.data(), l.k.get(), l.v.get(), l.lens_dev.get(),
                                   l.lens_host.data(), k_new.data(), kst.data(), v_new.data(), vst.data(),
                                   out.data(), ost.data(), (int64_t)batch, (int64_t)q.shape()[1],
                                   (int64_t)num_kv_heads, (int64_t)capacity, (int64_t)head_dim, scale ? 1 : 0,
                                   scale.value_or(0.f), ws, nullptr);
    if (rc != NNE_OK) return from_status(rc);
    l.engaged = true;
    return out;
}

Result<bool> KVCache::set_lengths(size_t layer_idx, const std::vector<int32_t>& lens) {
    auto ok = check_layer(layer_idx);
    if (ok.is_err()) return ok.error();
    if (lens.size() != batch) return EngineError::shape_mismatch({batch}, {lens.size()});
    for (int32_t L : lens)
        if (L < 0 || (size_t)L > capacity)
            return EngineError::invalid_argument("sequence length " + std::to_string(L) + " outside [0, " +
                                                 std::to_string(capacity) + "]");
    Layer& l = layers_[layer_idx];
    l.lens_host = lens;
    l.engaged = true;
    if (batch && nne_memcpy_h2d(l.lens_dev.get(), lens.data(), batch * 4, nullptr) != NNE_OK)
        return from_status(NNE_EHIP);
    return true;
}

// ---- RotaryEmbedding ------------------------------------------------------------

namespace {

size_t even_head_dim(size_t head_dim) {   // llama.rs:75
    if (head_dim % 2 != 0)
        throw std::invalid_argument("RoPE head_dim (" + std::to_string(head_dim) + ") must be even");
    return head_dim;
}

}  // namespace

RotaryEmbedding::RotaryEmbedding(size_t head_dim_, size_t max_seq_len_, float theta)
    : head_dim(even_head_dim(head_dim_)), max_seq_len(max_seq_len_) {
    std::vector<float> c(max_seq_len * head_dim), s(max_seq_len * head_dim);
    const int rc = nne_rope_tables(c.data(), s.data(), (int64_t)max_seq_len, (int64_t)head_dim, theta);
    if (rc != NNE_OK) throw std::invalid_argument(from_status(rc).to_string());
    cos_cached = RawTensor::from_vec(c, {1, 1, max_seq_len, head_dim});
    sin_cached = RawTensor::from_vec(s, {1, 1, max_seq_len, head_dim});
}

Result<RawTensor> RotaryEmbedding::apply(const RawTensor& x, size_t start_pos) const {
    const size_t b = x.ndim() == 4 ? x.shape()[0] : 0;
    return apply(x, std::vector<int32_t>(b, (int32_t)std::min<size_t>(start_pos, INT32_MAX)));
}

Result<RawTensor> RotaryEmbedding::apply(const RawTensor& x, const std::vector<int32_t>& start_pos) const {
    if (x.ndim() != 4)                                               // llama.rs:111-118
        return EngineError::invalid_argument("RoPE apply expects 4D tensor [Batch, Heads, SeqLen, HeadDim], got "
                                             "rank " + std::to_string(x.ndim()) + " with shape " + dims(x.shape()));
    if (x.shape()[3] != head_dim) return EngineError::shape_mismatch({head_dim}, {x.shape()[3]});   // :119-124
    if (start_pos.size() != x.shape()[0]) return EngineError::shape_mismatch({x.shape()[0]}, {start_pos.size()});
    RawTensor out = RawTensor::zeros(x.shape());
    auto pos_dev = device_alloc<int32_t>(start_pos.size());
    if (!start_pos.empty() && nne_memcpy_h2d(pos_dev.get(), start_pos.data(), start_pos.size() * 4, nullptr) != NNE_OK)
        return from_status(NNE_EHIP);
    const auto shape = as_i64(x.shape()), xst = as_i64(x.strides()), ost = as_i64(out.strides());
    const int rc = nne_rope_apply(x.data(), shape.data(), xst.data(), out.data(), ost.data(), cos_cached.data(),
                                  sin_cached.data(), (int64_t)max_seq_len, (int64_t)head_dim, pos_dev.get(),
                                  start_pos.data(), nullptr);
    if (rc != NNE_OK) return from_status(rc);
    if (nne_stream_sync(nullptr) != NNE_OK) return from_status(NNE_EHIP);   // pos_dev is freed on return
    return out;
}

// ---- GroupedQueryAttention --------------------------------------------------------

namespace {

size_t gqa_head_dim(size_t d_model, size_t num_heads, size_t num_kv_heads) {   // llama.rs:174-183
    if (num_heads == 0 || d_model % num_heads != 0)
        throw std::invalid_argument("d_model must be divisible by num_heads");
    if (num_kv_heads == 0 || num_heads % num_kv_heads != 0)
        throw std::invalid_argument("num_heads must be divisible by num_kv_heads for GQA");
    return d_model / num_heads;
}

}  // namespace

GroupedQueryAttention::GroupedQueryAttention(size_t d_model, size_t num_heads_, size_t num_kv_heads_,
                                             size_t max_seq_len, float rope_theta)
    : q_proj(Linear::without_bias(d_model, gqa_head_dim(d_model, num_heads_, num_kv_heads_) * num_heads_)),
      k_proj(Linear::without_bias(d_model, num_kv_heads_ * (d_model / num_heads_))),
      v_proj(Linear::without_bias(d_model, num_kv_heads_ * (d_model / num_heads_))),
      o_proj(Linear::without_bias(d_model, d_model)),
      rope(d_model / num_heads_, max_seq_len, rope_theta),
      num_heads(num_heads_), num_kv_heads(num_kv_heads_), head_dim(d_model / num_heads_),
      num_queries_per_kv(num_heads_ / num_kv_heads_) {
    repack();
}

void GroupedQueryAttention::repack() {
    const int64_t c = (int64_t)q_proj.in_features;
    const uint64_t bytes = nne_qkv_packed_bytes(c, (int64_t)num_heads, (int64_t)num_kv_heads, (int64_t)head_dim);
    if (bytes == 0) {
        w_packed_.reset();
        return;
    }
    w_packed_ = device_alloc<float>(bytes / 4);
    const int rc = nne_qkv_pack(q_proj.weight.data(), k_proj.weight.data(), v_proj.weight.data(), w_packed_.get(), c,
                                (int64_t)num_heads, (int64_t)num_kv_heads, (int64_t)head_dim, nullptr);
    if (rc != NNE_OK) throw std::runtime_error(from_status(rc).to_string());
}

Result<RawTensor> GroupedQueryAttention::forward_gqa_cached(const RawTensor& x, size_t start_pos, KVCache* cache,
                                                            size_t layer_idx) {
    if (x.ndim() != 3)                                               // llama.rs:211-217
        return EngineError::incompatible_shapes("GroupedQueryAttention forward (expected 3D input [B, T, C])",
                                                {x.shape()});
    const size_t b = x.shape()[0], t = x.shape()[1], c = x.shape()[2];
    const size_t hq = num_heads, hkv = num_kv_heads, d = head_dim;
    if (c != q_proj.in_features)
        return EngineError::incompatible_shapes("matmul_transposed_b", {x.shape(), q_proj.weight.shape()});
    if (cache) {
        if (layer_idx >= cache->num_layers())
            return EngineError::invalid_argument("KVCache layer index " + std::to_string(layer_idx) +
                                                 " out of range (total layers: " +
                                                 std::to_string(cache->num_layers()) + ")");
        if (cache->batch != b || cache->num_kv_heads != hkv || cache->head_dim != d)
            return EngineError::shape_mismatch({b, hkv, cache->capacity, d},
                                               {cache->batch, cache->num_kv_heads, cache->capacity, cache->head_dim});
        for (int32_t L : cache->lengths(layer_idx))
            if ((size_t)L != start_pos)
                return EngineError::invalid_argument("start_pos " + std::to_string(start_pos) +
                                                     " differs from a cached length " + std::to_string(L));
    }
    if (cache && t == 1 && w_packed_) {
        // Decode step: fused projection + RoPE, then append + attend (llama.rs:226-296, t = 1).
        RawTensor xc = x.to_contiguous();
        RawTensor q = RawTensor::zeros({b, hq, 1, d}), k_new = RawTensor::zeros({b, hkv, 1, d}),
                  v_new = RawTensor::zeros({b, hkv, 1, d});
        const int rc = nne_qkv_rope(xc.data(), (int64_t)c, w_packed_.get(), nullptr, nullptr, nullptr,
                                    rope.cos_cached.data(), rope.sin_cached.data(), (int64_t)rope.max_seq_len,
                                    (int64_t)rope.head_dim, cache->lengths_device(layer_idx),
                                    cache->lengths(layer_idx).data(), q.data(), k_new.data(), v_new.data(),
                                    (int64_t)b, (int64_t)c, (int64_t)hq, (int64_t)hkv, (int64_t)d, nullptr);
        if (rc != NNE_OK) return from_status(rc);
        auto ctx = cache->decode_step(layer_idx, q, k_new, v_new);
        if (ctx.is_err()) return ctx.error();
        auto merged = ctx.value().reshape({b, 1, hq * d});          // [B, Hq, 1, d] is [B, 1, Hq * d]
        if (merged.is_err()) return merged.error();
        return o_proj.forward(merged.value());
    }
    // 1. projections, [B, T, H, d] -> [B, H, T, d] views (llama.rs:222-233)
    auto qp = q_proj.forward(x);
    if (qp.is_err()) return qp.error();
    auto kp = k_proj.forward(x);
    if (kp.is_err()) return kp.error();
    auto vp = v_proj.forward(x);
    if (vp.is_err()) return vp.error();
    auto heads = [&](const RawTensor& y, size_t h) {
        return y.reshape({b, t, h, d}).value().transpose(1, 2).value();
    };
    // 2. RoPE (:235-236)
    auto q = rope.apply(heads(qp.value(), hq), start_pos);
    if (q.is_err()) return q.error();
    auto k = rope.apply(heads(kp.value(), hkv), start_pos);
    if (k.is_err()) return k.error();
    RawTensor v = heads(vp.value(), hkv);
    // 3. cache append (:238-251)
    RawTensor k_all = k.value(), v_all = v;
    if (cache) {
        auto kv = cache->update(layer_idx, k.value(), v);
        if (kv.is_err()) return kv.error();
        k_all = kv.value().first;
        v_all = kv.value().second;
    }
    // 4-7. attention with the causal mask of :277-292 for t > 1, written
    // straight into [B, T, H, d] = [B, T, C]
    RawTensor merged = RawTensor::zeros({b, t, hq * d});
    const std::vector<int64_t> qs = as_i64(q.value().shape()), qst = as_i64(q.value().strides());
    const std::vector<int64_t> ks = as_i64(k_all.shape()), kst = as_i64(k_all.strides());
    const std::vector<int64_t> vs = as_i64(v_all.shape()), vst = as_i64(v_all.strides());
    const std::vector<int64_t> ost{(int64_t)(t * hq * d), (int64_t)d, (int64_t)(hq * d), 1};
    const int rc = nne_attention_forward(q.value().data(), qs.data(), qst.data(), k_all.data(), ks.data(),
                                         kst.data(), v_all.data(), vs.data(), vst.data(), merged.data(), ost.data(),
                                         t > 1 ? 1 : 0, (int64_t)start_pos, 0, 0.f, nullptr);
    if (rc != NNE_OK) return from_status(rc);
    // 8. output projection (:298)
    return o_proj.forward(merged);
}

Result<RawTensor> GroupedQueryAttention::forward_gqa_cached(const RawTensor& x, size_t start_pos,
                                                            std::optional<KVCache::Slot> layer_cache) {
    if (!layer_cache || !layer_cache->has_value()) return forward_gqa_cached(x, start_pos, nullptr, 0);
    return forward_gqa_cached(x, start_pos, &layer_cache->cache(), layer_cache->layer_idx());
}

// ---- MultiHeadAttention -----------------------------------------------------------

MultiHeadAttention::MultiHeadAttention(size_t d_model_, size_t num_heads_, bool is_causal_)
    : q_proj(divisible_d_model(d_model_, num_heads_), d_model_), k_proj(d_model_, d_model_),
      v_proj(d_model_, d_model_), out_proj(d_model_, d_model_), num_heads(num_heads_), d_model(d_model_),
      head_dim(d_model_ / num_heads_), is_causal(is_causal_) {
    repack();
}

void MultiHeadAttention::repack() {
    const int64_t c = (int64_t)d_model, h = (int64_t)num_heads;
    const uint64_t bytes = nne_qkv_packed_bytes(c, h, h, (int64_t)head_dim);
    if (bytes == 0) {
        w_packed_.reset();
        return;
    }
    w_packed_ = device_alloc<float>(bytes / 4);
    const int rc = nne_qkv_pack(q_proj.weight.data(), k_proj.weight.data(), v_proj.weight.data(), w_packed_.get(), c,
                                h, h, (int64_t)head_dim, nullptr);
    if (rc != NNE_OK) throw std::runtime_error(from_status(rc).to_string());
}

namespace {

// Attention of q [B, H, Tq, d] over k/v [B, H, Tk, d] written into [B, Tq, C].
Result<RawTensor> attend_merged(const RawTensor& q, const RawTensor& k, const RawTensor& v, bool causal,
                                int64_t q_offset) {
    const size_t b = q.shape()[0], h = q.shape()[1], t = q.shape()[2], d = q.shape()[3];
    RawTensor merged = RawTensor::zeros({b, t, h * d});
    const std::vector<int64_t> qs = as_i64(q.shape()), qst = as_i64(q.strides());
    const std::vector<int64_t> ks = as_i64(k.shape()), kst = as_i64(k.strides());
    const std::vector<int64_t> vs = as_i64(v.shape()), vst = as_i64(v.strides());
    const std::vector<int64_t> ost{(int64_t)(t * h * d), (int64_t)d, (int64_t)(h * d), 1};
    const int rc = nne_attention_forward(q.data(), qs.data(), qst.data(), k.data(), ks.data(), kst.data(), v.data(),
                                         vs.data(), vst.data(), merged.data(), ost.data(), causal ? 1 : 0, q_offset,
                                         0, 0.f, nullptr);
    if (rc != NNE_OK) return from_status(rc);
    return merged;
}

}  // namespace

Result<RawTensor> MultiHeadAttention::forward_attention_cached(const RawTensor& x, KVCache* cache,
                                                               size_t layer_idx) {
    if (x.ndim() != 3)                                               // attention.rs:56-62
        return EngineError::incompatible_shapes("MultiHeadAttention forward (expected 3D input [B, T, C])",
                                                {x.shape()});
    const size_t b = x.shape()[0], t = x.shape()[1], c = x.shape()[2], h = num_heads, d = head_dim;
    if (c != d_model) return EngineError::incompatible_shapes("matmul_transposed_b", {x.shape(), q_proj.weight.shape()});
    if (cache) {
        if (layer_idx >= cache->num_layers())
            return EngineError::invalid_argument("KVCache layer index " + std::to_string(layer_idx) +
                                                 " out of range (total layers: " +
                                                 std::to_string(cache->num_layers()) + ")");
        if (cache->batch != b || cache->num_kv_heads != h || cache->head_dim != d)
            return EngineError::shape_mismatch({b, h, cache->capacity, d},
                                               {cache->batch, cache->num_kv_heads, cache->capacity, cache->head_dim});
        // Checked before anything is appended, so a refused step leaves the
        // cache as it was.
        const auto& lens = cache->lengths(layer_idx);
        for (int32_t L : lens)
            if (t > 1 && L != lens[0])
                return EngineError::invalid_argument("multi-token steps need equal cached lengths");
    }
    if (cache && t == 1) {
        // Decode step: biased projections (no rotation), then append + attend
        // with each sequence seeing its own rows (ragged lengths).
        RawTensor q, k_new, v_new;
        if (w_packed_) {
            RawTensor xc = x.to_contiguous();
            q = RawTensor::zeros({b, h, 1, d});
            k_new = RawTensor::zeros({b, h, 1, d});
            v_new = RawTensor::zeros({b, h, 1, d});
            const int rc = nne_qkv_rope(xc.data(), (int64_t)c, w_packed_.get(), q_proj.bias->data(),
                                        k_proj.bias->data(), v_proj.bias->data(), nullptr, nullptr, 0, (int64_t)d,
                                        nullptr, nullptr, q.data(), k_new.data(), v_new.data(), (int64_t)b,
                                        (int64_t)c, (int64_t)h, (int64_t)h, (int64_t)d, nullptr);
            if (rc != NNE_OK) return from_status(rc);
        } else {
            auto head_view = [&](const Linear& lin) -> Result<RawTensor> {
                auto y = lin.forward(x);                             // [B, 1, C]
                if (y.is_err()) return y.error();
                return y.value().reshape({b, 1, h, d}).value().transpose(1, 2).value().to_contiguous();
            };
            auto qp = head_view(q_proj), kp = head_view(k_proj), vp = head_view(v_proj);
            if (qp.is_err()) return qp.error();
            if (kp.is_err()) return kp.error();
            if (vp.is_err()) return vp.error();
            q = qp.value();
            k_new = kp.value();
            v_new = vp.value();
        }
        auto ctx = cache->decode_step(layer_idx, q, k_new, v_new);
        if (ctx.is_err()) return ctx.error();
        auto merged = ctx.value().reshape({b, 1, c});
        if (merged.is_err()) return merged.error();
        return out_proj.forward(merged.value());
    }
    auto qp = q_proj.forward(x);                                     // :66-75
    if (qp.is_err()) return qp.error();
    auto kp = k_proj.forward(x);
    if (kp.is_err()) return kp.error();
    auto vp = v_proj.forward(x);
    if (vp.is_err()) return vp.error();
    auto heads = [&](const RawTensor& y) { return y.reshape({b, t, h, d}).value().transpose(1, 2).value(); };
    RawTensor q = heads(qp.value()), k_all = heads(kp.value()), v_all = heads(vp.value());
    size_t total = t;
    if (cache) {                                                     // :78-91
        auto kv = cache->update(layer_idx, k_all, v_all);
        if (kv.is_err()) return kv.error();
        k_all = kv.value().first;
        v_all = kv.value().second;
        total = b ? (size_t)cache->lengths(layer_idx)[0] : 0;
    }
    // :93-122: mask c > (L - T) + r only for causal multi-token steps
    auto merged = attend_merged(q, k_all, v_all, is_causal && t > 1, (int64_t)(total - t));
    if (merged.is_err()) return merged.error();
    return out_proj.forward(merged.value());                         // :124-128
}

Result<RawTensor> MultiHeadAttention::forward_attention_cached(const RawTensor& x,
                                                               std::optional<KVCache::Slot> layer_cache) {
    if (!layer_cache || !layer_cache->has_value()) return forward_attention_cached(x, nullptr, 0);
    return forward_attention_cached(x, &layer_cache->cache(), layer_cache->layer_idx());
}

Result<RawTensor> MultiHeadAttention::forward_cross_attention_cached(
    const RawTensor& x, const RawTensor& memory, std::optional<std::pair<RawTensor, RawTensor>>* slot) {
    if (x.ndim() != 3 || memory.ndim() != 3)                         // attention.rs:148-153
        return EngineError::incompatible_shapes("MultiHeadAttention cross-attention (expected 3D query [B, T_q, C] "
                                                "and 3D memory [B, T_kv, C])",
                                                {x.shape(), memory.shape()});
    if (x.shape()[0] != memory.shape()[0] || x.shape()[2] != memory.shape()[2])   // :155-160
        return EngineError::incompatible_shapes(
            "MultiHeadAttention cross-attention (batch size and channel dim must match)", {x.shape(), memory.shape()});
    const size_t b = x.shape()[0], tq = x.shape()[1], tkv = memory.shape()[1], h = num_heads, d = head_dim;
    auto qp = q_proj.forward(x);
    if (qp.is_err()) return qp.error();
    RawTensor q = qp.value().reshape({b, tq, h, d}).value().transpose(1, 2).value();
    std::pair<RawTensor, RawTensor> kv;
    if (slot && slot->has_value()) {
        kv = slot->value();
    } else {
        auto kp = k_proj.forward(memory);
        if (kp.is_err()) return kp.error();
        auto vp = v_proj.forward(memory);
        if (vp.is_err()) return vp.error();
        kv = {kp.value().reshape({b, tkv, h, d}).value().transpose(1, 2).value(),
              vp.value().reshape({b, tkv, h, d}).value().transpose(1, 2).value()};
        if (slot) *slot = kv;
    }
    auto merged = attend_merged(q, kv.first, kv.second, false, 0);
    if (merged.is_err()) return merged.error();
    return out_proj.forward(merged.value());
}

}  // namespace nne
