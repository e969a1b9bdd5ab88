// mq4.hpp -- header-only C++ host API over the C ABI of libmq4 (include/mq4.h),
// mirroring the reference's interface for the quantized path so that a C++
// caller can replace the MLX ops at the same call sites:
//
//   marlin::QuantizedTensor      src/core/types.h:75-82
//   quantize_weight              src/model/weights.cpp:45-56 (:180-194 lm_head)
//   quantize_weights             the loader loop of those, src/model/weights.cpp:97-104, 147-160
//   qmatmul                      src/model/marlin.cpp:18-25
//   mlp_forward                  src/model/marlin.cpp:31-35 (+ :141-142)
//   lm_head                      src/model/marlin.cpp:161-169
//   sample_token (greedy)        src/sampling/sampler.cpp:9-16
//
// Device memory is owned by DeviceBuffer (hipMalloc/hipFree); every call is
// stream-ordered on the given hipStream_t.  Errors come back as
// mq4::Result<T> (a value or an Error with the library's message), the
// C++17 counterpart of the reference's std::expected Result<T>
// (src/core/types.h:13-19); no exception crosses the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <initializer_list>
#include <random>
#include <string>
#include <utility>
#include <variant>
#include <vector>

#include "mq4.h"

namespace mq4 {

struct Error {
    int code = 0;
    std::string message;
};

template <typename T>
class Result {
public:
    Result(T v) : v_(std::move(v)) {}
    Result(Error e) : v_(std::move(e)) {}
    bool ok() const { return v_.index() == 0; }
    explicit operator bool() const { return ok(); }
    T& value() { return std::get<0>(v_); }
    const Error& error() const { return std::get<1>(v_); }

private:
    std::variant<T, Error> v_;
};

inline Error last_error(int code) { return Error{code, mq4_last_error()}; }

// Owning device allocation.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) : bytes_(bytes) {
        if (bytes && hipMalloc(&p_, bytes) != hipSuccess) {
            p_ = nullptr;
            bytes_ = 0;
        }
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), bytes_(o.bytes_) { o.p_ = nullptr; o.bytes_ = 0; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            reset();
            p_ = o.p_;
            bytes_ = o.bytes_;
            o.p_ = nullptr;
            o.bytes_ = 0;
        }
        return *this;
    }
    ~DeviceBuffer() { reset(); }
    void reset() {
        if (p_) (void)hipFree(p_);
        p_ = nullptr;
        bytes_ = 0;
    }
    void* get() const { return p_; }
    size_t bytes() const { return bytes_; }
    template <typename T>
    T* as() const { return static_cast<T*>(p_); }

private:
    void* p_ = nullptr;
    size_t bytes_ = 0;
};

// MLX-layout Q4 weight: weight uint32 [N, K/8], scales/biases bf16 [N, K/64].
struct QuantizedTensor {
    DeviceBuffer weight, scales, biases;
    int64_t out_features = 0;   // N
    int64_t in_features = 0;    // K
    int group_size = 64;
    int bits = 4;
    bool quantized = false;

    const uint32_t* wq() const { return weight.as<uint32_t>(); }
    const uint16_t* s() const { return scales.as<uint16_t>(); }
    const uint16_t* b() const { return biases.as<uint16_t>(); }
};

// quantize_weight (src/model/weights.cpp:45-56): w is a device bf16 [N, K].
inline Result<QuantizedTensor> quantize_weight(const uint16_t* w, int64_t N, int64_t K,
                                               hipStream_t stream, int bits = 4, int group_size = 64) {
    QuantizedTensor q;
    q.out_features = N;
    q.in_features = K;
    q.bits = bits;
    q.group_size = group_size;
    q.weight = DeviceBuffer((size_t)N * (size_t)K / 8 * 4);
    q.scales = DeviceBuffer((size_t)N * (size_t)(K / (group_size > 0 ? group_size : 1)) * 2);
    q.biases = DeviceBuffer(q.scales.bytes());
    if (N > 0 && K > 0 && (!q.weight.get() || !q.scales.get() || !q.biases.get()))
        return Error{MQ4_ERR_HIP, "quantize_weight: device allocation failed"};
    const int rc = mq4_quantize(w, N, K, group_size, bits, q.weight.as<uint32_t>(), q.scales.as<uint16_t>(),
                                q.biases.as<uint16_t>(), stream);
    if (rc != MQ4_OK) return last_error(rc);
    q.quantized = true;
    return q;
}

// A bf16 [N, K] device weight to quantize (quantize_weights).
struct WeightView {
    const uint16_t* w;
    int64_t N, K;
};

// The loader's loop of quantize_weight calls (src/model/weights.cpp:97-104
// per layer at :147-160, and the lm_head at :180-194) as one batched call
// (mq4_quantize_batch); the tensors are bit-identical to quantize_weight's.
inline Result<std::vector<QuantizedTensor>> quantize_weights(const std::vector<WeightView>& ws,
                                                             hipStream_t stream, int bits = 4,
                                                             int group_size = 64) {
    std::vector<QuantizedTensor> out(ws.size());
    std::vector<mq4_quantize_job> jobs(ws.size());
    const int64_t gs = group_size > 0 ? group_size : 1;
    for (size_t i = 0; i < ws.size(); ++i) {
        QuantizedTensor& q = out[i];
        q.out_features = ws[i].N;
        q.in_features = ws[i].K;
        q.bits = bits;
        q.group_size = group_size;
        const bool shape_ok = ws[i].N > 0 && ws[i].K > 0;
        q.weight = DeviceBuffer(shape_ok ? (size_t)ws[i].N * (size_t)ws[i].K / 8 * 4 : 0);
        q.scales = DeviceBuffer(shape_ok ? (size_t)ws[i].N * (size_t)(ws[i].K / gs) * 2 : 0);
        q.biases = DeviceBuffer(q.scales.bytes());
        if (shape_ok && (!q.weight.get() || !q.scales.get() || !q.biases.get()))
            return Error{MQ4_ERR_HIP, "quantize_weights: device allocation failed"};
        jobs[i] = mq4_quantize_job{ws[i].w, ws[i].N, ws[i].K, q.weight.as<uint32_t>(), q.scales.as<uint16_t>(),
                                   q.biases.as<uint16_t>()};
    }
    const int rc = mq4_quantize_batch(jobs.data(), (int64_t)jobs.size(), group_size, bits, stream);
    if (rc != MQ4_OK) return last_error(rc);
    for (QuantizedTensor& q : out) q.quantized = true;
    return out;
}

// qmatmul (src/model/marlin.cpp:18-25): y[M, N] = x[M, K] @ dequant(W)^T.
inline Result<int> qmatmul(const uint16_t* x, int64_t M, const QuantizedTensor& w, uint16_t* y,
                           hipStream_t stream) {
    if (!w.quantized) return Error{MQ4_ERR_UNSUPPORTED, "qmatmul: unquantized weights are outside this library"};
    if (M == 0) return 0;   // no rows: nothing to compute (the C ABI rejects M = 0)
    const int rc = mq4_qmm(x, M, w.in_features, w.wq(), w.s(), w.b(), w.out_features, 1, w.group_size, w.bits, y,
                           stream);
    if (rc != MQ4_OK) return last_error(rc);
    return 0;
}

struct MLPWeights {   // src/model/marlin.h:17-21
    QuantizedTensor gate_proj, up_proj, down_proj;
};

// The fused entry points (mq4_mlp_residual, mq4_rmsnorm_gate_up_silu,
// mq4_qmm_residual, mq4_lm_head_argmax) take no format argument: they read
// the group-64, 4-bit layout only, so a tensor of another format (a cache
// file MLX wrote with group 128, say) is rejected here before its buffers
// reach them.
inline bool q4_format_ok(const QuantizedTensor& q) { return q.quantized && q.group_size == 64 && q.bits == 4; }

inline Result<int> check_q4(const char* fn, std::initializer_list<const QuantizedTensor*> qs) {
    for (const QuantizedTensor* q : qs)
        if (!q4_format_ok(*q))
            return Error{MQ4_ERR_UNSUPPORTED, std::string(fn) + ": needs group_size=64, bits=4 quantized weights"};
    return 0;
}

// hidden = hidden + mlp_forward(rms_norm(hidden, norm_weight)) in two kernels
// (src/model/marlin.cpp:141-142, 31-35); h is scratch of [M, intermediate].
inline Result<int> mlp_forward_residual(uint16_t* hidden, int64_t M, const uint16_t* norm_weight, float eps,
                                        const MLPWeights& w, uint16_t* h, hipStream_t stream) {
    const int64_t K = w.gate_proj.in_features, N = w.gate_proj.out_features;
    if (auto r = check_q4("mlp_forward_residual", {&w.gate_proj, &w.up_proj, &w.down_proj}); !r) return r.error();
    if (M == 0) return 0;
    int rc = norm_weight
                 ? mq4_rmsnorm_gate_up_silu(hidden, M, K, norm_weight, eps, w.gate_proj.wq(), w.gate_proj.s(),
                                            w.gate_proj.b(), w.up_proj.wq(), w.up_proj.s(), w.up_proj.b(), N, h,
                                            stream)
                 : mq4_mlp_gate_up_silu(hidden, M, K, w.gate_proj.wq(), w.gate_proj.s(), w.gate_proj.b(),
                                        w.up_proj.wq(), w.up_proj.s(), w.up_proj.b(), N, h, stream);
    if (rc != MQ4_OK) return last_error(rc);
    rc = mq4_qmm_residual(h, M, N, w.down_proj.wq(), w.down_proj.s(), w.down_proj.b(), w.down_proj.out_features,
                          hidden, hidden, stream);
    if (rc != MQ4_OK) return last_error(rc);
    return 0;
}

// hidden = hidden + mlp_forward(rms_norm(hidden, norm_weight)) in one call
// (src/model/marlin.cpp:141-142, 31-35), in place; the workspace holds
// mq4_mlp_workspace_size(max_rows, hidden size, intermediate size) bytes,
// which covers every call of at most max_rows rows (the size never shrinks
// as the row count grows).
class MlpResidual {
public:
    MlpResidual(int64_t max_rows, int64_t hidden, int64_t intermediate)
        : ws_(mq4_mlp_workspace_size(max_rows, hidden, intermediate)), max_rows_(max_rows) {}
    Result<int> operator()(uint16_t* x, int64_t M, const uint16_t* norm_weight, float eps, const MLPWeights& w,
                           hipStream_t stream) {
        if (M > max_rows_) return Error{MQ4_ERR_WORKSPACE, "MlpResidual: M exceeds max_rows"};
        if (auto r = check_q4("MlpResidual", {&w.gate_proj, &w.up_proj, &w.down_proj}); !r) return r.error();
        if (M == 0) return 0;
        const int rc = mq4_mlp_residual(x, M, w.gate_proj.in_features, norm_weight, eps, w.gate_proj.wq(),
                                        w.gate_proj.s(), w.gate_proj.b(), w.up_proj.wq(), w.up_proj.s(),
                                        w.up_proj.b(), w.down_proj.wq(), w.down_proj.s(), w.down_proj.b(),
                                        w.gate_proj.out_features, ws_.get(), ws_.bytes(), x, stream);
        if (rc != MQ4_OK) return last_error(rc);
        return 0;
    }

private:
    DeviceBuffer ws_;
    int64_t max_rows_;
};

// The MLP halves of a layer stack for M concurrent token rows (1 <= M <=
// max_rows <= 32), one launch per layer (mq4_mlp_layers; src/model/
// marlin.cpp:141-142 for M streams, src/core/engine.cpp:79-94): holds the
// layer table and its workspace, zero-filled here once.  x_out must overlap
// neither x nor the workspace; results agree with MlpResidual to fp32
// rounding.  Built for hidden 2048 / intermediate 6144.
class BatchedMlpLayers {
public:
    struct Layer {
        const uint16_t* post_attn_norm;
        const MLPWeights* mlp;
    };
    BatchedMlpLayers(const std::vector<Layer>& layers, int64_t max_rows)
        : ws_(mq4_mlp_layers_workspace_size(max_rows, 2048, 6144)), max_rows_(max_rows) {
        for (const Layer& l : layers) {
            const MLPWeights& w = *l.mlp;
            table_.push_back(mq4_mlp_layer{l.post_attn_norm, w.gate_proj.wq(), w.gate_proj.s(), w.gate_proj.b(),
                                           w.up_proj.wq(), w.up_proj.s(), w.up_proj.b(), w.down_proj.wq(),
                                           w.down_proj.s(), w.down_proj.b()});
            mlps_.push_back(l.mlp);
        }
        if (ws_.get() && hipMemset(ws_.get(), 0, ws_.bytes()) != hipSuccess) ws_.reset();
    }
    // layers [first, first + count) of the table over the M rows of x
    Result<int> operator()(const uint16_t* x, int64_t M, float eps, uint16_t* x_out, hipStream_t stream,
                           size_t first = 0, size_t count = SIZE_MAX) {
        if (!ws_.get()) return Error{MQ4_ERR_WORKSPACE, "BatchedMlpLayers: no workspace (unsupported sizes?)"};
        if (M > max_rows_) return Error{MQ4_ERR_WORKSPACE, "BatchedMlpLayers: M exceeds max_rows"};
        if (first >= table_.size()) return Error{MQ4_ERR_INVALID_ARG, "BatchedMlpLayers: no such layer"};
        if (count > table_.size() - first) count = table_.size() - first;
        for (size_t l = first; l < first + count; ++l) {
            const MLPWeights& w = *mlps_[l];
            if (auto r = check_q4("BatchedMlpLayers", {&w.gate_proj, &w.up_proj, &w.down_proj}); !r) return r.error();
        }
        if (M == 0) return 0;
        const int rc = mq4_mlp_layers(x, M, 2048, 6144, (int64_t)count, table_.data() + first, eps, x_out, ws_.get(),
                                      ws_.bytes(), stream);
        if (rc != MQ4_OK) return last_error(rc);
        return 0;
    }

private:
    DeviceBuffer ws_;
    int64_t max_rows_;
    std::vector<mq4_mlp_layer> table_;
    std::vector<const MLPWeights*> mlps_;
};

// Greedy next token(s): idx[m] = argmax(lm_head(rms_norm(hidden))) for each
// of the M rows (src/model/marlin.cpp:145, 161-169; src/sampling/sampler.cpp:14-16).
class GreedyLmHead {
public:
    GreedyLmHead(int64_t max_rows, int64_t vocab)
        : ws_(mq4_lm_head_argmax_workspace_size(max_rows, vocab)), max_rows_(max_rows) {}
    Result<int> operator()(const uint16_t* hidden, int64_t M, const uint16_t* final_norm, float eps,
                           const QuantizedTensor& lm, uint32_t* idx, uint16_t* logits, hipStream_t stream) {
        if (M > max_rows_) return Error{MQ4_ERR_WORKSPACE, "GreedyLmHead: M exceeds max_rows"};
        if (auto r = check_q4("GreedyLmHead", {&lm}); !r) return r.error();
        if (M == 0) return 0;
        const int rc = final_norm
                           ? mq4_rmsnorm_lm_head_argmax(hidden, M, lm.in_features, final_norm, eps, lm.wq(), lm.s(),
                                                        lm.b(), lm.out_features, idx, logits, ws_.get(), ws_.bytes(),
                                                        stream)
                           : mq4_lm_head_argmax(hidden, M, lm.in_features, lm.wq(), lm.s(), lm.b(),
                                                lm.out_features, idx, logits, ws_.get(), ws_.bytes(), stream);
        if (rc != MQ4_OK) return last_error(rc);
        return 0;
    }

    // The next token after a prompt: the reference computes the lm_head for
    // all S rows of the prefill hidden state (src/core/engine.cpp:64) and
    // sample_token keeps the last row (src/sampling/sampler.cpp:10-12); only
    // that row's logits matter for a greedy token, so only it is computed.
    // hidden is the [S, K] (or [1, S, K]) row-major prefill output.
    Result<int> last_row(const uint16_t* hidden, int64_t S, const uint16_t* final_norm, float eps,
                         const QuantizedTensor& lm, uint32_t* idx, uint16_t* logits, hipStream_t stream) {
        if (S <= 0) return Error{MQ4_ERR_INVALID_ARG, "GreedyLmHead::last_row: S must be positive"};
        return (*this)(hidden + (S - 1) * lm.in_features, 1, final_norm, eps, lm, idx, logits, stream);
    }

private:
    DeviceBuffer ws_;
    int64_t max_rows_;
};

// The sampling fields of the reference's SamplingConfig
// (src/core/config.h:60-63); seed drives this library's counter-based
// generator (the reference's seed field is unused and MLX's global key,
// seeded from the clock, draws).  seed = -1, the reference's default, takes
// a base drawn once per process from std::random_device, so separate
// processes draw different sequences, as they do in the reference.
struct SamplingConfig {
    float temperature = 0.0f;
    float top_p = 1.0f;
    int top_k = 0;
    int64_t seed = -1;
};

inline uint64_t process_seed() {
    static const uint64_t s = [] {
        std::random_device rd;
        return ((uint64_t)rd() << 32) ^ (uint64_t)rd();
    }();
    return s;
}

// sample_token over bf16 logits [M, vocab] (src/sampling/sampler.cpp:9-39),
// one token per row.  Each call draws with seed + the number of earlier
// calls, so successive tokens are independent, as the reference's advancing
// global key makes them; equal (seed, call count) give equal tokens.
class Sampler {
public:
    Sampler(int64_t max_rows, int64_t vocab) : max_rows_(max_rows), vocab_(vocab) {
        size_t need = 0;
        for (int64_t m = 1; m <= max_rows; ++m) {
            const size_t b = mq4_sample_workspace_size(m, vocab);
            need = b > need ? b : need;
        }
        ws_ = DeviceBuffer(need);
    }
    Result<int> operator()(const uint16_t* logits, int64_t M, const SamplingConfig& c, uint32_t* idx,
                           uint8_t* keep, hipStream_t stream) {
        if (M > max_rows_) return Error{MQ4_ERR_WORKSPACE, "Sampler: M exceeds max_rows"};
        const size_t need = mq4_sample_workspace_size(M, vocab_);
        if (need > ws_.bytes()) return Error{MQ4_ERR_WORKSPACE, "Sampler: workspace allocation failed"};
        const uint64_t base = c.seed < 0 ? process_seed() : (uint64_t)c.seed;
        const int rc = mq4_sample_bf16(logits, M, vocab_, c.temperature, c.top_k, c.top_p, base + calls_++, idx,
                                       keep, need ? ws_.get() : nullptr, need, stream);
        if (rc != MQ4_OK) return last_error(rc);
        return 0;
    }

private:
    DeviceBuffer ws_;
    int64_t max_rows_, vocab_;
    uint64_t calls_ = 0;
};

}  // namespace mq4
