// The dense operators of the reference's ops namespace on the GPU: add,
// linear, rms_norm, swiglu, RotaryEmbedding (reference
// tensor_cpp/src/ops.cpp:194-207, :315-369, :375-418, :493-509, :424-487),
// and two host operations: embedding, a gather of host rows (:278-309), and
// argmax (:213-272).  Each GPU call uploads its host tensors, runs one kernel
// of libsa_amd and returns a host tensor.
#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "device.h"
#include "tensor_cpp/ops.h"

namespace tensor_cpp {
namespace ops {

namespace {

using sa_compat::check;
using sa_compat::staging;
using sa_compat::to_device;
using sa_compat::to_host;

// Rows and width of a tensor read as [..., n] (at least 2-D, as the reference's
// linear and rms_norm require).
void rows_of(const Tensor& t, const char* op, size_t* rows, size_t* n) {
    if (t.ndim() < 2) throw std::invalid_argument(std::string(op) + " requires at least 2D input");
    *n = t.shape()[t.ndim() - 1];
    *rows = *n ? t.size() / *n : 0;
}

int as_int(size_t v, const char* what) {
    if (v > 0x7fffffffu) throw std::invalid_argument(std::string(what) + " exceeds the kernels' int range");
    return static_cast<int>(v);
}

}  // namespace

Tensor add(const Tensor& input, const Tensor& other, float alpha) {
    if (input.shape() != other.shape()) throw std::invalid_argument("Shape mismatch for addition");
    const size_t n = input.size();
    auto& st = staging();
    float* a = st.in[0].as<float>(n);
    float* b = st.in[1].as<float>(n);
    to_device(a, input.data(), n * sizeof(float));
    to_device(b, other.data(), n * sizeof(float));
    check(sa_axpby_f32(a, 1.0f, b, alpha, n, a, nullptr), "sa_axpby_f32");
    std::vector<float> out(n);
    to_host(out.data(), a, n * sizeof(float));
    return Tensor(std::move(out), input.shape());
}

Tensor embedding(const TensorL& indices, const Tensor& weight, long padding_idx) {
    if (weight.ndim() != 2) throw std::invalid_argument("embedding weight must be [num_embeddings, dim]");
    const size_t V = weight.shape()[0], H = weight.shape()[1];
    std::vector<float> out(indices.size() * H, 0.0f);
    for (size_t i = 0; i < indices.size(); ++i) {
        const long idx = indices[i];
        if (idx < 0 || idx >= static_cast<long>(V)) {
            if (padding_idx >= 0 && idx == padding_idx) continue;   // zero row
            throw std::out_of_range("Embedding index out of range");
        }
        std::copy(weight.data() + static_cast<size_t>(idx) * H, weight.data() + (static_cast<size_t>(idx) + 1) * H,
                  out.begin() + i * H);
    }
    Shape shape = indices.shape();
    shape.dims.push_back(H);
    return Tensor(std::move(out), shape);
}

Tensor linear(const Tensor& input, const Tensor& weight, const Tensor* bias) {
    size_t M, K;
    rows_of(input, "Linear", &M, &K);
    if (weight.ndim() != 2 || weight.shape()[1] != K)
        throw std::invalid_argument("Weight shape mismatch in linear layer");
    const size_t N = weight.shape()[0];
    if (bias && bias->size() != N) throw std::invalid_argument("bias must have out_features entries");
    std::vector<size_t> dims(input.shape().dims.begin(), input.shape().dims.end() - 1);
    dims.push_back(N);
    std::vector<float> out(M * N, 0.0f);
    if (M && N) {
        auto& st = staging();
        float* dx = st.in[0].as<float>(M * K);
        float* dw = st.in[1].as<float>(N * K);
        float* db = bias ? st.in[2].as<float>(N) : nullptr;
        float* dy = st.out.as<float>(M * N);
        to_device(dx, input.data(), M * K * sizeof(float));
        to_device(dw, weight.data(), N * K * sizeof(float));
        if (db) to_device(db, bias->data(), N * sizeof(float));
        check(sa_linear_f32(dx, as_int(M, "rows"), as_int(K, "in_features"), dw, as_int(N, "out_features"), db, dy,
                            nullptr),
              "sa_linear_f32");
        to_host(out.data(), dy, M * N * sizeof(float));
    }
    return Tensor(std::move(out), Shape(dims));
}

Tensor rms_norm(const Tensor& input, const Tensor* weight, float eps, int dim) {
    size_t rows, n;
    rows_of(input, "RMS norm", &rows, &n);
    if (dim != -1 && dim != static_cast<int>(input.ndim()) - 1)
        throw std::invalid_argument("rms_norm normalises the last dimension only");
    if (weight && weight->size() != n) throw std::invalid_argument("rms_norm weight must have hidden_size entries");
    std::vector<float> out(input.size());
    if (rows && n) {
        auto& st = staging();
        float* dx = st.in[0].as<float>(input.size());
        float* dw = weight ? st.in[1].as<float>(n) : nullptr;
        to_device(dx, input.data(), input.size() * sizeof(float));
        if (dw) to_device(dw, weight->data(), n * sizeof(float));
        check(sa_rms_norm_f32(dx, as_int(rows, "rows"), as_int(n, "hidden_size"), dw, eps, dx, nullptr),
              "sa_rms_norm_f32");
        to_host(out.data(), dx, input.size() * sizeof(float));
    }
    return Tensor(std::move(out), input.shape());
}

TensorL argmax(const Tensor& input, int dim, bool keepdim) {
    const size_t nd = input.ndim();
    if (dim == -1) {
        if (input.size() == 0) throw std::invalid_argument("argmax of an empty tensor");
        size_t best = 0;
        for (size_t i = 1; i < input.size(); ++i)
            if (input[i] > input[best]) best = i;
        return TensorL({static_cast<long>(best)}, Shape({1}));
    }
    if (dim != static_cast<int>(nd) - 1) throw std::runtime_error("argmax supports dim = -1 (global) or the last dim");
    if (nd < 2) throw std::invalid_argument("Argmax along last dim requires at least 2D input");
    const size_t n = input.shape()[nd - 1];
    if (n == 0) throw std::invalid_argument("argmax along an empty axis");
    const size_t rows = input.size() / n;
    std::vector<long> idx(rows);
    for (size_t r = 0; r < rows; ++r) {
        const float* x = input.data() + r * n;
        size_t best = 0;
        for (size_t i = 1; i < n; ++i)
            if (x[i] > x[best]) best = i;
        idx[r] = static_cast<long>(best);
    }
    // The reference's result shape: leading dims, the one before the last
    // kept only with keepdim; [1] when none remain.
    std::vector<size_t> dims;
    for (size_t i = 0; i + 1 < nd; ++i)
        if (keepdim || i + 2 < nd) dims.push_back(input.shape()[i]);
    if (dims.empty()) dims.push_back(1);
    return TensorL(idx, Shape(dims));
}

RotaryEmbedding::RotaryEmbedding(size_t dim, size_t max_seq_len, float theta)
    : dim_(dim), max_seq_len_(max_seq_len), theta_(theta) {
    if (dim % 2 != 0) throw std::invalid_argument("Rotary embedding dimension must be even");
    precompute_freqs_cis();
}

void RotaryEmbedding::precompute_freqs_cis() {
    const size_t half = dim_ / 2;
    std::vector<float> freq(half);
    for (size_t i = 0; i < half; ++i)
        freq[i] = 1.0f / std::pow(theta_, static_cast<float>(i) / static_cast<float>(dim_));
    cos_.resize(max_seq_len_ * half);
    sin_.resize(max_seq_len_ * half);
    for (size_t t = 0; t < max_seq_len_; ++t)
        for (size_t i = 0; i < half; ++i) {
            const float a = static_cast<float>(t) * freq[i];
            cos_[t * half + i] = std::cos(a);
            sin_[t * half + i] = std::sin(a);
        }
}

Tensor RotaryEmbedding::apply(const Tensor& input, size_t seq_len) {
    if (input.ndim() != 4) throw std::invalid_argument("RoPE requires 4D input: (batch, seq, heads, head_dim)");
    const size_t B = input.shape()[0], S = input.shape()[1], H = input.shape()[2], D = input.shape()[3];
    if (D != dim_) throw std::invalid_argument("Head dimension must match rotary embedding dimension");
    if (seq_len > S || seq_len > max_seq_len_)
        throw std::invalid_argument("seq_len exceeds the input's sequence axis or max_seq_len");
    std::vector<float> out(input.size(), 0.0f);
    const size_t per_b = seq_len * H * D;   // the rotated rows of one batch, contiguous
    if (B == 0 || per_b == 0) return Tensor(std::move(out), input.shape());
    const size_t rows = B * seq_len * H, half = D / 2;
    auto& st = staging();
    float* dx = st.in[0].as<float>(rows * D);
    float* dcos = st.in[2].as<float>(seq_len * half);
    float* dsin = st.in[3].as<float>(seq_len * half);
    int32_t* dpos = st.pos.as<int32_t>(rows);
    for (size_t b = 0; b < B; ++b) to_device(dx + b * per_b, input.data() + b * S * H * D, per_b * sizeof(float));
    to_device(dcos, cos_.data(), seq_len * half * sizeof(float));
    to_device(dsin, sin_.data(), seq_len * half * sizeof(float));
    std::vector<int32_t> pos(rows);
    for (size_t r = 0; r < rows; ++r) pos[r] = static_cast<int32_t>((r / H) % seq_len);
    to_device(dpos, pos.data(), rows * sizeof(int32_t));
    check(sa_qk_norm_rope(dx, as_int(rows, "rows"), as_int(D, "head_dim"), dpos, nullptr, 0.0f, dcos, dsin,
                          as_int(seq_len, "seq_len"), dx, nullptr),
          "sa_qk_norm_rope");
    for (size_t b = 0; b < B; ++b) to_host(out.data() + b * S * H * D, dx + b * per_b, per_b * sizeof(float));
    return Tensor(std::move(out), input.shape());
}

Tensor swiglu(const Tensor& x, const Tensor& gate) {
    if (x.shape() != gate.shape()) throw std::invalid_argument("Shape mismatch for SwiGLU");
    const size_t n = x.size();
    auto& st = staging();
    float* dx = st.in[0].as<float>(n);
    float* dg = st.in[1].as<float>(n);
    to_device(dx, x.data(), n * sizeof(float));
    to_device(dg, gate.data(), n * sizeof(float));
    check(sa_swiglu_f32(dg, dx, n, dx, nullptr), "sa_swiglu_f32");
    std::vector<float> out(n);
    to_host(out.data(), dx, n * sizeof(float));
    return Tensor(std::move(out), x.shape());
}

}  // namespace ops
}  // namespace tensor_cpp
