// Attention operators of the reference's ops namespace on the GPU
// (reference tensor_cpp/src/ops.cpp:514-738, 742-1017, 1027-1599).
#include "tensor_cpp/ops.h"
#include "tensor_cpp/attention_avx.h"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <string>

#include "attention.h"
#include "device.h"

namespace tensor_cpp {

int g_q_block_size = 32;
int g_kv_block_size = 64;

namespace ops {

bool g_streaming_scale_on_output = false;

namespace {

using sa_compat::check;
using sa_compat::staging;
using sa_compat::to_device;
using sa_compat::to_host;

struct Dims {
    size_t B, Hq, Sq, D, Hkv, Sk;
};

Dims check_qkv(const Tensor& q, const Tensor& k, const Tensor& v) {
    if (q.ndim() != 4 || k.ndim() != 4 || v.shape() != k.shape())
        throw std::invalid_argument("attention expects [batch, heads, seq, head_dim] query/key/value");
    Dims d{q.shape()[0], q.shape()[1], q.shape()[2], q.shape()[3], k.shape()[1], k.shape()[2]};
    if (k.shape()[0] != d.B || k.shape()[3] != d.D) throw std::invalid_argument("key shape does not match query");
    if (d.Hkv == 0 || d.Hq % d.Hkv) throw std::invalid_argument("query heads must be a multiple of key heads");
    return d;
}

// out[b, h, i, :] = softmax(scale q[b, h, i] k[b, h/rep]^T) v for every query
// row i (no mask), through the dense decode kernel: q goes up once as
// [Sq][B][Hq][D], one decode call per query row runs on the device without a
// host round trip between calls (they share the workspace in stream order),
// and the outputs come back once.
Tensor decode_rows(const Tensor& q, const Tensor& k, const Tensor& v, const Dims& d, float scale) {
    auto& st = staging();
    const size_t kv = k.size();
    float* dk = st.in[1].as<float>(kv);
    float* dv = st.in[2].as<float>(kv);
    to_device(dk, k.data(), kv * sizeof(float));
    to_device(dv, v.data(), kv * sizeof(float));
    const size_t nq = d.B * d.Hq * d.D;   // one query row of every (batch, head)
    float* dq = st.in[0].as<float>(nq * d.Sq);
    float* dout = st.out.as<float>(nq * d.Sq);
    const size_t ws_bytes = sa_decode_dense_ws_bytes((int)d.B, (int)d.Hq, (int)d.Sk, (int)d.D);
    void* ws = ws_bytes ? st.ws.ensure(ws_bytes) : nullptr;
    std::vector<float> rows(nq * d.Sq);
    for (size_t i = 0; i < d.Sq; ++i)
        for (size_t bh = 0; bh < d.B * d.Hq; ++bh)
            for (size_t x = 0; x < d.D; ++x) rows[(i * d.B * d.Hq + bh) * d.D + x] = q[(bh * d.Sq + i) * d.D + x];
    to_device(dq, rows.data(), rows.size() * sizeof(float));
    for (size_t i = 0; i < d.Sq; ++i)
        check(sa_decode_dense_f32(dq + i * nq, dk, dv, (int)d.B, (int)d.Hq, (int)d.Hkv, (int)d.Sk, (int)d.D, scale,
                                  dout + i * nq, ws, ws_bytes, nullptr),
              "sa_decode_dense_f32");
    to_host(rows.data(), dout, rows.size() * sizeof(float));
    std::vector<float> out(q.size());
    for (size_t i = 0; i < d.Sq; ++i)
        for (size_t bh = 0; bh < d.B * d.Hq; ++bh)
            for (size_t x = 0; x < d.D; ++x) out[(bh * d.Sq + i) * d.D + x] = rows[(i * d.B * d.Hq + bh) * d.D + x];
    return Tensor(std::move(out), q.shape());
}

// Causal prefill from position 0 on the MFMA kernel: query i sees keys 0..i.
Tensor causal_prefill(const Tensor& q, const Tensor& k, const Tensor& v, const Dims& d, float scale) {
    if (d.Sq > d.Sk) throw std::invalid_argument("causal prefill needs at least as many keys as queries");
    auto& st = staging();
    const size_t nq = q.size();
    const size_t nkv = d.B * d.Hkv * d.Sq * d.D;   // keys past Sq are never visible
    float* dq = st.in[0].as<float>(nq);
    float* dk = st.in[1].as<float>(nkv);
    float* dv = st.in[2].as<float>(nkv);
    float* dout = st.out.as<float>(nq);
    to_device(dq, q.data(), nq * sizeof(float));
    if (d.Sk == d.Sq) {
        to_device(dk, k.data(), nkv * sizeof(float));
        to_device(dv, v.data(), nkv * sizeof(float));
    } else {
        const size_t rows = d.Sq * d.D;
        for (size_t bh = 0; bh < d.B * d.Hkv; ++bh) {
            to_device(dk + bh * rows, k.data() + bh * d.Sk * d.D, rows * sizeof(float));
            to_device(dv + bh * rows, v.data() + bh * d.Sk * d.D, rows * sizeof(float));
        }
    }
    const size_t ws_bytes = sa_prefill_causal_ws_bytes(SA_DTYPE_F32, (int)d.B, (int)d.Hq, (int)d.Hkv, (int)d.Sq,
                                                       (int)d.D);
    void* ws = ws_bytes ? st.ws.ensure(ws_bytes) : nullptr;
    check(sa_prefill_causal_ws(dq, dk, dv, SA_DTYPE_F32, (int)d.B, (int)d.Hq, (int)d.Hkv, (int)d.Sq, (int)d.D,
                               scale, dout, ws, ws_bytes, nullptr),
          "sa_prefill_causal_ws");
    std::vector<float> out(nq);
    to_host(out.data(), dout, nq * sizeof(float));
    return Tensor(std::move(out), q.shape());
}

enum class MaskKind { kNone, kCausal, kOther };

MaskKind classify(const Tensor* mask, size_t Sq, size_t Sk) {
    if (!mask) return MaskKind::kNone;
    const size_t n = mask->size();
    if (n < Sq * Sk) return MaskKind::kOther;
    bool zero = true, causal = Sq == Sk;
    const float ninf = -std::numeric_limits<float>::infinity();
    for (size_t i = 0; i < Sq; ++i)
        for (size_t j = 0; j < Sk; ++j) {
            const float m = (*mask)[i * Sk + j];
            if (m != 0.0f) zero = false;
            if (causal && m != (j <= i ? 0.0f : ninf)) causal = false;
        }
    if (zero) return MaskKind::kNone;
    if (causal) return MaskKind::kCausal;
    return MaskKind::kOther;
}

// The -inf pattern of a self_attention_avx2 mask, read as the reference reads
// it (tensor_cpp/src/attention_avx.cpp:95-117): a mask whose dimension 2 is 1
// is one row for every query, any other is [Sq, Sk]; finite entries do not
// count.
MaskKind classify_ninf(const Tensor* mask, size_t Sq, size_t Sk) {
    if (!mask) return MaskKind::kNone;
    const float ninf = -std::numeric_limits<float>::infinity();
    const bool row = mask->ndim() >= 3 && mask->shape()[2] == 1;
    if (mask->size() < (row ? Sk : Sq * Sk)) throw std::invalid_argument("mask is smaller than the score matrix");
    bool none = true, causal = !row && Sq == Sk;
    for (size_t i = 0; i < (row ? 1 : Sq); ++i)
        for (size_t j = 0; j < Sk; ++j) {
            const bool masked = (*mask)[i * Sk + j] == ninf;
            if (masked) none = false;
            if (causal && masked != (j > i)) causal = false;
        }
    if (none) return MaskKind::kNone;
    if (causal) return MaskKind::kCausal;
    return MaskKind::kOther;
}

}  // namespace

Tensor self_attention(const Tensor& query, const Tensor& key, const Tensor& value, const Tensor* mask,
                      float scale) {
    const Dims d = check_qkv(query, key, value);
    switch (classify(mask, d.Sq, d.Sk)) {
        case MaskKind::kNone: return decode_rows(query, key, value, d, scale);
        case MaskKind::kCausal: return causal_prefill(query, key, value, d, scale);
        default: throw std::invalid_argument("self_attention supports no mask, an all-zero mask or the causal mask");
    }
}

Tensor cross_attention(const Tensor& query, const Tensor& key, const Tensor& value, const Tensor* /*mask*/,
                       float scale) {
    return decode_rows(query, key, value, check_qkv(query, key, value), scale);
}

std::vector<float> naive_attention_serial(const float* Q, const float* K, const float* V, int T, int d) {
    return ::naive_attention_serial(Q, K, V, T, d);
}

std::vector<float> streaming_attention_serial(const float* Q, const float* K, const float* V, int T, int d,
                                              int block_size) {
    return ::streaming_attention_serial(Q, K, V, T, d, block_size);
}

std::vector<float> streaming_attention_omp(const float* Q, const float* K, const float* V, int T, int d,
                                           int block_size, int num_threads) {
    return ::streaming_attention_omp(Q, K, V, T, d, block_size, num_threads);
}

Tensor self_attention_streaming(const Tensor& query, const Tensor& key, const Tensor& value, float scale,
                                int block_size) {
    if (block_size <= 0) throw std::invalid_argument("block_size must be positive");
    const Dims d = check_qkv(query, key, value);
    if (!g_streaming_scale_on_output) return decode_rows(query, key, value, d, scale);
    Tensor out = decode_rows(query, key, value, d, 1.0f);
    for (size_t i = 0; i < out.size(); ++i) out[i] *= scale;
    return out;
}

Tensor self_attention_streaming_blockwise(const Tensor& query, const Tensor& key, const Tensor& value,
                                          float scale, int q_block_size, int kv_block_size) {
    if (q_block_size <= 0 || kv_block_size <= 0) throw std::invalid_argument("block sizes must be positive");
    const Dims d = check_qkv(query, key, value);
    return causal_prefill(query, key, value, d, scale);
}

Tensor self_attention_streaming_blockwise_avx2(const Tensor& query, const Tensor& key, const Tensor& value,
                                               float scale, int q_block_size, int kv_block_size) {
    return self_attention_streaming_blockwise(query, key, value, scale, q_block_size, kv_block_size);
}

Tensor self_attention_streaming_blockwise_avx2_cache_optimized(const Tensor& query, const Tensor& key,
                                                               const Tensor& value, float scale,
                                                               int q_block_size, int kv_block_size) {
    return self_attention_streaming_blockwise(query, key, value, scale, q_block_size, kv_block_size);
}

namespace avx2 {

Tensor self_attention_avx2(const Tensor& query, const Tensor& key, const Tensor& value, const Tensor* mask,
                           float scale) {
    const Dims d = check_qkv(query, key, value);
    switch (classify_ninf(mask, d.Sq, d.Sk)) {
        case MaskKind::kNone: return decode_rows(query, key, value, d, scale);
        case MaskKind::kCausal: return causal_prefill(query, key, value, d, scale);
        default:
            throw std::invalid_argument("self_attention_avx2 supports a mask with no -inf entries or the causal one");
    }
}

Tensor linear_avx2(const Tensor& input, const Tensor& weight, const Tensor* bias) {
    return ops::linear(input, weight, bias);
}

}  // namespace avx2
}  // namespace ops
}  // namespace tensor_cpp
