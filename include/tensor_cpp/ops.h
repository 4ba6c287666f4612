/*
 * tensor_cpp/ops.h - the operators of the reference's ops namespace that the
 * Qwen3 layer uses (attention, linear, RMSNorm, SwiGLU, add, embedding),
 * served by the MI355X library.
 *
 * Same signatures as the reference (reference tensor_cpp/include/tensor_cpp/ops.h:35-329);
 * tensors are host fp32 as there (attention: [batch, heads, seq, head_dim]),
 * and each call runs the gfx950 kernels (split-KV decode, MFMA causal
 * prefill, fp32 MFMA linear) and returns a host tensor.  Beyond the reference, key/value may carry fewer heads than
 * the query (grouped KV heads: query head h reads KV head h / (H_q / H_kv)),
 * so repeat_kv is not needed.
 *
 * Supported attention shapes: single-query decode (q_len = 1) and causal
 * prefill from position 0 (q_len = kv_len).  self_attention accepts a null or
 * all-zero mask with q_len = 1, or the causal mask with q_len = kv_len; any
 * other mask throws std::invalid_argument.  cross_attention takes any q_len
 * and kv_len (every query row sees every key).  head_dim: 8, 16, 32, 64, 128
 * or 256 without a mask, 16, 32, 64 or 128 for causal prefill.
 *
 * The reference's all_reduce_sum and broadcast (MPI collectives, ops.h:338-339)
 * are not here: this library serves one GPU per process.
 */
#ifndef SA_AMD_TENSOR_CPP_OPS_H
#define SA_AMD_TENSOR_CPP_OPS_H

#include <cmath>
#include <complex>
#include <stdexcept>
#include <vector>

#include "tensor_cpp/tensor.h"

/* The reference's ops.h brings in OpenMP's API (ops.h:20); its benchmarks and
 * tests call omp_set_num_threads and the like through this header. */
#if __has_include(<omp.h>)
#include <omp.h>
#endif

/* Integer tensor of token ids (reference tensor_cpp/include/tensor_cpp/ops.h:35-52). */
class TensorL {
public:
    TensorL() = default;
    TensorL(const std::vector<long>& data, const tensor_cpp::Shape& shape) : data_(data), shape_(shape) {
        if (data.size() != shape.total()) throw std::invalid_argument("Data size does not match shape");
    }
    const tensor_cpp::Shape& shape() const { return shape_; }
    size_t size() const { return data_.size(); }
    const long* data() const { return data_.data(); }
    long operator[](size_t i) const { return data_[i]; }

private:
    std::vector<long> data_;
    tensor_cpp::Shape shape_;
};

namespace tensor_cpp {
namespace ops {

/* input + alpha * other, same shapes (reference tensor_cpp/src/ops.cpp:194-207).
 * On the GPU. */
Tensor add(const Tensor& input, const Tensor& other, float alpha = 1.0f);

/* Index of the largest element (reference tensor_cpp/src/ops.cpp:213-272),
 * the first of equal maxima.  dim = -1: over the whole tensor -> shape [1].
 * dim = ndim - 1 (ndim >= 2): one index per leading row, shaped as the
 * reference shapes it: the leading dims with keepdim, else those before the
 * last two, [1] if none remain; where that shape does not hold the row count
 * (say [B, V] with B > 1 and no keepdim) TensorL throws
 * std::invalid_argument, as the reference's does.  Other dims throw
 * std::runtime_error.  A host scan: the qwen3 functions return host logits. */
TensorL argmax(const Tensor& input, int dim = -1, bool keepdim = false);

/* Rows of weight [num_embeddings, dim] picked by indices -> [indices..., dim];
 * an index outside the table throws std::out_of_range unless it equals
 * padding_idx (a zero row) (reference tensor_cpp/src/ops.cpp:278-309).  A copy
 * of host rows: only the picked rows cross to the GPU in the layer path. */
Tensor embedding(const TensorL& indices, const Tensor& weight, long padding_idx = -1);

/* input [..., in] . weight[out, in]^T (+ bias [out]) -> [..., out], fp32 MFMA
 * on the GPU (reference tensor_cpp/src/ops.cpp:315-369). */
Tensor linear(const Tensor& input, const Tensor& weight, const Tensor* bias = nullptr);

/* x / sqrt(mean(x^2) + eps) * weight over the last axis, on the GPU
 * (reference tensor_cpp/src/ops.cpp:375-418).  Only dim = -1 (the last). */
Tensor rms_norm(const Tensor& input, const Tensor* weight = nullptr, float eps = 1e-8f, int dim = -1);

/* Rotary embedding on [batch, seq, heads, dim] (reference
 * tensor_cpp/include/tensor_cpp/ops.h:99-111, tensor_cpp/src/ops.cpp:424-487):
 * element i of a head is paired with element i + dim/2 and the pair is
 * rotated by the angle t * theta^(-i / dim) at sequence index t (the
 * reference's frequencies, i / dim rather than the 2i / dim of
 * compute_rope_freqs).  apply rotates the first seq_len positions on the GPU
 * and returns zeros for positions past seq_len, as the reference.  dim must
 * be even (the constructor throws std::invalid_argument otherwise, as the
 * reference); apply takes dim 8, 16, 32, 64, 128 or 256 and seq_len up to
 * max_seq_len and the input's seq axis (std::invalid_argument otherwise). */
class RotaryEmbedding {
public:
    RotaryEmbedding(size_t dim, size_t max_seq_len = 2048, float theta = 10000.0f);
    Tensor apply(const Tensor& input, size_t seq_len);

private:
    size_t dim_;
    size_t max_seq_len_;
    float theta_;
    std::vector<float> cos_, sin_;   // [max_seq_len][dim / 2]

    void precompute_freqs_cis();
};

/* x * silu(gate), elementwise on the GPU (reference tensor_cpp/src/ops.cpp:493-509). */
Tensor swiglu(const Tensor& x, const Tensor& gate);

/* softmax(scale * Q K^T + mask) V (reference tensor_cpp/src/ops.cpp:514-641). */
Tensor self_attention(const Tensor& query, const Tensor& key, const Tensor& value,
                      const Tensor* mask = nullptr, float scale = 1.0f);

/* softmax(scale * Q K^T) V with query [batch, heads, q_len, head_dim] and
 * key/value [batch, kv_heads, kv_len, head_dim] (reference
 * tensor_cpp/src/ops.cpp:647-738).  The reference takes a mask argument and
 * does not read it; so here. */
Tensor cross_attention(const Tensor& query, const Tensor& key, const Tensor& value,
                       const Tensor* mask = nullptr, float scale = 1.0f);

/* Single-query helpers (reference tensor_cpp/src/ops.cpp:742-958). */
std::vector<float> naive_attention_serial(const float* Q, const float* K, const float* V, int T, int d);
std::vector<float> streaming_attention_serial(const float* Q, const float* K, const float* V, int T, int d,
                                              int block_size);
std::vector<float> streaming_attention_omp(const float* Q, const float* K, const float* V, int T, int d,
                                           int block_size, int num_threads = 0);

/* Decode (query [B, H, 1, D]) with the online-softmax kernel (reference
 * tensor_cpp/src/ops.cpp:964-1017).  Returns softmax(scale q k^T) v.  The
 * reference instead computes softmax(q k^T) v * scale; set
 * g_streaming_scale_on_output to reproduce that. */
Tensor self_attention_streaming(const Tensor& query, const Tensor& key, const Tensor& value,
                                float scale = 1.0f, int block_size = 64);

/* Causal prefill from position 0 (reference tensor_cpp/src/ops.cpp:1027-1112,
 * 1383-1599).  Block sizes are the reference's tuning knobs; the GPU tiling
 * is fixed and the result does not depend on them beyond rounding. */
Tensor self_attention_streaming_blockwise(const Tensor& query, const Tensor& key, const Tensor& value,
                                          float scale = 1.0f, int q_block_size = 32, int kv_block_size = 64);
Tensor self_attention_streaming_blockwise_avx2(const Tensor& query, const Tensor& key, const Tensor& value,
                                               float scale = 1.0f, int q_block_size = 32,
                                               int kv_block_size = 64);
Tensor self_attention_streaming_blockwise_avx2_cache_optimized(const Tensor& query, const Tensor& key,
                                                               const Tensor& value, float scale = 1.0f,
                                                               int q_block_size = 32, int kv_block_size = 64);

/* When true, self_attention_streaming returns softmax(q k^T) v * scale, as the
 * reference's decode path does (default false: the correct attention). */
extern bool g_streaming_scale_on_output;

}  // namespace ops

/* The reference's process-wide block sizes for the prefill path
 * (reference tensor_cpp/include/tensor_cpp/ops.h:350-351). */
extern int g_q_block_size;
extern int g_kv_block_size;

}  // namespace tensor_cpp

#endif
