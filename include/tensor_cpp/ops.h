/*
 * tensor_cpp/ops.h - the attention operators of the reference's ops namespace,
 * served by the MI355X library.
 *
 * Same signatures as the reference (reference tensor_cpp/include/tensor_cpp/ops.h:133-329);
 * tensors are host [batch, heads, seq, head_dim] fp32 as there, and each call
 * runs the gfx950 kernels (split-KV decode, MFMA causal prefill) and returns
 * a host tensor.  Beyond the reference, key/value may carry fewer heads than
 * the query (grouped KV heads: query head h reads KV head h / (H_q / H_kv)),
 * so repeat_kv is not needed.
 *
 * Supported attention shapes: single-query decode (q_len = 1) and causal
 * prefill from position 0 (q_len = kv_len).  self_attention accepts a null or
 * all-zero mask with q_len = 1, or the causal mask with q_len = kv_len; any
 * other mask throws std::invalid_argument.
 */
#ifndef SA_AMD_TENSOR_CPP_OPS_H
#define SA_AMD_TENSOR_CPP_OPS_H

#include <vector>

#include "tensor_cpp/tensor.h"

namespace tensor_cpp {
namespace ops {

/* softmax(scale * Q K^T + mask) V (reference tensor_cpp/src/ops.cpp:514-641). */
Tensor self_attention(const Tensor& query, const Tensor& key, const Tensor& value,
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
