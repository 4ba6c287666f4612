/*
 * tensor_cpp/attention_avx.h - the reference's AVX2 attention operators
 * (reference tensor_cpp/include/tensor_cpp/attention_avx.h:14-57), served by
 * the MI355X library with the same namespace, names and signatures.
 *
 * self_attention_avx2 follows the reference's mask rule
 * (tensor_cpp/src/attention_avx.cpp:95-117): only -inf entries of the mask
 * count (finite values are ignored, not added), a mask whose dimension 2 is 1
 * ([1, 1, 1, k_seq_len]) applies to every query row, any other mask is read
 * as [q_seq_len, k_seq_len].  Supported -inf patterns: none (every query
 * attends to every key: the dense decode kernel) and the causal one
 * (q_seq_len == k_seq_len, -inf exactly above the diagonal: the causal
 * prefill kernel); any other pattern throws std::invalid_argument.  The
 * softmax is exact where the reference drops terms more than 20 below the
 * row max (attention_avx.cpp:110-115), a relative difference under e^-20 per
 * dropped term.  key/value may have fewer heads than query (GQA, query head h
 * reading key head h / (heads / kv_heads)); the reference requires equal
 * head counts, which is the case with kv_heads == heads.
 */
#ifndef SA_AMD_TENSOR_CPP_ATTENTION_AVX_H
#define SA_AMD_TENSOR_CPP_ATTENTION_AVX_H

#include <immintrin.h>

#include "tensor_cpp/tensor.h"

namespace tensor_cpp {
namespace ops {
namespace avx2 {

/* softmax(scale q k^T, -inf entries of mask excluded) v for query
 * [batch, heads, q_seq_len, head_dim] and key/value [batch, kv_heads,
 * k_seq_len, head_dim] (reference tensor_cpp/src/attention_avx.cpp:22-158). */
Tensor self_attention_avx2(const Tensor& query, const Tensor& key, const Tensor& value, const Tensor* mask,
                           float scale);

/* input [..., in_features] . weight [out_features, in_features]^T (+ bias),
 * as ops::linear (reference tensor_cpp/src/attention_avx.cpp:164-242). */
Tensor linear_avx2(const Tensor& input, const Tensor& weight, const Tensor* bias = nullptr);

}  // namespace avx2
}  // namespace ops
}  // namespace tensor_cpp

#endif  // SA_AMD_TENSOR_CPP_ATTENTION_AVX_H
