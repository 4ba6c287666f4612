/*
 * tensor_cpp/qwen3_ops_avx.h - the reference's AVX2 Qwen3 layer and forward,
 * served by the MI355X library.
 *
 * Same signatures as the reference (reference
 * tensor_cpp/include/tensor_cpp/qwen3_ops_avx.h:24-135).  These take the
 * separate q_proj / k_proj / v_proj weights, and normalise q and k per head as
 * the reference's AVX2 code does, x / (sqrt(mean(x^2)) + 1e-6) * w (eps added
 * to the root, tensor_cpp/src/qwen3_ops_avx.cpp:537, :566); everything else
 * is the GPU path of tensor_cpp/qwen3_ops.h.
 */
#ifndef SA_AMD_TENSOR_CPP_QWEN3_OPS_AVX_H
#define SA_AMD_TENSOR_CPP_QWEN3_OPS_AVX_H

#include <string>
#include <vector>

#include "tensor_cpp/qwen3_ops.h"
#include "tensor_cpp/tensor.h"

namespace tensor_cpp {
namespace qwen3 {
namespace avx2 {

/* qwen3_attention with separate projections (reference qwen3_ops_avx.cpp:25-146). */
Tensor qwen3_attention_avx(const Tensor& hidden_states, size_t num_attention_heads, size_t num_key_value_heads,
                           size_t head_dim, const Tensor& q_proj, const Tensor& k_proj, const Tensor& v_proj,
                           const Tensor& o_proj, const Tensor& q_norm_weight, const Tensor& k_norm_weight,
                           const Tensor& cos, const Tensor& sin);

/* One decoder layer without a cache (reference qwen3_ops_avx.cpp:329-377). */
Tensor qwen3_decoder_layer_avx(const Tensor& hidden_states, size_t num_attention_heads, size_t num_key_value_heads,
                               size_t head_dim, float rms_norm_eps, const Tensor& input_layernorm_weight,
                               const Tensor& q_proj, const Tensor& k_proj, const Tensor& v_proj,
                               const Tensor& o_proj, const Tensor& q_norm_weight, const Tensor& k_norm_weight,
                               const Tensor& post_attention_layernorm_weight, const Tensor& gate_mlp,
                               const Tensor& up_mlp, const Tensor& down_mlp, const Tensor& cos,
                               const Tensor& sin);

/* Logits [B, S, vocab] without a cache (reference qwen3_ops_avx.cpp:383-453). */
Tensor qwen3_forward_avx(const TensorL& input_ids, const Tensor& token_embedding,
                         const std::vector<Qwen3LayerWeights>& layers, const Tensor& norm_weight,
                         const Tensor& lm_head, size_t num_layers, size_t num_attention_heads,
                         size_t num_key_value_heads, size_t head_dim, float rms_norm_eps);

/* down(silu(gate(x)) * up(x)) (reference qwen3_ops_avx.cpp:456-463). */
Tensor qwen3_mlp_avx(const Tensor& hidden_states, const Tensor& gate_proj, const Tensor& up_proj,
                     const Tensor& down_proj);

/* qwen3_decoder_layer_with_cache with separate projections
 * (reference qwen3_ops_avx.cpp:469-754). */
Tensor qwen3_decoder_layer_avx_with_cache(const Tensor& hidden_states, KVCache* kv_cache, size_t layer_idx,
                                          size_t num_attention_heads, size_t num_key_value_heads,
                                          size_t head_dim, float rms_norm_eps,
                                          const Tensor& input_layernorm_weight, const Tensor& q_proj,
                                          const Tensor& k_proj, const Tensor& v_proj, const Tensor& o_proj,
                                          const Tensor& q_norm_weight, const Tensor& k_norm_weight,
                                          const Tensor& post_attention_layernorm_weight, const Tensor& gate_mlp,
                                          const Tensor& up_mlp, const Tensor& down_mlp, const Tensor& cos,
                                          const Tensor& sin, AttentionType attention_type = AttentionType::STANDARD);

/* qwen3_forward_with_cache over the layers' q_proj / k_proj / v_proj
 * (reference qwen3_ops_avx.cpp:760-843). */
Tensor qwen3_forward_avx_with_cache(const TensorL& input_ids, KVCache* kv_cache, const Tensor& token_embedding,
                                    const std::vector<Qwen3LayerWeights>& layers, const Tensor& norm_weight,
                                    const Tensor& lm_head, size_t num_layers, size_t num_attention_heads,
                                    size_t num_key_value_heads, size_t head_dim, float rms_norm_eps,
                                    AttentionType attention_type = AttentionType::STANDARD);

}  // namespace avx2
}  // namespace qwen3
}  // namespace tensor_cpp

#endif
