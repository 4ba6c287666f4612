/*
 * tensor_cpp/qwen3_ops.h - the reference's Qwen3 layer and forward, served by
 * the MI355X library.
 *
 * From the reference (reference tensor_cpp/include/tensor_cpp/qwen3_ops.h):
 * AttentionType, Qwen3LayerWeights, compute_rope_freqs, apply_rotary_pos_emb,
 * repeat_kv, create_causal_mask, qwen3_attention, qwen3_mlp,
 * qwen3_decoder_layer, qwen3_forward, qwen3_decoder_layer_with_cache and
 * qwen3_forward_with_cache, with the reference's signatures.  Weights and
 * activations are host fp32 tensors as there; each call uploads them, runs
 * the layer on the GPU in fp32 (fp32 MFMA projections, fused QK-norm + RoPE,
 * MFMA causal prefill or split-KV paged decode) and returns host tensors.
 * The forward keeps the hidden state on the GPU from the embedding to the
 * logits.  Also here: qwen3_attention_with_cache, the part of the layer
 * between the projections and o_proj, for callers with their own projections.
 *
 * Shapes the GPU path takes: head_dim 16, 32, 64 or 128; with a non-empty cache one
 * token per call (as the reference, whose concat appends one token).  Others
 * throw std::invalid_argument.
 */
#ifndef SA_AMD_TENSOR_CPP_QWEN3_OPS_H
#define SA_AMD_TENSOR_CPP_QWEN3_OPS_H

#include <utility>
#include <vector>

#include "tensor_cpp/kv_cache.h"
#include "tensor_cpp/ops.h"
#include "tensor_cpp/tensor.h"

namespace tensor_cpp {
namespace qwen3 {

enum class AttentionType {
    STANDARD,   // softmax attention (decode: all-zero mask, prefill: causal mask)
    STREAMING   // online softmax (decode: self_attention_streaming, prefill: blockwise)
};

/* One decoder layer's weights, nn.Linear layout [out, in]
 * (reference tensor_cpp/include/tensor_cpp/qwen3_ops.h:38-58).  The non-AVX
 * functions read qkv_projs (q rows, then k rows, then v rows); the avx2 ones
 * read q_proj, k_proj and v_proj. */
struct Qwen3LayerWeights {
    Tensor qkv_projs;      // [(Hq + 2 Hkv) * head_dim, hidden]
    Tensor q_proj;         // [Hq * head_dim, hidden]
    Tensor k_proj;         // [Hkv * head_dim, hidden]
    Tensor v_proj;         // [Hkv * head_dim, hidden]
    Tensor o_proj;         // [hidden, Hq * head_dim]
    Tensor q_norm_weight;  // [head_dim]
    Tensor k_norm_weight;  // [head_dim]
    Tensor input_layernorm_weight;            // [hidden]
    Tensor post_attention_layernorm_weight;   // [hidden]
    Tensor gate_proj;      // [intermediate, hidden]
    Tensor up_proj;        // [intermediate, hidden]
    Tensor down_proj;      // [hidden, intermediate]
};

/* cos, sin [seq_len, head_dim / 2] with inv_freq[i] = 1 / theta^(i / head_dim)
 * (reference tensor_cpp/src/qwen3_ops.cpp:70-104). */
std::pair<Tensor, Tensor> compute_rope_freqs(size_t seq_len, size_t head_dim, float theta = 10000.0f);

/* Rotate-half RoPE of q [B, Hq, S, D] and k [B, Hkv, S, D] with cos/sin rows
 * 0..S-1 (reference tensor_cpp/src/qwen3_ops.cpp:110-188). */
std::pair<Tensor, Tensor> apply_rotary_pos_emb(const Tensor& q, const Tensor& k, const Tensor& cos,
                                               const Tensor& sin);

/* [B, Hkv, S, D] -> [B, Hkv * n_rep, S, D], head h_kv * n_rep + r copies h_kv
 * (reference tensor_cpp/src/qwen3_ops.cpp:194-234). */
Tensor repeat_kv(const Tensor& hidden_states, int n_rep);

/* [seq_len, seq_len], 0 where j <= i, -inf elsewhere (reference qwen3_ops.cpp:240-259). */
Tensor create_causal_mask(size_t seq_len, float dtype = 0.0f);

/* The attention block of qwen3_decoder_layer_with_cache on the GPU.
 * q_proj_out [B, S, Hq * D], k_proj_out / v_proj_out [B, S, Hkv * D] (the
 * projection outputs before view/transpose); q_norm_weight / k_norm_weight
 * [D]; RoPE theta 1e6 at positions current_seq_len + s; eps inside the sqrt.
 * Appends K/V to kv_cache (layer_idx) without committing them: call
 * kv_cache->increment_seq_len(S) after the last layer, as
 * qwen3_forward_with_cache does.  With an empty cache the S queries attend
 * causally (prefill); otherwise S must be 1 (decode over the cache plus the
 * new token).  Returns the attention output [B, Hq, S, D] (before o_proj).
 * STREAMING decode honours ops::g_streaming_scale_on_output. */
Tensor qwen3_attention_with_cache(const Tensor& q_proj_out, const Tensor& k_proj_out,
                                  const Tensor& v_proj_out, KVCache* kv_cache, size_t layer_idx,
                                  size_t num_attention_heads, size_t num_key_value_heads, size_t head_dim,
                                  float rms_norm_eps, const Tensor& q_norm_weight,
                                  const Tensor& k_norm_weight,
                                  AttentionType attention_type = AttentionType::STANDARD);

/* Attention of a layer without a cache: q/k/v projections of hidden_states
 * [B, S, hidden] (already normed), per-head RMSNorm of q and k (eps 1e-6),
 * RoPE with rows 0..S-1 of cos/sin, causal attention, o_proj
 * -> [B, S, hidden] (reference tensor_cpp/src/qwen3_ops.cpp:302-431).
 * has_cache is accepted and ignored, as there. */
Tensor qwen3_attention(const Tensor& hidden_states, size_t num_attention_heads, size_t num_key_value_heads,
                       size_t head_dim, const Tensor& q_proj, const Tensor& k_proj, const Tensor& v_proj,
                       const Tensor& o_proj, const Tensor& q_norm_weight, const Tensor& k_norm_weight,
                       const Tensor& cos, const Tensor& sin, bool has_cache = false);

/* down(silu(gate(x)) * up(x)) (reference tensor_cpp/src/qwen3_ops.cpp:265-296). */
Tensor qwen3_mlp(const Tensor& hidden_states, const Tensor& gate_proj, const Tensor& up_proj,
                 const Tensor& down_proj);

/* One decoder layer without a cache: RMSNorm, qwen3_attention, residual,
 * RMSNorm, qwen3_mlp, residual (reference tensor_cpp/src/qwen3_ops.cpp:437-531). */
Tensor qwen3_decoder_layer(const Tensor& hidden_states, size_t num_attention_heads, size_t num_key_value_heads,
                           size_t head_dim, float rms_norm_eps, const Tensor& input_layernorm_weight,
                           const Tensor& qkv_projs, const Tensor& o_proj, const Tensor& q_norm_weight,
                           const Tensor& k_norm_weight, const Tensor& post_attention_layernorm_weight,
                           const Tensor& gate_mlp, const Tensor& up_mlp, const Tensor& down_mlp,
                           const Tensor& cos, const Tensor& sin);

/* Logits [B, S, vocab] of input_ids [B, S] without a cache
 * (reference tensor_cpp/src/qwen3_ops.cpp:537-614). */
Tensor qwen3_forward(const TensorL& input_ids, const Tensor& token_embedding,
                     const std::vector<Qwen3LayerWeights>& layers, const Tensor& norm_weight,
                     const Tensor& lm_head, size_t num_layers, size_t num_attention_heads,
                     size_t num_key_value_heads, size_t head_dim, float rms_norm_eps);

/* One decoder layer with a KV cache (reference tensor_cpp/src/qwen3_ops.cpp:620-934).
 * hidden_states [B, S, hidden].  kv_cache may be NULL (no cache: causal
 * attention over the S tokens).  With an empty cache the S tokens are a
 * prefill: RoPE with rows 0..S-1 of cos/sin, K (normed and rotated) and V
 * written to the cache, causal attention.  With current_seq_len = P > 0,
 * S must be 1: RoPE with row P, the token appended at P, attention over the
 * P + 1 tokens.  The cache length is not advanced (the forward does that once
 * per call).  STREAMING with one query honours ops::g_streaming_scale_on_output.
 * Returns [B, S, hidden]. */
Tensor qwen3_decoder_layer_with_cache(const Tensor& hidden_states, KVCache* kv_cache, size_t layer_idx,
                                      size_t num_attention_heads, size_t num_key_value_heads, size_t head_dim,
                                      float rms_norm_eps, const Tensor& input_layernorm_weight,
                                      const Tensor& qkv_projs, const Tensor& o_proj, const Tensor& q_norm_weight,
                                      const Tensor& k_norm_weight, const Tensor& post_attention_layernorm_weight,
                                      const Tensor& gate_mlp, const Tensor& up_mlp, const Tensor& down_mlp,
                                      const Tensor& cos, const Tensor& sin,
                                      AttentionType attention_type = AttentionType::STANDARD);

/* Logits [B, S, vocab] of input_ids [B, S]: embedding, the layers with the
 * cache, kv_cache->increment_seq_len(S) once, final RMSNorm, lm_head
 * (reference tensor_cpp/src/qwen3_ops.cpp:936-1014).  RoPE uses theta 1e6 at
 * positions current_seq_len + s.  kv_cache may be NULL. */
Tensor qwen3_forward_with_cache(const TensorL& input_ids, KVCache* kv_cache, const Tensor& token_embedding,
                                const std::vector<Qwen3LayerWeights>& layers, const Tensor& norm_weight,
                                const Tensor& lm_head, size_t num_layers, size_t num_attention_heads,
                                size_t num_key_value_heads, size_t head_dim, float rms_norm_eps,
                                AttentionType attention_type = AttentionType::STANDARD);

}  // namespace qwen3
}  // namespace tensor_cpp

#endif
