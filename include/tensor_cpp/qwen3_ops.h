/*
 * tensor_cpp/qwen3_ops.h - the attention path of the reference's Qwen3 layer,
 * served by the MI355X library.
 *
 * From the reference (reference tensor_cpp/include/tensor_cpp/qwen3_ops.h):
 * AttentionType, compute_rope_freqs, apply_rotary_pos_emb, repeat_kv,
 * create_causal_mask.  In place of qwen3_decoder_layer_with_cache, whose
 * projections, MLP and residuals are outside this library,
 * qwen3_attention_with_cache runs the part of it between the Q/K/V
 * projections and o_proj (reference tensor_cpp/src/qwen3_ops.cpp:697-909):
 * per-head RMSNorm of q and k, RoPE at position current_seq_len + s, append
 * to the cache, and causal prefill (cache empty) or decode attention.
 */
#ifndef SA_AMD_TENSOR_CPP_QWEN3_OPS_H
#define SA_AMD_TENSOR_CPP_QWEN3_OPS_H

#include <utility>

#include "tensor_cpp/kv_cache.h"
#include "tensor_cpp/ops.h"
#include "tensor_cpp/tensor.h"

namespace tensor_cpp {
namespace qwen3 {

enum class AttentionType {
    STANDARD,   // softmax attention (decode: all-zero mask, prefill: causal mask)
    STREAMING   // online softmax (decode: self_attention_streaming, prefill: blockwise)
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

}  // namespace qwen3
}  // namespace tensor_cpp

#endif
