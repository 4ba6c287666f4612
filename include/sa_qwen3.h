/*
 * sa_qwen3.h - the Qwen3 decoder around the attention path, on the GPU.
 *
 * One greedy decode step of a batch of sequences through the whole model:
 * token embedding, per layer RMSNorm -> q/k/v projections -> per-head q/k
 * RMSNorm + RoPE + K/V append (sa_qknorm_rope_append) -> paged GQA decode
 * (sa_paged_decode) -> o projection + residual -> RMSNorm -> SwiGLU MLP +
 * residual, then the final RMSNorm, lm_head and argmax.  This replaces
 * qwen3_forward_with_cache with a one-token input (reference
 * tensor_cpp/src/qwen3_ops.cpp:936-1014, the layer at :620-934, the MLP at
 * :265-296, ops::rms_norm / linear / embedding at tensor_cpp/src/ops.cpp:278-417).
 *
 * Weights are bf16 matrices in nn.Linear layout [out][in] and fp32 norm
 * weights; activations, accumulation and logits are fp32.  The K/V cache is
 * an sa_kvcache whose geometry matches the model (layers, KV heads, head_dim).
 */
#ifndef SA_QWEN3_H
#define SA_QWEN3_H

#include "sa_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sa_qwen3_desc {
    int num_layers;     /* 28 for Qwen3-0.6B */
    int hidden;         /* 1024 */
    int intermediate;   /* 3072 */
    int vocab;          /* 151936 */
    int n_q_heads;      /* 16 */
    int n_kv_heads;     /* 8 */
    int head_dim;       /* 128 */
    int max_pos;        /* rows of the RoPE tables: positions 0 .. max_pos-1 */
    float rms_eps;      /* 1e-6 */
    float rope_theta;   /* 1e6 */
} sa_qwen3_desc;

typedef struct sa_qwen3 sa_qwen3;

/* Weight tensors, per layer unless noted.  Shapes ([rows][cols], row-major):
 *   SA_QW_EMBED      [vocab][hidden]              bf16 (layer ignored)
 *   SA_QW_IN_NORM    [hidden]                     fp32
 *   SA_QW_QKV        [(Hq + 2 Hkv) D][hidden]     bf16, rows q | k | v
 *   SA_QW_Q_NORM     [D]                          fp32
 *   SA_QW_K_NORM     [D]                          fp32
 *   SA_QW_O          [hidden][Hq D]               bf16
 *   SA_QW_POST_NORM  [hidden]                     fp32
 *   SA_QW_GATE_UP    [2 intermediate][hidden]     bf16, rows gate | up
 *   SA_QW_DOWN       [hidden][intermediate]       bf16
 *   SA_QW_FINAL_NORM [hidden]                     fp32 (layer ignored)
 *   SA_QW_LM_HEAD    [vocab][hidden]              bf16 (layer ignored)      */
typedef enum sa_qwen3_tensor {
    SA_QW_EMBED = 0, SA_QW_IN_NORM, SA_QW_QKV, SA_QW_Q_NORM, SA_QW_K_NORM, SA_QW_O,
    SA_QW_POST_NORM, SA_QW_GATE_UP, SA_QW_DOWN, SA_QW_FINAL_NORM, SA_QW_LM_HEAD
} sa_qwen3_tensor;

/* Allocate the weights (uninitialised), RoPE tables and the activations of a
 * batch of up to max_batch sequences (max_batch <= 1024; the projections
 * tile rows by 64, the fused attention launches 64 sequences at a time).
 * Requirements:
 * hidden, Hq*D, (Hq+2Hkv)*D, 2*intermediate and vocab multiples of 64;
 * hidden, Hq*D and intermediate multiples of 32; D in {64, 128}. */
sa_status sa_qwen3_create(const sa_qwen3_desc* desc, int max_batch, sa_qwen3** out);
sa_status sa_qwen3_destroy(sa_qwen3* model);

/* The desc the model was created with (an accessor; no reference counterpart). */
sa_status sa_qwen3_get_desc(const sa_qwen3* model, sa_qwen3_desc* desc);

/* Device pointer, element count and dtype of one weight tensor. */
sa_status sa_qwen3_tensor_ptr(sa_qwen3* model, int layer, sa_qwen3_tensor which, void** ptr,
                              size_t* count, sa_dtype* dtype);

/* Synthetic weights: matrices std * N(0,1) rounded to bf16, norm weights
 * 1 + std * N(0,1).  Element i of a tensor is draw i of stream
 * (1000 + 16 * layer + which) of the seeded splitmix64 / Box-Muller
 * generator (seed * 0x9E3779B97F4A7C15 ^ stream << 32 ^ index, fp64 Box-Muller
 * on draws 2i and 2i+1, rounded to fp32), so any tensor can be rebuilt on a
 * host from (seed, stream). */
sa_status sa_qwen3_init_random(sa_qwen3* model, uint64_t seed, float std, sa_stream_t stream);

/* ---- Checkpoints in safetensors format (Hugging Face Qwen3 tensor names) ----
 * Replace load_qwen3_weights (reference tensor_cpp/src/qwen3_loader.cpp:
 * 188-296, declared in tensor_cpp/include/tensor_cpp/qwen3_loader.h:80-85).
 * Names read: model.embed_tokens.weight, model.norm.weight, lm_head.weight
 * (absent when the checkpoint ties it to the embedding: the embedding is
 * used), and per layer i model.layers.i.{input_layernorm, post_attention_
 * layernorm, self_attn.{q,k,v,o}_proj, self_attn.{q,k}_norm,
 * mlp.{gate,up,down}_proj}.weight.  Tensors may be BF16 or F32; matrices are
 * stored on the device in bf16 (F32 rounded to nearest even), norm weights
 * in fp32.  Host only, no GPU needed: */

/* The model shape the checkpoint holds: layer count from the layer names,
 * hidden and vocab from the embedding, head_dim from q_norm, head counts
 * from q_proj / k_proj rows, intermediate from gate_proj.  rms_eps = 1e-6
 * and rope_theta = 1e6 (Qwen3's values; the file does not carry them) and
 * max_pos = 0, for the caller to set.  SA_EIO: unreadable or malformed file;
 * SA_EINVAL: a tensor missing or of a shape that does not fit the others. */
sa_status sa_qwen3_desc_from_safetensors(const char* path, sa_qwen3_desc* desc);

/* Upload a checkpoint into a model created with a matching desc (same
 * layers, hidden, intermediate, vocab, heads and head_dim): q/k/v rows
 * fused q | k | v, gate/up fused gate | up.  Synchronous. */
sa_status sa_qwen3_load_safetensors(sa_qwen3* model, const char* path);

/* Prefill: a prompt of L tokens for each of sequences 0 .. batch-1, which
 * must be empty, in one forward (qwen3_forward_with_cache on an empty cache
 * with input [batch, L]; reference tensor_cpp/src/qwen3_ops.cpp:936-1014).
 * tokens: device int32 [batch][L].  Every layer appends the prompt's K/V
 * (positions 0 .. L-1) and attends causally over it; afterwards each
 * sequence's length is L.  next_tokens: device int32 [batch], the argmax of
 * the last position's logits; logits: device fp32 [batch][vocab] (that
 * position) or NULL.  The caller must have reserved L tokens of pages.
 * Activations of batch * L rows live in a grow-only device buffer of the
 * model (allocated on the first call of a larger size).  Asynchronous. */
sa_status sa_qwen3_prefill(sa_qwen3* model, sa_kvcache* cache, const int32_t* tokens, int batch, int L,
                           int32_t* next_tokens, float* logits, sa_stream_t stream);

/* One greedy decode step for sequences 0 .. batch-1 of the cache.
 * tokens: device int32 [batch] input ids; token i is appended to sequence i
 * at position sa_kvcache_len(cache, i), every layer attends over that
 * sequence's committed tokens plus the new one, and afterwards every
 * sequence's length grows by one (the reference's increment_seq_len after
 * the last layer).  next_tokens: device int32 [batch], argmax of the logits
 * (lowest index on ties).  logits: device fp32 [batch][vocab] or NULL.  The
 * caller must have reserved cache pages for the new tokens.  Input ids
 * outside [0, vocab) embed as zeros.  Asynchronous on stream; the first call
 * with a given cache geometry allocates the attention workspace. */
sa_status sa_qwen3_decode_step(sa_qwen3* model, sa_kvcache* cache, const int32_t* tokens, int batch,
                               int32_t* next_tokens, float* logits, sa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SA_QWEN3_H */
