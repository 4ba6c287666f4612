/*
 * tensor_cpp/qwen3_loader.h - the reference's Qwen3 weight loader, served by
 * the MI355X library.
 *
 * From the reference (reference tensor_cpp/include/tensor_cpp/qwen3_loader.h):
 * bf16_to_float, TensorInfo, Qwen3Weights, load_qwen3_weights and
 * test_qwen3_forward, with the reference's signatures.  The weights are host
 * fp32 tensors, as the qwen3_ops functions take them.
 *
 * load_qwen3_weights reads a Hugging Face Qwen3 checkpoint (one safetensors
 * file).  Where the reference reads every tensor as BF16 and assumes 28
 * layers, 16/8 heads and head_dim 128 (tensor_cpp/src/qwen3_loader.cpp:188,
 * :217-221), this one parses the header as JSON, takes BF16 or F32 tensors,
 * reads the model shape from the file (layers from the tensor names, head_dim
 * from q_norm, the head counts from the q_proj / k_proj rows) and checks
 * every tensor's shape against it; on Qwen3-0.6B both give the same weights.
 * A checkpoint without lm_head.weight (tied word embeddings) gets a copy of
 * the embedding as lm_head.  Errors throw std::runtime_error: "Failed to open
 * safetensors file: <path>" for a file that cannot be opened or whose header
 * is malformed, "Tensor not found: <name>" for a missing tensor (as the
 * reference), and a message naming the tensor for a wrong shape or dtype.
 */
#ifndef SA_AMD_TENSOR_CPP_QWEN3_LOADER_H
#define SA_AMD_TENSOR_CPP_QWEN3_LOADER_H

#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "tensor_cpp/qwen3_ops.h"
#include "tensor_cpp/tensor.h"

namespace tensor_cpp {
namespace qwen3 {

/* A bf16 bit pattern widened to fp32: the bf16 bits are the top half of the
 * fp32 word (reference tensor_cpp/include/tensor_cpp/qwen3_loader.h:25-35). */
inline float bf16_to_float(uint16_t bf16) {
    const uint32_t bits = static_cast<uint32_t>(bf16) << 16;
    float f;
    std::memcpy(&f, &bits, sizeof(f));
    return f;
}

/* One entry of a safetensors header (reference
 * tensor_cpp/include/tensor_cpp/qwen3_loader.h:40-51). */
struct TensorInfo {
    std::string dtype;
    std::vector<size_t> shape;
    size_t offset_start;
    size_t offset_end;

    size_t total_elements() const {
        size_t n = 1;
        for (size_t s : shape) n *= s;
        return n;
    }
};

/* The whole model's weights (reference
 * tensor_cpp/include/tensor_cpp/qwen3_loader.h:56-77).  Every layer holds both
 * qkv_projs (q rows, then k rows, then v rows) and the separate q/k/v_proj. */
struct Qwen3Weights {
    Tensor embed_tokens;   // [vocab_size, hidden_size]
    Tensor norm_weight;    // [hidden_size]
    Tensor lm_head;        // [vocab_size, hidden_size]
    std::vector<Qwen3LayerWeights> layers;

    size_t num_layers;
    size_t num_attention_heads;
    size_t num_key_value_heads;
    size_t head_dim;
    size_t hidden_size;
    size_t vocab_size;
};

/* The weights of the checkpoint at path (reference
 * tensor_cpp/src/qwen3_loader.cpp:163-296). */
Qwen3Weights load_qwen3_weights(const std::string& path);

/* Loads the checkpoint and runs the model over input_ids [batch, seq_len]
 * (input_shape), returning the final-norm hidden states [batch, seq_len,
 * hidden_size].  The reference's version (tensor_cpp/src/qwen3_loader.cpp:
 * 298-325) is a placeholder that returns zeros of that shape. */
Tensor test_qwen3_forward(const std::string& safetensors_path, const std::vector<long>& input_ids_data,
                          const std::vector<size_t>& input_shape);

}  // namespace qwen3
}  // namespace tensor_cpp

#endif  // SA_AMD_TENSOR_CPP_QWEN3_LOADER_H
