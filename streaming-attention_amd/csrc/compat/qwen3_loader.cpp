// The reference's load_qwen3_weights and test_qwen3_forward
// (tensor_cpp/src/qwen3_loader.cpp:163-325) over the library's safetensors
// reader: host fp32 tensors for the qwen3_ops functions.
#include "tensor_cpp/qwen3_loader.h"

#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "safetensors.h"

namespace tensor_cpp {
namespace qwen3 {

namespace {

struct Reader {
    const sa::Checkpoint& ck;

    // The tensor `name`, which must have the given shape, as a host fp32 tensor.
    Tensor load(const std::string& name, const std::vector<int64_t>& shape) const {
        if (!ck.find(name)) throw std::runtime_error("Tensor not found: " + name);
        const sa::StEntry* t = nullptr;
        if (ck.need(name, shape, &t) != SA_OK) throw std::runtime_error(sa_last_error());
        std::vector<float> v(static_cast<size_t>(t->numel()));
        ck.to_f32(*t, v.data());
        std::vector<size_t> dims(shape.begin(), shape.end());
        return Tensor(std::move(v), Shape(dims));
    }
};

// Rows of a, then of b, then of c (all [*, cols]).
Tensor concat_rows(const Tensor& a, const Tensor& b, const Tensor& c) {
    std::vector<float> v;
    v.reserve(a.size() + b.size() + c.size());
    v.insert(v.end(), a.data(), a.data() + a.size());
    v.insert(v.end(), b.data(), b.data() + b.size());
    v.insert(v.end(), c.data(), c.data() + c.size());
    const size_t rows = a.shape()[0] + b.shape()[0] + c.shape()[0];
    return Tensor(std::move(v), Shape({rows, a.shape()[1]}));
}

}  // namespace

Qwen3Weights load_qwen3_weights(const std::string& path) {
    sa::Checkpoint ck;
    if (ck.open_file(path.c_str()) != SA_OK)
        throw std::runtime_error("Failed to open safetensors file: " + path + " (" + sa_last_error() + ")");
    if (!ck.find("model.embed_tokens.weight")) throw std::runtime_error("Tensor not found: model.embed_tokens.weight");
    sa_qwen3_desc d{};
    if (sa::read_qwen3_desc(ck, &d) != SA_OK) throw std::runtime_error(sa_last_error());
    const int64_t H = d.hidden, I = d.intermediate, V = d.vocab, D = d.head_dim;
    const int64_t Nq = d.n_q_heads * D, Nk = d.n_kv_heads * D;
    const Reader r{ck};

    Qwen3Weights w;
    w.num_layers = static_cast<size_t>(d.num_layers);
    w.num_attention_heads = static_cast<size_t>(d.n_q_heads);
    w.num_key_value_heads = static_cast<size_t>(d.n_kv_heads);
    w.head_dim = static_cast<size_t>(D);
    w.hidden_size = static_cast<size_t>(H);
    w.vocab_size = static_cast<size_t>(V);
    w.embed_tokens = r.load("model.embed_tokens.weight", {V, H});
    w.norm_weight = r.load("model.norm.weight", {H});
    w.lm_head = ck.find("lm_head.weight") ? r.load("lm_head.weight", {V, H}) : w.embed_tokens;
    w.layers.resize(w.num_layers);
    for (int l = 0; l < d.num_layers; ++l) {
        auto name = [l](const char* leaf) { return sa::layer_tensor_name(l, leaf); };
        Qwen3LayerWeights& L = w.layers[l];
        L.input_layernorm_weight = r.load(name("input_layernorm.weight"), {H});
        L.post_attention_layernorm_weight = r.load(name("post_attention_layernorm.weight"), {H});
        L.q_proj = r.load(name("self_attn.q_proj.weight"), {Nq, H});
        L.k_proj = r.load(name("self_attn.k_proj.weight"), {Nk, H});
        L.v_proj = r.load(name("self_attn.v_proj.weight"), {Nk, H});
        L.q_norm_weight = r.load(name("self_attn.q_norm.weight"), {D});
        L.k_norm_weight = r.load(name("self_attn.k_norm.weight"), {D});
        L.o_proj = r.load(name("self_attn.o_proj.weight"), {H, Nq});
        L.gate_proj = r.load(name("mlp.gate_proj.weight"), {I, H});
        L.up_proj = r.load(name("mlp.up_proj.weight"), {I, H});
        L.down_proj = r.load(name("mlp.down_proj.weight"), {H, I});
        L.qkv_projs = concat_rows(L.q_proj, L.k_proj, L.v_proj);
    }
    return w;
}

Tensor test_qwen3_forward(const std::string& safetensors_path, const std::vector<long>& input_ids_data,
                          const std::vector<size_t>& input_shape) {
    if (input_shape.size() != 2 || input_shape[0] * input_shape[1] != input_ids_data.size())
        throw std::invalid_argument("input_shape must be [batch, seq_len] holding input_ids_data");
    const Qwen3Weights w = load_qwen3_weights(safetensors_path);
    const TensorL ids(input_ids_data, Shape(input_shape));
    // lm_head = I: the "logits" are the final-norm hidden states themselves.
    return qwen3_forward(ids, w.embed_tokens, w.layers, w.norm_weight, Tensor::eye(w.hidden_size), w.num_layers,
                         w.num_attention_heads, w.num_key_value_heads, w.head_dim, 1e-6f);
}

}  // namespace qwen3
}  // namespace tensor_cpp
