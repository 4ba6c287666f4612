// Test driver: the library's reference-shaped C++ API (tensor_cpp/qwen3_ops.h,
// tensor_cpp/qwen3_ops_avx.h, tensor_cpp/kv_cache.h, tensor_cpp/ops.h) driven
// exactly as oracle/ref_shim.cpp drives the reference, behind the same plain
// array arguments, so tests can put the GPU results beside the reference's
// golden vectors.  Built as tests/cpp/bin/libdrive_compat.so.
#include <cstdint>
#include <cstring>
#include <exception>
#include <stdexcept>
#include <string>
#include <vector>

#include "tensor_cpp/attention_avx.h"
#include "tensor_cpp/kv_cache.h"
#include "tensor_cpp/ops.h"
#include "tensor_cpp/qwen3_loader.h"
#include "tensor_cpp/qwen3_ops.h"
#include "tensor_cpp/qwen3_ops_avx.h"

using tensor_cpp::Shape;
using tensor_cpp::Tensor;
namespace q3 = tensor_cpp::qwen3;

namespace {

std::string g_error;

Tensor make(const float* p, std::vector<size_t> dims) {
    size_t n = 1;
    for (size_t d : dims) n *= d;
    return Tensor(std::vector<float>(p, p + n), Shape(dims));
}

int failed(const std::exception& e) {
    g_error = e.what();
    return -1;
}

// "E:" + what() with E the exception's kind: I invalid_argument, O out_of_range,
// R runtime_error (other than those), X anything else.
int failed_kind(const std::exception& e) {
    const char* k = dynamic_cast<const std::invalid_argument*>(&e) ? "I:"
                    : dynamic_cast<const std::out_of_range*>(&e)   ? "O:"
                    : dynamic_cast<const std::runtime_error*>(&e)  ? "R:"
                                                                   : "X:";
    g_error = std::string(k) + e.what();
    return -1;
}

// Layer weights from the flat arrays of drv_qwen3_forward (layout below).
std::vector<q3::Qwen3LayerWeights> layer_weights(int nl, int H, int I, int Hq, int Hkv, int D, const float* in_norm,
                                                 const float* qkv, const float* q_norm, const float* k_norm,
                                                 const float* o, const float* post_norm, const float* gate_up,
                                                 const float* down) {
    const size_t qd = (size_t)Hq * D, kd = (size_t)Hkv * D, proj = qd + 2 * kd;
    std::vector<q3::Qwen3LayerWeights> layers(nl);
    for (int l = 0; l < nl; ++l) {
        auto& w = layers[l];
        w.input_layernorm_weight = make(in_norm + (size_t)l * H, {(size_t)H});
        const float* wqkv = qkv + (size_t)l * proj * H;
        w.qkv_projs = make(wqkv, {proj, (size_t)H});
        w.q_proj = make(wqkv, {qd, (size_t)H});
        w.k_proj = make(wqkv + qd * H, {kd, (size_t)H});
        w.v_proj = make(wqkv + (qd + kd) * H, {kd, (size_t)H});
        w.q_norm_weight = make(q_norm + (size_t)l * D, {(size_t)D});
        w.k_norm_weight = make(k_norm + (size_t)l * D, {(size_t)D});
        w.o_proj = make(o + (size_t)l * H * qd, {(size_t)H, qd});
        w.post_attention_layernorm_weight = make(post_norm + (size_t)l * H, {(size_t)H});
        const float* gu = gate_up + (size_t)l * 2 * I * H;
        w.gate_proj = make(gu, {(size_t)I, (size_t)H});
        w.up_proj = make(gu + (size_t)I * H, {(size_t)I, (size_t)H});
        w.down_proj = make(down + (size_t)l * H * I, {(size_t)H, (size_t)I});
    }
    return layers;
}

}  // namespace

extern "C" {

const char* drv_last_error() { return g_error.c_str(); }

// One decoder layer with a KVCache through a prompt of prompt_len tokens and
// then n_steps single-token steps, wired so that its attention output appears
// verbatim in its output (the arguments and wiring of ref_layer_attention in
// oracle/ref_shim.cpp): hidden rows [q | k | v | 0], combined projection
// [I | 0], o_proj into the zero block, zero MLP, RMSNorm weights 1.
// streaming selects AttentionType::STREAMING with the reference's
// scale-on-output single-query kernel.  Returns 0, or -1 on an exception.
int drv_layer_attention(int Hq, int Hkv, int D, int prompt_len, int n_steps, const float* q_in, const float* k_in,
                        const float* v_in, const float* wq, const float* wk, float eps, int max_seq, int avx2,
                        int streaming, float* attn_out, float* qkv_eff) {
    const bool saved = tensor_cpp::ops::g_streaming_scale_on_output;
    try {
        tensor_cpp::ops::g_streaming_scale_on_output = streaming != 0;
        const size_t qd = (size_t)Hq * D, kd = (size_t)Hkv * D;
        const size_t proj = qd + 2 * kd;
        const size_t W = proj + qd;
        std::vector<float> qkv(proj * W, 0.0f), qp(qd * W, 0.0f), kp(kd * W, 0.0f), vp(kd * W, 0.0f);
        for (size_t r = 0; r < proj; ++r) qkv[r * W + r] = 1.0f;
        for (size_t r = 0; r < qd; ++r) qp[r * W + r] = 1.0f;
        for (size_t r = 0; r < kd; ++r) kp[r * W + qd + r] = 1.0f;
        for (size_t r = 0; r < kd; ++r) vp[r * W + qd + kd + r] = 1.0f;
        std::vector<float> op(W * qd, 0.0f);
        for (size_t c = 0; c < qd; ++c) op[(proj + c) * qd + c] = 1.0f;
        Tensor t_qkv(qkv, Shape({proj, W}));
        Tensor t_qp(qp, Shape({qd, W})), t_kp(kp, Shape({kd, W})), t_vp(vp, Shape({kd, W}));
        Tensor t_op(op, Shape({W, qd}));
        Tensor ones(std::vector<float>(W, 1.0f), Shape({W}));
        Tensor t_wq = make(wq, {(size_t)D});
        Tensor t_wk = make(wk, {(size_t)D});
        const size_t I = 8;
        Tensor gate(std::vector<float>(I * W, 0.0f), Shape({I, W}));
        Tensor up(std::vector<float>(I * W, 0.0f), Shape({I, W}));
        Tensor down(std::vector<float>(W * I, 0.0f), Shape({W, I}));

        q3::KVCache cache(1, 1, Hkv, D, max_seq);
        auto cs = q3::compute_rope_freqs(cache.max_seq_len, D, 1000000.0f);
        const auto type = streaming ? q3::AttentionType::STREAMING : q3::AttentionType::STANDARD;

        int t0 = 0;
        for (int call = 0; call <= n_steps; ++call) {
            const int S = call == 0 ? prompt_len : 1;
            std::vector<float> h((size_t)S * W, 0.0f);
            for (int s = 0; s < S; ++s) {
                const int t = t0 + s;
                std::memcpy(&h[s * W], q_in + (size_t)t * qd, qd * sizeof(float));
                std::memcpy(&h[s * W + qd], k_in + (size_t)t * kd, kd * sizeof(float));
                std::memcpy(&h[s * W + qd + kd], v_in + (size_t)t * kd, kd * sizeof(float));
            }
            Tensor hidden(h, Shape({1, (size_t)S, W}));
            Tensor normed = tensor_cpp::ops::rms_norm(hidden, &ones, eps);
            for (int s = 0; s < S; ++s)
                std::memcpy(qkv_eff + (size_t)(t0 + s) * proj, normed.data() + (size_t)s * W, proj * sizeof(float));
            Tensor out;
            if (avx2)
                out = q3::avx2::qwen3_decoder_layer_avx_with_cache(hidden, &cache, 0, Hq, Hkv, D, eps, ones, t_qp,
                                                                   t_kp, t_vp, t_op, t_wq, t_wk, ones, gate, up, down,
                                                                   cs.first, cs.second, type);
            else
                out = q3::qwen3_decoder_layer_with_cache(hidden, &cache, 0, Hq, Hkv, D, eps, ones, t_qkv, t_op, t_wq,
                                                         t_wk, ones, gate, up, down, cs.first, cs.second, type);
            for (int s = 0; s < S; ++s)
                std::memcpy(attn_out + (size_t)(t0 + s) * qd, out.data() + (size_t)s * W + proj, qd * sizeof(float));
            cache.increment_seq_len(S);
            t0 += S;
        }
        tensor_cpp::ops::g_streaming_scale_on_output = saved;
        return 0;
    } catch (const std::exception& e) {
        tensor_cpp::ops::g_streaming_scale_on_output = saved;
        return failed(e);
    }
}

// Teacher-forced forwards through qwen3_forward_with_cache (avx2:
// qwen3_forward_avx_with_cache), STANDARD attention: a P-token prompt, then
// n_steps one-token forwards; logits [n_steps + 1][B][V] at the last position
// of each (the arguments of ref_qwen3_forward in oracle/ref_shim.cpp).
// Weights, row-major fp32: embed [V][H], in_norm [nl][H],
// qkv [nl][(Hq+2Hkv)D][H], q_norm/k_norm [nl][D], o [nl][H][Hq D],
// post_norm [nl][H], gate_up [nl][2I][H], down [nl][H][I], final_norm [H],
// lm_head [V][H].
int drv_qwen3_forward(int nl, int H, int I, int V, int Hq, int Hkv, int D, float eps, int B, int P, int n_steps,
                      const int* tokens, const float* embed, const float* in_norm, const float* qkv,
                      const float* q_norm, const float* k_norm, const float* o, const float* post_norm,
                      const float* gate_up, const float* down, const float* final_norm, const float* lm_head,
                      int avx2, float* logits) {
    try {
        const auto layers = layer_weights(nl, H, I, Hq, Hkv, D, in_norm, qkv, q_norm, k_norm, o, post_norm, gate_up,
                                          down);
        Tensor t_embed = make(embed, {(size_t)V, (size_t)H});
        Tensor t_norm = make(final_norm, {(size_t)H});
        Tensor t_head = make(lm_head, {(size_t)V, (size_t)H});
        q3::KVCache cache(nl, B, Hkv, D, P + n_steps + 1);
        const int N = P + n_steps;
        int t0 = 0;
        for (int call = 0; call <= n_steps; ++call) {
            const int S = call == 0 ? P : 1;
            std::vector<long> ids((size_t)B * S);
            for (int b = 0; b < B; ++b)
                for (int s = 0; s < S; ++s) ids[(size_t)b * S + s] = tokens[(size_t)b * N + t0 + s];
            TensorL input(ids, Shape({(size_t)B, (size_t)S}));
            Tensor out = avx2 ? q3::avx2::qwen3_forward_avx_with_cache(input, &cache, t_embed, layers, t_norm, t_head,
                                                                        nl, Hq, Hkv, D, eps,
                                                                        q3::AttentionType::STANDARD)
                              : q3::qwen3_forward_with_cache(input, &cache, t_embed, layers, t_norm, t_head, nl, Hq,
                                                             Hkv, D, eps, q3::AttentionType::STANDARD);
            for (int b = 0; b < B; ++b)
                std::memcpy(logits + ((size_t)call * B + b) * V, out.data() + ((size_t)b * S + S - 1) * V,
                            (size_t)V * sizeof(float));
            t0 += S;
        }
        return 0;
    } catch (const std::exception& e) {
        return failed(e);
    }
}

// One forward without a cache (qwen3_forward, avx2: qwen3_forward_avx) over
// all N tokens of tokens [B][N]: logits [B][N][V] at every position.  Same
// weight layout as drv_qwen3_forward.
int drv_qwen3_forward_nocache(int nl, int H, int I, int V, int Hq, int Hkv, int D, float eps, int B, int N,
                              const int* tokens, const float* embed, const float* in_norm, const float* qkv,
                              const float* q_norm, const float* k_norm, const float* o, const float* post_norm,
                              const float* gate_up, const float* down, const float* final_norm, const float* lm_head,
                              int avx2, float* logits) {
    try {
        const auto layers = layer_weights(nl, H, I, Hq, Hkv, D, in_norm, qkv, q_norm, k_norm, o, post_norm, gate_up,
                                          down);
        Tensor t_embed = make(embed, {(size_t)V, (size_t)H});
        Tensor t_norm = make(final_norm, {(size_t)H});
        Tensor t_head = make(lm_head, {(size_t)V, (size_t)H});
        std::vector<long> ids((size_t)B * N);
        for (size_t i = 0; i < ids.size(); ++i) ids[i] = tokens[i];
        TensorL input(ids, Shape({(size_t)B, (size_t)N}));
        Tensor out = avx2 ? q3::avx2::qwen3_forward_avx(input, t_embed, layers, t_norm, t_head, nl, Hq, Hkv, D, eps)
                          : q3::qwen3_forward(input, t_embed, layers, t_norm, t_head, nl, Hq, Hkv, D, eps);
        std::memcpy(logits, out.data(), out.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        return failed(e);
    }
}

// load_qwen3_weights(path).  meta[7] receives num_layers, heads, kv heads,
// head_dim, hidden, vocab and the float count of the flat copy; when out is
// non-null and cap covers that count, out receives embed_tokens, norm_weight,
// lm_head, then per layer input_layernorm, post_attention_layernorm,
// qkv_projs, q_proj, k_proj, v_proj, q_norm, k_norm, o_proj, gate_proj,
// up_proj, down_proj, each row-major.  Returns 0, or -1 with the exception's
// kind and text in drv_last_error.
int drv_load_weights(const char* path, int64_t* meta, float* out, int64_t cap) {
    try {
        const q3::Qwen3Weights w = q3::load_qwen3_weights(path);
        std::vector<const Tensor*> parts = {&w.embed_tokens, &w.norm_weight, &w.lm_head};
        for (const auto& L : w.layers)
            for (const Tensor* t : {&L.input_layernorm_weight, &L.post_attention_layernorm_weight, &L.qkv_projs,
                                    &L.q_proj, &L.k_proj, &L.v_proj, &L.q_norm_weight, &L.k_norm_weight, &L.o_proj,
                                    &L.gate_proj, &L.up_proj, &L.down_proj})
                parts.push_back(t);
        int64_t total = 0;
        for (const Tensor* t : parts) total += (int64_t)t->size();
        const int64_t m[7] = {(int64_t)w.num_layers, (int64_t)w.num_attention_heads, (int64_t)w.num_key_value_heads,
                              (int64_t)w.head_dim, (int64_t)w.hidden_size, (int64_t)w.vocab_size, total};
        std::memcpy(meta, m, sizeof(m));
        if (out && cap >= total)
            for (const Tensor* t : parts) {
                std::memcpy(out, t->data(), t->size() * sizeof(float));
                out += t->size();
            }
        return 0;
    } catch (const std::exception& e) {
        return failed_kind(e);
    }
}

// test_qwen3_forward(path, tokens [B][N]) -> hidden [B][N][hidden].
int drv_test_forward(const char* path, const int* tokens, int B, int N, float* hidden, int64_t cap) {
    try {
        std::vector<long> ids((size_t)B * N);
        for (size_t i = 0; i < ids.size(); ++i) ids[i] = tokens[i];
        const Tensor h = q3::test_qwen3_forward(path, ids, {(size_t)B, (size_t)N});
        if ((int64_t)h.size() > cap) throw std::length_error("hidden buffer too small");
        std::memcpy(hidden, h.data(), h.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        return failed_kind(e);
    }
}

// ops::RotaryEmbedding(D, max_seq, theta).apply(x [B][S][H][D], seq_len).
int drv_rotary(const float* x, int B, int S, int H, int D, int max_seq, float theta, int seq_len, float* out) {
    try {
        tensor_cpp::ops::RotaryEmbedding rope((size_t)D, (size_t)max_seq, theta);
        const Tensor y = rope.apply(make(x, {(size_t)B, (size_t)S, (size_t)H, (size_t)D}), (size_t)seq_len);
        std::memcpy(out, y.data(), y.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        return failed_kind(e);
    }
}

// ops::argmax, the arguments and results of ref_argmax in oracle/ref_shim.cpp.
long drv_argmax(const float* x, const int64_t* dims, int nd, int dim, int keepdim, int64_t* idx, long cap,
                int64_t* shape_out, int* out_nd) {
    try {
        const TensorL r = tensor_cpp::ops::argmax(make(x, std::vector<size_t>(dims, dims + nd)), dim, keepdim != 0);
        const long count = (long)r.size();
        for (long i = 0; i < count && i < cap; ++i) idx[i] = r[i];
        *out_nd = (int)r.shape().ndim();
        for (int i = 0; i < *out_nd && i < 8; ++i) shape_out[i] = (int64_t)r.shape()[i];
        return count;
    } catch (const std::exception& e) {
        return failed_kind(e);
    }
}

// ops::cross_attention(q [B][Hq][Sq][D], k/v [B][Hkv][Sk][D], mask, scale);
// mask [Sq][Sk] or null.
int drv_cross_attention(const float* q, const float* k, const float* v, int B, int Hq, int Hkv, int Sq, int Sk, int D,
                        float scale, const float* mask, float* out) {
    try {
        const Tensor tq = make(q, {(size_t)B, (size_t)Hq, (size_t)Sq, (size_t)D});
        const Tensor tk = make(k, {(size_t)B, (size_t)Hkv, (size_t)Sk, (size_t)D});
        const Tensor tv = make(v, {(size_t)B, (size_t)Hkv, (size_t)Sk, (size_t)D});
        Tensor tm;
        if (mask) tm = make(mask, {(size_t)Sq, (size_t)Sk});
        const Tensor y = tensor_cpp::ops::cross_attention(tq, tk, tv, mask ? &tm : nullptr, scale);
        std::memcpy(out, y.data(), y.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        return failed_kind(e);
    }
}

// ops::avx2::self_attention_avx2(q [B][Hq][Sq][D], k/v [B][Hkv][Sk][D], mask,
// scale); mask [1][1][mrows][Sk] (mrows 1 or Sq) or null.
int drv_self_attention_avx2(const float* q, const float* k, const float* v, int B, int Hq, int Hkv, int Sq, int Sk,
                            int D, float scale, const float* mask, int mrows, float* out) {
    try {
        const Tensor tq = make(q, {(size_t)B, (size_t)Hq, (size_t)Sq, (size_t)D});
        const Tensor tk = make(k, {(size_t)B, (size_t)Hkv, (size_t)Sk, (size_t)D});
        const Tensor tv = make(v, {(size_t)B, (size_t)Hkv, (size_t)Sk, (size_t)D});
        Tensor tm;
        if (mask) tm = make(mask, {1, 1, (size_t)mrows, (size_t)Sk});
        const Tensor y = tensor_cpp::ops::avx2::self_attention_avx2(tq, tk, tv, mask ? &tm : nullptr, scale);
        std::memcpy(out, y.data(), y.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        return failed_kind(e);
    }
}

// ops::avx2::linear_avx2(x [M][K], w [N][K], bias [N] or null).
int drv_linear_avx2(const float* x, const float* w, const float* bias, int M, int K, int N, float* out) {
    try {
        const Tensor tx = make(x, {(size_t)M, (size_t)K});
        const Tensor tw = make(w, {(size_t)N, (size_t)K});
        Tensor tb;
        if (bias) tb = make(bias, {(size_t)N});
        const Tensor y = tensor_cpp::ops::avx2::linear_avx2(tx, tw, bias ? &tb : nullptr);
        std::memcpy(out, y.data(), y.size() * sizeof(float));
        return 0;
    } catch (const std::exception& e) {
        return failed_kind(e);
    }
}

}  // extern "C"
