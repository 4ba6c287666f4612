// ref_shim.cpp - extern "C" entry points into the reference implementation.
//
// TEST INFRASTRUCTURE ONLY.  Compiled together with the reference's own
// sources (attention/src, tensor_cpp/src) by oracle/Makefile into
// oracle/_ref/libsa_ref.so; used by tests/golden/make_golden.py to write
// golden vectors, by tests to pin the oracle, and by bench.py as the timed
// CPU baseline.  Nothing here re-implements the reference: each function only
// marshals plain arrays into the reference's API and back.
#include <omp.h>

#include <chrono>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "attention.h"
#include "tensor_cpp/attention_avx.h"
#include "tensor_cpp/kv_cache.h"
#include "tensor_cpp/ops.h"
#include "tensor_cpp/qwen3_ops.h"
#include "tensor_cpp/qwen3_loader.h"
#include "tensor_cpp/qwen3_ops_avx.h"

using tensor_cpp::Shape;
using tensor_cpp::Tensor;
namespace q3 = tensor_cpp::qwen3;

namespace {
Tensor make(const float* p, std::vector<size_t> dims) {
    size_t n = 1;
    for (size_t d : dims) n *= d;
    return Tensor(std::vector<float>(p, p + n), Shape(dims));
}
void put(const Tensor& t, float* out) { std::memcpy(out, t.data(), t.size() * sizeof(float)); }
void put(const std::vector<float>& v, float* out) { std::memcpy(out, v.data(), v.size() * sizeof(float)); }

// Timing fill: values uniform in [-amp, amp) from a 64-bit LCG (the values
// only need to be finite and non-denormal; no result is checked).
Tensor filled(std::vector<size_t> dims, float amp, uint64_t& state) {
    size_t n = 1;
    for (size_t d : dims) n *= d;
    std::vector<float> v(n);
    for (auto& x : v) {
        state = state * 6364136223846793005ULL + 1442695040888963407ULL;
        x = amp * (2.0f * (float)(state >> 40) / 16777216.0f - 1.0f);
    }
    return Tensor(std::move(v), Shape(dims));
}

// Teacher-forced forwards through qwen3_forward_with_cache, or with avx2
// qwen3_forward_avx_with_cache (STANDARD attention, dense KVCache): a P-token
// prompt, then n_steps one-token forwards; logits [n_steps + 1][B][V] at the
// last position of each.
void run_forward(const std::vector<q3::Qwen3LayerWeights>& layers, const Tensor& embed, const Tensor& norm,
                 const Tensor& head, int nl, int Hq, int Hkv, int D, float eps, int B, int P, int n_steps,
                 const int* tokens, int V, int avx2, float* logits) {
    q3::KVCache cache(nl, B, Hkv, D, P + n_steps + 1);
    const int N = P + n_steps;
    int t0 = 0;
    for (int call = 0; call <= n_steps; ++call) {
        const int S = call == 0 ? P : 1;
        std::vector<long> ids((size_t)B * S);
        for (int b = 0; b < B; ++b)
            for (int s = 0; s < S; ++s) ids[(size_t)b * S + s] = tokens[(size_t)b * N + t0 + s];
        TensorL input(ids, Shape({(size_t)B, (size_t)S}));
        Tensor out = avx2 ? tensor_cpp::qwen3::avx2::qwen3_forward_avx_with_cache(
                                input, &cache, embed, layers, norm, head, nl, Hq, Hkv, D, eps,
                                q3::AttentionType::STANDARD)
                          : q3::qwen3_forward_with_cache(input, &cache, embed, layers, norm, head, nl, Hq, Hkv, D,
                                                         eps, q3::AttentionType::STANDARD);
        for (int b = 0; b < B; ++b)
            std::memcpy(logits + ((size_t)call * B + b) * V, out.data() + ((size_t)b * S + S - 1) * V,
                        (size_t)V * sizeof(float));
        t0 += S;
    }
}
}  // namespace

extern "C" {

void ref_streaming_serial(const float* Q, const float* K, const float* V, int T, int d, int block,
                          float* O) {
    put(streaming_attention_serial(Q, K, V, T, d, block), O);
}

void ref_naive_serial(const float* Q, const float* K, const float* V, int T, int d, float* O) {
    put(naive_attention_serial(Q, K, V, T, d), O);
}

void ref_streaming_omp(const float* Q, const float* K, const float* V, int T, int d, int block,
                       int nthreads, float* O) {
    put(streaming_attention_omp(Q, K, V, T, d, block, nthreads), O);
}

void ref_naive_omp(const float* Q, const float* K, const float* V, int T, int d, int nthreads,
                   float* O) {
    put(naive_attention_omp(Q, K, V, T, d, nthreads), O);
}

void ref_set_threads(int n) { omp_set_num_threads(n); }

float ref_l2_error(const float* a, const float* b, int n) { return compute_l2_error(a, b, n); }
float ref_max_error(const float* a, const float* b, int n) { return compute_max_error(a, b, n); }

// compute_rope_freqs(seq_len, head_dim, theta) -> cos, sin [seq_len][D/2]
void ref_rope_freqs(int seq_len, int D, float theta, float* cos_out, float* sin_out) {
    auto cs = q3::compute_rope_freqs(seq_len, D, theta);
    put(cs.first, cos_out);
    put(cs.second, sin_out);
}

// apply_rotary_pos_emb on q [B][Hq][S][D], k [B][Hkv][S][D] with cos/sin [S][D/2]
void ref_apply_rope(const float* q, const float* k, int B, int Hq, int Hkv, int S, int D,
                    const float* cos_t, const float* sin_t, float* q_out, float* k_out) {
    Tensor tq = make(q, {(size_t)B, (size_t)Hq, (size_t)S, (size_t)D});
    Tensor tk = make(k, {(size_t)B, (size_t)Hkv, (size_t)S, (size_t)D});
    Tensor tc = make(cos_t, {(size_t)S, (size_t)D / 2});
    Tensor ts = make(sin_t, {(size_t)S, (size_t)D / 2});
    auto r = q3::apply_rotary_pos_emb(tq, tk, tc, ts);
    put(r.first, q_out);
    put(r.second, k_out);
}

void ref_repeat_kv(const float* x, int B, int Hkv, int S, int D, int n_rep, float* out) {
    put(q3::repeat_kv(make(x, {(size_t)B, (size_t)Hkv, (size_t)S, (size_t)D}), n_rep), out);
}

// ops::self_attention on [B][H][Sq][D] x [B][H][Sk][D]; causal != 0 adds the
// [Sk][Sk] causal mask (prefill), otherwise an all-zero [1,1,1,Sk] mask (decode).
void ref_self_attention(const float* q, const float* k, const float* v, int B, int H, int Sq, int Sk,
                        int D, int causal, float scale, float* out) {
    Tensor tq = make(q, {(size_t)B, (size_t)H, (size_t)Sq, (size_t)D});
    Tensor tk = make(k, {(size_t)B, (size_t)H, (size_t)Sk, (size_t)D});
    Tensor tv = make(v, {(size_t)B, (size_t)H, (size_t)Sk, (size_t)D});
    Tensor mask;
    if (causal) {
        mask = q3::create_causal_mask(Sk).view({1, 1, (size_t)Sk, (size_t)Sk});
    } else {
        mask = Tensor(std::vector<float>((size_t)Sk, 0.0f), Shape({1, 1, 1, (size_t)Sk}));
    }
    put(tensor_cpp::ops::self_attention(tq, tk, tv, &mask, scale), out);
}

// nthreads > 0 sets the OpenMP thread count for the call (restored afterwards).
void ref_self_attention_streaming(const float* q, const float* k, const float* v, int B, int H, int L,
                                  int D, float scale, int block, int nthreads, float* out) {
    const int saved = omp_get_max_threads();
    if (nthreads > 0) omp_set_num_threads(nthreads);
    Tensor tq = make(q, {(size_t)B, (size_t)H, 1, (size_t)D});
    Tensor tk = make(k, {(size_t)B, (size_t)H, (size_t)L, (size_t)D});
    Tensor tv = make(v, {(size_t)B, (size_t)H, (size_t)L, (size_t)D});
    put(tensor_cpp::ops::self_attention_streaming(tq, tk, tv, scale, block), out);
    omp_set_num_threads(saved);
}

// variant: 0 = self_attention_streaming_blockwise, 1 = _avx2, 2 = _avx2_cache_optimized
void ref_blockwise(const float* q, const float* k, const float* v, int B, int H, int L, int D,
                   float scale, int q_block, int kv_block, int variant, float* out) {
    Tensor tq = make(q, {(size_t)B, (size_t)H, (size_t)L, (size_t)D});
    Tensor tk = make(k, {(size_t)B, (size_t)H, (size_t)L, (size_t)D});
    Tensor tv = make(v, {(size_t)B, (size_t)H, (size_t)L, (size_t)D});
    namespace ops = tensor_cpp::ops;
    if (variant == 1)
        put(ops::self_attention_streaming_blockwise_avx2(tq, tk, tv, scale, q_block, kv_block), out);
    else if (variant == 2)
        put(ops::self_attention_streaming_blockwise_avx2_cache_optimized(tq, tk, tv, scale, q_block,
                                                                          kv_block), out);
    else
        put(ops::self_attention_streaming_blockwise(tq, tk, tv, scale, q_block, kv_block), out);
}

// Drive one reference decoder layer with a KVCache through a prompt of
// prompt_len tokens and then n_steps single-token steps, and recover the
// attention output of every call.
//
// The layer is wired so that its attention output appears verbatim in its
// output: hidden rows are [q | k | v | 0] (width W = 2*Hq*D + 2*Hkv*D), the
// combined QKV projection is [I | 0], o_proj writes into the zero block, and
// the MLP weights are zero.  The input RMSNorm (weight 1) rescales each row,
// so the q/k/v the attention saw are x / sqrt(mean(x^2) + eps); they are
// returned in qkv_eff so callers can feed the same values elsewhere.
//
// q_in [N][Hq*D], k_in/v_in [N][Hkv*D] with N = prompt_len + n_steps;
// attn_out [N][Hq*D]; qkv_eff [N][(Hq+2Hkv)*D].
// avx2 selects qwen3_decoder_layer_avx_with_cache; streaming selects
// AttentionType::STREAMING.  Returns 0 on success, -1 on a reference exception.
int ref_layer_attention(int Hq, int Hkv, int D, int prompt_len, int n_steps, const float* q_in,
                        const float* k_in, const float* v_in, const float* wq, const float* wk,
                        float eps, int max_seq, int avx2, int streaming, float* attn_out,
                        float* qkv_eff) {
    try {
        const size_t qd = (size_t)Hq * D, kd = (size_t)Hkv * D;
        const size_t proj = qd + 2 * kd;
        const size_t W = proj + qd;
        // Combined projection [I | 0] : [proj][W]; separate q/k/v for the AVX2 path.
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
                std::memcpy(qkv_eff + (size_t)(t0 + s) * proj, normed.data() + (size_t)s * W,
                            proj * sizeof(float));
            Tensor out;
            if (avx2)
                out = tensor_cpp::qwen3::avx2::qwen3_decoder_layer_avx_with_cache(
                    hidden, &cache, 0, Hq, Hkv, D, eps, ones, t_qp, t_kp, t_vp, t_op, t_wq, t_wk, ones,
                    gate, up, down, cs.first, cs.second, type);
            else
                out = q3::qwen3_decoder_layer_with_cache(hidden, &cache, 0, Hq, Hkv, D, eps, ones,
                                                         t_qkv, t_op, t_wq, t_wk, ones, gate, up, down,
                                                         cs.first, cs.second, type);
            // Residual of the attention block is hidden itself: zero on the output columns.
            for (int s = 0; s < S; ++s)
                std::memcpy(attn_out + (size_t)(t0 + s) * qd, out.data() + (size_t)s * W + proj,
                            qd * sizeof(float));
            cache.increment_seq_len(S);
            t0 += S;
        }
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Timing only (the CPU baseline of the decode benchmarks): n_steps one-token
// forwards of one reference decoder layer,
// qwen3_decoder_layer_avx_with_cache (tensor_cpp/src/qwen3_ops_avx.cpp:469-754)
// with AttentionType::STREAMING, for B sequences whose KVCache already holds
// L0 tokens (written with KVCache::update, then increment_seq_len(L0)).
// Hidden size H, MLP width I; weights and inputs are LCG fill.  Each call
// does everything the reference does per layer and token: RMSNorm, q/k/v
// projections, q/k RMSNorm, RoPE, the cache read, concat and update,
// repeat_kv, self_attention_streaming, o_proj and the MLP.  The RoPE table is
// built once beforehand (the reference rebuilds it once per forward, outside
// the layer).  secs[i] = wall seconds of call i.  Returns 0, or -1 on a
// reference exception.
int ref_time_decode_layer(int H, int I, int Hq, int Hkv, int D, int B, int L0, int n_steps,
                          int nthreads, double* secs) {
    try {
        const int saved = omp_get_max_threads();
        if (nthreads > 0) omp_set_num_threads(nthreads);
        uint64_t st = 0x5eed0001ULL;
        const size_t qd = (size_t)Hq * D, kd = (size_t)Hkv * D;
        Tensor ones_h(std::vector<float>((size_t)H, 1.0f), Shape({(size_t)H}));
        Tensor ones_d(std::vector<float>((size_t)D, 1.0f), Shape({(size_t)D}));
        Tensor qp = filled({qd, (size_t)H}, 0.02f, st), kp = filled({kd, (size_t)H}, 0.02f, st);
        Tensor vp = filled({kd, (size_t)H}, 0.02f, st), op = filled({(size_t)H, qd}, 0.02f, st);
        Tensor gate = filled({(size_t)I, (size_t)H}, 0.02f, st), up = filled({(size_t)I, (size_t)H}, 0.02f, st);
        Tensor down = filled({(size_t)H, (size_t)I}, 0.02f, st);
        q3::KVCache cache(1, B, Hkv, D, L0 + n_steps + 1);
        if (L0 > 0) {
            cache.update(0, filled({(size_t)B, (size_t)Hkv, (size_t)L0, (size_t)D}, 1.0f, st),
                         filled({(size_t)B, (size_t)Hkv, (size_t)L0, (size_t)D}, 1.0f, st));
            cache.increment_seq_len(L0);
        }
        auto cs = q3::compute_rope_freqs(cache.max_seq_len, D, 1000000.0f);
        for (int i = 0; i < n_steps; ++i) {
            Tensor hidden = filled({(size_t)B, 1, (size_t)H}, 1.0f, st);
            const auto t0 = std::chrono::steady_clock::now();
            Tensor out = tensor_cpp::qwen3::avx2::qwen3_decoder_layer_avx_with_cache(
                hidden, &cache, 0, Hq, Hkv, D, 1e-6f, ones_h, qp, kp, vp, op, ones_d, ones_d, ones_h,
                gate, up, down, cs.first, cs.second, q3::AttentionType::STREAMING);
            const auto t1 = std::chrono::steady_clock::now();
            secs[i] = std::chrono::duration<double>(t1 - t0).count();
            cache.increment_seq_len(1);
        }
        omp_set_num_threads(saved);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Whole-model forward through the reference (qwen3_forward_with_cache,
// tensor_cpp/src/qwen3_ops.cpp:936-1014) with its dense KVCache and STANDARD
// attention: a prompt of P tokens per sequence, then n_steps one-token
// forwards fed the given tokens (teacher forcing).  tokens [B][P + n_steps];
// logits [n_steps + 1][B][V]: the last position of each forward.  avx2
// selects qwen3_forward_avx_with_cache (tensor_cpp/src/qwen3_ops_avx.cpp:760-843),
// which reads the layers' q_proj/k_proj/v_proj (filled here from qkv).
// Weights, all row-major fp32: embed [V][H], in_norm [nl][H],
// qkv [nl][(Hq+2Hkv)D][H], q_norm/k_norm [nl][D], o [nl][H][Hq D],
// post_norm [nl][H], gate_up [nl][2I][H] (gate rows then up rows),
// down [nl][H][I], final_norm [H], lm_head [V][H].
int ref_qwen3_forward(int nl, int H, int I, int V, int Hq, int Hkv, int D, float eps, int B, int P,
                      int n_steps, const int* tokens, const float* embed, const float* in_norm,
                      const float* qkv, const float* q_norm, const float* k_norm, const float* o,
                      const float* post_norm, const float* gate_up, const float* down,
                      const float* final_norm, const float* lm_head, int avx2, float* logits) {
    try {
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
        Tensor t_embed = make(embed, {(size_t)V, (size_t)H});
        Tensor t_norm = make(final_norm, {(size_t)H});
        Tensor t_head = make(lm_head, {(size_t)V, (size_t)H});
        run_forward(layers, t_embed, t_norm, t_head, nl, Hq, Hkv, D, eps, B, P, n_steps, tokens, V, avx2, logits);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// The same forwards with the weights read by the reference's own loader,
// load_qwen3_weights (tensor_cpp/src/qwen3_loader.cpp:188-296), from a
// safetensors file.  That loader assumes 28 layers, 16/8 heads and head_dim
// 128 and takes hidden and vocab from the embedding.  Returns -1 on a
// reference exception (for example a missing tensor).
int ref_qwen3_forward_file(const char* path, float eps, int B, int P, int n_steps, const int* tokens,
                           float* logits) {
    try {
        q3::Qwen3Weights w = q3::load_qwen3_weights(path);
        run_forward(w.layers, w.embed_tokens, w.norm_weight, w.lm_head, (int)w.num_layers,
                    (int)w.num_attention_heads, (int)w.num_key_value_heads, (int)w.head_dim, eps, B, P, n_steps,
                    tokens, (int)w.vocab_size, 0, logits);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// load_qwen3_weights (tensor_cpp/src/qwen3_loader.cpp:163-296) itself:
// meta[7] = num_layers, heads, kv heads, head_dim, hidden, vocab and the
// float count of the flat copy; with out non-null and cap large enough, out
// receives embed_tokens, norm_weight, lm_head, then per layer
// input_layernorm, post_attention_layernorm, qkv_projs, q_proj, k_proj,
// v_proj, q_norm, k_norm, o_proj, gate_proj, up_proj, down_proj.  Returns -1
// on a reference exception.
int ref_load_weights(const char* path, int64_t* meta, float* out, int64_t cap) {
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
    } catch (const std::exception&) {
        return -1;
    }
}

// ops::RotaryEmbedding(D, max_seq, theta).apply(x [B][S][H][D], seq_len)
// (tensor_cpp/src/ops.cpp:424-487).  Returns -1 on a reference exception.
int ref_rotary(const float* x, int B, int S, int H, int D, int max_seq, float theta, int seq_len, float* out) {
    try {
        tensor_cpp::ops::RotaryEmbedding rope((size_t)D, (size_t)max_seq, theta);
        Tensor in(std::vector<float>(x, x + (size_t)B * S * H * D), Shape({(size_t)B, (size_t)S, (size_t)H, (size_t)D}));
        put(rope.apply(in, (size_t)seq_len), out);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// ops::argmax(x of shape dims[nd], dim, keepdim) (tensor_cpp/src/ops.cpp:213-272):
// idx receives the indices (up to cap), shape_out[8] the result's dims, *out_nd
// their count.  Returns the index count, or -1 on a reference exception.
long ref_argmax(const float* x, const int64_t* dims, int nd, int dim, int keepdim, int64_t* idx, long cap,
                int64_t* shape_out, int* out_nd) {
    try {
        std::vector<size_t> d(dims, dims + nd);
        size_t n = 1;
        for (size_t v : d) n *= v;
        Tensor in(std::vector<float>(x, x + n), Shape(d));
        TensorL r = tensor_cpp::ops::argmax(in, dim, keepdim != 0);
        const long count = (long)r.size();
        for (long i = 0; i < count && i < cap; ++i) idx[i] = r[i];
        *out_nd = (int)r.shape().ndim();
        for (int i = 0; i < *out_nd && i < 8; ++i) shape_out[i] = (int64_t)r.shape()[i];
        return count;
    } catch (const std::exception&) {
        return -1;
    }
}

// ops::cross_attention(q [B][H][Sq][D], k/v [B][H][Sk][D], mask = nullptr,
// scale) (tensor_cpp/src/ops.cpp:647-738).
void ref_cross_attention(const float* q, const float* k, const float* v, int B, int H, int Sq, int Sk, int D,
                         float scale, float* out) {
    const Shape qs({(size_t)B, (size_t)H, (size_t)Sq, (size_t)D}), ks({(size_t)B, (size_t)H, (size_t)Sk, (size_t)D});
    Tensor tq(std::vector<float>(q, q + qs.total()), qs);
    Tensor tk(std::vector<float>(k, k + ks.total()), ks);
    Tensor tv(std::vector<float>(v, v + ks.total()), ks);
    put(tensor_cpp::ops::cross_attention(tq, tk, tv, nullptr, scale), out);
}

// ops::avx2::self_attention_avx2(q [B][H][Sq][D], k/v [B][H][Sk][D], mask
// [1][1][mrows][Sk] or null, scale) (tensor_cpp/src/attention_avx.cpp:22-158).
void ref_self_attention_avx2(const float* q, const float* k, const float* v, int B, int H, int Sq, int Sk, int D,
                             float scale, const float* mask, int mrows, float* out) {
    const Shape qs({(size_t)B, (size_t)H, (size_t)Sq, (size_t)D}), ks({(size_t)B, (size_t)H, (size_t)Sk, (size_t)D});
    Tensor tq(std::vector<float>(q, q + qs.total()), qs);
    Tensor tk(std::vector<float>(k, k + ks.total()), ks);
    Tensor tv(std::vector<float>(v, v + ks.total()), ks);
    Tensor tm;
    if (mask) {
        const Shape ms({1, 1, (size_t)mrows, (size_t)Sk});
        tm = Tensor(std::vector<float>(mask, mask + ms.total()), ms);
    }
    put(tensor_cpp::ops::avx2::self_attention_avx2(tq, tk, tv, mask ? &tm : nullptr, scale), out);
}

}  // extern "C"
