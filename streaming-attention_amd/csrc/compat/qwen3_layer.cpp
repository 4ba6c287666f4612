// The Qwen3 decoder layer and forward of the API mirror on the GPU
// (reference tensor_cpp/src/qwen3_ops.cpp:70-104, :265-1014 and
// tensor_cpp/src/qwen3_ops_avx.cpp:25-843).
//
// One engine serves every variant.  A layer call uploads the caller's host
// weights and hidden state, then runs on the device: RMSNorm, the q/k/v
// projections (fp32 MFMA), per-head RMSNorm + RoPE of q and k, the K/V append
// to the cache, causal prefill or paged decode attention, o_proj, the
// residual, RMSNorm, the SwiGLU MLP and the second residual.  The forward
// keeps the hidden state on the device from the embedding rows to the logits.
// Everything is fp32, as the reference computes it.
#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

#include "device.h"
#include "tensor_cpp/qwen3_ops.h"
#include "tensor_cpp/qwen3_ops_avx.h"

namespace tensor_cpp {
namespace qwen3 {

namespace {

using sa_compat::check;
using sa_compat::DevBuf;
using sa_compat::to_device;
using sa_compat::to_host;

constexpr float kRopeTheta = 1000000.0f;   // the forwards' RoPE base (reference qwen3_ops.cpp:958)
constexpr float kQkNormEps = 1e-6f;        // the q/k RMSNorm's eps, fixed in the reference (qwen3_ops.cpp:716)

// cos/sin rows p0 .. p0 + n - 1 of the RoPE table, each [head_dim / 2], with
// exactly compute_rope_freqs' arithmetic (reference qwen3_ops.cpp:70-104).
void rope_rows(size_t p0, size_t n, size_t head_dim, float theta, float* cos_out, float* sin_out) {
    if (head_dim % 2 != 0) throw std::invalid_argument("head_dim must be even for RoPE");
    const size_t half = head_dim / 2;
    std::vector<float> inv(half);
    for (size_t i = 0; i < half; ++i)
        inv[i] = 1.0f / std::pow(theta, static_cast<float>(i) / static_cast<float>(head_dim));
    for (size_t r = 0; r < n; ++r)
        for (size_t i = 0; i < half; ++i) {
            const float a = static_cast<float>(p0 + r) * inv[i];
            cos_out[r * half + i] = std::cos(a);
            sin_out[r * half + i] = std::sin(a);
        }
}

struct Geometry {
    size_t B = 0, S = 0, H = 0, Hq = 0, Hkv = 0, D = 0;
    size_t M() const { return B * S; }
    size_t qd() const { return Hq * D; }
    size_t kd() const { return Hkv * D; }
};

// What separates the avx2 twins and the attention types.
struct Variant {
    bool avx2 = false;   // q/k RMSNorm x / (sqrt(mean(x^2)) + eps)
    AttentionType type = AttentionType::STANDARD;
};

// A layer's host weights: pointers into the caller's tensors.  Null entries
// are parts a call does not use.
struct HostWeights {
    const float* in_norm = nullptr;
    const float* q = nullptr;
    const float* k = nullptr;
    const float* v = nullptr;
    const float* o = nullptr;
    const float* q_norm = nullptr;
    const float* k_norm = nullptr;
    const float* post_norm = nullptr;
    const float* gate = nullptr;
    const float* up = nullptr;
    const float* down = nullptr;
    size_t I = 0;   // MLP width
};

struct DevWeights {
    float *in_norm, *q, *k, *v, *o, *q_norm, *k_norm, *post_norm, *gate, *up, *down;
};

// Device buffers of one thread's layer calls, grown on demand and reused.
struct Buffers {
    DevBuf weights, x, t, q, k, v, attn, h, mlp, g, u, rope, pos, ws;
};
Buffers& buffers() {
    thread_local Buffers b;
    return b;
}

[[noreturn]] void bad(const std::string& what) { throw std::invalid_argument(what); }

int as_int(size_t v, const char* what) {
    if (v > 0x7fffffffu) bad(std::string(what) + " exceeds the kernels' int range");
    return static_cast<int>(v);
}

void expect_matrix(const Tensor& t, size_t rows, size_t cols, const char* name) {
    if (t.ndim() != 2 || t.shape()[0] != rows || t.shape()[1] != cols)
        bad(std::string(name) + " must be [" + std::to_string(rows) + ", " + std::to_string(cols) + "]");
}

void expect_vector(const Tensor& t, size_t n, const char* name) {
    if (t.size() != n) bad(std::string(name) + " must have " + std::to_string(n) + " entries");
}

// Head counts and size the GPU kernels take (fp32 causal prefill: head_dim
// 16, 32, 64 or 128).
void check_heads(size_t Hq, size_t Hkv, size_t D) {
    if (Hq == 0 || Hkv == 0 || Hq % Hkv) bad("num_attention_heads must be a multiple of num_key_value_heads");
    if (D != 16 && D != 32 && D != 64 && D != 128)
        bad("head_dim must be 16, 32, 64 or 128 on the GPU (got " + std::to_string(D) + ")");
}

Geometry geometry(const Tensor& hidden, size_t Hq, size_t Hkv, size_t D) {
    if (hidden.ndim() != 3) bad("hidden_states must be [batch, seq_len, hidden_size]");
    check_heads(Hq, Hkv, D);
    return Geometry{hidden.shape()[0], hidden.shape()[1], hidden.shape()[2], Hq, Hkv, D};
}

// Attention weights: combined qkv_projs (q, k, v rows) or separate q/k/v.
void attention_weights(const Geometry& g, const Tensor* qkv, const Tensor* q, const Tensor* k, const Tensor* v,
                       const Tensor& o, const Tensor& q_norm, const Tensor& k_norm, HostWeights* w) {
    if (qkv) {
        expect_matrix(*qkv, g.qd() + 2 * g.kd(), g.H, "qkv_projs");
        w->q = qkv->data();
        w->k = w->q + g.qd() * g.H;
        w->v = w->k + g.kd() * g.H;
    } else {
        expect_matrix(*q, g.qd(), g.H, "q_proj");
        expect_matrix(*k, g.kd(), g.H, "k_proj");
        expect_matrix(*v, g.kd(), g.H, "v_proj");
        w->q = q->data();
        w->k = k->data();
        w->v = v->data();
    }
    expect_matrix(o, g.H, g.qd(), "o_proj");
    expect_vector(q_norm, g.D, "q_norm_weight");
    expect_vector(k_norm, g.D, "k_norm_weight");
    w->o = o.data();
    w->q_norm = q_norm.data();
    w->k_norm = k_norm.data();
}

void mlp_weights(const Geometry& g, const Tensor& gate, const Tensor& up, const Tensor& down, HostWeights* w) {
    if (gate.ndim() != 2) bad("gate_proj must be [intermediate_size, hidden_size]");
    const size_t I = gate.shape()[0];
    expect_matrix(gate, I, g.H, "gate_proj");
    expect_matrix(up, I, g.H, "up_proj");
    expect_matrix(down, g.H, I, "down_proj");
    w->gate = gate.data();
    w->up = up.data();
    w->down = down.data();
    w->I = I;
}

// Checks that the cache can take this call (before anything is written).
void check_cache(const Geometry& g, const KVCache* c, size_t last_layer) {
    if (!c) return;
    if (last_layer >= c->num_layers) throw std::out_of_range("Layer index out of range");
    if (g.B != c->batch_size || g.Hkv != c->num_kv_heads || g.D != c->head_dim)
        bad("KV cache shape does not match the layer");
    if (c->current_seq_len + g.S > c->max_seq_len) throw std::runtime_error("KV cache full, cannot append more tokens");
    if (c->current_seq_len > 0 && g.S != 1) bad("with a non-empty cache one token is decoded per call");
}

// Uploads the non-null host weights into one packed device buffer.
DevWeights upload(const Geometry& g, const HostWeights& hw) {
    struct Part {
        const float* src;
        size_t n;
        float** dst;
    };
    DevWeights w{};
    const size_t H = g.H, qd = g.qd(), kd = g.kd(), I = hw.I;
    Part parts[] = {{hw.in_norm, H, &w.in_norm},    {hw.q, qd * H, &w.q},          {hw.k, kd * H, &w.k},
                    {hw.v, kd * H, &w.v},           {hw.o, H * qd, &w.o},          {hw.q_norm, g.D, &w.q_norm},
                    {hw.k_norm, g.D, &w.k_norm},    {hw.post_norm, H, &w.post_norm}, {hw.gate, I * H, &w.gate},
                    {hw.up, I * H, &w.up},          {hw.down, H * I, &w.down}};
    auto padded = [](size_t n) { return (n + 63) / 64 * 64; };   // 256-byte aligned parts
    size_t total = 0;
    for (const Part& p : parts)
        if (p.src) total += padded(p.n);
    float* base = buffers().weights.as<float>(total);
    size_t off = 0;
    for (const Part& p : parts) {
        if (!p.src) continue;
        *p.dst = base + off;
        to_device(*p.dst, p.src, p.n * sizeof(float));
        off += padded(p.n);
    }
    return w;
}

// The attention of one call on device buffers.  q [M][Hq D], k and v
// [M][Hkv D] are the projection outputs, token-major.  q and k are normalised
// and rotated in place with rope rows 0 .. S-1 (positions pos0 .. pos0+S-1),
// K and V are appended to the cache when there is one, and attn receives the
// attention, token-major [B][S][Hq][D] or, with head_major, [B][Hq][S][D].
// qk_eps: the eps of the q/k RMSNorm.
void attention_dev(const Geometry& g, const Variant& var, const float* q_norm, const float* k_norm, float qk_eps,
                   const float* rope_cos, const float* rope_sin, KVCache* cache, size_t layer, float* q, float* k,
                   const float* v, bool head_major, float* attn) {
    Buffers& b = buffers();
    const size_t M = g.M();
    const int S = as_int(g.S, "seq_len"), D = as_int(g.D, "head_dim");
    std::vector<int32_t> pos(M * (g.Hq + g.Hkv));
    for (size_t r = 0; r < M * g.Hq; ++r) pos[r] = static_cast<int32_t>((r / g.Hq) % g.S);
    for (size_t r = 0; r < M * g.Hkv; ++r) pos[M * g.Hq + r] = static_cast<int32_t>((r / g.Hkv) % g.S);
    int32_t* dpos = b.pos.as<int32_t>(pos.size());
    to_device(dpos, pos.data(), pos.size() * sizeof(int32_t));
    const sa_norm_mode mode = var.avx2 ? SA_NORM_EPS_OUTSIDE : SA_NORM_EPS_INSIDE;
    check(sa_qk_norm_rope_ex(q, as_int(M * g.Hq, "query rows"), D, dpos, q_norm, qk_eps, mode, rope_cos, rope_sin,
                             S, q, nullptr),
          "q norm + RoPE");
    check(sa_qk_norm_rope_ex(k, as_int(M * g.Hkv, "key rows"), D, dpos + M * g.Hq, k_norm, qk_eps, mode, rope_cos,
                             rope_sin, S, k, nullptr),
          "k norm + RoPE");
    const size_t pos0 = cache ? cache->current_seq_len : 0;
    if (cache)
        check(sa_qknorm_rope_append(cache->handle(), static_cast<int>(layer), nullptr, k, v, static_cast<int>(g.B), S,
                                    nullptr, static_cast<int>(g.Hq), nullptr, nullptr, 0.0f, nullptr, nullptr, 0,
                                    nullptr, nullptr),
              "KV cache append");

    const float scale = 1.0f / std::sqrt(static_cast<float>(g.D));
    // The reference's single-query streaming kernel computes softmax(q k^T) v
    // and multiplies by scale afterwards (ops::g_streaming_scale_on_output).
    const bool scale_out = var.type == AttentionType::STREAMING && g.S == 1 && ops::g_streaming_scale_on_output;
    const int B = static_cast<int>(g.B), Hq = static_cast<int>(g.Hq), Hkv = static_cast<int>(g.Hkv);
    if (pos0 == 0) {
        const int64_t qs[3] = {(int64_t)(g.S * g.qd()), (int64_t)g.D, (int64_t)g.qd()};
        const int64_t kvs[3] = {(int64_t)(g.S * g.kd()), (int64_t)g.D, (int64_t)g.kd()};
        const int64_t os_tok[3] = {(int64_t)(g.S * g.qd()), (int64_t)g.D, (int64_t)g.qd()};
        const int64_t os_head[3] = {(int64_t)(g.S * g.qd()), (int64_t)(g.S * g.D), (int64_t)g.D};
        const size_t ws_bytes = sa_prefill_causal_ws_bytes(SA_DTYPE_F32, B, Hq, Hkv, S, D);
        void* ws = ws_bytes ? b.ws.ensure(ws_bytes) : nullptr;
        check(sa_prefill_causal_strided_ws(q, k, v, SA_DTYPE_F32, B, Hq, Hkv, S, D, qs, kvs,
                                           head_major ? os_head : os_tok, scale, attn, ws, ws_bytes, nullptr),
              "causal prefill");
    } else {
        const size_t ws_bytes = sa_paged_decode_ws_bytes(cache->handle(), B, Hq);
        void* ws = ws_bytes ? b.ws.ensure(ws_bytes) : nullptr;
        check(sa_paged_decode(cache->handle(), static_cast<int>(layer), q, B, nullptr, Hq, 1, scale_out ? 1.0f : scale,
                              attn, ws, ws_bytes, nullptr),
              "paged decode");
    }
    if (scale_out) check(sa_axpby_f32(attn, scale, nullptr, 0.0f, M * g.qd(), attn, nullptr), "output scale");
}

// attn_out [M][H] = o_proj(attention(q/k/v projections of normed [M][H])).
void attention_block_dev(const Geometry& g, const Variant& var, const DevWeights& w, const float* rope_cos,
                         const float* rope_sin, KVCache* cache, size_t layer, const float* normed, float* attn_out) {
    Buffers& b = buffers();
    const size_t M = g.M();
    const int iM = as_int(M, "tokens"), iH = as_int(g.H, "hidden_size");
    float* q = b.q.as<float>(M * g.qd());
    float* k = b.k.as<float>(M * g.kd());
    float* v = b.v.as<float>(M * g.kd());
    float* attn = b.attn.as<float>(M * g.qd());
    check(sa_linear_f32(normed, iM, iH, w.q, as_int(g.qd(), "q rows"), nullptr, q, nullptr), "q_proj");
    check(sa_linear_f32(normed, iM, iH, w.k, as_int(g.kd(), "k rows"), nullptr, k, nullptr), "k_proj");
    check(sa_linear_f32(normed, iM, iH, w.v, as_int(g.kd(), "v rows"), nullptr, v, nullptr), "v_proj");
    attention_dev(g, var, w.q_norm, w.k_norm, kQkNormEps, rope_cos, rope_sin, cache, layer, q, k, v, false, attn);
    check(sa_linear_f32(attn, iM, as_int(g.qd(), "q width"), w.o, iH, nullptr, attn_out, nullptr), "o_proj");
}

// out [M][H] = down(silu(gate(x)) * up(x)); out must not overlap x.
void mlp_dev(const Geometry& g, const DevWeights& w, size_t I, const float* x, float* out) {
    Buffers& b = buffers();
    const size_t M = g.M();
    const int iM = as_int(M, "tokens"), iH = as_int(g.H, "hidden_size"), iI = as_int(I, "intermediate_size");
    float* gt = b.g.as<float>(M * I);
    float* up = b.u.as<float>(M * I);
    check(sa_linear_f32(x, iM, iH, w.gate, iI, nullptr, gt, nullptr), "gate_proj");
    check(sa_linear_f32(x, iM, iH, w.up, iI, nullptr, up, nullptr), "up_proj");
    check(sa_swiglu_f32(gt, up, M * I, gt, nullptr), "SwiGLU");
    check(sa_linear_f32(gt, iM, iI, w.down, iH, nullptr, out, nullptr), "down_proj");
}

// One decoder layer, x [M][H] in place on the device.
void layer_dev(const Geometry& g, const Variant& var, const HostWeights& hw, float eps, const float* rope_cos,
               const float* rope_sin, KVCache* cache, size_t layer, float* x) {
    Buffers& b = buffers();
    const DevWeights w = upload(g, hw);
    const size_t M = g.M(), n = M * g.H;
    const int iM = as_int(M, "tokens"), iH = as_int(g.H, "hidden_size");
    float* t = b.t.as<float>(n);
    float* h = b.h.as<float>(n);
    check(sa_rms_norm_f32(x, iM, iH, w.in_norm, eps, t, nullptr), "input_layernorm");
    attention_block_dev(g, var, w, rope_cos, rope_sin, cache, layer, t, h);
    check(sa_axpby_f32(x, 1.0f, h, 1.0f, n, h, nullptr), "residual");               // h = x + attn
    check(sa_rms_norm_f32(h, iM, iH, w.post_norm, eps, t, nullptr), "post_attention_layernorm");
    float* mlp = b.mlp.as<float>(n);
    mlp_dev(g, w, hw.I, t, mlp);
    check(sa_axpby_f32(h, 1.0f, mlp, 1.0f, n, x, nullptr), "residual");             // x = h + mlp
}

// Uploads cos/sin rows p0 .. p0 + S - 1 of host tables [rows, head_dim / 2]
// into the rope buffer; returns the device cos (sin follows S rows later).
float* upload_rope(const Tensor& cos, const Tensor& sin, size_t p0, size_t S, size_t D) {
    const size_t half = D / 2;
    if (cos.size() != sin.size() || cos.size() < (p0 + S) * half)
        bad("cos/sin must hold rows for positions " + std::to_string(p0) + " .. " + std::to_string(p0 + S - 1));
    float* d = buffers().rope.as<float>(2 * S * half);
    to_device(d, cos.data() + p0 * half, S * half * sizeof(float));
    to_device(d + S * half, sin.data() + p0 * half, S * half * sizeof(float));
    return d;
}

Tensor download(const float* d, const Shape& shape) {
    std::vector<float> out(shape.total());
    to_host(out.data(), d, out.size() * sizeof(float));
    return Tensor(std::move(out), shape);
}

// The layer with a cache, for both weight layouts.
Tensor layer_call(const Tensor& hidden, KVCache* cache, size_t layer, size_t Hq, size_t Hkv, size_t D, float eps,
                  const Tensor& in_norm, const Tensor* qkv, const Tensor* q, const Tensor* k, const Tensor* v,
                  const Tensor& o, const Tensor& q_norm, const Tensor& k_norm, const Tensor& post_norm,
                  const Tensor& gate, const Tensor& up, const Tensor& down, const Tensor& cos, const Tensor& sin,
                  const Variant& var) {
    const Geometry g = geometry(hidden, Hq, Hkv, D);
    HostWeights hw;
    attention_weights(g, qkv, q, k, v, o, q_norm, k_norm, &hw);
    mlp_weights(g, gate, up, down, &hw);
    expect_vector(in_norm, g.H, "input_layernorm_weight");
    expect_vector(post_norm, g.H, "post_attention_layernorm_weight");
    hw.in_norm = in_norm.data();
    hw.post_norm = post_norm.data();
    check_cache(g, cache, layer);
    if (g.M() == 0) return Tensor(std::vector<float>(), hidden.shape());
    const size_t pos0 = cache ? cache->current_seq_len : 0;
    const float* rope = upload_rope(cos, sin, pos0, g.S, g.D);
    float* x = buffers().x.as<float>(g.M() * g.H);
    to_device(x, hidden.data(), g.M() * g.H * sizeof(float));
    layer_dev(g, var, hw, eps, rope, rope + g.S * g.D / 2, cache, layer, x);
    return download(x, hidden.shape());
}

// The forward with a cache, for both weight layouts.
Tensor forward_call(const TensorL& ids, KVCache* cache, const Tensor& embed, const std::vector<Qwen3LayerWeights>& layers,
                    const Tensor& norm_w, const Tensor& lm_head, size_t nl, size_t Hq, size_t Hkv, size_t D, float eps,
                    const Variant& var) {
    if (ids.shape().ndim() != 2) bad("input_ids must be [batch, seq_len]");
    if (embed.ndim() != 2) bad("token_embedding must be [vocab_size, hidden_size]");
    if (layers.size() < nl) bad("fewer layer weights than num_layers");
    check_heads(Hq, Hkv, D);
    const Geometry g{ids.shape()[0], ids.shape()[1], embed.shape()[1], Hq, Hkv, D};
    if (lm_head.ndim() != 2 || lm_head.shape()[1] != g.H) bad("lm_head must be [vocab_size, hidden_size]");
    expect_vector(norm_w, g.H, "norm_weight");
    std::vector<HostWeights> hws(nl);
    for (size_t l = 0; l < nl; ++l) {
        const Qwen3LayerWeights& L = layers[l];
        if (var.avx2)
            attention_weights(g, nullptr, &L.q_proj, &L.k_proj, &L.v_proj, L.o_proj, L.q_norm_weight,
                              L.k_norm_weight, &hws[l]);
        else
            attention_weights(g, &L.qkv_projs, nullptr, nullptr, nullptr, L.o_proj, L.q_norm_weight,
                              L.k_norm_weight, &hws[l]);
        mlp_weights(g, L.gate_proj, L.up_proj, L.down_proj, &hws[l]);
        expect_vector(L.input_layernorm_weight, g.H, "input_layernorm_weight");
        expect_vector(L.post_attention_layernorm_weight, g.H, "post_attention_layernorm_weight");
        hws[l].in_norm = L.input_layernorm_weight.data();
        hws[l].post_norm = L.post_attention_layernorm_weight.data();
    }
    if (nl > 0) check_cache(g, cache, nl - 1);
    else if (cache && cache->current_seq_len + g.S > cache->max_seq_len)
        throw std::runtime_error("KV cache full, cannot append more tokens");
    const Tensor x0 = ops::embedding(ids, embed);   // std::out_of_range on a bad id
    const size_t V = lm_head.shape()[0], M = g.M();
    Shape out_shape({g.B, g.S, V});
    if (M == 0) {
        if (cache) cache->increment_seq_len(g.S);
        return Tensor(std::vector<float>(), out_shape);
    }

    const size_t pos0 = cache ? cache->current_seq_len : 0;
    const size_t half = g.D / 2;
    std::vector<float> rope_h(2 * g.S * half);
    rope_rows(pos0, g.S, g.D, kRopeTheta, rope_h.data(), rope_h.data() + g.S * half);
    Buffers& b = buffers();
    float* rope = b.rope.as<float>(rope_h.size());
    to_device(rope, rope_h.data(), rope_h.size() * sizeof(float));
    float* x = b.x.as<float>(M * g.H);
    to_device(x, x0.data(), M * g.H * sizeof(float));
    for (size_t l = 0; l < nl; ++l) layer_dev(g, var, hws[l], eps, rope, rope + g.S * half, cache, l, x);
    if (cache) cache->increment_seq_len(g.S);

    // Final RMSNorm and lm_head: the weights buffer is free again by now.
    float* head = b.weights.as<float>(V * g.H + g.H);
    to_device(head, lm_head.data(), V * g.H * sizeof(float));
    to_device(head + V * g.H, norm_w.data(), g.H * sizeof(float));
    float* t = b.t.as<float>(M * g.H);
    float* logits = b.g.as<float>(M * V);
    check(sa_rms_norm_f32(x, as_int(M, "tokens"), as_int(g.H, "hidden_size"), head + V * g.H, eps, t, nullptr),
          "final norm");
    check(sa_linear_f32(t, as_int(M, "tokens"), as_int(g.H, "hidden_size"), head, as_int(V, "vocab_size"), nullptr,
                        logits, nullptr),
          "lm_head");
    return download(logits, out_shape);
}

// qwen3_attention / qwen3_attention_avx: no cache, normed hidden in.
Tensor attention_call(const Tensor& hidden, size_t Hq, size_t Hkv, size_t D, const Tensor& q, const Tensor& k,
                      const Tensor& v, const Tensor& o, const Tensor& q_norm, const Tensor& k_norm, const Tensor& cos,
                      const Tensor& sin, const Variant& var) {
    const Geometry g = geometry(hidden, Hq, Hkv, D);
    HostWeights hw;
    attention_weights(g, nullptr, &q, &k, &v, o, q_norm, k_norm, &hw);
    if (g.M() == 0) return Tensor(std::vector<float>(), hidden.shape());
    const DevWeights w = upload(g, hw);
    const float* rope = upload_rope(cos, sin, 0, g.S, g.D);
    Buffers& b = buffers();
    float* x = b.x.as<float>(g.M() * g.H);
    float* out = b.h.as<float>(g.M() * g.H);
    to_device(x, hidden.data(), g.M() * g.H * sizeof(float));
    attention_block_dev(g, var, w, rope, rope + g.S * g.D / 2, nullptr, 0, x, out);
    return download(out, hidden.shape());
}

Tensor mlp_call(const Tensor& hidden, const Tensor& gate, const Tensor& up, const Tensor& down) {
    if (hidden.ndim() < 2) bad("hidden_states must be [..., hidden_size]");
    Geometry g;
    g.H = hidden.shape()[hidden.ndim() - 1];
    g.B = g.H ? hidden.size() / g.H : 0;
    g.S = 1;
    HostWeights hw;
    mlp_weights(g, gate, up, down, &hw);
    if (g.M() == 0 || g.H == 0) return Tensor(std::vector<float>(hidden.size()), hidden.shape());
    const DevWeights w = upload(g, hw);
    Buffers& b = buffers();
    float* x = b.x.as<float>(g.M() * g.H);
    float* out = b.h.as<float>(g.M() * g.H);
    to_device(x, hidden.data(), g.M() * g.H * sizeof(float));
    mlp_dev(g, w, hw.I, x, out);
    return download(out, hidden.shape());
}

}  // namespace

std::pair<Tensor, Tensor> compute_rope_freqs(size_t seq_len, size_t head_dim, float theta) {
    if (head_dim % 2 != 0) throw std::invalid_argument("head_dim must be even for RoPE");
    const size_t half = head_dim / 2;
    std::vector<float> c(seq_len * half), s(seq_len * half);
    rope_rows(0, seq_len, head_dim, theta, c.data(), s.data());
    return {Tensor(std::move(c), Shape({seq_len, half})), Tensor(std::move(s), Shape({seq_len, half}))};
}

Tensor qwen3_attention(const Tensor& hidden_states, size_t Hq, size_t Hkv, size_t D, const Tensor& q_proj,
                       const Tensor& k_proj, const Tensor& v_proj, const Tensor& o_proj, const Tensor& q_norm_weight,
                       const Tensor& k_norm_weight, const Tensor& cos, const Tensor& sin, bool /*has_cache*/) {
    return attention_call(hidden_states, Hq, Hkv, D, q_proj, k_proj, v_proj, o_proj, q_norm_weight, k_norm_weight,
                          cos, sin, Variant{});
}

Tensor qwen3_mlp(const Tensor& hidden_states, const Tensor& gate_proj, const Tensor& up_proj,
                 const Tensor& down_proj) {
    return mlp_call(hidden_states, gate_proj, up_proj, down_proj);
}

Tensor qwen3_decoder_layer(const Tensor& hidden_states, size_t Hq, size_t Hkv, size_t D, float eps,
                           const Tensor& input_layernorm_weight, const Tensor& qkv_projs, const Tensor& o_proj,
                           const Tensor& q_norm_weight, const Tensor& k_norm_weight,
                           const Tensor& post_attention_layernorm_weight, const Tensor& gate_mlp,
                           const Tensor& up_mlp, const Tensor& down_mlp, const Tensor& cos, const Tensor& sin) {
    return layer_call(hidden_states, nullptr, 0, Hq, Hkv, D, eps, input_layernorm_weight, &qkv_projs, nullptr,
                      nullptr, nullptr, o_proj, q_norm_weight, k_norm_weight, post_attention_layernorm_weight,
                      gate_mlp, up_mlp, down_mlp, cos, sin, Variant{});
}

Tensor qwen3_forward(const TensorL& input_ids, const Tensor& token_embedding,
                     const std::vector<Qwen3LayerWeights>& layers, const Tensor& norm_weight, const Tensor& lm_head,
                     size_t num_layers, size_t Hq, size_t Hkv, size_t D, float eps) {
    return forward_call(input_ids, nullptr, token_embedding, layers, norm_weight, lm_head, num_layers, Hq, Hkv, D,
                        eps, Variant{});
}

Tensor qwen3_decoder_layer_with_cache(const Tensor& hidden_states, KVCache* kv_cache, size_t layer_idx, size_t Hq,
                                      size_t Hkv, size_t D, float eps, const Tensor& input_layernorm_weight,
                                      const Tensor& qkv_projs, const Tensor& o_proj, const Tensor& q_norm_weight,
                                      const Tensor& k_norm_weight, const Tensor& post_attention_layernorm_weight,
                                      const Tensor& gate_mlp, const Tensor& up_mlp, const Tensor& down_mlp,
                                      const Tensor& cos, const Tensor& sin, AttentionType attention_type) {
    return layer_call(hidden_states, kv_cache, layer_idx, Hq, Hkv, D, eps, input_layernorm_weight, &qkv_projs,
                      nullptr, nullptr, nullptr, o_proj, q_norm_weight, k_norm_weight,
                      post_attention_layernorm_weight, gate_mlp, up_mlp, down_mlp, cos, sin,
                      Variant{false, attention_type});
}

Tensor qwen3_forward_with_cache(const TensorL& input_ids, KVCache* kv_cache, const Tensor& token_embedding,
                                const std::vector<Qwen3LayerWeights>& layers, const Tensor& norm_weight,
                                const Tensor& lm_head, size_t num_layers, size_t Hq, size_t Hkv, size_t D, float eps,
                                AttentionType attention_type) {
    return forward_call(input_ids, kv_cache, token_embedding, layers, norm_weight, lm_head, num_layers, Hq, Hkv, D,
                        eps, Variant{false, attention_type});
}

Tensor qwen3_attention_with_cache(const Tensor& q_proj_out, const Tensor& k_proj_out, const Tensor& v_proj_out,
                                  KVCache* kv_cache, size_t layer_idx, size_t Hq, size_t Hkv, size_t D, float eps,
                                  const Tensor& q_norm_weight, const Tensor& k_norm_weight,
                                  AttentionType attention_type) {
    if (!kv_cache) bad("qwen3_attention_with_cache needs a KV cache");
    if (q_proj_out.ndim() != 3) bad("q_proj_out must be [batch, seq_len, heads * head_dim]");
    check_heads(Hq, Hkv, D);
    const Geometry g{q_proj_out.shape()[0], q_proj_out.shape()[1], 0, Hq, Hkv, D};
    if (q_proj_out.shape()[2] != g.qd() || k_proj_out.size() != g.M() * g.kd() || v_proj_out.size() != g.M() * g.kd())
        bad("projection outputs do not match the head counts");
    expect_vector(q_norm_weight, D, "q_norm_weight");
    expect_vector(k_norm_weight, D, "k_norm_weight");
    check_cache(g, kv_cache, layer_idx);
    const Shape out_shape({g.B, Hq, g.S, D});
    if (g.M() == 0) return Tensor(std::vector<float>(), out_shape);
    Buffers& b = buffers();
    const size_t nq = g.M() * g.qd(), nkv = g.M() * g.kd(), half = D / 2;
    float* q = b.q.as<float>(nq);
    float* k = b.k.as<float>(nkv);
    float* v = b.v.as<float>(nkv);
    float* w = b.weights.as<float>(2 * D + 2 * g.S * half);
    float* rope = w + 2 * D;
    float* attn = b.attn.as<float>(nq);
    to_device(q, q_proj_out.data(), nq * sizeof(float));
    to_device(k, k_proj_out.data(), nkv * sizeof(float));
    to_device(v, v_proj_out.data(), nkv * sizeof(float));
    to_device(w, q_norm_weight.data(), D * sizeof(float));
    to_device(w + D, k_norm_weight.data(), D * sizeof(float));
    std::vector<float> rope_h(2 * g.S * half);
    rope_rows(kv_cache->current_seq_len, g.S, D, kRopeTheta, rope_h.data(), rope_h.data() + g.S * half);
    to_device(rope, rope_h.data(), rope_h.size() * sizeof(float));
    attention_dev(g, Variant{false, attention_type}, w, w + D, eps, rope, rope + g.S * half, kv_cache, layer_idx, q,
                  k, v, true, attn);
    return download(attn, out_shape);
}

namespace avx2 {

Tensor qwen3_attention_avx(const Tensor& hidden_states, size_t Hq, size_t Hkv, size_t D, const Tensor& q_proj,
                           const Tensor& k_proj, const Tensor& v_proj, const Tensor& o_proj,
                           const Tensor& q_norm_weight, const Tensor& k_norm_weight, const Tensor& cos,
                           const Tensor& sin) {
    return attention_call(hidden_states, Hq, Hkv, D, q_proj, k_proj, v_proj, o_proj, q_norm_weight, k_norm_weight,
                          cos, sin, Variant{true, AttentionType::STANDARD});
}

Tensor qwen3_decoder_layer_avx(const Tensor& hidden_states, size_t Hq, size_t Hkv, size_t D, float eps,
                               const Tensor& input_layernorm_weight, const Tensor& q_proj, const Tensor& k_proj,
                               const Tensor& v_proj, const Tensor& o_proj, const Tensor& q_norm_weight,
                               const Tensor& k_norm_weight, const Tensor& post_attention_layernorm_weight,
                               const Tensor& gate_mlp, const Tensor& up_mlp, const Tensor& down_mlp, const Tensor& cos,
                               const Tensor& sin) {
    return layer_call(hidden_states, nullptr, 0, Hq, Hkv, D, eps, input_layernorm_weight, nullptr, &q_proj, &k_proj,
                      &v_proj, o_proj, q_norm_weight, k_norm_weight, post_attention_layernorm_weight, gate_mlp,
                      up_mlp, down_mlp, cos, sin, Variant{true, AttentionType::STANDARD});
}

Tensor qwen3_forward_avx(const TensorL& input_ids, const Tensor& token_embedding,
                         const std::vector<Qwen3LayerWeights>& layers, const Tensor& norm_weight,
                         const Tensor& lm_head, size_t num_layers, size_t Hq, size_t Hkv, size_t D, float eps) {
    return forward_call(input_ids, nullptr, token_embedding, layers, norm_weight, lm_head, num_layers, Hq, Hkv, D,
                        eps, Variant{true, AttentionType::STANDARD});
}

Tensor qwen3_mlp_avx(const Tensor& hidden_states, const Tensor& gate_proj, const Tensor& up_proj,
                     const Tensor& down_proj) {
    return mlp_call(hidden_states, gate_proj, up_proj, down_proj);
}

Tensor qwen3_decoder_layer_avx_with_cache(const Tensor& hidden_states, KVCache* kv_cache, size_t layer_idx,
                                          size_t Hq, size_t Hkv, size_t D, float eps,
                                          const Tensor& input_layernorm_weight, const Tensor& q_proj,
                                          const Tensor& k_proj, const Tensor& v_proj, const Tensor& o_proj,
                                          const Tensor& q_norm_weight, const Tensor& k_norm_weight,
                                          const Tensor& post_attention_layernorm_weight, const Tensor& gate_mlp,
                                          const Tensor& up_mlp, const Tensor& down_mlp, const Tensor& cos,
                                          const Tensor& sin, AttentionType attention_type) {
    return layer_call(hidden_states, kv_cache, layer_idx, Hq, Hkv, D, eps, input_layernorm_weight, nullptr, &q_proj,
                      &k_proj, &v_proj, o_proj, q_norm_weight, k_norm_weight, post_attention_layernorm_weight,
                      gate_mlp, up_mlp, down_mlp, cos, sin, Variant{true, attention_type});
}

Tensor qwen3_forward_avx_with_cache(const TensorL& input_ids, KVCache* kv_cache, const Tensor& token_embedding,
                                    const std::vector<Qwen3LayerWeights>& layers, const Tensor& norm_weight,
                                    const Tensor& lm_head, size_t num_layers, size_t Hq, size_t Hkv, size_t D,
                                    float eps, AttentionType attention_type) {
    return forward_call(input_ids, kv_cache, token_embedding, layers, norm_weight, lm_head, num_layers, Hq, Hkv, D,
                        eps, Variant{true, attention_type});
}

}  // namespace avx2
}  // namespace qwen3
}  // namespace tensor_cpp
