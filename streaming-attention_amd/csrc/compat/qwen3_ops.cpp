// The Qwen3 attention path of the API mirror on the GPU (reference
// tensor_cpp/src/qwen3_ops.cpp:30-259 and the attention block of
// qwen3_decoder_layer_with_cache, :697-909).
#include "tensor_cpp/qwen3_ops.h"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <vector>

#include "device.h"

namespace tensor_cpp {
namespace qwen3 {

namespace {

using sa_compat::check;
using sa_compat::DevBuf;
using sa_compat::to_device;
using sa_compat::to_host;

constexpr float kQwen3Theta = 1000000.0f;

// RoPE tables on the device, rebuilt only when a longer one is needed.
struct RopeTables {
    DevBuf cos_t, sin_t;
    int max_pos = 0, dim = 0;
    float theta = 0.0f;

    void ensure(int need_pos, int d, float th) {
        if (need_pos <= max_pos && d == dim && th == theta) return;
        const int n = std::max(need_pos, 64);
        float* c = cos_t.as<float>((size_t)n * d / 2);
        float* s = sin_t.as<float>((size_t)n * d / 2);
        check(sa_rope_table_init(c, s, n, d, th, nullptr), "sa_rope_table_init");
        max_pos = n;
        dim = d;
        theta = th;
    }
    const float* cos_ptr() { return static_cast<const float*>(cos_t.ensure(0)); }
    const float* sin_ptr() { return static_cast<const float*>(sin_t.ensure(0)); }
};

RopeTables& rope_tables() {
    thread_local RopeTables t;
    return t;
}

}  // namespace

std::pair<Tensor, Tensor> compute_rope_freqs(size_t seq_len, size_t head_dim, float theta) {
    if (head_dim % 2 != 0) throw std::invalid_argument("head_dim must be even for RoPE");
    const size_t half = head_dim / 2;
    std::vector<float> inv(half), c(seq_len * half), s(seq_len * half);
    for (size_t i = 0; i < half; ++i)
        inv[i] = 1.0f / std::pow(theta, static_cast<float>(i) / static_cast<float>(head_dim));
    for (size_t p = 0; p < seq_len; ++p)
        for (size_t i = 0; i < half; ++i) {
            const float a = static_cast<float>(p) * inv[i];
            c[p * half + i] = std::cos(a);
            s[p * half + i] = std::sin(a);
        }
    return {Tensor(std::move(c), Shape({seq_len, half})), Tensor(std::move(s), Shape({seq_len, half}))};
}

std::pair<Tensor, Tensor> apply_rotary_pos_emb(const Tensor& q, const Tensor& k, const Tensor& cos,
                                               const Tensor& sin) {
    if (q.ndim() != 4 || k.ndim() != 4) throw std::invalid_argument("q and k must be [batch, heads, seq, head_dim]");
    const size_t S = q.shape()[2], D = q.shape()[3];
    if (D % 2 != 0) throw std::invalid_argument("head_dim must be even for RoPE");
    if (k.shape()[2] != S || k.shape()[3] != D) throw std::invalid_argument("k shape does not match q");
    if (cos.size() < S * D / 2 || sin.size() != cos.size())
        throw std::invalid_argument("cos/sin must hold seq_len rows of head_dim/2");
    auto& st = sa_compat::staging();
    float* dcos = st.in[2].as<float>(S * D / 2);
    float* dsin = st.in[3].as<float>(S * D / 2);
    to_device(dcos, cos.data(), S * D / 2 * sizeof(float));
    to_device(dsin, sin.data(), S * D / 2 * sizeof(float));
    auto rotate = [&](const Tensor& x) {
        const size_t rows = x.size() / D;
        std::vector<int32_t> pos(rows);
        for (size_t r = 0; r < rows; ++r) pos[r] = static_cast<int32_t>(r % S);
        int32_t* dpos = st.pos.as<int32_t>(rows);
        float* dx = st.in[0].as<float>(x.size());
        to_device(dpos, pos.data(), rows * sizeof(int32_t));
        to_device(dx, x.data(), x.size() * sizeof(float));
        check(sa_qk_norm_rope(dx, static_cast<int>(rows), static_cast<int>(D), dpos, nullptr, 0.0f, dcos, dsin,
                              static_cast<int>(S), dx, nullptr),
              "sa_qk_norm_rope");
        std::vector<float> out(x.size());
        to_host(out.data(), dx, x.size() * sizeof(float));
        return Tensor(std::move(out), x.shape());
    };
    Tensor qo = rotate(q);
    Tensor ko = rotate(k);
    return {qo, ko};
}

Tensor repeat_kv(const Tensor& x, int n_rep) {
    if (n_rep <= 0) throw std::invalid_argument("n_rep must be positive");
    if (n_rep == 1) return x;
    const size_t B = x.shape()[0], H = x.shape()[1], S = x.shape()[2], D = x.shape()[3];
    std::vector<float> out(B * H * n_rep * S * D);
    const size_t blk = S * D;
    for (size_t b = 0; b < B; ++b)
        for (size_t h = 0; h < H; ++h)
            for (int r = 0; r < n_rep; ++r)
                std::copy(x.data() + (b * H + h) * blk, x.data() + (b * H + h + 1) * blk,
                          out.begin() + ((b * H + h) * n_rep + r) * blk);
    return Tensor(std::move(out), Shape({B, H * n_rep, S, D}));
}

Tensor create_causal_mask(size_t seq_len, float /*dtype*/) {
    std::vector<float> m(seq_len * seq_len);
    for (size_t i = 0; i < seq_len; ++i)
        for (size_t j = 0; j < seq_len; ++j)
            m[i * seq_len + j] = j <= i ? 0.0f : -std::numeric_limits<float>::infinity();
    return Tensor(std::move(m), Shape({seq_len, seq_len}));
}

Tensor qwen3_attention_with_cache(const Tensor& q_proj_out, const Tensor& k_proj_out, const Tensor& v_proj_out,
                                  KVCache* kv_cache, size_t layer_idx, size_t Hq, size_t Hkv, size_t D,
                                  float eps, const Tensor& q_norm_weight, const Tensor& k_norm_weight,
                                  AttentionType attention_type) {
    if (!kv_cache) throw std::invalid_argument("qwen3_attention_with_cache needs a KV cache");
    if (layer_idx >= kv_cache->num_layers) throw std::out_of_range("Layer index out of range");
    if (q_proj_out.ndim() != 3) throw std::invalid_argument("q_proj_out must be [batch, seq_len, heads * head_dim]");
    const size_t B = q_proj_out.shape()[0], S = q_proj_out.shape()[1];
    if (q_proj_out.shape()[2] != Hq * D || k_proj_out.size() != B * S * Hkv * D ||
        v_proj_out.size() != B * S * Hkv * D)
        throw std::invalid_argument("projection outputs do not match the head counts");
    if (B != kv_cache->batch_size || Hkv != kv_cache->num_kv_heads || D != kv_cache->head_dim)
        throw std::invalid_argument("KV cache shape does not match the layer");
    if (q_norm_weight.size() != D || k_norm_weight.size() != D)
        throw std::invalid_argument("norm weights must have head_dim entries");
    const size_t pos0 = kv_cache->current_seq_len;
    if (pos0 + S > kv_cache->max_seq_len) throw std::runtime_error("KV cache full, cannot append more tokens");
    if (pos0 > 0 && S != 1) throw std::invalid_argument("with a non-empty cache one token is decoded at a time");
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));

    auto& st = sa_compat::staging();
    const size_t nq = B * S * Hq * D, nkv = B * S * Hkv * D;
    float* dq = st.in[0].as<float>(nq);
    float* dk = st.in[1].as<float>(nkv);
    float* dv = st.in[2].as<float>(nkv);
    float* dw = st.in[3].as<float>(2 * D);
    float* dout = st.out.as<float>(nq + nq);   // [0, nq): roped q, [nq, 2 nq): attention
    to_device(dq, q_proj_out.data(), nq * sizeof(float));
    to_device(dk, k_proj_out.data(), nkv * sizeof(float));
    to_device(dv, v_proj_out.data(), nkv * sizeof(float));
    to_device(dw, q_norm_weight.data(), D * sizeof(float));
    to_device(dw + D, k_norm_weight.data(), D * sizeof(float));
    RopeTables& rope = rope_tables();
    rope.ensure(static_cast<int>(kv_cache->max_seq_len), static_cast<int>(D), kQwen3Theta);

    sa_kvcache* c = kv_cache->handle();
    float* q_roped = dout;
    float* attn = dout + nq;
    check(sa_qknorm_rope_append(c, static_cast<int>(layer_idx), dq, dk, dv, static_cast<int>(B), static_cast<int>(S),
                                nullptr, static_cast<int>(Hq), dw, dw + D, eps, rope.cos_ptr(), rope.sin_ptr(),
                                rope.max_pos, q_roped, nullptr),
          "sa_qknorm_rope_append");

    std::vector<float> host(nq);
    if (pos0 == 0) {
        // Prefill: causal attention over the S new tokens.  q comes roped from
        // the append kernel; k is normed and roped again here into dk (the
        // cache holds the same values), v is used as given.
        std::vector<int32_t> pos(B * S * Hkv);
        for (size_t r = 0; r < pos.size(); ++r) pos[r] = static_cast<int32_t>((r / Hkv) % S);
        int32_t* dpos = st.pos.as<int32_t>(pos.size());
        to_device(dpos, pos.data(), pos.size() * sizeof(int32_t));
        check(sa_qk_norm_rope(dk, static_cast<int>(B * S * Hkv), static_cast<int>(D), dpos, dw + D, eps,
                              rope.cos_ptr(), rope.sin_ptr(), rope.max_pos, dk, nullptr),
              "sa_qk_norm_rope");
        // token-major inputs [B][S][H][D]; output [B][Hq][S][D]
        const int64_t qs[3] = {(int64_t)(S * Hq * D), (int64_t)D, (int64_t)(Hq * D)};
        const int64_t kvs[3] = {(int64_t)(S * Hkv * D), (int64_t)D, (int64_t)(Hkv * D)};
        const int64_t os[3] = {(int64_t)(Hq * S * D), (int64_t)(S * D), (int64_t)D};
        check(sa_prefill_causal_strided(q_roped, dk, dv, SA_DTYPE_F32, static_cast<int>(B), static_cast<int>(Hq),
                                        static_cast<int>(Hkv), static_cast<int>(S), static_cast<int>(D), qs, kvs,
                                        os, scale, attn, nullptr),
              "sa_prefill_causal_strided");
        to_host(host.data(), attn, nq * sizeof(float));
        return Tensor(std::move(host), Shape({B, Hq, S, D}));
    }
    // Decode: the new token attends over the cache plus itself (one pending token).
    const bool scale_out = attention_type == AttentionType::STREAMING && ops::g_streaming_scale_on_output;
    const size_t ws_bytes = sa_paged_decode_ws_bytes(c, static_cast<int>(B), static_cast<int>(Hq));
    void* ws = ws_bytes ? st.ws.ensure(ws_bytes) : nullptr;
    check(sa_paged_decode(c, static_cast<int>(layer_idx), q_roped, static_cast<int>(B), nullptr, static_cast<int>(Hq),
                          1, scale_out ? 1.0f : scale, attn, ws, ws_bytes, nullptr),
          "sa_paged_decode");
    to_host(host.data(), attn, nq * sizeof(float));
    if (scale_out)
        for (float& x : host) x *= scale;
    return Tensor(std::move(host), Shape({B, Hq, S, D}));
}

}  // namespace qwen3
}  // namespace tensor_cpp
