// RoPE application, repeat_kv and the causal mask of the API mirror
// (reference tensor_cpp/src/qwen3_ops.cpp:110-259).
#include "tensor_cpp/qwen3_ops.h"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <vector>

#include "device.h"

namespace tensor_cpp {
namespace qwen3 {

using sa_compat::check;
using sa_compat::to_device;
using sa_compat::to_host;

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

}  // namespace qwen3
}  // namespace tensor_cpp
