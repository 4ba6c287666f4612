// KVCache of the API mirror over the paged device cache (reference
// tensor_cpp/include/tensor_cpp/kv_cache.h:27-238).
#include "tensor_cpp/kv_cache.h"

#include <stdexcept>
#include <utility>
#include <vector>

#include "device.h"

namespace tensor_cpp {
namespace qwen3 {

using sa_compat::check;

KVCache::KVCache(size_t n_layers, size_t batch, size_t n_kv_heads, size_t dim, size_t max_len,
                 sa_dtype kv_dtype)
    : num_layers(n_layers),
      batch_size(batch),
      num_kv_heads(n_kv_heads),
      head_dim(dim),
      max_seq_len(max_len),
      current_seq_len(0),
      dtype_(kv_dtype) {
    if (n_layers == 0 || batch == 0 || n_kv_heads == 0 || max_len == 0)
        throw std::invalid_argument("KVCache dimensions must be positive");
    const int pages_per_seq = static_cast<int>((max_len + SA_PAGE_TOKENS - 1) / SA_PAGE_TOKENS);
    sa_kv_desc d{};
    d.num_layers = static_cast<int>(n_layers);
    d.num_kv_heads = static_cast<int>(n_kv_heads);
    d.head_dim = static_cast<int>(dim);
    d.max_seqs = static_cast<int>(batch);
    d.max_pages_per_seq = pages_per_seq;
    d.num_pages = pages_per_seq * static_cast<int>(batch);
    d.kv_dtype = kv_dtype;
    check(sa_kvcache_create(&d, &cache_), "sa_kvcache_create");
    for (size_t b = 0; b < batch; ++b)
        check(sa_kvcache_reserve(cache_, static_cast<int>(b), pages_per_seq * SA_PAGE_TOKENS, nullptr),
              "sa_kvcache_reserve");
}

KVCache::~KVCache() {
    if (cache_) sa_kvcache_destroy(cache_);
}

KVCache::KVCache(KVCache&& o) noexcept
    : num_layers(o.num_layers),
      batch_size(o.batch_size),
      num_kv_heads(o.num_kv_heads),
      head_dim(o.head_dim),
      max_seq_len(o.max_seq_len),
      current_seq_len(o.current_seq_len),
      cache_(o.cache_),
      dtype_(o.dtype_) {
    o.cache_ = nullptr;
}

KVCache& KVCache::operator=(KVCache&& o) noexcept {
    if (this != &o) {
        if (cache_) sa_kvcache_destroy(cache_);
        num_layers = o.num_layers;
        batch_size = o.batch_size;
        num_kv_heads = o.num_kv_heads;
        head_dim = o.head_dim;
        max_seq_len = o.max_seq_len;
        current_seq_len = o.current_seq_len;
        cache_ = o.cache_;
        dtype_ = o.dtype_;
        o.cache_ = nullptr;
    }
    return *this;
}

void KVCache::update(size_t layer_idx, const Tensor& new_keys, const Tensor& new_values) {
    if (layer_idx >= num_layers) throw std::out_of_range("Layer index out of range");
    const Shape& s = new_keys.shape();
    if (s.ndim() != 4 || new_values.shape() != s || s[0] != batch_size || s[1] != num_kv_heads ||
        s[3] != head_dim)
        throw std::invalid_argument("update expects [batch, num_kv_heads, seq_len, head_dim] keys and values");
    const size_t S = s[2];
    if (current_seq_len + S > max_seq_len) throw std::runtime_error("KV cache full, cannot append more tokens");
    if (S == 0) return;
    // [B, Hkv, S, D] -> token-major [B, S, Hkv, D] for the append kernel.
    const Tensor k_t = new_keys.transpose(1, 2);
    const Tensor v_t = new_values.transpose(1, 2);
    auto& st = sa_compat::staging();
    const size_t n = k_t.size();
    float* dk = st.in[0].as<float>(n);
    float* dv = st.in[1].as<float>(n);
    sa_compat::to_device(dk, k_t.data(), n * sizeof(float));
    sa_compat::to_device(dv, v_t.data(), n * sizeof(float));
    check(sa_qknorm_rope_append(cache_, static_cast<int>(layer_idx), nullptr, dk, dv,
                                static_cast<int>(batch_size), static_cast<int>(S), nullptr, 0, nullptr,
                                nullptr, 0.0f, nullptr, nullptr, 0, nullptr, nullptr),
          "sa_qknorm_rope_append");
    sa_compat::hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
}

void KVCache::increment_seq_len(size_t amount) {
    if (amount == 0) return;
    check(sa_kvcache_commit(cache_, nullptr, static_cast<int>(batch_size), static_cast<int>(amount), nullptr),
          "KV cache full, cannot append more tokens");
    current_seq_len += amount;
}

void KVCache::reset() {
    check(sa_kvcache_reset(cache_, nullptr), "sa_kvcache_reset");
    const int pages_per_seq = static_cast<int>((max_seq_len + SA_PAGE_TOKENS - 1) / SA_PAGE_TOKENS);
    for (size_t b = 0; b < batch_size; ++b)
        check(sa_kvcache_reserve(cache_, static_cast<int>(b), pages_per_seq * SA_PAGE_TOKENS, nullptr),
              "sa_kvcache_reserve");
    sa_compat::hip_check(hipStreamSynchronize(nullptr), "hipStreamSynchronize");
    current_seq_len = 0;
}

Tensor KVCache::gather(size_t layer_idx, size_t seq_len, bool keys) const {
    if (layer_idx >= num_layers) throw std::out_of_range("Layer index out of range");
    if (seq_len > current_seq_len) throw std::runtime_error("Requested seq_len exceeds cached length");
    std::vector<float> out(batch_size * num_kv_heads * seq_len * head_dim);
    if (seq_len > 0) {
        const size_t per = num_kv_heads * seq_len * head_dim;
        float* d = sa_compat::staging().out.as<float>(per);
        for (size_t b = 0; b < batch_size; ++b) {
            check(sa_kvcache_gather(cache_, static_cast<int>(layer_idx), static_cast<int>(b),
                                    static_cast<int>(seq_len), keys ? d : nullptr, keys ? nullptr : d, nullptr),
                  "sa_kvcache_gather");
            sa_compat::to_host(out.data() + b * per, d, per * sizeof(float));
        }
    }
    return Tensor(std::move(out), Shape({batch_size, num_kv_heads, seq_len, head_dim}));
}

Tensor KVCache::get_cached_keys(size_t layer_idx, size_t seq_len) const { return gather(layer_idx, seq_len, true); }

Tensor KVCache::get_cached_values(size_t layer_idx, size_t seq_len) const {
    return gather(layer_idx, seq_len, false);
}

}  // namespace qwen3
}  // namespace tensor_cpp
