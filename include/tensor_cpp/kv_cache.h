/*
 * tensor_cpp/kv_cache.h - the reference's KVCache, kept resident on the GPU.
 *
 * Replaces tensor_cpp::qwen3::KVCache (reference
 * tensor_cpp/include/tensor_cpp/kv_cache.h:27-238) with the same public
 * fields, constructor and methods.  Storage is the paged device cache of
 * libsa_amd (sa_kvcache): every batch row owns ceil(max_seq_len / 64) pages
 * of 64 tokens, fp32 by default or bf16.
 *
 * Semantics kept from the reference: update() writes new keys/values at
 * current_seq_len without advancing it; increment_seq_len() commits; reset()
 * zeroes everything; get_cached_keys/values() return dense host copies
 * [batch, num_kv_heads, seq_len, head_dim].  The exceptions are the
 * reference's: std::out_of_range for a bad layer, std::runtime_error for a
 * full cache or an over-long read.
 *
 * Not kept: the per-layer host tensors key_cache / value_cache (the data
 * lives on the device; use get_cached_* or handle()).  increment_seq_len()
 * past the page capacity throws std::runtime_error (the reference defers the
 * error to the next update()).
 */
#ifndef SA_AMD_TENSOR_CPP_KV_CACHE_H
#define SA_AMD_TENSOR_CPP_KV_CACHE_H

#include <cstddef>

#include "sa_amd.h"
#include "tensor_cpp/tensor.h"

namespace tensor_cpp {
namespace qwen3 {

struct KVCache {
    size_t num_layers;       ///< Number of layers
    size_t batch_size;       ///< Batch size
    size_t num_kv_heads;     ///< Number of key-value heads
    size_t head_dim;         ///< Head dimension
    size_t max_seq_len;      ///< Maximum sequence length
    size_t current_seq_len;  ///< Committed sequence length (all rows)

    KVCache(size_t num_layers, size_t batch_size, size_t num_kv_heads, size_t head_dim,
            size_t max_seq_len = 4096, sa_dtype kv_dtype = SA_DTYPE_F32);
    ~KVCache();
    KVCache(const KVCache&) = delete;
    KVCache& operator=(const KVCache&) = delete;
    KVCache(KVCache&& other) noexcept;
    KVCache& operator=(KVCache&& other) noexcept;

    /** Write new_keys / new_values [batch, num_kv_heads, seq_len, head_dim] at
     *  current_seq_len (does not advance it). */
    void update(size_t layer_idx, const Tensor& new_keys, const Tensor& new_values);
    /** Commit `amount` appended tokens for every batch row. */
    void increment_seq_len(size_t amount = 1);
    /** Length 0 and zeroed storage. */
    void reset();
    /** Dense copies [batch, num_kv_heads, seq_len, head_dim] of the first seq_len tokens. */
    Tensor get_cached_keys(size_t layer_idx, size_t seq_len) const;
    Tensor get_cached_values(size_t layer_idx, size_t seq_len) const;

    /** The device cache, for callers that drive the kernels directly. */
    sa_kvcache* handle() const { return cache_; }
    sa_dtype kv_dtype() const { return dtype_; }

private:
    Tensor gather(size_t layer_idx, size_t seq_len, bool keys) const;
    sa_kvcache* cache_ = nullptr;
    sa_dtype dtype_ = SA_DTYPE_F32;
};

}  // namespace qwen3
}  // namespace tensor_cpp

#endif
