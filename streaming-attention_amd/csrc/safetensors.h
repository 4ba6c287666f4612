// A read-only view of a safetensors checkpoint: the 8-byte little-endian
// header length N, N bytes of JSON (tensor name -> {"dtype", "shape",
// "data_offsets": [begin, end]}, plus an optional "__metadata__" entry), then
// the tensor data with offsets relative to the end of the header.  Shared by
// the device loader (sa_qwen3_load_safetensors) and the host mirror of the
// reference's load_qwen3_weights.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "sa_amd.h"
#include "sa_qwen3.h"

namespace sa {

struct StEntry {
    std::string dtype;
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t s : shape) n *= s;
        return n;
    }
};

// The file mapped read-only, its header parsed and every entry checked (byte
// range inside the file and equal to shape x dtype size for BF16 / F32).
// Errors return a status and set the library's last error.
class Checkpoint {
public:
    Checkpoint() = default;
    Checkpoint(const Checkpoint&) = delete;
    Checkpoint& operator=(const Checkpoint&) = delete;
    ~Checkpoint();

    sa_status open_file(const char* path);
    // 2 for BF16, 4 for F32, 0 for any other dtype.
    static int elem_size(const std::string& dtype);
    const StEntry* find(const std::string& name) const;
    // The tensor `name` with exactly the given shape, in BF16 or F32.
    sa_status need(const std::string& name, const std::vector<int64_t>& shape, const StEntry** out) const;
    const unsigned char* bytes(const StEntry& t) const { return data_ + t.begin; }
    // Values of t widened to fp32 into dst[t.numel()] (BF16 or F32 only).
    void to_f32(const StEntry& t, float* dst) const;
    // 1 + the largest i of any "model.layers.<i>." tensor (0 if none).
    int num_layers() const;

private:
    int fd_ = -1;
    void* map_ = nullptr;
    size_t size_ = 0;
    const unsigned char* data_ = nullptr;
    size_t data_size_ = 0;
    std::map<std::string, StEntry> tensors_;
};

std::string layer_tensor_name(int layer, const char* leaf);

// Model shape read from the checkpoint: vocab and hidden from the embedding,
// head_dim from q_norm, heads from q_proj / k_proj rows, intermediate from
// gate_proj, layers from the names; rms_eps 1e-6, rope_theta 1e6, max_pos 0.
sa_status read_qwen3_desc(const Checkpoint& ck, sa_qwen3_desc* d);

}  // namespace sa
