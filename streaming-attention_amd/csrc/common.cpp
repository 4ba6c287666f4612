// Error state and device queries shared by the C ABI entry points.
#include "sa_internal.h"

#include <atomic>
#include <mutex>
#include <vector>

namespace sa {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

sa_status fail(sa_status st, const std::string& msg) {
    g_last_error = msg;
    return st;
}

sa_status hip_fail(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return SA_EHIP;
}

int device_cu_count() {
    static std::mutex mu;
    static std::vector<int> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
    if (cache[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cache[dev] = n;
    }
    return cache[dev];
}

namespace {
std::atomic<int> g_q_block{0};
std::atomic<int> g_kv_block{0};
}  // namespace

int attn_q_block() { return g_q_block.load(std::memory_order_relaxed); }
int attn_kv_block() { return g_kv_block.load(std::memory_order_relaxed); }

}  // namespace sa

extern "C" const char* sa_last_error(void) { return sa::g_last_error.c_str(); }

extern "C" sa_status sa_set_attention_blocks(int q_block, int kv_block) {
    sa::clear_error();
    if (q_block != 0 && q_block != 32 && q_block != 64 && q_block != 128)
        return sa::fail(SA_EINVAL, "q_block_size must be 32, 64 or 128 (0: automatic)");
    if (kv_block != 0 && (kv_block < 64 || kv_block > 16384 || kv_block % 64 != 0))
        return sa::fail(SA_EINVAL, "kv_block_size must be a multiple of 64 in [64, 16384] (0: automatic)");
    sa::g_q_block.store(q_block, std::memory_order_relaxed);
    sa::g_kv_block.store(kv_block, std::memory_order_relaxed);
    return SA_OK;
}

extern "C" sa_status sa_get_attention_blocks(int* q_block, int* kv_block) {
    sa::clear_error();
    if (!q_block || !kv_block) return sa::fail(SA_EINVAL, "null pointer");
    *q_block = sa::attn_q_block();
    *kv_block = sa::attn_kv_block();
    return SA_OK;
}
