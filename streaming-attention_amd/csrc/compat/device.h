// Host-side plumbing for the C++ API mirror: device staging buffers that grow
// and are reused per thread, synchronous copies, and sa_status -> exception.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <stdexcept>
#include <string>

#include "sa_amd.h"

namespace sa_compat {

[[noreturn]] void throw_status(sa_status st, const char* what);

inline void check(sa_status st, const char* what) {
    if (st != SA_OK) throw_status(st, what);
}

void hip_check(hipError_t e, const char* what);

// A device allocation that only grows.
class DevBuf {
public:
    DevBuf() = default;
    ~DevBuf();
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    void* ensure(size_t bytes);
    template <class T>
    T* as(size_t count) { return static_cast<T*>(ensure(count * sizeof(T))); }

private:
    void* ptr_ = nullptr;
    size_t bytes_ = 0;
};

// Per-thread staging buffers (inputs, outputs, workspace).
struct Staging {
    DevBuf in[4];
    DevBuf out;
    DevBuf ws;
    DevBuf pos;
};
Staging& staging();

void to_device(void* dst, const void* src, size_t bytes);
void to_host(void* dst, const void* src, size_t bytes);

}  // namespace sa_compat
