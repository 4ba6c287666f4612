#include "device.h"

namespace sa_compat {

void throw_status(sa_status st, const char* what) {
    std::string msg = std::string(what) + ": " + sa_last_error();
    switch (st) {
        case SA_EINVAL: throw std::invalid_argument(msg);
        case SA_ERANGE: throw std::out_of_range(msg);
        default: throw std::runtime_error(msg);
    }
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

DevBuf::~DevBuf() {
    if (ptr_) (void)hipFree(ptr_);
}

void* DevBuf::ensure(size_t bytes) {
    if (bytes == 0) bytes = 16;
    if (bytes > bytes_) {
        if (ptr_) hip_check(hipFree(ptr_), "hipFree");
        ptr_ = nullptr;
        bytes_ = 0;
        hip_check(hipMalloc(&ptr_, bytes), "hipMalloc");
        bytes_ = bytes;
    }
    return ptr_;
}

Staging& staging() {
    thread_local Staging s;
    return s;
}

void to_device(void* dst, const void* src, size_t bytes) {
    if (bytes) hip_check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
}

void to_host(void* dst, const void* src, size_t bytes) {
    if (bytes) hip_check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}

}  // namespace sa_compat
