// The reference's raw-pointer vector operators (tensor_cpp/src/ops_avx.cpp)
// on the GPU: each call uploads its host arrays, runs one kernel of
// libsa_amd (fp32 MFMA linear, RMSNorm, axpby) and copies the result back.
#include "tensor_cpp/ops_avx.h"

#include <stdexcept>
#include <string>
#include <vector>

#include "device.h"

namespace tensor_cpp {
namespace ops {
namespace avx {

namespace {

using sa_compat::check;
using sa_compat::staging;
using sa_compat::to_device;
using sa_compat::to_host;

size_t count(int v, const char* what) {
    if (v < 0) throw std::invalid_argument(std::string(what) + " must be >= 0");
    return static_cast<size_t>(v);
}

}  // namespace

std::vector<float> matmul_avx(const float* A, const float* B, int M, int N, int K) {
    const size_t m = count(M, "M"), n = count(N, "N"), k = count(K, "K");
    std::vector<float> C(m * n, 0.0f);
    if (m == 0 || n == 0) return C;
    auto& st = staging();
    float* da = k ? st.in[0].as<float>(m * k) : nullptr;
    float* db = k ? st.in[1].as<float>(n * k) : nullptr;
    float* dc = st.out.as<float>(m * n);
    if (k) {
        to_device(da, A, m * k * sizeof(float));
        to_device(db, B, n * k * sizeof(float));
    }
    check(sa_linear_f32(da, M, K, db, N, nullptr, dc, nullptr), "sa_linear_f32");
    to_host(C.data(), dc, m * n * sizeof(float));
    return C;
}

float dot_avx(const float* x, const float* y, int size) {
    return matmul_avx(x, y, 1, 1, size)[0];
}

void add_avx(const float* x, const float* y, float scale, int size, float* result) {
    const size_t n = count(size, "size");
    if (n == 0) return;
    auto& st = staging();
    float* dx = st.in[0].as<float>(n);
    float* dy = st.in[1].as<float>(n);
    to_device(dx, x, n * sizeof(float));
    to_device(dy, y, n * sizeof(float));
    check(sa_axpby_f32(dx, 1.0f, dy, scale, n, dx, nullptr), "sa_axpby_f32");
    to_host(result, dx, n * sizeof(float));
}

void rms_norm_avx(const float* input, const float* weight, int batch_size, int hidden_size, float eps,
                  float* result) {
    const size_t rows = count(batch_size, "batch_size"), n = count(hidden_size, "hidden_size");
    if (rows == 0 || n == 0) return;
    auto& st = staging();
    float* dx = st.in[0].as<float>(rows * n);
    float* dw = weight ? st.in[1].as<float>(n) : nullptr;
    to_device(dx, input, rows * n * sizeof(float));
    if (dw) to_device(dw, weight, n * sizeof(float));
    check(sa_rms_norm_f32(dx, batch_size, hidden_size, dw, eps, dx, nullptr), "sa_rms_norm_f32");
    to_host(result, dx, rows * n * sizeof(float));
}

bool is_avx2_supported() { return __builtin_cpu_supports("avx2"); }

bool is_avx512_supported() { return __builtin_cpu_supports("avx512f"); }

}  // namespace avx
}  // namespace ops
}  // namespace tensor_cpp
