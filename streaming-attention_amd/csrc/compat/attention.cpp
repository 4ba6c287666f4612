// attention.h on the GPU: every variant stages Q/K/V to the device, runs the
// split-KV kernel (sa_stream_attn_f32, unscaled as the reference is) and
// copies O back.  Reference: attention/src/attention.h:27-208.
#include "attention.h"

#include <cmath>
#include <stdexcept>
#include <string>

#include "device.h"

namespace {

std::vector<float> run_single(const float* Q, const float* K, const float* V, int T, int d,
                              int block_size) {
    using namespace sa_compat;
    if (d != 8 && d != 16 && d != 32 && d != 64 && d != 128 && d != 256)
        throw std::invalid_argument("d must be 8, 16, 32, 64, 128 or 256 (got " + std::to_string(d) + ")");
    if (block_size <= 0) throw std::invalid_argument("block_size must be positive");
    std::vector<float> out(d, 0.0f);
    if (T <= 0) return out;
    if (!Q || !K || !V) throw std::invalid_argument("null input");
    Staging& s = staging();
    const size_t kv = (size_t)T * d;
    float* dq = s.in[0].as<float>(d);
    float* dk = s.in[1].as<float>(kv);
    float* dv = s.in[2].as<float>(kv);
    float* dout = s.out.as<float>(d);
    const size_t ws_bytes = sa_stream_attn_ws_bytes(T, d);
    void* ws = ws_bytes ? s.ws.ensure(ws_bytes) : nullptr;
    to_device(dq, Q, d * sizeof(float));
    to_device(dk, K, kv * sizeof(float));
    to_device(dv, V, kv * sizeof(float));
    check(sa_stream_attn_f32(dq, dk, dv, T, d, block_size, 1.0f, dout, ws, ws_bytes, nullptr),
          "sa_stream_attn_f32");
    to_host(out.data(), dout, d * sizeof(float));
    return out;
}

// The naive form is the same softmax(QK^T)V; block 64 is only a label here.
constexpr int kNaiveBlock = 64;

void single_rank(int T_local, int T_global) {
    if (T_local != T_global)
        throw std::invalid_argument("one process holds the whole sequence: T_local must equal T_global");
}

}  // namespace

std::vector<float> naive_attention_serial(const float* Q, const float* K, const float* V, int T, int d) {
    return run_single(Q, K, V, T, d, kNaiveBlock);
}

std::vector<float> naive_attention_omp(const float* Q, const float* K, const float* V, int T, int d,
                                       int /*num_threads*/) {
    return run_single(Q, K, V, T, d, kNaiveBlock);
}

std::vector<float> naive_attention_mpi(const float* Q_local, const float* K_local, const float* V_local,
                                       int T_local, int T_global, int d, int /*num_omp_threads*/,
                                       MPI_Comm /*comm*/) {
    single_rank(T_local, T_global);
    return run_single(Q_local, K_local, V_local, T_local, d, kNaiveBlock);
}

std::vector<float> naive_attention_mpi_simple(const float* Q_local, const float* K_local,
                                              const float* V_local, int T_local, int T_global, int d,
                                              MPI_Comm /*comm*/) {
    single_rank(T_local, T_global);
    return run_single(Q_local, K_local, V_local, T_local, d, kNaiveBlock);
}

std::vector<float> streaming_attention_serial(const float* Q, const float* K, const float* V, int T, int d,
                                              int block_size) {
    return run_single(Q, K, V, T, d, block_size);
}

std::vector<float> streaming_attention_omp(const float* Q, const float* K, const float* V, int T, int d,
                                           int block_size, int /*num_threads*/) {
    return run_single(Q, K, V, T, d, block_size);
}

std::vector<float> streaming_attention_omp_numa(const float* Q, const float* K, const float* V, int T,
                                                int d, int block_size, int /*num_threads*/) {
    return run_single(Q, K, V, T, d, block_size);
}

std::vector<float> streaming_attention_mpi_simple(const float* Q_local, const float* K_local,
                                                  const float* V_local, int T_local, int T_global, int d,
                                                  int block_size, MPI_Comm /*comm*/) {
    single_rank(T_local, T_global);
    return run_single(Q_local, K_local, V_local, T_local, d, block_size);
}

// Error metrics, as defined by the reference (attention/src/naive_serial.cpp:75-98):
// relative L2 with an absolute fallback, and max |a - b|.  Host arithmetic on
// the caller's vectors, like the reference.
float compute_l2_error(const float* a, const float* b, int size) {
    float sum_sq = 0.0f, sum_ref = 0.0f;
    for (int i = 0; i < size; ++i) {
        const float diff = a[i] - b[i];
        sum_sq += diff * diff;
        sum_ref += b[i] * b[i];
    }
    const float ref_norm = std::sqrt(sum_ref);
    return ref_norm < 1e-10f ? std::sqrt(sum_sq) : std::sqrt(sum_sq) / ref_norm;
}

float compute_max_error(const float* a, const float* b, int size) {
    float m = 0.0f;
    for (int i = 0; i < size; ++i) m = std::max(m, std::fabs(a[i] - b[i]));
    return m;
}
