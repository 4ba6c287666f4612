/*
 * tensor_cpp/ops_avx.h - the reference's raw-pointer vector operators
 * (reference tensor_cpp/include/tensor_cpp/ops_avx.h:14-95), served by the
 * MI355X library: same names and signatures, host fp32 arrays in and out,
 * the arithmetic on the GPU (fp32 MFMA for matmul_avx and dot_avx; the
 * library's RMSNorm and axpby kernels).
 */
#ifndef SA_AMD_TENSOR_CPP_OPS_AVX_H
#define SA_AMD_TENSOR_CPP_OPS_AVX_H

#include <vector>

#include "tensor_cpp/tensor.h"

namespace tensor_cpp {
namespace ops {
namespace avx {

/* C [M, N] = A [M, K] . B [N, K]^T (reference tensor_cpp/src/ops_avx.cpp:50-150). */
std::vector<float> matmul_avx(const float* A, const float* B, int M, int N, int K);

/* sum_i x[i] y[i] (reference tensor_cpp/src/ops_avx.cpp:152-210). */
float dot_avx(const float* x, const float* y, int size);

/* result = x + scale * y (reference tensor_cpp/src/ops_avx.cpp:214-244);
 * result may alias x or y. */
void add_avx(const float* x, const float* y, float scale, int size, float* result);

/* Per row of [batch_size, hidden_size]: x / sqrt(mean(x^2) + eps) * weight,
 * weight [hidden_size] or null (reference tensor_cpp/src/ops_avx.cpp:249-315);
 * result may alias input. */
void rms_norm_avx(const float* input, const float* weight, int batch_size, int hidden_size, float eps, float* result);

/* Whether the host CPU has AVX2 / AVX-512F (the reference reports its own
 * build flags, ops_avx.cpp:30-45).  The operators above run on the GPU either
 * way. */
bool is_avx2_supported();
bool is_avx512_supported();

}  // namespace avx
}  // namespace ops
}  // namespace tensor_cpp

#endif
