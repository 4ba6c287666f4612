// Dense fp32 operators of the Qwen3 decoder layer on gfx950: the linear
// projection (fp32 MFMA), RMSNorm, SwiGLU and the scaled add of residuals.
//
// They serve the reference's host-tensor layer API (tensor_cpp/src/ops.cpp
// linear :315-369, rms_norm :375-418, add :194-207, swiglu :493-509;
// tensor_cpp/src/qwen3_ops.cpp qwen3_mlp :265-296) with fp32 weights, so the
// layer keeps fp32 arithmetic end to end.  Every operator reads and writes
// HBM once per element; the linear is the only one with data reuse.
#include <stdint.h>

#include "sa_internal.h"

namespace sa {
namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// y[M][N] = x[M][K] . w[N][K]^T (+ bias[N]), fp32 in and out.
//
// Workgroup (bx, by) owns the 64 x 64 output tile at rows 64 by, columns
// 64 bx; wave w computes its 32 x 32 quadrant (w >> 1, w & 1) as 2 x 2 tiles
// of v_mfma_f32_16x16x4_f32.  Per 32-wide k step the workgroup stages the
// 64 x 32 blocks of x and w through LDS, k-major, so that a fragment read
// (lane l: row l & 15 at k = l >> 4) is 16 consecutive floats per k.  Rows,
// columns and k past the matrix read as zero; stores are bounds-checked.
// VEC: K % 4 == 0 and 16-byte aligned x and w, so blocks load as float4.
// ---------------------------------------------------------------------------
constexpr int kLinTile = 64;
constexpr int kLinK = 32;
constexpr int kLinStride = kLinTile + 4;   // floats per LDS k row

template <bool VEC>
__device__ __forceinline__ void stage_block(const float* __restrict__ src, int rows, int K, int r0, int k0,
                                            float (*dst)[kLinStride]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int slot = threadIdx.x + i * 256;   // 512 slots of 4 floats: 64 rows x 8
        const int r = slot >> 3, kq = (slot & 7) * 4;
        const int row = r0 + r, k = k0 + kq;
        f32x4_t v = {0.f, 0.f, 0.f, 0.f};
        if (row < rows) {
            const float* p = src + (size_t)row * K + k;
            if constexpr (VEC) {
                if (k < K) v = *reinterpret_cast<const f32x4_t*>(p);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (k + j < K) v[j] = p[j];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) dst[kq + j][r] = v[j];
    }
}

template <bool VEC>
__global__ void __launch_bounds__(256)
linear_f32_kernel(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ bias,
                  float* __restrict__ y, int M, int N, int K) {
    __shared__ float xs[kLinK][kLinStride];
    __shared__ float ws[kLinK][kLinStride];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.y * kLinTile, n0 = blockIdx.x * kLinTile;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int c = lane & 15, kl = lane >> 4;
    f32x4_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < K; k0 += kLinK) {
        stage_block<VEC>(x, M, K, m0, k0, xs);
        stage_block<VEC>(w, N, K, n0, k0, ws);
        __syncthreads();
#pragma unroll
        for (int ks = 0; ks < kLinK; ks += 4) {
            const int kk = ks + kl;
            const float a0 = xs[kk][wm + c], a1 = xs[kk][wm + 16 + c];
            const float b0 = ws[kk][wn + c], b1 = ws[kk][wn + 16 + c];
            acc[0][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a1, b1, acc[1][1], 0, 0, 0);
        }
        __syncthreads();
    }
    // Output fragment: lane l holds column l & 15 of rows 4 (l >> 4) + r.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int col = n0 + wn + 16 * j + c;
        if (col >= N) continue;
        const float b = bias ? bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm + 16 * i + 4 * kl + r;
                if (row < M) y[(size_t)row * N + col] = acc[i][j][r] + b;
            }
    }
}

// ---------------------------------------------------------------------------
// Row RMSNorm, one workgroup per row: y = (x / sqrt(sum(x^2) / n + eps)) * w.
// y may alias x (each element is read before it is written, by one thread).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
rms_norm_f32_kernel(const float* x, int n, const float* __restrict__ w, float eps, float* y) {
    __shared__ float red[4];
    const float* xr = x + (size_t)blockIdx.x * n;
    float* yr = y + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) ss = fmaf(xr[i], xr[i], ss);
    ss = group_reduce<OpSum, 1, kWave>(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (red[0] + red[1]) + (red[2] + red[3]);
    const float rms = sqrtf(total / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = xr[i] / rms;
        yr[i] = w ? v * w[i] : v;
    }
}

// out = up * (gate * sigmoid(gate)), sigmoid(g) = 1 / (1 + exp(-g)).
__global__ void __launch_bounds__(256)
swiglu_f32_kernel(const float* gate, const float* up, size_t n, float* out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const float g = gate[i];
        const float silu = g * (1.0f / (1.0f + expf(-g)));
        out[i] = up[i] * silu;
    }
}

// out = a x + b y (y == NULL: out = a x).
__global__ void __launch_bounds__(256)
axpby_f32_kernel(const float* x, float a, const float* y, float b, size_t n, float* out) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        out[i] = y ? fmaf(a, x[i], b * y[i]) : a * x[i];
}

// Enough workgroups to cover n once, at most 8 per CU (grid-stride beyond).
dim3 elementwise_grid(size_t n) {
    const size_t want = (n + 255) / 256;
    const size_t cap = (size_t)device_cu_count() * 8;
    return dim3((unsigned)(want < cap ? (want ? want : 1) : cap));
}

}  // namespace
}  // namespace sa

using namespace sa;

extern "C" sa_status sa_linear_f32(const float* x, int M, int K, const float* w, int N, const float* bias,
                                   float* y, sa_stream_t stream) {
    clear_error();
    if (!y || (K > 0 && (!x || !w))) return fail(SA_EINVAL, "null pointer");
    if (M < 0 || N < 0 || K < 0) return fail(SA_EINVAL, "M, N and K must be >= 0");
    if (M == 0 || N == 0) return SA_OK;
    const dim3 grid((N + kLinTile - 1) / kLinTile, (M + kLinTile - 1) / kLinTile);
    if (grid.y > 65535u) return fail(SA_EINVAL, "M too large for one launch");
    hipStream_t st = as_stream(stream);
    if (K % 4 == 0 && aligned16(x) && aligned16(w))
        hipLaunchKernelGGL(linear_f32_kernel<true>, grid, dim3(256), 0, st, x, w, bias, y, M, N, K);
    else
        hipLaunchKernelGGL(linear_f32_kernel<false>, grid, dim3(256), 0, st, x, w, bias, y, M, N, K);
    SA_CHECK_LAUNCH();
    return SA_OK;
}

extern "C" sa_status sa_rms_norm_f32(const float* x, int rows, int n, const float* w, float eps, float* y,
                                     sa_stream_t stream) {
    clear_error();
    if (!x || !y) return fail(SA_EINVAL, "null pointer");
    if (rows < 0 || n <= 0) return fail(SA_EINVAL, "rows must be >= 0 and n > 0");
    if (rows == 0) return SA_OK;
    hipLaunchKernelGGL(rms_norm_f32_kernel, dim3(rows), dim3(256), 0, as_stream(stream), x, n, w, eps, y);
    SA_CHECK_LAUNCH();
    return SA_OK;
}

extern "C" sa_status sa_swiglu_f32(const float* gate, const float* up, size_t n, float* out,
                                   sa_stream_t stream) {
    clear_error();
    if (!gate || !up || !out) return fail(SA_EINVAL, "null pointer");
    if (n == 0) return SA_OK;
    hipLaunchKernelGGL(swiglu_f32_kernel, elementwise_grid(n), dim3(256), 0, as_stream(stream), gate, up, n,
                       out);
    SA_CHECK_LAUNCH();
    return SA_OK;
}

extern "C" sa_status sa_axpby_f32(const float* x, float a, const float* y, float b, size_t n, float* out,
                                  sa_stream_t stream) {
    clear_error();
    if (!x || !out) return fail(SA_EINVAL, "null pointer");
    if (n == 0) return SA_OK;
    hipLaunchKernelGGL(axpby_f32_kernel, elementwise_grid(n), dim3(256), 0, as_stream(stream), x, a, y, b, n,
                       out);
    SA_CHECK_LAUNCH();
    return SA_OK;
}
