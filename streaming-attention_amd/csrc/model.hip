// Qwen3 greedy decode step on gfx950: the decoder around the attention path.
//
// Reference: qwen3_forward_with_cache and qwen3_decoder_layer_with_cache
// (tensor_cpp/src/qwen3_ops.cpp:620-1014), qwen3_mlp (:265-296), and the ops
// they call: embedding (tensor_cpp/src/ops.cpp:278-313), linear (:315-372),
// rms_norm (:375-417).  The attention block itself runs on the fused
// append + paged decode launch of sa_append_decode (decode step) and on
// sa_qknorm_rope_append + the causal prefill kernel (prompt), both reading
// q, k and v straight from the qkv projection's split-K partials.
//
// Layout: the batch of B <= kMaxBatch token rows stays fp32 in a residual stream
// x[B][hidden]; every projection is one GEMM Y = X W^T with bf16 weights in
// nn.Linear layout [out][in] and fp32 accumulation, split over K into
// fixed-order partial sums when the output is narrow, so results do not
// depend on scheduling.  Epilogue kernels fold the partial sums into the next
// step: the attention launches (q | k | v), residual add + RMSNorm, SwiGLU.
#include <math.h>

#include <algorithm>
#include <vector>

#include "sa_internal.h"
#include "sa_qwen3.h"

struct sa_qwen3 {
    struct Layer {
        float* in_norm;
        uint16_t* qkv;
        float* q_norm;
        float* k_norm;
        uint16_t* o;
        float* post_norm;
        uint16_t* gate_up;
        uint16_t* down;
    };
    sa_qwen3_desc d{};
    int max_batch = 0;
    int device = 0;
    std::vector<void*> allocs;
    uint16_t* embed = nullptr;
    uint16_t* lm_head = nullptr;
    float* final_norm = nullptr;
    std::vector<Layer> layers;
    float* rope_cos = nullptr;
    float* rope_sin = nullptr;
    // activations for max_batch rows
    float* x = nullptr;        // residual stream [B][hidden]
    float* h = nullptr;        // normed input of the next projection [B][hidden]
    float* q = nullptr;        // [B][Hq D]
    float* k = nullptr;        // [B][Hkv D]
    float* v = nullptr;        // [B][Hkv D]
    float* q_rope = nullptr;   // [B][Hq D]
    float* attn = nullptr;     // [B][Hq D]
    float* act = nullptr;      // [B][intermediate]
    float* part = nullptr;     // split-K partial sums
    float* logits = nullptr;   // [B][vocab]
    float* am_val = nullptr;   // argmax partials [B][kArgBlocks]
    int32_t* am_idx = nullptr;
    void* ws = nullptr;        // paged decode workspace (grow-only)
    size_t ws_bytes = 0;
    void* pf = nullptr;        // prefill activations for batch x prompt rows (grow-only)
    size_t pf_bytes = 0;
    // Interleaved decode steps (two half-batches): the second half's
    // split-K partials, decode workspace, stream (default priority) and the
    // events that fork and join it; created on the first interleaved step.
    float* part2 = nullptr;
    void* ws2 = nullptr;
    size_t ws2_bytes = 0;
    hipStream_t side = nullptr;
    std::vector<hipEvent_t> events;   // fork, join, the first half's first attention done
};

namespace sa {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMaxRows = 64;     // batch rows one GEMM tile covers (more rows: more tiles)
constexpr int kMaxBatch = 1024;  // decode batch rows per model (activations and logits sized for them)
constexpr int kGN = 64;          // GEMM output columns per workgroup
constexpr int kGK = 32;          // GEMM k chunk
constexpr int kArgBlocks = 64;   // argmax workgroups per row
// A decode step interleaves two half-batches when the attention streams at
// least this many cached K/V bytes per layer.
constexpr long long kInterleaveBytes = 1LL << 30;

// ---------------------------------------------------------------------------
// Synthetic weights: the splitmix64 / Box-Muller generator of the test
// harness, element i = draw i of (seed, stream).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ double unit_draw(uint64_t key, uint64_t i) {
    return (double)((splitmix64(key ^ i) >> 11) + 1) * 0x1.0p-53;
}

__device__ __forceinline__ float normal_draw(uint64_t key, uint64_t i, double scale) {
    const double u1 = unit_draw(key, 2 * i), u2 = unit_draw(key, 2 * i + 1);
    const double z = sqrt(-2.0 * log(u1)) * cos(2.0 * M_PI * u2);
    return (float)(z * scale);
}

__global__ void init_bf16_kernel(uint16_t* out, size_t n, uint64_t key, double scale) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = f32_to_bf16_rne(normal_draw(key, i, scale));
}

__global__ void init_norm_kernel(float* out, size_t n, uint64_t key, double scale) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = 1.0f + normal_draw(key, i, scale);
}

// ---------------------------------------------------------------------------
// Row reductions (256 threads)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = group_reduce<OpSum, 1, 64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();   // red may still be read by a previous call
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) s += red[w];
    return s;
}

// x[m] and h[m] = rms_norm(x[m]) * w, as ops::rms_norm: x / sqrt(mean(x^2) + eps) * w.
__device__ __forceinline__ void norm_row(const float* xr, int H, const float* w, float eps, float* hr,
                                         float* red) {
    float ss = 0.f;
    for (int j = threadIdx.x; j < H; j += blockDim.x) ss += xr[j] * xr[j];
    ss = block_sum(ss, red);
    const float rms = sqrtf(ss / (float)H + eps);
    for (int j = threadIdx.x; j < H; j += blockDim.x) hr[j] = (xr[j] / rms) * w[j];
}

// Embedding gather (bf16 -> fp32) and the first layer's input RMSNorm.
__global__ void __launch_bounds__(256)
embed_norm_kernel(const uint16_t* embed, const int32_t* tokens, int vocab, int H, const float* w, float eps,
                  float* x, float* h) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    const int tok = tokens[m];
    const bool ok = tok >= 0 && tok < vocab;
    float* xr = x + (size_t)m * H;
    for (int j = threadIdx.x; j < H; j += blockDim.x) {
        const uint16_t b = ok ? embed[(size_t)tok * H + j] : (uint16_t)0;
        xr[j] = __uint_as_float((uint32_t)b << 16);
    }
    __syncthreads();
    norm_row(xr, H, w, eps, h + (size_t)m * H, red);
}

// ---------------------------------------------------------------------------
// GEMM: P[s][m][n] = sum over k in split s of X[m][k] * W[n][k].
// X fp32 [M][K], W bf16 [N][K]; N % 64 == 0, split % 32 == 0.
// Workgroup (x, y, z) owns rows 64 z .. 64 z + 63 (rows past M read as zero),
// columns 64 x .. 64 x + 63 and split y; wave w computes columns
// 64 x + 16 w .. + 15 for all 64 rows with v_mfma_f32_16x16x32_bf16.
//
// The bf16 MFMA takes fp32 X as kGemmTerms bf16 terms: t_0 = rne(x),
// t_i = rne(x - t_0 - ... - t_{i-1}) (each difference is exact in fp32), so
// |x - sum t_i| <= 2^-9(kGemmTerms) |x|.  Every product t_i * w is exact in
// fp32 (the weights are bf16) and accumulates in fp32: the result is the fp32
// GEMM's to within that truncation of X.  Per 32-wide k step the workgroup
// converts its 64 x 32 block of X into LDS (double-buffered, one barrier per
// step); W fragments stream from global memory into registers kGemmRing steps
// ahead of their use, X blocks kGemmXRing steps ahead; the per-step barrier
// orders LDS only, so those loads stay in flight across it.  (With
// __syncthreads, which waits for every outstanding global load, each k-step
// cost about one memory round trip: 46.7 us per projection for a 512-row
// prompt at the Qwen3-0.6B shape.)
// ---------------------------------------------------------------------------
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kGemmTerms = 3;     // bf16 terms of each activation (2^-27 |x| left over)
constexpr int kGemmRing = 8;      // W fragments in flight per wave (k steps)
constexpr int kGemmXRing = 4;     // X blocks in flight per thread (k steps); divides kGemmRing
constexpr int kGemmXStride = kGK + 8;   // bf16 per LDS row of X: conflict-free fragment reads

template <int CW>
__global__ void __launch_bounds__(256)
gemm_xwt_kernel(const float* __restrict__ X, int M, int K, const uint16_t* __restrict__ W, int N, int split,
                float* __restrict__ P) {
    __shared__ __align__(16) uint16_t Xb[2][kGemmTerms][kMaxRows][kGemmXStride];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r16 = lane & 15, g = lane >> 4;
    const int n0 = blockIdx.x * kGN * CW + 16 * CW * wave;
    const int k_begin = blockIdx.y * split;
    const int m0 = blockIdx.z * kMaxRows;
    const int Mt = min(M - m0, kMaxRows);
    const int nsteps = split / kGK;

    // W fragment c of step j (A operand): lane (r16, g) holds
    // W[n0 + 16 c + r16][k + 8 g .. + 7].
    const uint16_t* Wl = W + (size_t)(n0 + r16) * K + k_begin + 8 * g;
    auto load_w = [&](int j, int c) { return *reinterpret_cast<const bf16x8_t*>(Wl + (size_t)c * 16 * K + j * kGK); };
    // X block of step j: thread t converts X[m0 + t / 4][k + 8 (t % 4) .. + 7].
    // Rows past M load row M - 1 and are zeroed when converted.  Every load of
    // the loop below is issued unconditionally (steps past the last clamp to
    // it): a load behind a branch leaves the compiler unable to count the
    // loads in flight, and it then waits for all of them (vmcnt(0)) before
    // the first use of any, which drains the prefetch rings every step.
    const int xr = tid >> 2, xc = 8 * (tid & 3);
    const bool x_on = xr < Mt;
    const float* Xl = X + (size_t)(m0 + min(xr, Mt - 1)) * K + k_begin + xc;
    auto load_x = [&](int j, f32x4_t& a, f32x4_t& b) {
        a = *reinterpret_cast<const f32x4_t*>(Xl + j * kGK);
        b = *reinterpret_cast<const f32x4_t*>(Xl + j * kGK + 4);
    };
    auto store_x = [&](int buf, f32x4_t a, f32x4_t b) {
        a = x_on ? a : f32x4_t{};
        b = x_on ? b : f32x4_t{};
        f32x2_t v[4] = {{a[0], a[1]}, {a[2], a[3]}, {b[0], b[1]}, {b[2], b[3]}};
#pragma unroll
        for (int t = 0; t < kGemmTerms; ++t) {
            u32x4_t packed;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const bf16x2_t h = __builtin_convertvector(v[e], bf16x2_t);
                const uint32_t bits = __builtin_bit_cast(uint32_t, h);
                packed[e] = bits;
                v[e] -= f32x2_t{bf16_lo(bits), bf16_hi(bits)};
            }
            *reinterpret_cast<u32x4_t*>(&Xb[buf][t][xr][xc]) = packed;
        }
    };

    const int last = nsteps - 1;
    bf16x8_t ring[kGemmRing][CW];
#pragma unroll
    for (int u = 0; u < kGemmRing; ++u)
#pragma unroll
        for (int c = 0; c < CW; ++c) ring[u][c] = load_w(min(u, last), c);
    // acc[mt]: element i is row m0 + 16 mt + r16, column n0 + 4 g + i.  Term
    // by term, the four row blocks in turn: consecutive MFMAs write
    // different accumulators (each accumulator still adds its terms in
    // order 0, 1, 2).
    f32x4_t acc[kMaxRows / 16][CW] = {};
    auto mfma_step = [&](const bf16x8_t (&wf)[CW], int buf) {
#pragma unroll
        for (int t = 0; t < kGemmTerms; ++t)
#pragma unroll
            for (int mt = 0; mt < kMaxRows / 16; ++mt) {
                const bf16x8_t xf = *reinterpret_cast<const bf16x8_t*>(&Xb[buf][t][16 * mt + r16][8 * g]);
#pragma unroll
                for (int c = 0; c < CW; ++c)
                    acc[mt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[c], xf, acc[mt][c], 0, 0, 0);
            }
    };
    static_assert(kGemmRing % kGemmXRing == 0, "the X ring index follows the unrolled W ring index");
    // xr_a/xr_b[i]: the X block of the step s with s % kGemmXRing == i.
    f32x4_t xr_a[kGemmXRing], xr_b[kGemmXRing];
#pragma unroll
    for (int i = 0; i < kGemmXRing; ++i) load_x(min(i, last), xr_a[i], xr_b[i]);
    store_x(0, xr_a[0], xr_b[0]);
    __syncthreads();

    // Step j = j0 + u, with u = j % kGemmRing known at compile time.
    auto step = [&](int j, int u) {
        const int buf = u & 1;       // kGemmRing is even, so j & 1 == u & 1
        bf16x8_t wf[CW];
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            wf[c] = ring[u][c];
            ring[u][c] = load_w(min(j + kGemmRing, last), c);
        }
        mfma_step(wf, buf);
        // the other buffer was last read before the previous barrier
        const int nx = (u + 1) % kGemmXRing;
        if (j + 1 < nsteps) store_x(buf ^ 1, xr_a[nx], xr_b[nx]);
        // slot u % kGemmXRing held step j, stored one step ago
        const int cx = u % kGemmXRing;
        load_x(min(j + kGemmXRing, last), xr_a[cx], xr_b[cx]);
        lds_barrier();
    };
    // Whole groups of kGemmRing steps with no exit inside (an exit after each
    // step made the compiler wait there for the loads its epilogue's
    // registers were still receiving), then the last partial group.
    const int full = nsteps / kGemmRing * kGemmRing;
    for (int j0 = 0; j0 < full; j0 += kGemmRing) {
#pragma unroll
        for (int u = 0; u < kGemmRing; ++u) step(j0 + u, u);
    }
#pragma unroll
    for (int u = 0; u < kGemmRing; ++u) {
        if (full + u >= nsteps) break;
        step(full + u, u);
    }
    float* out = P + (size_t)blockIdx.y * M * N + (size_t)m0 * N + n0 + 4 * g;
#pragma unroll
    for (int mt = 0; mt < kMaxRows / 16; ++mt) {
        const int m = 16 * mt + r16;
        if (m < Mt) {
#pragma unroll
            for (int c = 0; c < CW; ++c) *reinterpret_cast<f32x4_t*>(out + (size_t)m * N + 16 * c) = acc[mt][c];
        }
    }
}

// Sum of the split-K partials of elements (m, n .. n+3), in split order; the
// loads of 8 splits are issued together.
__device__ __forceinline__ float4 psum4(const float* P, int S, int M, int N, int m, int n) {
    const size_t split = (size_t)M * N;
    const float* p = P + (size_t)m * N + n;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    int i = 0;
    for (; i + 8 <= S; i += 8) {
        float4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = *reinterpret_cast<const float4*>(p + (i + u) * split);
#pragma unroll
        for (int u = 0; u < 8; ++u) { s.x += v[u].x; s.y += v[u].y; s.z += v[u].z; s.w += v[u].w; }
    }
    for (; i < S; ++i) {
        const float4 v = *reinterpret_cast<const float4*>(p + i * split);
        s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    return s;
}

// x[m] += projection output; h[m] = rms_norm(x[m]) * w (the next block's norm).
// One workgroup per row; H <= 4096 and a multiple of 4.
__global__ void __launch_bounds__(256)
residual_norm_kernel(const float* P, int S, int M, int H, float* x, const float* w, float eps, float* h) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    float* xr = x + (size_t)m * H;
    float4 xv[4];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int n = (c * 256 + threadIdx.x) * 4;
        if (n < H) {
            const float4 y = psum4(P, S, M, H, m, n);
            float4 t = *reinterpret_cast<const float4*>(xr + n);
            t.x += y.x; t.y += y.y; t.z += y.z; t.w += y.w;
            *reinterpret_cast<float4*>(xr + n) = t;
            xv[c] = t;
            ss += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
        }
    }
    ss = block_sum(ss, red);
    const float rms = sqrtf(ss / (float)H + eps);
    float* hr = h + (size_t)m * H;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int n = (c * 256 + threadIdx.x) * 4;
        if (n < H) {
            const float4 wv = *reinterpret_cast<const float4*>(w + n);
            *reinterpret_cast<float4*>(hr + n) = make_float4((xv[c].x / rms) * wv.x, (xv[c].y / rms) * wv.y,
                                                             (xv[c].z / rms) * wv.z, (xv[c].w / rms) * wv.w);
        }
    }
}

// act[m][i] = silu(gate) * up, silu(g) = g * (1 / (1 + exp(-g))) (qwen3_ops.cpp:287).
__global__ void __launch_bounds__(256) swiglu_kernel(const float* P, int S, int M, int I, float* act) {
    const size_t groups = (size_t)M * (I / 4);
    for (size_t e = (size_t)blockIdx.x * blockDim.x + threadIdx.x; e < groups; e += (size_t)gridDim.x * blockDim.x) {
        const int m = (int)(e / (I / 4)), i = (int)(e % (I / 4)) * 4;
        const float4 g = psum4(P, S, M, 2 * I, m, i);
        const float4 u = psum4(P, S, M, 2 * I, m, I + i);
        const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
        float r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = gv[j] * (1.0f / (1.0f + expf(-gv[j]))) * uv[j];
        *reinterpret_cast<float4*>(act + (size_t)m * I + i) = make_float4(r[0], r[1], r[2], r[3]);
    }
}

// ---------------------------------------------------------------------------
// Greedy argmax over the vocabulary (lowest index among equal maxima).
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) { return v > bv || (v == bv && i < bi); }

__device__ __forceinline__ void block_argmax(float& v, int& idx, float* sv, int* si) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (better(ov, oi, v, idx)) { v = ov; idx = oi; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { sv[wave] = v; si[wave] = idx; }
    __syncthreads();
    v = sv[0]; idx = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
        if (better(sv[w], si[w], v, idx)) { v = sv[w]; idx = si[w]; }
}

__global__ void __launch_bounds__(256)
argmax_partial_kernel(const float* logits, int V, float* pv, int32_t* pi) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int m = blockIdx.y;
    const int chunk = (V + gridDim.x - 1) / gridDim.x;
    const int b0 = blockIdx.x * chunk, b1 = min(V, b0 + chunk);
    const float* row = logits + (size_t)m * V;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = b0 + threadIdx.x; i < b1; i += blockDim.x)
        if (better(row[i], i, v, idx)) { v = row[i]; idx = i; }
    block_argmax(v, idx, sv, si);
    if (threadIdx.x == 0) { pv[m * gridDim.x + blockIdx.x] = v; pi[m * gridDim.x + blockIdx.x] = idx; }
}

__global__ void argmax_final_kernel(const float* pv, const int32_t* pi, int nb, int32_t* out) {
    const int m = blockIdx.x;
    if (threadIdx.x != 0) return;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int b = 0; b < nb; ++b)
        if (better(pv[m * nb + b], pi[m * nb + b], v, idx)) { v = pv[m * nb + b]; idx = pi[m * nb + b]; }
    out[m] = idx == 0x7fffffff ? 0 : idx;
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------
// Split-K count for an M-row projection: doubled while the grid has fewer
// than two workgroups per CU, each split keeping at least min_steps k-steps
// and the partials at most max_cols * M floats (the partial buffer).
int pick_split(int N, int K, int cus, int M = kMaxRows, int min_steps = 2, long long max_cols = 1LL << 30,
               int cw = 1) {
    const int nb = N / (kGN * cw), chunks = K / kGK, mt = (M + kMaxRows - 1) / kMaxRows;
    int s = 1;
    while (s * 2 <= 32 && (long long)nb * s * mt < 2LL * cus && chunks % (s * 2) == 0 &&
           chunks / (s * 2) >= min_steps && (long long)N * s * 2 <= max_cols)
        s *= 2;
    return s;
}

// cw: 16-column W fragments per wave (1, or 2 for 128-column workgroups).
struct Gemm { int N, K, S, cw = 1; };

sa_status gemm(const float* X, int M, const uint16_t* W, const Gemm& g, float* P, hipStream_t st) {
    const dim3 grid(g.N / (kGN * g.cw), g.S, (M + kMaxRows - 1) / kMaxRows);
    if (g.cw == 2)
        hipLaunchKernelGGL(gemm_xwt_kernel<2>, grid, dim3(256), 0, st, X, M, g.K, W, g.N, g.K / g.S, P);
    else
        hipLaunchKernelGGL(gemm_xwt_kernel<1>, grid, dim3(256), 0, st, X, M, g.K, W, g.N, g.K / g.S, P);
    SA_CHECK_LAUNCH();
    return SA_OK;
}

uint64_t stream_key(uint64_t seed, uint32_t stream) {
    return (seed * 0x9E3779B97F4A7C15ull) ^ ((uint64_t)stream << 32);
}

}  // namespace
}  // namespace sa

using namespace sa;

namespace {

struct Shapes {
    int H, I, V, Hq, Hkv, D, Nq, Nk, Nqkv;
    Gemm qkv, o, gate_up, down, lm;
};

Shapes shapes_of(const sa_qwen3_desc& d, int cus) {
    Shapes s;
    s.H = d.hidden; s.I = d.intermediate; s.V = d.vocab;
    s.Hq = d.n_q_heads; s.Hkv = d.n_kv_heads; s.D = d.head_dim;
    s.Nq = s.Hq * s.D; s.Nk = s.Hkv * s.D; s.Nqkv = s.Nq + 2 * s.Nk;
    // Decode-step projections (64 rows per tile): splits of at least 8 k-steps,
    // 4 for the 1024-column o and down projections (16 column blocks: 256
    // workgroups instead of 128).  Measured on the 28-layer B = 64 step:
    // 20.79 ms against 20.98 ms with 2-step splits everywhere (the partials'
    // traffic outweighed the extra workgroups); o/down at 4 / 8 / 16 steps
    // 20.76 / 20.78 / 21.00 ms on one box.  128-column workgroups for qkv
    // and gate_up measured slower (20.72 ms, 20.79 with 4-step splits,
    // against 20.67 ms on another box).
    s.qkv = {s.Nqkv, s.H, pick_split(s.Nqkv, s.H, cus, kMaxRows, 8)};
    const int od_steps = 4;
    s.o = {s.H, s.Nq, pick_split(s.H, s.Nq, cus, kMaxRows, od_steps)};
    s.gate_up = {2 * s.I, s.H, pick_split(2 * s.I, s.H, cus, kMaxRows, 8)};
    s.down = {s.H, s.I, pick_split(s.H, s.I, cus, kMaxRows, od_steps)};
    // lm_head: 128-column workgroups halve the activation re-reads; at
    // vocab 151936, 64 rows: 93.7 us against 111 us per call.
    s.lm = {s.V, s.H, 1, s.V % (2 * kGN) == 0 ? 2 : 1};
    return s;
}

template <class T>
sa_status dev_alloc(sa_qwen3* m, T** p, size_t count) {
    void* raw = nullptr;
    const hipError_t e = hipMalloc(&raw, std::max<size_t>(count, 1) * sizeof(T));
    if (e != hipSuccess) return fail(SA_ENOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    m->allocs.push_back(raw);
    *p = static_cast<T*>(raw);
    return SA_OK;
}

void release(sa_qwen3* m) {
    if (m->side) (void)hipStreamSynchronize(m->side);
    for (hipEvent_t e : m->events) (void)hipEventDestroy(e);
    m->events.clear();
    if (m->side) (void)hipStreamDestroy(m->side);
    m->side = nullptr;
    for (void* p : m->allocs) (void)hipFree(p);
    m->allocs.clear();
    if (m->ws) (void)hipFree(m->ws);
    m->ws = nullptr;
    if (m->ws2) (void)hipFree(m->ws2);
    m->ws2 = nullptr;
    if (m->pf) (void)hipFree(m->pf);
    m->pf = nullptr;
}

// Grow-only device buffer.
sa_status grow(void** p, size_t* have, size_t need) {
    if (need <= *have) return SA_OK;
    if (*p) SA_HIP_TRY(hipFree(*p));
    *p = nullptr;
    *have = 0;
    SA_HIP_TRY(hipMalloc(p, need));
    *have = need;
    return SA_OK;
}

// The second stream, its partial buffer and the ordering events of an
// interleaved step, made once per model (on the model's device).
sa_status make_side(sa_qwen3* m, size_t part_floats) {
    if (m->side) return SA_OK;
    if (!m->part2) {
        void* p = nullptr;
        SA_HIP_TRY(hipMalloc(&p, std::max<size_t>(part_floats, 1) * sizeof(float)));
        m->allocs.push_back(p);
        m->part2 = static_cast<float*>(p);
    }
    const size_t n_ev = 3;
    while (m->events.size() < n_ev) {
        hipEvent_t e;
        SA_HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
        m->events.push_back(e);
    }
    SA_HIP_TRY(hipStreamCreateWithFlags(&m->side, hipStreamNonBlocking));
    return SA_OK;
}

}  // namespace

extern "C" sa_status sa_qwen3_create(const sa_qwen3_desc* desc, int max_batch, sa_qwen3** out) {
    clear_error();
    if (!desc || !out) return fail(SA_EINVAL, "null argument");
    *out = nullptr;
    const sa_qwen3_desc& d = *desc;
    if (d.num_layers <= 0 || d.hidden <= 0 || d.intermediate <= 0 || d.vocab <= 0 || d.n_q_heads <= 0 ||
        d.n_kv_heads <= 0 || d.n_q_heads % d.n_kv_heads || d.max_pos <= 0)
        return fail(SA_EINVAL, "bad model shape");
    if (d.head_dim != 64 && d.head_dim != 128) return fail(SA_EINVAL, "head_dim must be 64 or 128");
    const int nq = d.n_q_heads * d.head_dim, nqkv = nq + 2 * d.n_kv_heads * d.head_dim;
    if (d.hidden % kGN || nq % kGN || nqkv % kGN || (2 * d.intermediate) % kGN || d.vocab % kGN ||
        d.hidden % kGK || nq % kGK || d.intermediate % kGK)
        return fail(SA_EINVAL, "projection sizes must be multiples of 64 (outputs) and 32 (inputs)");
    if (d.hidden > 4096) return fail(SA_EINVAL, "hidden must be at most 4096");
    if (max_batch < 1 || max_batch > kMaxBatch) return fail(SA_ERANGE, "max_batch must be in [1, 1024]");
    sa_qwen3* m = new sa_qwen3();
    m->d = d;
    m->max_batch = max_batch;
    auto cleanup = [&](sa_status s) {
        release(m);
        delete m;
        return s;
    };
    if (hipGetDevice(&m->device) != hipSuccess) return cleanup(fail(SA_EHIP, "hipGetDevice failed"));
    const Shapes s = shapes_of(d, device_cu_count());
    const size_t H = s.H, V = s.V, B = max_batch;
    sa_status st;
    if ((st = dev_alloc(m, &m->embed, V * H)) != SA_OK) return cleanup(st);
    if ((st = dev_alloc(m, &m->lm_head, V * H)) != SA_OK) return cleanup(st);
    if ((st = dev_alloc(m, &m->final_norm, H)) != SA_OK) return cleanup(st);
    m->layers.resize(d.num_layers);
    for (auto& L : m->layers) {
        if ((st = dev_alloc(m, &L.in_norm, H)) != SA_OK) return cleanup(st);
        if ((st = dev_alloc(m, &L.qkv, (size_t)s.Nqkv * H)) != SA_OK) return cleanup(st);
        if ((st = dev_alloc(m, &L.q_norm, s.D)) != SA_OK) return cleanup(st);
        if ((st = dev_alloc(m, &L.k_norm, s.D)) != SA_OK) return cleanup(st);
        if ((st = dev_alloc(m, &L.o, H * s.Nq)) != SA_OK) return cleanup(st);
        if ((st = dev_alloc(m, &L.post_norm, H)) != SA_OK) return cleanup(st);
        if ((st = dev_alloc(m, &L.gate_up, 2 * (size_t)s.I * H)) != SA_OK) return cleanup(st);
        if ((st = dev_alloc(m, &L.down, H * s.I)) != SA_OK) return cleanup(st);
    }
    const size_t half = (size_t)d.max_pos * (d.head_dim / 2);
    if ((st = dev_alloc(m, &m->rope_cos, half)) != SA_OK) return cleanup(st);
    if ((st = dev_alloc(m, &m->rope_sin, half)) != SA_OK) return cleanup(st);
    if ((st = sa_rope_table_init(m->rope_cos, m->rope_sin, d.max_pos, d.head_dim, d.rope_theta, nullptr)) != SA_OK)
        return cleanup(st);
    size_t part = 0;
    for (const Gemm* g : {&s.qkv, &s.o, &s.gate_up, &s.down}) part = std::max(part, (size_t)g->S * B * g->N);
    if ((st = dev_alloc(m, &m->x, B * H)) != SA_OK || (st = dev_alloc(m, &m->h, B * H)) != SA_OK ||
        (st = dev_alloc(m, &m->q, B * s.Nq)) != SA_OK || (st = dev_alloc(m, &m->k, B * s.Nk)) != SA_OK ||
        (st = dev_alloc(m, &m->v, B * s.Nk)) != SA_OK || (st = dev_alloc(m, &m->q_rope, B * s.Nq)) != SA_OK ||
        (st = dev_alloc(m, &m->attn, B * s.Nq)) != SA_OK || (st = dev_alloc(m, &m->act, B * s.I)) != SA_OK ||
        (st = dev_alloc(m, &m->part, part)) != SA_OK || (st = dev_alloc(m, &m->logits, B * V)) != SA_OK ||
        (st = dev_alloc(m, &m->am_val, B * kArgBlocks)) != SA_OK ||
        (st = dev_alloc(m, &m->am_idx, B * kArgBlocks)) != SA_OK)
        return cleanup(st);
    if (hipDeviceSynchronize() != hipSuccess) return cleanup(fail(SA_EHIP, "RoPE table init failed"));
    *out = m;
    return SA_OK;
}

extern "C" sa_status sa_qwen3_destroy(sa_qwen3* m) {
    clear_error();
    if (!m) return SA_OK;
    release(m);
    delete m;
    return SA_OK;
}

extern "C" sa_status sa_qwen3_get_desc(const sa_qwen3* m, sa_qwen3_desc* desc) {
    clear_error();
    if (!m || !desc) return fail(SA_EINVAL, "null argument");
    *desc = m->d;
    return SA_OK;
}

extern "C" sa_status sa_qwen3_tensor_ptr(sa_qwen3* m, int layer, sa_qwen3_tensor which, void** ptr, size_t* count,
                                         sa_dtype* dtype) {
    clear_error();
    if (!m || !ptr || !count || !dtype) return fail(SA_EINVAL, "null argument");
    const Shapes s = shapes_of(m->d, 1);
    const size_t H = s.H;
    const bool global = which == SA_QW_EMBED || which == SA_QW_FINAL_NORM || which == SA_QW_LM_HEAD;
    if (!global && (layer < 0 || layer >= m->d.num_layers)) return fail(SA_ERANGE, "layer out of range");
    const sa_qwen3::Layer* L = global ? nullptr : &m->layers[layer];
    switch (which) {
        case SA_QW_EMBED: *ptr = m->embed; *count = (size_t)s.V * H; *dtype = SA_DTYPE_BF16; break;
        case SA_QW_LM_HEAD: *ptr = m->lm_head; *count = (size_t)s.V * H; *dtype = SA_DTYPE_BF16; break;
        case SA_QW_FINAL_NORM: *ptr = m->final_norm; *count = H; *dtype = SA_DTYPE_F32; break;
        case SA_QW_IN_NORM: *ptr = L->in_norm; *count = H; *dtype = SA_DTYPE_F32; break;
        case SA_QW_QKV: *ptr = L->qkv; *count = (size_t)s.Nqkv * H; *dtype = SA_DTYPE_BF16; break;
        case SA_QW_Q_NORM: *ptr = L->q_norm; *count = s.D; *dtype = SA_DTYPE_F32; break;
        case SA_QW_K_NORM: *ptr = L->k_norm; *count = s.D; *dtype = SA_DTYPE_F32; break;
        case SA_QW_O: *ptr = L->o; *count = H * s.Nq; *dtype = SA_DTYPE_BF16; break;
        case SA_QW_POST_NORM: *ptr = L->post_norm; *count = H; *dtype = SA_DTYPE_F32; break;
        case SA_QW_GATE_UP: *ptr = L->gate_up; *count = 2 * (size_t)s.I * H; *dtype = SA_DTYPE_BF16; break;
        case SA_QW_DOWN: *ptr = L->down; *count = H * s.I; *dtype = SA_DTYPE_BF16; break;
        default: return fail(SA_EINVAL, "unknown weight tensor");
    }
    return SA_OK;
}

extern "C" sa_status sa_qwen3_init_random(sa_qwen3* m, uint64_t seed, float stdev, sa_stream_t stream) {
    clear_error();
    if (!m) return fail(SA_EINVAL, "null model");
    hipStream_t st = as_stream(stream);
    const int grid = 4 * device_cu_count();
    for (int layer = -1; layer < m->d.num_layers; ++layer) {
        for (int w = SA_QW_EMBED; w <= SA_QW_LM_HEAD; ++w) {
            const bool global = w == SA_QW_EMBED || w == SA_QW_FINAL_NORM || w == SA_QW_LM_HEAD;
            if (global != (layer < 0)) continue;
            void* p;
            size_t n;
            sa_dtype dt;
            SA_TRY(sa_qwen3_tensor_ptr(m, layer < 0 ? 0 : layer, (sa_qwen3_tensor)w, &p, &n, &dt));
            const uint32_t stream_id = 1000u + 16u * (uint32_t)(layer < 0 ? 0 : layer) + (uint32_t)w;
            const uint64_t key = stream_key(seed, stream_id);
            if (dt == SA_DTYPE_BF16)
                hipLaunchKernelGGL(init_bf16_kernel, dim3(grid), dim3(256), 0, st, static_cast<uint16_t*>(p), n, key,
                                   (double)stdev);
            else
                hipLaunchKernelGGL(init_norm_kernel, dim3(grid), dim3(256), 0, st, static_cast<float*>(p), n, key,
                                   (double)stdev);
            SA_CHECK_LAUNCH();
        }
    }
    return SA_OK;
}

// A prompt of L tokens for each of sequences 0 .. batch-1 (all empty), run
// as one causal prefill: the activations are batch * L token rows, the
// projections the same GEMMs over row tiles (split-K where the column tiles
// are few), the attention
// block q/k RMSNorm + RoPE at positions 0 .. L-1, the K/V append, and the
// causal prefill kernel over the dense token-major q/k/v.  Reference:
// qwen3_forward_with_cache with an empty cache and S = L
// (tensor_cpp/src/qwen3_ops.cpp:936-1014, layer :620-934; the prefill attention
// there is self_attention with a causal mask or
// self_attention_streaming_blockwise, :894-909).
extern "C" sa_status sa_qwen3_prefill(sa_qwen3* m, sa_kvcache* cache, const int32_t* tokens, int batch, int L,
                                      int32_t* next_tokens, float* logits, sa_stream_t stream) {
    clear_error();
    if (!m || !cache || !tokens || !next_tokens) return fail(SA_EINVAL, "null argument");
    if (batch < 1 || batch > m->max_batch) return fail(SA_ERANGE, "batch outside [1, max_batch]");
    const sa_qwen3_desc& d = m->d;
    if (L < 1 || L > d.max_pos) return fail(SA_ERANGE, "prompt length outside [1, max_pos]");
    sa_kv_desc kd;
    SA_TRY(sa_kvcache_get_desc(cache, &kd));
    if (kd.num_layers != d.num_layers || kd.num_kv_heads != d.n_kv_heads || kd.head_dim != d.head_dim)
        return fail(SA_EINVAL, "cache geometry does not match the model");
    if (batch > kd.max_seqs) return fail(SA_ERANGE, "batch exceeds the cache's sequences");
    if ((long long)L > (long long)kd.max_pages_per_seq * 64)
        return fail(SA_EFULL, "prompt longer than a sequence's page table");
    for (int i = 0; i < batch; ++i) {
        if (sa_kvcache_len(cache, i) != 0) return fail(SA_EINVAL, "prefill needs empty sequences");
        if (sa_kvcache_capacity(cache, i) < L) return fail(SA_EFULL, "KV cache full, reserve pages for the prompt");
    }
    hipStream_t st = as_stream(stream);
    const Shapes s = shapes_of(d, device_cu_count());
    const long long M = (long long)batch * L;
    if (M > 0x7fffffffLL / std::max({s.Nqkv, 2 * s.I, s.H}))
        return fail(SA_ERANGE, "batch * prompt too large");
    // Split-K only where the row tiles alone leave CUs idle (o_proj and down
    // at hidden 1024: 16 column tiles; measured for a 512-token prompt at the
    // Qwen3-0.6B shape, 61.7 us per call unsplit), with at least 8 k-steps
    // per split and the partials within the qkv / gate_up width.
    const int cus = device_cu_count();
    const long long part_cols = std::max({s.Nqkv, 2 * s.I, s.H});
    const int m_rows = (int)std::min<long long>(M, 0x7fffffff);
    // 128-column workgroups (each X fragment read from LDS feeds two MFMAs)
    // for prompts of more than four 64-row blocks, 64 columns below.
    // Measured at the Qwen3-0.6B shape through benchmark_qwen3 (tok/s, same
    // box, interleaved; 64 / 128 columns): 128 tokens 42,100 / 35,900, 256:
    // 73,200 / 67,200, 384: 88,000 / 89,700, 512: 107,800 / 111,500, 1024:
    // 128,100 / 141,100, 2048: 118,800 / 133,300.  Shorter prompts give
    // 128-column grids too few workgroups once split-K keeps its minimum
    // k-steps per split.
    auto shape = [&](int N, int K) {
        const int cw = m_rows > 4 * kMaxRows && N % (2 * kGN) == 0 ? 2 : 1;
        return Gemm{N, K, pick_split(N, K, cus, m_rows, 8, part_cols, cw), cw};
    };
    const Gemm g_qkv = shape(s.Nqkv, s.H);
    const Gemm g_o = shape(s.H, s.Nq);
    const Gemm g_gu = shape(2 * s.I, s.H);
    const Gemm g_down = shape(s.H, s.I);

    // activations of the M token rows, carved from one grow-only buffer
    const size_t f_x = M * s.H, f_q = M * s.Nq, f_k = M * s.Nk, f_act = M * s.I;
    const size_t f_part = M * part_cols;
    // the attention's workspace (paired key ranges of short prompts) after
    // the activations, at a 256-byte boundary
    const size_t ws_attn = sa_prefill_causal_ws_bytes(SA_DTYPE_F32, batch, s.Hq, s.Hkv, L, s.D);
    const size_t f_act_all = (2 * f_x + 2 * f_q + 2 * f_k + f_act + f_part + (size_t)batch * s.H + 63) / 64 * 64;
    const size_t floats = f_act_all + (ws_attn + 255) / 256 * 64;
    const size_t need = floats * sizeof(float);
    if (need > m->pf_bytes) {
        if (m->pf) SA_HIP_TRY(hipFree(m->pf));
        m->pf = nullptr;
        m->pf_bytes = 0;
        if (hipMalloc(&m->pf, need) != hipSuccess) return fail(SA_ENOMEM, "prefill activations");
        m->pf_bytes = need;
    }
    float* x = static_cast<float*>(m->pf);
    float* h = x + f_x;
    float* q = h + f_x;
    float* attn = q + f_q;
    float* k = attn + f_q;
    float* v = k + f_k;
    float* act = v + f_k;
    float* part = act + f_act;
    float* h_last = part + f_part;
    float* attn_ws = ws_attn ? static_cast<float*>(m->pf) + f_act_all : nullptr;
    const float eps = d.rms_eps;
    const float scale = 1.0f / sqrtf((float)d.head_dim);
    float* out_logits = logits ? logits : m->logits;

    hipLaunchKernelGGL(embed_norm_kernel, dim3((unsigned)M), dim3(256), 0, st, m->embed, tokens, s.V, s.H,
                       m->layers[0].in_norm, eps, x, h);
    SA_CHECK_LAUNCH();
    const int ew_grid = (int)std::min<long long>(4LL * device_cu_count(), (M * s.I / 4 + 255) / 256);
    const int64_t q_str[3] = {(int64_t)L * s.Nq, s.D, s.Nq};
    const int64_t kv_str[3] = {(int64_t)L * s.Nk, s.D, s.Nk};
    for (int l = 0; l < d.num_layers; ++l) {
        const sa_qwen3::Layer& Ly = m->layers[l];
        // ---- attention block ----
        SA_TRY(gemm(h, (int)M, Ly.qkv, g_qkv, part, st));
        // q, k, v summed from the projection's split-K partials, q and k
        // normed and rotated (positions 0 .. L-1: the cache is empty), K and V
        // appended to the cache, q, k, v written for the attention: one launch.
        SA_TRY(qknorm_rope_append_partials(cache, l, part, g_qkv.S, batch, L, s.Hq, Ly.q_norm, Ly.k_norm, eps,
                                           m->rope_cos, m->rope_sin, d.max_pos, q, k, v, st));
        SA_TRY(sa_prefill_causal_strided_ws(q, k, v, SA_DTYPE_F32, batch, s.Hq, s.Hkv, L, s.D, q_str, kv_str, q_str,
                                            scale, attn, attn_ws, ws_attn, stream));
        SA_TRY(gemm(attn, (int)M, Ly.o, g_o, part, st));
        hipLaunchKernelGGL(residual_norm_kernel, dim3((unsigned)M), dim3(256), 0, st, part, g_o.S, (int)M, s.H, x,
                           Ly.post_norm, eps, h);
        SA_CHECK_LAUNCH();
        // ---- MLP ----
        SA_TRY(gemm(h, (int)M, Ly.gate_up, g_gu, part, st));
        hipLaunchKernelGGL(swiglu_kernel, dim3(ew_grid), dim3(256), 0, st, part, g_gu.S, (int)M, s.I, act);
        SA_CHECK_LAUNCH();
        SA_TRY(gemm(act, (int)M, Ly.down, g_down, part, st));
        const float* next_norm = l + 1 < d.num_layers ? m->layers[l + 1].in_norm : m->final_norm;
        hipLaunchKernelGGL(residual_norm_kernel, dim3((unsigned)M), dim3(256), 0, st, part, g_down.S, (int)M, s.H,
                           x, next_norm, eps, h);
        SA_CHECK_LAUNCH();
    }
    // ---- the last position of each sequence: lm_head, greedy argmax ----
    SA_HIP_TRY(hipMemcpy2DAsync(h_last, (size_t)s.H * sizeof(float), h + (size_t)(L - 1) * s.H,
                                (size_t)L * s.H * sizeof(float), (size_t)s.H * sizeof(float), batch,
                                hipMemcpyDeviceToDevice, st));
    SA_TRY(gemm(h_last, batch, m->lm_head, s.lm, out_logits, st));
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks, batch), dim3(256), 0, st, out_logits, s.V, m->am_val,
                       m->am_idx);
    SA_CHECK_LAUNCH();
    hipLaunchKernelGGL(argmax_final_kernel, dim3(batch), dim3(64), 0, st, m->am_val, m->am_idx, kArgBlocks,
                       next_tokens);
    SA_CHECK_LAUNCH();
    return sa_kvcache_commit(cache, nullptr, batch, L, stream);
}

extern "C" sa_status sa_qwen3_decode_step(sa_qwen3* m, sa_kvcache* cache, const int32_t* tokens, int batch,
                                          int32_t* next_tokens, float* logits, sa_stream_t stream) {
    clear_error();
    if (!m || !cache || !tokens || !next_tokens) return fail(SA_EINVAL, "null argument");
    if (batch < 1 || batch > m->max_batch) return fail(SA_ERANGE, "batch outside [1, max_batch]");
    sa_kv_desc kd;
    SA_TRY(sa_kvcache_get_desc(cache, &kd));
    const sa_qwen3_desc& d = m->d;
    if (kd.num_layers != d.num_layers || kd.num_kv_heads != d.n_kv_heads || kd.head_dim != d.head_dim)
        return fail(SA_EINVAL, "cache geometry does not match the model");
    if (batch > kd.max_seqs) return fail(SA_ERANGE, "batch exceeds the cache's sequences");
    for (int i = 0; i < batch; ++i) {
        const int len = sa_kvcache_len(cache, i);
        if (len < 0 || len >= d.max_pos) return fail(SA_ERANGE, "position outside the RoPE table");
        if (len + 1 > sa_kvcache_capacity(cache, i)) return fail(SA_EFULL, "KV cache full, cannot append more tokens");
    }
    hipStream_t st = as_stream(stream);
    const size_t need = sa_paged_decode_ws_bytes(cache, batch, d.n_q_heads);
    SA_TRY(grow(&m->ws, &m->ws_bytes, need));
    const Shapes s = shapes_of(d, device_cu_count());
    const int M = batch;
    const float eps = d.rms_eps;
    const float scale = 1.0f / sqrtf((float)d.head_dim);
    float* out_logits = logits ? logits : m->logits;

    // Rows [r0, r0 + n) of the batch on one stream: its own split-K partials
    // and decode workspace; x, h, attn and act rows at the same offsets.
    struct Rows {
        int r0, n;
        float* part;
        void* ws;
        size_t ws_bytes;
        hipStream_t st;
        std::vector<int32_t> ids;
    };
    const int ew_grid_full = std::min(4 * device_cu_count(), (M * s.I / 4 + 255) / 256);
    auto qkv = [&](const Rows& r, int l) {
        return gemm(m->h + (size_t)r.r0 * s.H, r.n, m->layers[l].qkv, s.qkv, r.part, r.st);
    };
    // The split-K sum of the projection, q/k norm + RoPE, the K/V append and
    // the paged decode in one launch per 64 sequences (plus the LSE merge of
    // multi-chunk sequences); the last layer's call also commits the token.
    // (A separate split kernel cost 4.7 us per layer.)
    auto attention = [&](const Rows& r, int l) {
        const sa_qwen3::Layer& L = m->layers[l];
        return sa::append_decode_partials(cache, l, r.part, s.qkv.S, r.n, r.ids.data(), s.Hq, L.q_norm, L.k_norm,
                                          eps, m->rope_cos, m->rope_sin, d.max_pos, scale,
                                          m->attn + (size_t)r.r0 * s.Nq, nullptr, r.ws, r.ws_bytes,
                                          l + 1 == d.num_layers ? 1 : 0, r.st);
    };
    // o projection, residual + norm, MLP, residual + the next block's norm.
    auto rest = [&](const Rows& r, int l) -> sa_status {
        const sa_qwen3::Layer& L = m->layers[l];
        float* x = m->x + (size_t)r.r0 * s.H;
        float* h = m->h + (size_t)r.r0 * s.H;
        float* act = m->act + (size_t)r.r0 * s.I;
        SA_TRY(gemm(m->attn + (size_t)r.r0 * s.Nq, r.n, L.o, s.o, r.part, r.st));
        hipLaunchKernelGGL(residual_norm_kernel, dim3(r.n), dim3(256), 0, r.st, r.part, s.o.S, r.n, s.H, x,
                           L.post_norm, eps, h);
        SA_CHECK_LAUNCH();
        SA_TRY(gemm(h, r.n, L.gate_up, s.gate_up, r.part, r.st));
        const int ew_grid = std::min(ew_grid_full, (r.n * s.I / 4 + 255) / 256);
        hipLaunchKernelGGL(swiglu_kernel, dim3(ew_grid), dim3(256), 0, r.st, r.part, s.gate_up.S, r.n, s.I, act);
        SA_CHECK_LAUNCH();
        SA_TRY(gemm(act, r.n, L.down, s.down, r.part, r.st));
        const float* next_norm = l + 1 < d.num_layers ? m->layers[l + 1].in_norm : m->final_norm;
        hipLaunchKernelGGL(residual_norm_kernel, dim3(r.n), dim3(256), 0, r.st, r.part, s.down.S, r.n, s.H, x,
                           next_norm, eps, h);
        SA_CHECK_LAUNCH();
        return SA_OK;
    };

    hipLaunchKernelGGL(embed_norm_kernel, dim3(M), dim3(256), 0, st, m->embed, tokens, s.V, s.H,
                       m->layers[0].in_norm, eps, m->x, m->h);
    SA_CHECK_LAUNCH();
    // Interleaving: with enough context, the batch runs as two half-batches
    // on two streams, the second starting its first attention when the
    // first half's ends.  From then on the halves run free, half a layer
    // apart: each half's projections, norms and MLP (latency-bound launches)
    // run while the other half's attention streams the cache, and each
    // attention launch's tail overlaps the other's.  The halves split the
    // cached tokens evenly; SA_DECODE_INTERLEAVE=0 / 1 forces it off / on.
    // Measured on the 28-layer, 64-sequence bf16 step (979-31,078 tokens,
    // same box): 19.61 ms against 20.48 ms on one stream; with the halves'
    // attention launches strictly alternating (an event wait before each),
    // 20.78 ms: a cross-stream wait costs ~12 us and each half-batch launch
    // has a tail of its own.
    long long total = 0;
    std::vector<long long> prefix(M + 1, 0);
    for (int i = 0; i < M; ++i) prefix[i + 1] = prefix[i] + sa_kvcache_len(cache, i) + 1;
    total = prefix[M];
    const int kv_elem = kd.kv_dtype == SA_DTYPE_BF16 ? 2 : 4;
    const long long attn_bytes = total * d.n_kv_heads * d.head_dim * 2LL * kv_elem;
    const char* fenv = std::getenv("SA_DECODE_INTERLEAVE");
    const bool interleave = M >= 2 && (fenv ? std::atoi(fenv) != 0 : attn_bytes >= kInterleaveBytes);
    if (!interleave) {
        Rows all{0, M, m->part, m->ws, m->ws_bytes, st, {}};
        for (int i = 0; i < M; ++i) all.ids.push_back(i);
        for (int l = 0; l < d.num_layers; ++l) {
            SA_TRY(qkv(all, l));
            SA_TRY(attention(all, l));
            SA_TRY(rest(all, l));
        }
    } else {
        size_t part_floats = 0;
        for (const Gemm* g : {&s.qkv, &s.o, &s.gate_up, &s.down})
            part_floats = std::max(part_floats, (size_t)g->S * m->max_batch * g->N);
        SA_TRY(make_side(m, part_floats));
        SA_TRY(grow(&m->ws2, &m->ws2_bytes, need));
        int cut = 1;
        while (cut < M - 1 && 2 * prefix[cut] < total) ++cut;
        Rows a{0, cut, m->part, m->ws, m->ws_bytes, st, {}};
        Rows b{cut, M - cut, m->part2, m->ws2, m->ws2_bytes, m->side, {}};
        for (int i = 0; i < M; ++i) (i < cut ? a.ids : b.ids).push_back(i);
        hipEvent_t fork = m->events[0], join = m->events[1], a_first = m->events[2];
        SA_HIP_TRY(hipEventRecord(fork, st));
        SA_HIP_TRY(hipStreamWaitEvent(m->side, fork, 0));
        auto layers = [&]() -> sa_status {
            SA_TRY(qkv(a, 0));
            SA_TRY(qkv(b, 0));
            for (int l = 0; l < d.num_layers; ++l) {
                SA_TRY(attention(a, l));
                if (l == 0) SA_HIP_TRY(hipEventRecord(a_first, st));
                SA_TRY(rest(a, l));
                if (l + 1 < d.num_layers) SA_TRY(qkv(a, l + 1));
                if (l == 0) SA_HIP_TRY(hipStreamWaitEvent(m->side, a_first, 0));
                SA_TRY(attention(b, l));
                SA_TRY(rest(b, l));
                if (l + 1 < d.num_layers) SA_TRY(qkv(b, l + 1));
            }
            return SA_OK;
        };
        const sa_status ls = layers();
        // Joined on failure too, so the caller's stream orders after whatever
        // the side stream was given.
        SA_HIP_TRY(hipEventRecord(join, m->side));
        SA_HIP_TRY(hipStreamWaitEvent(st, join, 0));
        if (ls != SA_OK) return ls;
    }
    // ---- final norm (folded above), lm_head, greedy argmax ----
    SA_TRY(gemm(m->h, M, m->lm_head, s.lm, out_logits, st));
    hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgBlocks, M), dim3(256), 0, st, out_logits, s.V, m->am_val,
                       m->am_idx);
    SA_CHECK_LAUNCH();
    hipLaunchKernelGGL(argmax_final_kernel, dim3(M), dim3(64), 0, st, m->am_val, m->am_idx, kArgBlocks,
                       next_tokens);
    SA_CHECK_LAUNCH();
    return SA_OK;   // the last layer's sa_append_decode committed the token
}
