// Internal helpers shared by the gfx950 kernels and the C ABI glue.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "sa_amd.h"

namespace sa {

// ---------------------------------------------------------------------------
// Host-side error reporting: one message per thread, returned by sa_last_error.
// ---------------------------------------------------------------------------
void set_error(const std::string& msg);
void clear_error();
sa_status fail(sa_status st, const std::string& msg);
sa_status hip_fail(hipError_t e, const char* what);
int device_cu_count();

// Process-wide tile settings (sa_set_attention_blocks); 0 = the launch's own
// choice.  q: query rows per prefill workgroup and head; kv: tokens per
// split-KV chunk of decode attention.
int attn_q_block();
int attn_kv_block();

#define SA_HIP_TRY(expr)                                   \
    do {                                                   \
        hipError_t _e = (expr);                            \
        if (_e != hipSuccess) return ::sa::hip_fail(_e, #expr); \
    } while (0)

#define SA_TRY(expr)                                       \
    do {                                                   \
        sa_status _s = (expr);                             \
        if (_s != SA_OK) return _s;                        \
    } while (0)

#define SA_CHECK_LAUNCH()                                  \
    do {                                                   \
        hipError_t _e = hipGetLastError();                 \
        if (_e != hipSuccess) return ::sa::hip_fail(_e, "kernel launch"); \
    } while (0)

inline hipStream_t as_stream(sa_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
constexpr int kWave = 64;

// bf16 is stored as raw uint16 bits; widening is exact.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16 with round-to-nearest-even; NaN stays a quiet NaN.
__host__ __device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// DPP lane exchanges inside a row of 16 lanes.  After a full-group sum/max the
// values are uniform inside each group, so mirror patterns act as xor 4 / 8.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within 16

// Lane i <-> i ^ M within 32 lanes (ds_swizzle bit mode: and_mask 0x1f,
// or_mask 0, xor_mask M).
template <int M>
__device__ __forceinline__ float swz_xor(float v) {
    static_assert(M > 0 && M < 32, "ds_swizzle xor masks stay inside 32 lanes");
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (M << 10) | 0x1F));
}
__device__ __forceinline__ float swz_xor16(float v) { return swz_xor<16>(v); }
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// waits for every outstanding global access of the wave (s_waitcnt
// vmcnt(0)), which drains loads issued ahead of their use; here they stay in
// flight and the compiler waits for each where its value is used.  For
// kernels whose waves exchange data through LDS only.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

struct OpSum { __device__ static float apply(float a, float b) { return a + b; } };
struct OpMax { __device__ static float apply(float a, float b) { return fmaxf(a, b); } };

// Reduce over lane groups: combine across the xor masks FROM, 2*FROM, ... < TO.
// With FROM = 1 the result is the reduction over aligned groups of TO lanes,
// uniform inside each group.  FROM > 1 is only valid when values are already
// uniform inside groups of FROM lanes.
template <class Op, int FROM, int TO>
__device__ __forceinline__ float group_reduce(float v) {
    if constexpr (FROM <= 1 && TO > 1) v = Op::apply(v, dpp<kDppXor1>(v));
    if constexpr (FROM <= 2 && TO > 2) v = Op::apply(v, dpp<kDppXor2>(v));
    if constexpr (FROM <= 4 && TO > 4) v = Op::apply(v, dpp<kDppHalfMirror>(v));
    if constexpr (FROM <= 8 && TO > 8) v = Op::apply(v, dpp<kDppMirror>(v));
    if constexpr (FROM <= 16 && TO > 16) v = Op::apply(v, swz_xor16(v));
    if constexpr (FROM <= 32 && TO > 32) v = Op::apply(v, xor32(v));
    return v;
}

// The same reduction for values that differ inside the groups of FROM lanes
// (say, one column of a row per lane): every step pairs lane i with lane
// i ^ mask, so lanes are combined only with lanes of the same position in
// their group.
template <class Op, int FROM, int TO>
__device__ __forceinline__ float group_reduce_xor(float v) {
    if constexpr (FROM <= 1 && TO > 1) v = Op::apply(v, dpp<kDppXor1>(v));
    if constexpr (FROM <= 2 && TO > 2) v = Op::apply(v, dpp<kDppXor2>(v));
    if constexpr (FROM <= 4 && TO > 4) v = Op::apply(v, swz_xor<4>(v));
    if constexpr (FROM <= 8 && TO > 8) v = Op::apply(v, swz_xor<8>(v));
    if constexpr (FROM <= 16 && TO > 16) v = Op::apply(v, swz_xor<16>(v));
    if constexpr (FROM <= 32 && TO > 32) v = Op::apply(v, xor32(v));
    return v;
}

// One head row held by a wave as rotate-half pairs: lane j owns elements
// i and i + D/2 for i = j, j + 64, ...
template <int D>
struct RowPairs {
    static constexpr int H = D / 2;
    static constexpr int NP = (H + kWave - 1) / kWave;
    float lo[NP], hi[NP];

    __device__ __forceinline__ void load(const float* x, int lane) {
#pragma unroll
        for (int c = 0; c < NP; ++c) {
            const int i = lane + c * kWave;
            lo[c] = (i < H) ? x[i] : 0.f;
            hi[c] = (i < H) ? x[i + H] : 0.f;
        }
    }
    // The row as the sum, in split order, of S split-K partial rows
    // x[s * split] .. (s = 0 .. S-1).
    __device__ __forceinline__ void load_sum(const float* x, size_t split, int S, int lane) {
#pragma unroll
        for (int c = 0; c < NP; ++c) {
            const int i = lane + c * kWave;
            float a = 0.f, b = 0.f;
            if (i < H) {
                for (int t = 0; t < S; ++t) {
                    a += x[t * split + i];
                    b += x[t * split + i + H];
                }
            }
            lo[c] = a;
            hi[c] = b;
        }
    }
    // y = (x / sqrt(mean(x^2) + eps)) * w, eps inside the sqrt (reference
    // tensor_cpp/src/qwen3_ops.cpp:716-717), or with eps_outside
    // y = (x / (sqrt(mean(x^2)) + eps)) * w, as the reference's AVX2 layer
    // (tensor_cpp/src/qwen3_ops_avx.cpp:537, :566).
    __device__ __forceinline__ void rms_norm(const float* w, float eps, int lane, bool eps_outside = false) {
        float wl[NP], wh[NP];
        load_pairs(w, lane, wl, wh);
        rms_norm_with(wl, wh, eps, eps_outside);
    }
    // The same with this lane's weight pairs already loaded (load_pairs).
    // Products and sums are rounded as written (no contraction), so every
    // kernel that uses these rows computes the same bits.
    __device__ __forceinline__ void rms_norm_with(const float (&wl)[NP], const float (&wh)[NP], float eps,
                                                  bool eps_outside = false) {
#pragma clang fp contract(off)
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < NP; ++c) ss = fmaf(lo[c], lo[c], fmaf(hi[c], hi[c], ss));
        ss = group_reduce<OpSum, 1, kWave>(ss);
        const float rms = eps_outside ? sqrtf(ss / (float)D) + eps : sqrtf(ss / (float)D + eps);
#pragma unroll
        for (int c = 0; c < NP; ++c) {
            lo[c] = (lo[c] / rms) * wl[c];
            hi[c] = (hi[c] / rms) * wh[c];
        }
    }
    // x' = x cos + rotate_half(x) sin with rotate_half(x) = [-x2, x1], cos/sin
    // of row pos (reference tensor_cpp/src/qwen3_ops.cpp:30-64, 110-188).
    __device__ __forceinline__ void rope(const float* cos_t, const float* sin_t, int pos, int lane) {
        float cs[NP], sn[NP];
        load_row(cos_t + (size_t)pos * H, lane, cs);
        load_row(sin_t + (size_t)pos * H, lane, sn);
        rope_with(cs, sn);
    }
    // The same with this lane's cos/sin already loaded (load_row of row pos).
    __device__ __forceinline__ void rope_with(const float (&cs)[NP], const float (&sn)[NP]) {
#pragma clang fp contract(off)
#pragma unroll
        for (int c = 0; c < NP; ++c) {
            const float l2 = lo[c] * cs[c] - hi[c] * sn[c];
            const float h2 = hi[c] * cs[c] + lo[c] * sn[c];
            lo[c] = l2;
            hi[c] = h2;
        }
    }
    // This lane's elements i and i + D/2 (i = lane, lane + 64, ...) of x[D].
    __device__ static __forceinline__ void load_pairs(const float* x, int lane, float (&l)[NP], float (&h)[NP]) {
#pragma unroll
        for (int c = 0; c < NP; ++c) {
            const int i = lane + c * kWave;
            l[c] = (i < H) ? x[i] : 0.f;
            h[c] = (i < H) ? x[i + H] : 0.f;
        }
    }
    // This lane's elements i = lane, lane + 64, ... of a row of D/2.
    __device__ static __forceinline__ void load_row(const float* x, int lane, float (&v)[NP]) {
#pragma unroll
        for (int c = 0; c < NP; ++c) {
            const int i = lane + c * kWave;
            v[c] = (i < H) ? x[i] : 0.f;
        }
    }
    __device__ __forceinline__ void store(float* y, int lane) const {
#pragma unroll
        for (int c = 0; c < NP; ++c) {
            const int i = lane + c * kWave;
            if (i < H) { y[i] = lo[c]; y[i + H] = hi[c]; }
        }
    }
};

// Cache rows of the sequences of one launch, passed by value in the kernel
// arguments (the host has checked every one of them against the page table).
constexpr int kRowsPerLaunch = 64;
struct RowList {
    int32_t row[kRowsPerLaunch];
};

// ---------------------------------------------------------------------------
// Entry points implemented in decode.hip, used by the cache glue.
// ---------------------------------------------------------------------------
struct PagedView {
    const void* k_pool;
    const void* v_pool;
    const int32_t* block_table;
    const int32_t* seq_lens;
    int n_kv, d, max_pages, num_pages;
    bool bf16;
};

// sa_qknorm_rope_append with an optional k_out: K normed and rotated, as
// q_out receives q (either may alias its input).
sa_status qknorm_rope_append(sa_kvcache* c, int layer, const float* q, const float* k, const float* v, int n_seq,
                             int S, const int32_t* seq_ids, int n_q_heads, const float* q_norm_w,
                             const float* k_norm_w, float eps, const float* rope_cos, const float* rope_sin,
                             int rope_max_pos, float* q_out, float* k_out, hipStream_t st);

// The same with q, k and v read as the sum of n_part split-K partials of a
// [n_seq * S][(n_q_heads + 2 n_kv) * D] projection (q columns, then k, then
// v; partial t at part + t * rows * cols), and v written to v_out as well.
sa_status qknorm_rope_append_partials(sa_kvcache* c, int layer, const float* part, int n_part, int n_seq, int S,
                                      int n_q_heads, const float* q_norm_w, const float* k_norm_w, float eps,
                                      const float* rope_cos, const float* rope_sin, int rope_max_pos, float* q_out,
                                      float* k_out, float* v_out, hipStream_t st);

// sa_append_decode with q, k and v read from split-K partials (FusedAppend).
sa_status append_decode_partials(sa_kvcache* c, int layer, const float* part, int n_part, int n_seq,
                                 const int32_t* seq_ids, int n_q_heads, const float* q_norm_w,
                                 const float* k_norm_w, float eps, const float* rope_cos, const float* rope_sin,
                                 int rope_max_pos, float scale, float* out, float* q_out, void* ws,
                                 size_t ws_bytes, int commit, hipStream_t st);

size_t paged_ws(int n_seq, int n_q, int n_kv, int d, int max_pages);
// seq_ids: host array of cache rows (NULL: 0 .. n_seq-1), already checked.
// lens: the rows' committed lengths (host array in call order, the page
// table's mirror): the launches read them instead of the device lengths and
// size their grids to the chunks that hold tokens.
sa_status decode_paged(const PagedView& c, const float* q, int n_seq, const int32_t* seq_ids,
                       const int32_t* lens, int n_q, int n_pending, int max_len, long long total_len,
                       float scale, float* out, void* ws, size_t ws_bytes, hipStream_t st);

// The append half of a fused decode step: the new token of every sequence
// (raw q [n_seq][n_q][D] is decode_paged's q; k, v [n_seq][n_kv][D]), its
// per-head RMSNorm weights (NULL: none) and RoPE tables (NULL: none), the
// position of the token in each sequence (its committed length, host array
// in call order), and whether to commit it (seq_lens[row] = pos + 1).
struct FusedAppend {
    const float* k;
    const float* v;
    const float* wq;
    const float* wk;
    float eps;
    const float* cos_t;
    const float* sin_t;
    int rope_max_pos;
    float* q_out;              // NULL, or receives the normed, rotated q
    int32_t* lens;             // the cache's device lengths (written on commit)
    const int32_t* pos;        // host, [n_seq]
    bool commit;
    // Optional: q, k and v (then unused) read as the sum of part_S split-K
    // partials of an [part_M][(n_q + 2 n_kv) * D] projection (q columns, then
    // k, then v; partial t at part + t * part_M * cols), row i for sequence i.
    const float* part = nullptr;
    int part_S = 0;
    int part_M = 0;
};

// decode_paged with the step's append folded in: one launch per
// kRowsPerLaunch sequences when every sequence fits one chunk, plus the LSE
// merge launch otherwise.  max_len / total_len count the new token.
sa_status decode_paged_fused(const PagedView& c, const float* q, int n_seq, const int32_t* seq_ids, int n_q,
                             const FusedAppend& f, int max_len, long long total_len, float scale, float* out,
                             void* ws, size_t ws_bytes, hipStream_t st);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace sa
