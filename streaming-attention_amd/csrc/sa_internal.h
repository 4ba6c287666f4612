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

__device__ __forceinline__ float swz_xor16(float v) {
    // ds_swizzle bit mode: and_mask 0x1f, or_mask 0, xor_mask 0x10
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ float xor32(float v) { return __shfl_xor(v, 32, 64); }

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

size_t paged_ws(int n_seq, int n_q, int n_kv, int d, int max_pages);
// seq_ids: host array of cache rows (NULL: 0 .. n_seq-1), already checked.
sa_status decode_paged(const PagedView& c, const float* q, int n_seq, const int32_t* seq_ids,
                       int n_q, int n_pending, int max_len, long long total_len, float scale,
                       float* out, void* ws, size_t ws_bytes, hipStream_t st);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace sa
