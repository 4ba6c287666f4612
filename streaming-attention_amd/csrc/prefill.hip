// Causal prefill attention on gfx950 MFMA (flash-style, block-tiled).
//
// Reference: ops::self_attention_streaming_blockwise (reference
// tensor_cpp/src/ops.cpp:1027-1112): each query i keeps an online-softmax
// state (utils/softmax_online.h:40-87) over KV blocks restricted to keys
// 0..i, scores = (q.k) * scale.  GQA: query head h reads KV head h / (Hq/Hkv)
// (the repeat_kv map of tensor_cpp/src/qwen3_ops.cpp:194-234), no copy.
//
// Tiling: a workgroup of 4 waves owns 128 queries of one head (32 per wave,
// as two 16-query groups) and walks 64-key tiles staged in LDS.  Scores are
// computed transposed, S^T = K Q^T, with 16x16 MFMA blocks: lane l then holds
// query l%16 and 4 keys per block, so row max / row sum are in-lane plus two
// cross-lane steps, and P^T is already in the B-operand layout of the
// O^T += V^T P^T product.  bf16 inputs use v_mfma_f32_16x16x32_bf16 (P is
// rounded to bf16, accumulation fp32); fp32 inputs use v_mfma_f32_16x16x4f32.
// Tiles entirely above the diagonal are never loaded; only tiles that cross
// the diagonal apply the element mask.
#include "sa_internal.h"

namespace sa {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kQTile = 128;   // queries per workgroup
constexpr int kKTile = 64;    // keys per LDS tile
constexpr int kPThreads = 256;
constexpr float kLog2eP = 1.4426950408889634f;

template <bool BF16, int D>
struct PrefillLds {
    // K row-major [64][D + pad]; V: fp32 row-major [64][D + pad], bf16
    // transposed [D][64 + pad] so a lane can read 4 consecutive keys of one d.
    static constexpr int KPAD = BF16 ? 8 : 4;
    static constexpr int K_STRIDE = D + KPAD;
    static constexpr int V_STRIDE = BF16 ? (kKTile + 8) : (D + 4);
    static constexpr int V_ROWS = BF16 ? D : kKTile;
    using elem = typename std::conditional<BF16, uint16_t, float>::type;
    static constexpr int BYTES = (kKTile * K_STRIDE + V_ROWS * V_STRIDE) * sizeof(elem);
};

struct PrefillArgs {
    const void* q;
    const void* k;
    const void* v;
    float* out;
    long long qs[3];    // element strides {batch, head, row} of q
    long long kvs[3];   // of k and v
    long long os[3];    // of out
    int Hq, Hkv, L;
    float scale;
};

__device__ __forceinline__ float xsum16_32(float v) {
    v += swz_xor16(v);
    v += xor32(v);
    return v;
}
__device__ __forceinline__ float xmax16_32(float v) {
    v = fmaxf(v, swz_xor16(v));
    v = fmaxf(v, xor32(v));
    return v;
}

template <bool BF16, int D>
__global__ void __launch_bounds__(kPThreads)
prefill_causal_kernel(PrefillArgs pa) {
    const int Hq = pa.Hq, Hkv = pa.Hkv, L = pa.L;
    const float scale = pa.scale;
    using Lds = PrefillLds<BF16, D>;
    using elem = typename Lds::elem;
    constexpr int NDB = D / 16;            // 16-wide d blocks of the output
    extern __shared__ __align__(16) unsigned char smem[];
    elem* sK = reinterpret_cast<elem*>(smem);
    elem* sV = sK + kKTile * Lds::K_STRIDE;

    const int n_qt = (L + kQTile - 1) / kQTile;
    const int qt = n_qt - 1 - blockIdx.x;      // heaviest tiles first
    const int bh = blockIdx.y;                 // b * Hq + h
    const int b = bh / Hq, h = bh % Hq;
    const int kvh = h / (Hq / Hkv);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;                   // lane group 0..3
    const int c16 = lane & 15;

    const elem* Q = static_cast<const elem*>(pa.q) + b * pa.qs[0] + h * pa.qs[1];
    const elem* K = static_cast<const elem*>(pa.k) + b * pa.kvs[0] + kvh * pa.kvs[1];
    const elem* V = static_cast<const elem*>(pa.v) + b * pa.kvs[0] + kvh * pa.kvs[1];
    const long long q_row = pa.qs[2], kv_row = pa.kvs[2];

    const int q_wave0 = qt * kQTile + wave * 32;   // first query of this wave

    // Q^T fragments (B operand) per 16-query group.
    constexpr int QF = BF16 ? D / 32 : D / 4;      // k-steps over D
    using qfrag_t = typename std::conditional<BF16, bf16x8_t, float>::type;
    qfrag_t qf[2][QF];
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
        const int qi = q_wave0 + gq * 16 + c16;
        const bool ok = qi < L;
#pragma unroll
        for (int s = 0; s < QF; ++s) {
            if constexpr (BF16) {
                uint4 raw = ok ? *reinterpret_cast<const uint4*>(Q + qi * q_row + s * 32 + g * 8)
                               : make_uint4(0, 0, 0, 0);
                qf[gq][s] = __builtin_bit_cast(bf16x8_t, raw);
            } else {
                qf[gq][s] = ok ? Q[qi * q_row + s * 4 + g] : 0.f;
            }
        }
    }

    f32x4_t acc[2][NDB];
#pragma unroll
    for (int gq = 0; gq < 2; ++gq)
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[gq][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.f, 0.f};

    const int q_last_wg = min(L, (qt + 1) * kQTile) - 1;
    const int n_kt = q_last_wg / kKTile + 1;

    for (int kt = 0; kt < n_kt; ++kt) {
        const int key0 = kt * kKTile;
        __syncthreads();
        // ---- stage K and V tile ----
        {
            constexpr int EPV = 16 / sizeof(elem);     // elements per 16 B
            constexpr int CPR = D / EPV;               // 16 B chunks per row
            for (int idx = threadIdx.x; idx < kKTile * CPR; idx += kPThreads) {
                const int r = idx / CPR, cchunk = idx % CPR;
                const int key = key0 + r;
                uint4 kr = make_uint4(0, 0, 0, 0), vr = make_uint4(0, 0, 0, 0);
                if (key < L) {
                    kr = *reinterpret_cast<const uint4*>(K + key * kv_row + cchunk * EPV);
                    vr = *reinterpret_cast<const uint4*>(V + key * kv_row + cchunk * EPV);
                }
                *reinterpret_cast<uint4*>(sK + r * Lds::K_STRIDE + cchunk * EPV) = kr;
                if constexpr (BF16) {
                    const uint16_t* ve = reinterpret_cast<const uint16_t*>(&vr);
#pragma unroll
                    for (int e = 0; e < 8; ++e) sV[(cchunk * 8 + e) * Lds::V_STRIDE + r] = ve[e];
                } else {
                    *reinterpret_cast<uint4*>(sV + r * Lds::V_STRIDE + cchunk * EPV) = vr;
                }
            }
        }
        __syncthreads();
        if (key0 > q_wave0 + 31) continue;   // whole wave above the diagonal
        const bool diag = key0 + kKTile - 1 > q_wave0;

#pragma unroll
        for (int gq = 0; gq < 2; ++gq) {
            const int qi = q_wave0 + gq * 16 + c16;
            // ---- S^T = K Q^T for 4 blocks of 16 keys ----
            f32x4_t st[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                f32x4_t s = {0.f, 0.f, 0.f, 0.f};
                const elem* krow = sK + (c * 16 + c16) * Lds::K_STRIDE;
#pragma unroll
                for (int ks = 0; ks < QF; ++ks) {
                    if constexpr (BF16) {
                        bf16x8_t a = __builtin_bit_cast(
                            bf16x8_t, *reinterpret_cast<const uint4*>(krow + ks * 32 + g * 8));
                        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[gq][ks], s, 0, 0, 0);
                    } else {
                        s = __builtin_amdgcn_mfma_f32_16x16x4f32(krow[ks * 4 + g], qf[gq][ks], s, 0, 0, 0);
                    }
                }
                st[c] = s;
            }
            // ---- scale, mask, online softmax (per query = per lane) ----
            float mt = -INFINITY;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = key0 + c * 16 + g * 4 + i;
                    float sv = st[c][i] * scale;
                    if (diag && (key > qi || key >= L)) sv = -INFINITY;
                    st[c][i] = sv;
                    mt = fmaxf(mt, sv);
                }
            mt = xmax16_32(mt);
            const float m_new = fmaxf(m_run[gq], mt);
            const float alpha = __builtin_amdgcn_exp2f((m_run[gq] - m_new) * kLog2eP);
            float rs = 0.f;
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = __builtin_amdgcn_exp2f((st[c][i] - m_new) * kLog2eP);
                    st[c][i] = p;
                    rs += p;
                }
            rs = xsum16_32(rs);
            l_run[gq] = l_run[gq] * alpha + rs;
            m_run[gq] = m_new;
#pragma unroll
            for (int db = 0; db < NDB; ++db) acc[gq][db] *= alpha;

            // ---- O^T += V^T P^T ----
            if constexpr (BF16) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int c0 = 2 * j, c1 = 2 * j + 1;
                    uint32_t pw[4];
                    pw[0] = f32_to_bf16_rne(st[c0][0]) | ((uint32_t)f32_to_bf16_rne(st[c0][1]) << 16);
                    pw[1] = f32_to_bf16_rne(st[c0][2]) | ((uint32_t)f32_to_bf16_rne(st[c0][3]) << 16);
                    pw[2] = f32_to_bf16_rne(st[c1][0]) | ((uint32_t)f32_to_bf16_rne(st[c1][1]) << 16);
                    pw[3] = f32_to_bf16_rne(st[c1][2]) | ((uint32_t)f32_to_bf16_rne(st[c1][3]) << 16);
                    const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, make_uint4(pw[0], pw[1], pw[2], pw[3]));
#pragma unroll
                    for (int db = 0; db < NDB; ++db) {
                        const elem* vrow = sV + (db * 16 + c16) * Lds::V_STRIDE;
                        const uint2 lo = *reinterpret_cast<const uint2*>(vrow + c0 * 16 + g * 4);
                        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + c1 * 16 + g * 4);
                        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
                        acc[gq][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, acc[gq][db], 0, 0, 0);
                    }
                }
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float pv = st[c][i];
                        const elem* vrow = sV + (c * 16 + g * 4 + i) * Lds::V_STRIDE;
#pragma unroll
                        for (int db = 0; db < NDB; ++db)
                            acc[gq][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[db * 16 + c16], pv,
                                                                               acc[gq][db], 0, 0, 0);
                    }
            }
        }
    }

    // ---- normalise and store: lane holds O^T[d = db*16 + 4g + i][q = c16] ----
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
        const int qi = q_wave0 + gq * 16 + c16;
        if (qi >= L) continue;
        const float inv = 1.0f / l_run[gq];
        float* orow = pa.out + b * pa.os[0] + h * pa.os[1] + qi * pa.os[2];
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            float4 o4 = make_float4(acc[gq][db][0] * inv, acc[gq][db][1] * inv, acc[gq][db][2] * inv,
                                    acc[gq][db][3] * inv);
            *reinterpret_cast<float4*>(orow + db * 16 + g * 4) = o4;
        }
    }
}

template <bool BF16, int D>
sa_status launch_prefill(const PrefillArgs& pa, int B, hipStream_t st) {
    using Lds = PrefillLds<BF16, D>;
    if constexpr (Lds::BYTES > 65536) {
        // The fp32 D=128 tile needs more than 64 KiB of LDS: opt in per device.
        static thread_local int opted_device = -1;
        int dev = 0;
        SA_HIP_TRY(hipGetDevice(&dev));
        if (opted_device != dev) {
            SA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&prefill_causal_kernel<BF16, D>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, Lds::BYTES));
            opted_device = dev;
        }
    }
    dim3 grid((pa.L + kQTile - 1) / kQTile, B * pa.Hq);
    hipLaunchKernelGGL((prefill_causal_kernel<BF16, D>), grid, dim3(kPThreads), Lds::BYTES, st, pa);
    SA_CHECK_LAUNCH();
    return SA_OK;
}

sa_status prefill(const void* q, const void* k, const void* v, sa_dtype dtype, int batch, int n_q_heads,
                  int n_kv_heads, int L, int D, const int64_t* qs, const int64_t* kvs, const int64_t* os,
                  float scale, float* out, hipStream_t st) {
    if (!q || !k || !v || !out || !qs || !kvs || !os) return fail(SA_EINVAL, "null pointer");
    if (batch <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads)
        return fail(SA_EINVAL, "bad head counts");
    if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16) return fail(SA_EINVAL, "dtype must be F32 or BF16");
    if (D != 64 && D != 128) return fail(SA_EINVAL, "prefill head_dim must be 64 or 128");
    if (L <= 0) return SA_OK;
    const int elem = dtype == SA_DTYPE_BF16 ? 2 : 4;
    const int64_t align_in = 16 / elem, align_out = 4;
    for (int i = 0; i < 3; ++i) {
        if (qs[i] % align_in || kvs[i] % align_in || os[i] % align_out || qs[i] < 0 || kvs[i] < 0 || os[i] < 0)
            return fail(SA_EINVAL, "strides must keep every row 16-byte aligned");
    }
    if (qs[2] < D || kvs[2] < D || os[2] < D) return fail(SA_EINVAL, "row stride shorter than head_dim");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return fail(SA_EINVAL, "q, k, v and out must be 16-byte aligned");
    PrefillArgs pa{};
    pa.q = q; pa.k = k; pa.v = v; pa.out = out;
    for (int i = 0; i < 3; ++i) { pa.qs[i] = qs[i]; pa.kvs[i] = kvs[i]; pa.os[i] = os[i]; }
    pa.Hq = n_q_heads; pa.Hkv = n_kv_heads; pa.L = L; pa.scale = scale;
    if (dtype == SA_DTYPE_BF16)
        return D == 64 ? launch_prefill<true, 64>(pa, batch, st) : launch_prefill<true, 128>(pa, batch, st);
    return D == 64 ? launch_prefill<false, 64>(pa, batch, st) : launch_prefill<false, 128>(pa, batch, st);
}

}  // namespace
}  // namespace sa

extern "C" sa_status sa_prefill_causal(const void* q, const void* k, const void* v, sa_dtype dtype,
                                       int batch, int n_q_heads, int n_kv_heads, int L, int D,
                                       float scale, float* out, sa_stream_t stream) {
    sa::clear_error();
    const int64_t Ld = (int64_t)L * D;
    const int64_t qs[3] = {n_q_heads * Ld, Ld, D};
    const int64_t kvs[3] = {n_kv_heads * Ld, Ld, D};
    return sa::prefill(q, k, v, dtype, batch, n_q_heads, n_kv_heads, L, D, qs, kvs, qs, scale, out,
                       sa::as_stream(stream));
}

extern "C" sa_status sa_prefill_causal_strided(const void* q, const void* k, const void* v, sa_dtype dtype,
                                               int batch, int n_q_heads, int n_kv_heads, int L, int D,
                                               const int64_t q_strides[3], const int64_t kv_strides[3],
                                               const int64_t out_strides[3], float scale, float* out,
                                               sa_stream_t stream) {
    sa::clear_error();
    return sa::prefill(q, k, v, dtype, batch, n_q_heads, n_kv_heads, L, D, q_strides, kv_strides, out_strides,
                       scale, out, sa::as_stream(stream));
}
