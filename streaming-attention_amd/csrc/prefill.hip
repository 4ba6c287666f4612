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
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

constexpr int kQTile = 128;   // queries per workgroup
constexpr int kKTile = 64;    // keys per LDS tile
constexpr int kPThreads = 256;
constexpr float kLog2eP = 1.4426950408889634f;

template <bool BF16, int D>
struct PrefillLds {
    // Two stages.  K row-major [64][D + pad]; V fp32 row-major [64][D + pad],
    // bf16 transposed [D][64 + pad] so a lane reads 4 consecutive keys of one d.
    static constexpr int KPAD = BF16 ? 8 : 4;
    static constexpr int K_STRIDE = D + KPAD;
    static constexpr int V_STRIDE = BF16 ? (kKTile + 8) : (D + 4);
    static constexpr int V_ROWS = BF16 ? D : kKTile;
    using elem = typename std::conditional<BF16, uint16_t, float>::type;
    static constexpr int STAGE = kKTile * K_STRIDE + V_ROWS * V_STRIDE;   // elements
    static constexpr int BYTES = 2 * STAGE * (int)sizeof(elem);
    // 16-byte global loads per thread per tile, for K and for V.
    static constexpr int EPV = 16 / (int)sizeof(elem);
    static constexpr int CPR = D / EPV;                 // 16 B chunks per row
    static constexpr int NK = kKTile * CPR / 256;       // K loads per thread
    static constexpr int NV = NK;                       // V loads per thread
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
struct TileStage {
    uint4 k[PrefillLds<BF16, D>::NK];
    uint4 v[PrefillLds<BF16, D>::NV];
};

// Global -> registers for the K/V tile starting at key0.  K: thread t reads
// row t / CPR (consecutive lanes cover whole rows).  bf16 V: thread t reads
// the row pair (2 rp, 2 rp + 1), rp = t % 32, at chunk t / 32, so the
// transposed LDS writes of a wave land on distinct banks.  Rows past L read 0.
template <bool BF16, int D>
__device__ __forceinline__ void load_tile(TileStage<BF16, D>& st, const typename PrefillLds<BF16, D>::elem* K,
                                          const typename PrefillLds<BF16, D>::elem* V, long long kv_row,
                                          int key0, int L) {
    using Lds = PrefillLds<BF16, D>;
    constexpr int CPR = Lds::CPR, EPV = Lds::EPV;
#pragma unroll
    for (int i = 0; i < Lds::NK; ++i) {
        const int idx = threadIdx.x + i * kPThreads;
        const int r = idx / CPR, c = idx % CPR;
        const int key = key0 + r;
        st.k[i] = key < L ? *reinterpret_cast<const uint4*>(K + key * kv_row + c * EPV) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < Lds::NV; ++i) {
        int r, c;
        if constexpr (BF16) {
            const int item = threadIdx.x + (i / 2) * kPThreads;   // (row pair, chunk)
            r = 2 * (item % 32) + (i & 1);
            c = item / 32;
        } else {
            const int idx = threadIdx.x + i * kPThreads;
            r = idx / CPR;
            c = idx % CPR;
        }
        const int key = key0 + r;
        st.v[i] = key < L ? *reinterpret_cast<const uint4*>(V + key * kv_row + c * EPV) : make_uint4(0, 0, 0, 0);
    }
}

// Registers -> LDS stage (K row-major; bf16 V transposed with one 4-byte
// store per (d, key pair)).
template <bool BF16, int D>
__device__ __forceinline__ void store_tile(const TileStage<BF16, D>& st, typename PrefillLds<BF16, D>::elem* sK,
                                           typename PrefillLds<BF16, D>::elem* sV) {
    using Lds = PrefillLds<BF16, D>;
    constexpr int CPR = Lds::CPR, EPV = Lds::EPV;
#pragma unroll
    for (int i = 0; i < Lds::NK; ++i) {
        const int idx = threadIdx.x + i * kPThreads;
        *reinterpret_cast<uint4*>(sK + (idx / CPR) * Lds::K_STRIDE + (idx % CPR) * EPV) = st.k[i];
    }
    if constexpr (BF16) {
#pragma unroll
        for (int i = 0; i < Lds::NV; i += 2) {
            const int item = threadIdx.x + (i / 2) * kPThreads;
            const int rp = item % 32, c = item / 32;
            const uint32_t* lo = reinterpret_cast<const uint32_t*>(&st.v[i]);
            const uint32_t* hi = reinterpret_cast<const uint32_t*>(&st.v[i + 1]);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                // elements 2w, 2w+1 of the chunk for keys 2rp (lo) and 2rp+1 (hi)
                const uint32_t e0 = (lo[w] & 0xffffu) | (hi[w] << 16);
                const uint32_t e1 = (lo[w] >> 16) | (hi[w] & 0xffff0000u);
                *reinterpret_cast<uint32_t*>(sV + (c * 8 + 2 * w) * Lds::V_STRIDE + 2 * rp) = e0;
                *reinterpret_cast<uint32_t*>(sV + (c * 8 + 2 * w + 1) * Lds::V_STRIDE + 2 * rp) = e1;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < Lds::NV; ++i) {
            const int idx = threadIdx.x + i * kPThreads;
            *reinterpret_cast<uint4*>(sV + (idx / CPR) * Lds::V_STRIDE + (idx % CPR) * EPV) = st.v[i];
        }
    }
}

template <bool BF16, int D>
__global__ void __launch_bounds__(kPThreads)
prefill_causal_kernel(PrefillArgs pa) {
    const int Hq = pa.Hq, Hkv = pa.Hkv, L = pa.L;
    // Scores go to the log2 domain once: p = 2^(s - m) with s = q.k * scale * log2(e).
    const float sl2 = pa.scale * kLog2eP;
    using Lds = PrefillLds<BF16, D>;
    using elem = typename Lds::elem;
    constexpr int NDB = D / 16;            // 16-wide d blocks of the output
    extern __shared__ __align__(16) unsigned char smem[];
    elem* stage_base = reinterpret_cast<elem*>(smem);

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
    const int q_last_wg = min(L, (qt + 1) * kQTile) - 1;
    const int n_kt = q_last_wg / kKTile + 1;

    // Tile 0 in flight while Q is read.
    TileStage<BF16, D> next;
    load_tile<BF16, D>(next, K, V, kv_row, 0, L);

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

    store_tile<BF16, D>(next, stage_base, stage_base + kKTile * Lds::K_STRIDE);
    __syncthreads();

    for (int kt = 0; kt < n_kt; ++kt) {
        const int key0 = kt * kKTile;
        elem* sK = stage_base + (kt & 1) * Lds::STAGE;
        elem* sV = sK + kKTile * Lds::K_STRIDE;
        const bool more = kt + 1 < n_kt;
        // Next tile's loads fly during this tile's MFMAs.
        if (more) load_tile<BF16, D>(next, K, V, kv_row, key0 + kKTile, L);

        if (key0 <= q_wave0 + 31) {   // else the whole wave is above the diagonal
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
                // ---- mask, online softmax in the log2 domain (per query = per lane) ----
                float mt = -INFINITY;
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float sv = st[c][i] * sl2;
                        if (diag) {
                            const int key = key0 + c * 16 + g * 4 + i;
                            if (key > qi || key >= L) sv = -INFINITY;
                        }
                        st[c][i] = sv;
                        mt = fmaxf(mt, sv);
                    }
                mt = xmax16_32(mt);
                const float m_new = fmaxf(m_run[gq], mt);
                const float alpha = __builtin_amdgcn_exp2f(m_run[gq] - m_new);
                float rs = 0.f;
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float p = __builtin_amdgcn_exp2f(st[c][i] - m_new);
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
                        // hardware RNE conversion, two values per instruction
                        bf16x2_t p01 = __builtin_convertvector(f32x2_t{st[c0][0], st[c0][1]}, bf16x2_t);
                        bf16x2_t p23 = __builtin_convertvector(f32x2_t{st[c0][2], st[c0][3]}, bf16x2_t);
                        bf16x2_t p45 = __builtin_convertvector(f32x2_t{st[c1][0], st[c1][1]}, bf16x2_t);
                        bf16x2_t p67 = __builtin_convertvector(f32x2_t{st[c1][2], st[c1][3]}, bf16x2_t);
                        const bf16x8_t pb = __builtin_bit_cast(
                            bf16x8_t, make_uint4(__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23),
                                                 __builtin_bit_cast(uint32_t, p45), __builtin_bit_cast(uint32_t, p67)));
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
        if (more) {
            // The other stage was last read in the previous iteration, before
            // the barrier that ended it.
            elem* nK = stage_base + ((kt + 1) & 1) * Lds::STAGE;
            store_tile<BF16, D>(next, nK, nK + kKTile * Lds::K_STRIDE);
        }
        __syncthreads();
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
