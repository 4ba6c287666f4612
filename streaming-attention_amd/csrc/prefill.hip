// Causal prefill attention on gfx950 MFMA (flash-style, block-tiled).
//
// Reference: ops::self_attention_streaming_blockwise (reference
// tensor_cpp/src/ops.cpp:1027-1112): each query i keeps an online-softmax
// state (utils/softmax_online.h:40-87) over KV blocks restricted to keys
// 0..i, scores = (q.k) * scale.  GQA: query head h reads KV head h / (Hq/Hkv)
// (the repeat_kv map of tensor_cpp/src/qwen3_ops.cpp:194-234), no copy.
//
// Both kernels compute scores transposed, S^T = K Q^T, so a lane owns one
// query column and the row max / row sum need almost no cross-lane work, and
// P^T comes out of the score MFMA already in the B-operand layout of the
// O^T += V^T P^T product.  Softmax runs in the log2 domain, p = 2^(s*c - m)
// with c = scale * log2(e).  Tiles entirely above the diagonal are never
// computed; only the tile that crosses a wave's diagonal applies the mask.
//
// bf16 inputs (v_mfma_f32_32x32x16_bf16, fp32 accumulation): a wave owns 64
// queries as two 32-query blocks, a workgroup of 4 waves 256 queries.  The
// running max is raised lazily: a wave rescales its accumulators only when
// some score exceeds the current max by more than 2^8, so p stays below 256
// and the common tile does no rescale at all.  P is rounded to bf16 for the
// PV product; the row sums use the fp32 p.
//
// fp32 inputs (v_mfma_f32_16x16x4f32): a wave owns 32 queries as two
// 16-query blocks, a workgroup 128 queries, eager rescale.
#include <type_traits>

#include "sa_internal.h"

namespace sa {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
// Staging registers use the native vector type: HIP's uint4 is a struct whose
// copies lower to memcpy and end up in scratch memory.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kKTile = 64;    // keys per LDS tile (both kernels)
constexpr float kLog2eP = 1.4426950408889634f;

struct PrefillArgs {
    const void* q;
    const void* k;
    const void* v;
    float* out;
    long long qs[3];    // element strides {batch, head, row} of q
    long long kvs[3];   // of k and v
    long long os[3];    // of out
    int Hq, Hkv, L;
    int n_qt;           // query tiles per head
    int xcd_groups;     // KV groups per XCD when the grid maps groups to XCDs, else 0
    float sl2;          // |scale| * log2(e)
    uint32_t q_sign;    // 0x80008000 to negate bf16 q pairs (negative scale), else 0
    float scale;        // signed scale (fp32 kernel)
};

// Work mapping shared by both kernels.  A KV group is one (batch, kv head);
// its G = Hq/Hkv query heads read the same K/V.  When the number of groups is
// a multiple of 8, hardware workgroup i (dispatched to XCD i % 8) takes work
// slot i / 8 of the groups owned by that XCD, so each XCD's L2 holds the K/V
// of its own groups only.  Inside an XCD (or the whole grid otherwise) slots
// run heaviest query tile first, which balances the causal triangle.
struct Work { int b, h, kvh, qt; };
__device__ __forceinline__ Work map_work(const PrefillArgs& pa, int i) {
    const int G = pa.Hq / pa.Hkv;
    int x = 0, j = i, span = gridDim.x / (G * pa.n_qt);   // groups in this slot range
    if (pa.xcd_groups) { x = i & 7; j = i >> 3; span = pa.xcd_groups; }
    const int per_qt = span * G;
    Work w;
    w.qt = pa.n_qt - 1 - j / per_qt;
    const int rem = j % per_qt;
    const int group = x * span + rem / G;
    w.b = group / pa.Hkv;
    w.kvh = group % pa.Hkv;
    w.h = w.kvh * G + rem % G;
    return w;
}

// ===========================================================================
// bf16 kernel
// ===========================================================================
// A wave owns QB 32-query blocks; a workgroup of W waves owns W * QB * 32
// queries and streams 64-key K/V tiles through two LDS stages.
constexpr float kLazyRescale = 8.f;              // log2 headroom before a rescale

template <int D, int W>
struct BfLds {
    static constexpr int THREADS = W * 64;
    static constexpr int K_STRIDE = D + 8;           // K row-major [64][D + 8]
    static constexpr int V_STRIDE = kKTile + 8;      // V transposed [D][64 + 8]
    static constexpr int K_ELEMS = kKTile * K_STRIDE;
    static constexpr int STAGE = K_ELEMS + D * V_STRIDE;   // bf16 elements per stage
    static constexpr int BYTES = 2 * STAGE * 2;            // two stages
    static constexpr int CPR = D / 8;                // 16-byte chunks per row
    static constexpr int K_ITEMS = kKTile * CPR;     // 16-byte K chunks per tile
    static constexpr int V_ITEMS = 32 * CPR;         // (row pair, chunk) V items per tile
    static constexpr int NK = (K_ITEMS + THREADS - 1) / THREADS;
    static constexpr int NVI = (V_ITEMS + THREADS - 1) / THREADS;
    static_assert(K_ITEMS % THREADS == 0 || THREADS % K_ITEMS == 0, "K items must tile the workgroup");
    static_assert(V_ITEMS % THREADS == 0 || THREADS % V_ITEMS == 0, "V items must tile the workgroup");
};

// The K rows a lane feeds to the score MFMA are permuted within each 32-key
// block (bits 2 and 3 of the row swapped).  With the 32x32 output layout
// (lane l: column l%32, rows 8*(j/4) + 4*(l/32) + j%4 for element j) this
// makes element j of lane l the score of key 16*(j/8) + 8*(l/32) + j%8: each
// lane's 8-element groups are 8 consecutive keys, exactly what the B operand
// of the 32x32x16 PV step needs, and what one 16-byte read of V^T supplies.
__device__ __forceinline__ int swap_bits23(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

template <int D, int W>
struct BfStage {
    u32x4_t k[BfLds<D, W>::NK];
    u32x4_t v[2 * BfLds<D, W>::NVI];
};

// Per-thread element offsets of the tile loads, relative to the tile's first
// row.  K: chunk idx = tid + i*THREADS -> row idx / CPR.  V: item = tid +
// i*THREADS -> row pair item % 32 (rows 2rp, 2rp + 1), chunk item / 32.
// Threads past the item count (small head dims, many waves) idle; that split
// falls on whole waves.
template <int D, int W>
struct BfLoadMap {
    using Lds = BfLds<D, W>;
    int k_row[Lds::NK], k_col[Lds::NK];
    int v_row[Lds::NVI], v_col[Lds::NVI];
    bool k_on, v_on;
    __device__ __forceinline__ BfLoadMap() {
        k_on = threadIdx.x < Lds::K_ITEMS;
        v_on = threadIdx.x < Lds::V_ITEMS;
#pragma unroll
        for (int i = 0; i < Lds::NK; ++i) {
            const int idx = threadIdx.x + i * Lds::THREADS;
            k_row[i] = idx / Lds::CPR;
            k_col[i] = (idx % Lds::CPR) * 8;
        }
#pragma unroll
        for (int i = 0; i < Lds::NVI; ++i) {
            const int item = threadIdx.x + i * Lds::THREADS;
            v_row[i] = 2 * (item % 32);
            v_col[i] = (item / 32) * 8;
        }
    }
};

// Global -> registers.  Rows past the end of the sequence are clamped to the
// last row: they only feed keys that the causal mask removes.
template <int D, int W>
__device__ __forceinline__ void bf_load(BfStage<D, W>& st, const BfLoadMap<D, W>& mp, const uint16_t* K,
                                        const uint16_t* V, int kv_row, int key0, int L) {
    using Lds = BfLds<D, W>;
    const uint16_t* Kt = K + (long long)key0 * kv_row;
    const uint16_t* Vt = V + (long long)key0 * kv_row;
    const int rmax = L - 1 - key0;
    if (mp.k_on) {
#pragma unroll
        for (int i = 0; i < Lds::NK; ++i)
            st.k[i] = *reinterpret_cast<const u32x4_t*>(Kt + min(mp.k_row[i], rmax) * kv_row + mp.k_col[i]);
    }
    if (mp.v_on) {
#pragma unroll
        for (int i = 0; i < Lds::NVI; ++i) {
            st.v[2 * i] = *reinterpret_cast<const u32x4_t*>(Vt + min(mp.v_row[i], rmax) * kv_row + mp.v_col[i]);
            st.v[2 * i + 1] =
                *reinterpret_cast<const u32x4_t*>(Vt + min(mp.v_row[i] + 1, rmax) * kv_row + mp.v_col[i]);
        }
    }
}

// Registers -> LDS stage.  K row-major; V transposed with one 4-byte store
// per (d, key pair): lanes of a wave cover 32 consecutive key pairs of one d,
// so each store instruction touches 32 distinct banks per half-wave.
template <int D, int W>
__device__ __forceinline__ void bf_store(const BfStage<D, W>& st, const BfLoadMap<D, W>& mp, uint16_t* sK,
                                         uint16_t* sV) {
    using Lds = BfLds<D, W>;
    if (mp.k_on) {
#pragma unroll
        for (int i = 0; i < Lds::NK; ++i)
            *reinterpret_cast<u32x4_t*>(sK + mp.k_row[i] * Lds::K_STRIDE + mp.k_col[i]) = st.k[i];
    }
    if (mp.v_on) {
#pragma unroll
        for (int i = 0; i < Lds::NVI; ++i) {
            const u32x4_t lo = st.v[2 * i], hi = st.v[2 * i + 1];
            uint16_t* col = sV + mp.v_col[i] * Lds::V_STRIDE + mp.v_row[i];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                // elements 2w, 2w+1 of the chunk: key pair (lo, hi) for each
                *reinterpret_cast<uint32_t*>(col + (2 * w) * Lds::V_STRIDE) =
                    __builtin_amdgcn_perm(hi[w], lo[w], 0x05040100u);
                *reinterpret_cast<uint32_t*>(col + (2 * w + 1) * Lds::V_STRIDE) =
                    __builtin_amdgcn_perm(hi[w], lo[w], 0x07060302u);
            }
        }
    }
}

__device__ __forceinline__ bf16x8_t lds_b128(const uint16_t* p) { return *reinterpret_cast<const bf16x8_t*>(p); }

template <int D, int QB, int W>
__global__ void __launch_bounds__(W * 64)
prefill_bf16_kernel(PrefillArgs pa) {
    using Lds = BfLds<D, W>;
    constexpr int NKS = D / 16;     // k-steps of the score product
    constexpr int NDB = D / 32;     // 32-row d blocks of O^T
    constexpr int QWAVE = 32 * QB;  // queries per wave
    constexpr int QTILE = W * QWAVE;
    extern __shared__ __align__(16) unsigned char smem[];
    uint16_t* stage_base = reinterpret_cast<uint16_t*>(smem);

    const int L = pa.L;
    const Work wk = map_work(pa, blockIdx.x);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 31;        // query column inside a 32-query block
    const int hh = lane >> 5;       // lane half
    const float sl2 = pa.sl2;

    const uint16_t* Q = static_cast<const uint16_t*>(pa.q) + wk.b * pa.qs[0] + wk.h * pa.qs[1];
    const uint16_t* K = static_cast<const uint16_t*>(pa.k) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const uint16_t* V = static_cast<const uint16_t*>(pa.v) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const int kv_row = static_cast<int>(pa.kvs[2]);

    const int q_wave0 = wk.qt * QTILE + wave * QWAVE;
    const int n_kt = (min(L, (wk.qt + 1) * QTILE) - 1) / kKTile + 1;
    // Tiles this wave computes: keys up to its last query.  The last one is
    // the diagonal tile; dq is the wave's first query relative to it.
    const int wave_kt = q_wave0 < L ? (q_wave0 + QWAVE - 1) / kKTile + 1 : 0;
    const int dq = q_wave0 - (wave_kt - 1) * kKTile;

    const BfLoadMap<D, W> mp;
    BfStage<D, W> next;
    bf_load<D, W>(next, mp, K, V, kv_row, 0, L);

    // Q^T fragments (B operand): lane holds q[n][16 ks + 8 hh .. + 7].
    bf16x8_t qf[QB][NKS];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int qi = min(q_wave0 + qb * 32 + n, L - 1);
        const uint16_t* qrow = Q + qi * pa.qs[2] + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
            const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(qrow + ks * 16) ^ pa.q_sign;
            qf[qb][ks] = __builtin_bit_cast(bf16x8_t, raw);
            // MFMA sources may be AGPRs: Q waits there, leaving VGPRs to the softmax.
            asm("" : "+a"(qf[qb][ks]));
        }
    }

    f32x16_t acc[QB][NDB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[qb][db] = f32x16_t{};
    float ms[QB], lp[QB];   // running max (log2 domain, equal in both lane halves); row-sum part
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) { ms[qb] = -INFINITY; lp[qb] = 0.f; }

    // Per-lane LDS read offsets (elements) inside a stage.
    const int k_off = swap_bits23(n) * Lds::K_STRIDE + 8 * hh;
    const int v_off = Lds::K_ELEMS + n * Lds::V_STRIDE + 8 * hh;

    bf_store<D, W>(next, mp, stage_base, stage_base + Lds::K_ELEMS);
    __syncthreads();

    for (int kt = 0; kt < n_kt; ++kt) {
        const uint16_t* sK = stage_base + (kt & 1) * Lds::STAGE;
        // Next tile's loads fly during this tile's MFMAs.  Past the last tile
        // they read clamped, in-range rows into a stage nobody reads.
        bf_load<D, W>(next, mp, K, V, kv_row, (kt + 1) * kKTile, L);

        // One tile, as two 32-key halves kb.  Per half: the K fragments are
        // read up front, the score MFMAs of all query blocks share them; the
        // V fragments are issued next so their latency hides behind the
        // softmax; the softmax assumes the running max holds and a rare fix-up
        // handles a raised max; then the PV MFMAs.  DIAG instantiates the
        // diagonal tile's mask.
        auto tile = [&](auto diag_tag) {
            constexpr bool DIAG = decltype(diag_tag)::value;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                // ---- S^T = K Q^T for keys 32 kb .. 32 kb + 31 ----
                bf16x8_t kf[NKS];
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) kf[ks] = lds_b128(sK + k_off + kb * 32 * Lds::K_STRIDE + ks * 16);
                f32x16_t s[QB];
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) s[qb] = f32x16_t{};
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb)
                        s[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[qb][ks], s[qb], 0, 0, 0);
                bf16x8_t vf[NDB][2];
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
                        vf[db][t] = lds_b128(sK + v_off + db * 32 * Lds::V_STRIDE + kb * 32 + t * 16);

                // Element j of s[qb] is key kt*64 + 32 kb + 16 (j/8) + 8 hh + j%8
                // for query q_wave0 + 32 qb + n.  On the diagonal tile keys past
                // the query are removed (query - kt*64 = dq + 32 qb + n).
                auto masked = [&](int qb, int j) {
                    return DIAG && 32 * kb + 16 * (j / 8) + 8 * hh + (j % 8) > dq + 32 * qb + n;
                };
                float mt[QB];
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    if constexpr (DIAG) {
#pragma unroll
                        for (int j = 0; j < 16; ++j)
                            if (masked(qb, j)) s[qb][j] = -INFINITY;
                    }
                    mt[qb] = s[qb][0];
#pragma unroll
                    for (int j = 1; j < 16; ++j) mt[qb] = fmaxf(mt[qb], s[qb][j]);
                }
                bf16x8_t pb[QB][2];
                float rs[QB];
                auto softmax = [&](int qb) {
                    const float nm = -ms[qb];
                    float p[16];
                    rs[qb] = 0.f;
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[qb][j], sl2, nm));
                        if (masked(qb, j)) p[j] = 0.f;   // exact zero also for a zero scale
                        rs[qb] += p[j];
                    }
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const bf16x2_t p01 = __builtin_convertvector(f32x2_t{p[8 * t + 0], p[8 * t + 1]}, bf16x2_t);
                        const bf16x2_t p23 = __builtin_convertvector(f32x2_t{p[8 * t + 2], p[8 * t + 3]}, bf16x2_t);
                        const bf16x2_t p45 = __builtin_convertvector(f32x2_t{p[8 * t + 4], p[8 * t + 5]}, bf16x2_t);
                        const bf16x2_t p67 = __builtin_convertvector(f32x2_t{p[8 * t + 6], p[8 * t + 7]}, bf16x2_t);
                        pb[qb][t] = __builtin_bit_cast(
                            bf16x8_t, make_uint4(__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23),
                                                 __builtin_bit_cast(uint32_t, p45), __builtin_bit_cast(uint32_t, p67)));
                    }
                };
                bool up = false;
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    softmax(qb);
                    // Keep the common-case softmax ahead of the branch (the
                    // compiler would otherwise sink it into the no-rescale path).
                    asm volatile("" : "+v"(pb[qb][0]), "+v"(pb[qb][1]), "+v"(rs[qb]));
                    up = up || mt[qb] * sl2 > ms[qb] + kLazyRescale;
                }
                if (__any(up)) {
                    // Raise the max to the exact row max of this half (both
                    // lane halves agree), rescale, redo the softmax.
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb) {
                        const float mq = fmaxf(mt[qb], __shfl_xor(mt[qb], 32, 64));
                        const float m_new = fmaxf(ms[qb], mq * sl2);
                        const float alpha = ms[qb] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms[qb] - m_new);
#pragma unroll
                        for (int db = 0; db < NDB; ++db) acc[qb][db] *= alpha;
                        lp[qb] *= alpha;
                        ms[qb] = m_new;
                        softmax(qb);
                    }
                }
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) lp[qb] += rs[qb];
                // ---- O^T += V^T P^T over the same 32 keys ----
#pragma unroll
                for (int db = 0; db < NDB; ++db)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
#pragma unroll
                        for (int qb = 0; qb < QB; ++qb)
                            acc[qb][db] =
                                __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][t], pb[qb][t], acc[qb][db], 0, 0, 0);
            }
        };
        if (kt + 1 < wave_kt) tile(std::false_type{});
        else if (kt + 1 == wave_kt) tile(std::true_type{});

        // The other stage was last read before the barrier that ended the
        // previous iteration.
        uint16_t* nK = stage_base + ((kt + 1) & 1) * Lds::STAGE;
        bf_store<D, W>(next, mp, nK, nK + Lds::K_ELEMS);
        __syncthreads();
    }

    // ---- normalise and store: element j of acc[qb][db] is
    //      O[q_wave0 + 32 qb + n][32 db + 8 (j/4) + 4 hh + j%4] ----
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float l = lp[qb] + __shfl_xor(lp[qb], 32, 64);
        const int qi = q_wave0 + qb * 32 + n;
        if (qi >= L) continue;
        const float inv = 1.0f / l;
        float* orow = pa.out + wk.b * pa.os[0] + wk.h * pa.os[1] + qi * pa.os[2] + 4 * hh;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                *reinterpret_cast<float4*>(orow + 32 * db + 8 * jj) =
                    make_float4(acc[qb][db][4 * jj] * inv, acc[qb][db][4 * jj + 1] * inv,
                                acc[qb][db][4 * jj + 2] * inv, acc[qb][db][4 * jj + 3] * inv);
    }
}

// ===========================================================================
// fp32 kernel
// ===========================================================================
constexpr int kFQTile = 128;    // queries per workgroup
constexpr int kFThreads = 256;

template <int D>
struct F32Lds {
    static constexpr int K_STRIDE = D + 4;           // K row-major [64][D + 4]
    static constexpr int V_STRIDE = D + 4;           // V row-major [64][D + 4]
    static constexpr int K_ELEMS = kKTile * K_STRIDE;
    static constexpr int STAGE = K_ELEMS + kKTile * V_STRIDE;   // floats per stage
    static constexpr int BYTES = 2 * STAGE * 4;
    static constexpr int CPR = D / 4;                // 16-byte chunks per row
    static constexpr int NK = kKTile * CPR / kFThreads;
};

template <int D>
struct F32Stage {
    u32x4_t k[F32Lds<D>::NK];
    u32x4_t v[F32Lds<D>::NK];
};

template <int D>
__device__ __forceinline__ void f32_load(F32Stage<D>& st, const float* K, const float* V, long long kv_row,
                                         int key0, int L) {
    using Lds = F32Lds<D>;
    const int rmax = L - 1 - key0;
#pragma unroll
    for (int i = 0; i < Lds::NK; ++i) {
        const int idx = threadIdx.x + i * kFThreads;
        const long long off = min(idx / Lds::CPR, rmax) * kv_row + (idx % Lds::CPR) * 4;
        st.k[i] = *reinterpret_cast<const u32x4_t*>(K + key0 * kv_row + off);
        st.v[i] = *reinterpret_cast<const u32x4_t*>(V + key0 * kv_row + off);
    }
}

template <int D>
__device__ __forceinline__ void f32_store(const F32Stage<D>& st, float* sK, float* sV) {
    using Lds = F32Lds<D>;
#pragma unroll
    for (int i = 0; i < Lds::NK; ++i) {
        const int idx = threadIdx.x + i * kFThreads;
        const int r = idx / Lds::CPR, c = (idx % Lds::CPR) * 4;
        *reinterpret_cast<u32x4_t*>(sK + r * Lds::K_STRIDE + c) = st.k[i];
        *reinterpret_cast<u32x4_t*>(sV + r * Lds::V_STRIDE + c) = st.v[i];
    }
}

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

template <int D>
__global__ void __launch_bounds__(kFThreads)
prefill_f32_kernel(PrefillArgs pa) {
    using Lds = F32Lds<D>;
    const int L = pa.L;
    const float sl2 = pa.scale * kLog2eP;
    constexpr int NDB = D / 16;            // 16-wide d blocks of the output
    constexpr int QF = D / 4;              // k-steps over D
    extern __shared__ __align__(16) unsigned char smem[];
    float* stage_base = reinterpret_cast<float*>(smem);

    const Work wk = map_work(pa, blockIdx.x);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int g = lane >> 4;                   // lane group 0..3
    const int c16 = lane & 15;

    const float* Q = static_cast<const float*>(pa.q) + wk.b * pa.qs[0] + wk.h * pa.qs[1];
    const float* K = static_cast<const float*>(pa.k) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const float* V = static_cast<const float*>(pa.v) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const long long q_row = pa.qs[2], kv_row = pa.kvs[2];

    const int q_wave0 = wk.qt * kFQTile + wave * 32;   // first query of this wave
    const int n_kt = (min(L, (wk.qt + 1) * kFQTile) - 1) / kKTile + 1;

    F32Stage<D> next;
    f32_load<D>(next, K, V, kv_row, 0, L);

    // Q^T fragments (B operand) per 16-query group.
    float qf[2][QF];
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
        const int qi = min(q_wave0 + gq * 16 + c16, L - 1);
#pragma unroll
        for (int s = 0; s < QF; ++s) qf[gq][s] = Q[qi * q_row + s * 4 + g];
    }

    f32x4_t acc[2][NDB];
#pragma unroll
    for (int gq = 0; gq < 2; ++gq)
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[gq][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.f, 0.f};

    f32_store<D>(next, stage_base, stage_base + Lds::K_ELEMS);
    __syncthreads();

    for (int kt = 0; kt < n_kt; ++kt) {
        const int key0 = kt * kKTile;
        const float* sK = stage_base + (kt & 1) * Lds::STAGE;
        const float* sV = sK + Lds::K_ELEMS;
        const bool more = kt + 1 < n_kt;
        if (more) f32_load<D>(next, K, V, kv_row, key0 + kKTile, L);

        if (key0 <= q_wave0 + 31 && q_wave0 < L) {   // else the whole wave is above the diagonal
            const bool diag = key0 + kKTile - 1 > q_wave0;
#pragma unroll
            for (int gq = 0; gq < 2; ++gq) {
                const int qi = q_wave0 + gq * 16 + c16;
                // ---- S^T = K Q^T for 4 blocks of 16 keys ----
                f32x4_t st[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    f32x4_t s = {0.f, 0.f, 0.f, 0.f};
                    const float* krow = sK + (c * 16 + c16) * Lds::K_STRIDE;
#pragma unroll
                    for (int ks = 0; ks < QF; ++ks)
                        s = __builtin_amdgcn_mfma_f32_16x16x4f32(krow[ks * 4 + g], qf[gq][ks], s, 0, 0, 0);
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
                            if (key > qi) sv = -INFINITY;
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
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float pv = st[c][i];
                        const float* vrow = sV + (c * 16 + g * 4 + i) * Lds::V_STRIDE;
#pragma unroll
                        for (int db = 0; db < NDB; ++db)
                            acc[gq][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[db * 16 + c16], pv,
                                                                               acc[gq][db], 0, 0, 0);
                    }
            }
        }
        if (more) {
            // The other stage was last read before the barrier that ended the
            // previous iteration.
            float* nK = stage_base + ((kt + 1) & 1) * Lds::STAGE;
            f32_store<D>(next, nK, nK + Lds::K_ELEMS);
        }
        __syncthreads();
    }

    // ---- normalise and store: lane holds O^T[d = db*16 + 4g + i][q = c16] ----
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
        const int qi = q_wave0 + gq * 16 + c16;
        if (qi >= L) continue;
        const float inv = 1.0f / l_run[gq];
        float* orow = pa.out + wk.b * pa.os[0] + wk.h * pa.os[1] + qi * pa.os[2];
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            float4 o4 = make_float4(acc[gq][db][0] * inv, acc[gq][db][1] * inv, acc[gq][db][2] * inv,
                                    acc[gq][db][3] * inv);
            *reinterpret_cast<float4*>(orow + db * 16 + g * 4) = o4;
        }
    }
}

// ===========================================================================
// Launch
// ===========================================================================
template <class Kernel>
sa_status opt_in_lds(Kernel* kernel, int bytes) {
    if (bytes <= 65536) return SA_OK;
    // Tiles above 64 KiB of LDS need the per-device opt-in.
    static thread_local int opted_device = -1;
    int dev = 0;
    SA_HIP_TRY(hipGetDevice(&dev));
    if (opted_device != dev) {
        SA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
        opted_device = dev;
    }
    return SA_OK;
}

// bf16 shape: W waves of QB 32-query blocks each.  Measured at L = 8192 on
// MI355X: 4 waves x 64 queries (one wave per SIMD) 0.383 ms, 8 waves x 32
// queries (two per SIMD) 0.414 ms.
constexpr int kBfQB = 2;
constexpr int kBfW = 4;

template <int D, int QB, int W>
sa_status launch_bf16(const PrefillArgs& pa, dim3 grid, hipStream_t st) {
    constexpr int bytes = BfLds<D, W>::BYTES;
    sa_status s = opt_in_lds(&prefill_bf16_kernel<D, QB, W>, bytes);
    if (s != SA_OK) return s;
    hipLaunchKernelGGL((prefill_bf16_kernel<D, QB, W>), grid, dim3(W * 64), bytes, st, pa);
    return SA_OK;
}

sa_status launch(PrefillArgs pa, int B, bool bf16, int D, hipStream_t st) {
    const int q_tile = bf16 ? kBfW * kBfQB * 32 : kFQTile;
    pa.n_qt = (pa.L + q_tile - 1) / q_tile;
    const int groups = B * pa.Hkv;
    pa.xcd_groups = groups % 8 == 0 ? groups / 8 : 0;
    const long long n_wg = (long long)B * pa.Hq * pa.n_qt;
    if (n_wg > 0x7fffffffLL) return fail(SA_ERANGE, "prefill grid too large");
    const dim3 grid(static_cast<unsigned>(n_wg));
    sa_status s = SA_OK;
    if (bf16) {
        s = D == 64 ? launch_bf16<64, kBfQB, kBfW>(pa, grid, st) : launch_bf16<128, kBfQB, kBfW>(pa, grid, st);
    } else if (D == 64) {
        s = opt_in_lds(&prefill_f32_kernel<64>, F32Lds<64>::BYTES);
        if (s == SA_OK)
            hipLaunchKernelGGL(prefill_f32_kernel<64>, grid, dim3(kFThreads), F32Lds<64>::BYTES, st, pa);
    } else {
        s = opt_in_lds(&prefill_f32_kernel<128>, F32Lds<128>::BYTES);
        if (s == SA_OK)
            hipLaunchKernelGGL(prefill_f32_kernel<128>, grid, dim3(kFThreads), F32Lds<128>::BYTES, st, pa);
    }
    if (s != SA_OK) return s;
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
    // The kernels index rows inside one (batch, head) with 32-bit element offsets.
    if ((int64_t)L * qs[2] >= (1LL << 31) || (int64_t)L * kvs[2] >= (1LL << 31) ||
        (int64_t)L * os[2] >= (1LL << 31))
        return fail(SA_ERANGE, "L * row stride must stay below 2^31 elements");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return fail(SA_EINVAL, "q, k, v and out must be 16-byte aligned");
    PrefillArgs pa{};
    pa.q = q; pa.k = k; pa.v = v; pa.out = out;
    for (int i = 0; i < 3; ++i) { pa.qs[i] = qs[i]; pa.kvs[i] = kvs[i]; pa.os[i] = os[i]; }
    pa.Hq = n_q_heads; pa.Hkv = n_kv_heads; pa.L = L;
    pa.scale = scale;
    pa.sl2 = fabsf(scale) * kLog2eP;
    pa.q_sign = scale < 0.f ? 0x80008000u : 0u;
    return launch(pa, batch, dtype == SA_DTYPE_BF16, D, st);
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
