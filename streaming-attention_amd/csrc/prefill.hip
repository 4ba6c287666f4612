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
// bf16 inputs (v_mfma_f32_32x32x16_bf16, fp32 accumulation): a wave owns 32
// queries; a workgroup of 8 waves (4 when the grid would not fill the CUs
// twice) serves the query heads of one KV group (GQA 2 with 8 waves: 4 waves
// x 32 queries for each of the two heads), so every K/V tile staged in LDS
// feeds all of them.  The running max is raised lazily: a wave
// rescales its accumulators only when some score exceeds the current max by
// more than 2^8, and then after the PV product (exact), so the common tile
// has no branch between softmax and PV.  P is rounded to bf16 for the PV
// product; the row sums use the fp32 p.  Prompts too short to give every CU
// a workgroup run 32-query workgroups that split each key range between two
// wave groups and merge the halves in LDS.
//
// fp32 inputs (v_mfma_f32_16x16x4f32): a wave owns 32 queries as two
// 16-query blocks, a workgroup 128 queries, eager rescale.
#include <cstdlib>
#include <numeric>
#include <type_traits>

#include "prefill_shared.h"

namespace sa {
namespace {
using namespace pf;


// ===========================================================================
// bf16 kernel
// ===========================================================================
// A wave owns QB 32-query blocks; a workgroup of W waves owns W * QB * 32
// queries and streams 64-key K/V tiles through two LDS stages.
constexpr float kLazyRescale = 8.f;              // log2 headroom before a rescale
constexpr float kHugeExcess = 64.f;              // beyond this the softmax waits for the rescale

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
    extern __shared__ __align__(16) unsigned char smem[];
    uint16_t* stage_base = reinterpret_cast<uint16_t*>(smem);

    const int L = pa.L;
    const Work wk = map_work(pa, blockIdx.x);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n = lane & 31;        // query column inside a 32-query block
    const int hh = lane >> 5;       // lane half
    const float sl2 = pa.sl2;
    // In an 8-wave workgroup waves w and w + 4 share a SIMD.  The first of
    // each pair runs at a raised priority throughout, so when both are ready to issue it goes
    // first and the pair drifts out of phase: one wave's MFMAs overlap the
    // other's softmax instead of the two interleaving MFMA for MFMA.
    if (W >= 8 && __builtin_amdgcn_readfirstlane(wave) < W / 2) __builtin_amdgcn_s_setprio(1);

    // The workgroup's gh query heads share every K/V tile: W / gh waves per
    // head, each wave QWAVE consecutive queries of its head.
    const int wph = W / pa.gh;
    const int qtile = wph * QWAVE;                   // query positions per workgroup
    const int h = wk.h0 + wave / wph;
    const uint16_t* Q = static_cast<const uint16_t*>(pa.q) + wk.b * pa.qs[0] + h * pa.qs[1];
    const uint16_t* K = static_cast<const uint16_t*>(pa.k) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const uint16_t* V = static_cast<const uint16_t*>(pa.v) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const int kv_row = static_cast<int>(pa.kvs[2]);

    const int q_wave0 = wk.qt * qtile + (wave % wph) * QWAVE;
    const int n_kt = (min(L, (wk.qt + 1) * qtile) - 1) / kKTile + 1;
    // Tiles this wave computes: keys up to its last query.  The last one is
    // the diagonal tile; dq is the wave's first query relative to it.
    const int wave_kt = q_wave0 < L ? (q_wave0 + QWAVE - 1) / kKTile + 1 : 0;
    const int dq = q_wave0 - (wave_kt - 1) * kKTile;

    const BfLoadMap<D, W> mp;
    // Tile registers: tile kt+1 waits in one set while tile kt+2 is in flight
    // in the other, so a tile's global loads have two tiles of compute to land.
    BfStage<D, W> ra, rb;
    bf_load<D, W>(ra, mp, K, V, kv_row, 0, L);

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

    bf_store<D, W>(ra, mp, stage_base, stage_base + Lds::K_ELEMS);
    bf_load<D, W>(rb, mp, K, V, kv_row, kKTile, L);
    bf_load<D, W>(ra, mp, K, V, kv_row, 2 * kKTile, L);
    __syncthreads();

    // One iteration: compute tile kt from LDS stage kt & 1, move tile kt+1
    // (held) into the other stage, and issue tile kt+3's loads into held.
    // Past the last tile the loads read clamped, in-range rows into stages
    // nobody reads.
    auto step = [&](int kt, BfStage<D, W>& held) {
        const uint16_t* sK = stage_base + (kt & 1) * Lds::STAGE;

        // One tile, as two 32-key halves kb.  Per half, for each query block
        // qb: scores, a softmax relative to the current running max m, the PV
        // product.  A raised max is applied after the PV product: with
        // p' = 2^(s c - m) and a = 2^(m - m_new), a O + PV(p' a) = a (O + PV(p')),
        // exact as long as p' stays finite, so the common path has no branch
        // between softmax and PV and the softmax of block 0 overlaps the score
        // MFMAs of block 1, the softmax of block 1 the PV MFMAs of block 0.
        // Only an excess above 2^kHugeExcess (a wave's first tile, in practice)
        // rescales before the softmax.  DIAG instantiates the diagonal mask.
        // LDS fragment reads run ahead of their use: the V fragments of a half
        // are read before its softmax, the K fragments of the second half
        // before the first half's PV product.
        auto tile = [&](auto diag_tag) {
            constexpr bool DIAG = decltype(diag_tag)::value;
            bf16x8_t kf[NKS];
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) kf[ks] = lds_b128(sK + k_off + ks * 16);
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                // Element j of a score block is key kt*64 + 32 kb + 16 (j/8) + 8 hh + j%8
                // for query q_wave0 + 32 qb + n.  On the diagonal tile keys past
                // the query are removed (query - kt*64 = dq + 32 qb + n).
                auto masked = [&](int qb, int j) {
                    return DIAG && 32 * kb + 16 * (j / 8) + 8 * hh + (j % 8) > dq + 32 * qb + n;
                };
                auto scores = [&](int qb) {
                    f32x16_t sc = {};
#pragma unroll
                    for (int ks = 0; ks < NKS; ++ks)
                        sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[qb][ks], sc, 0, 0, 0);
                    if constexpr (DIAG) {
#pragma unroll
                        for (int j = 0; j < 16; ++j)
                            if (masked(qb, j)) sc[j] = -INFINITY;
                    }
                    return sc;
                };
                auto row_max = [&](const f32x16_t& sc) {
                    float mt = sc[0];
#pragma unroll
                    for (int j = 1; j < 16; ++j) mt = fmaxf(mt, sc[j]);
                    return mt;
                };
                // Raise m to this half's exact row max (both lane halves agree)
                // and scale what was accumulated; returns the scale factor.
                auto raise = [&](int qb, float mt) {
                    const float mq = fmaxf(mt, __shfl_xor(mt, 32, 64));
                    const float m_new = fmaxf(ms[qb], mq * sl2);
                    const float alpha = ms[qb] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms[qb] - m_new);
#pragma unroll
                    for (int db = 0; db < NDB; ++db) acc[qb][db] *= alpha;
                    lp[qb] *= alpha;
                    ms[qb] = m_new;
                };
                auto softmax = [&](int qb, const f32x16_t& sc, bf16x8_t (&pb)[2]) {
                    const float nm = -ms[qb];
                    float p[16];
                    float rs = 0.f;
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[j], sl2, nm));
                        if (masked(qb, j)) p[j] = 0.f;   // exact zero also for a zero scale
                        rs += p[j];
                    }
                    lp[qb] += rs;
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const bf16x2_t p01 = __builtin_convertvector(f32x2_t{p[8 * t + 0], p[8 * t + 1]}, bf16x2_t);
                        const bf16x2_t p23 = __builtin_convertvector(f32x2_t{p[8 * t + 2], p[8 * t + 3]}, bf16x2_t);
                        const bf16x2_t p45 = __builtin_convertvector(f32x2_t{p[8 * t + 4], p[8 * t + 5]}, bf16x2_t);
                        const bf16x2_t p67 = __builtin_convertvector(f32x2_t{p[8 * t + 6], p[8 * t + 7]}, bf16x2_t);
                        pb[t] = __builtin_bit_cast(
                            bf16x8_t, make_uint4(__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23),
                                                 __builtin_bit_cast(uint32_t, p45), __builtin_bit_cast(uint32_t, p67)));
                    }
                };
                f32x16_t s[QB];
                float mt[QB];
                bf16x8_t pb[QB][2];
                bf16x8_t vf[NDB][2];
                auto load_v = [&]() {
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int t = 0; t < 2; ++t)
                            vf[db][t] = lds_b128(sK + v_off + db * 32 * Lds::V_STRIDE + kb * 32 + t * 16);
                };
                // ---- O^T += V^T P^T over these 32 keys ----
                auto pv = [&](int qb) {
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
#pragma unroll
                        for (int t = 0; t < 2; ++t)
                            acc[qb][db] =
                                __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][t], pb[qb][t], acc[qb][db], 0, 0, 0);
                };
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    s[qb] = scores(qb);
                    if (qb == QB - 1) load_v();
                    mt[qb] = row_max(s[qb]);
                    if (__any(mt[qb] * sl2 > ms[qb] + kHugeExcess)) raise(qb, mt[qb]);
                    softmax(qb, s[qb], pb[qb]);
                }
                if (kb == 0) {
#pragma unroll
                    for (int ks = 0; ks < NKS; ++ks) kf[ks] = lds_b128(sK + k_off + 32 * Lds::K_STRIDE + ks * 16);
                }
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) pv(qb);
                // A max that rose by more than 2^kLazyRescale: rescale now (after PV, exact).
                bool up = false;
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) up = up || mt[qb] * sl2 > ms[qb] + kLazyRescale;
                if (__any(up)) {
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb) raise(qb, mt[qb]);
                }
            }
        };
        if (kt + 1 < wave_kt) tile(std::false_type{});
        else if (kt + 1 == wave_kt) tile(std::true_type{});

        // The other stage was last read before the barrier that ended the
        // previous iteration.
        uint16_t* nK = stage_base + ((kt + 1) & 1) * Lds::STAGE;
        bf_store<D, W>(held, mp, nK, nK + Lds::K_ELEMS);
        bf_load<D, W>(held, mp, K, V, kv_row, (kt + 3) * kKTile, L);
        __syncthreads();
    };
    for (int kt = 0; kt < n_kt; kt += 2) {
        step(kt, rb);
        if (kt + 1 < n_kt) step(kt + 1, ra);
    }

    // ---- normalise and store: element j of acc[qb][db] is
    //      O[q_wave0 + 32 qb + n][32 db + 8 (j/4) + 4 hh + j%4] ----
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const float l = lp[qb] + __shfl_xor(lp[qb], 32, 64);
        const int qi = q_wave0 + qb * 32 + n;
        if (qi >= L) continue;
        const float inv = 1.0f / l;
        float* orow = pa.out + wk.b * pa.os[0] + h * pa.os[1] + qi * pa.os[2] + 4 * hh;
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
// bf16 kernel, head_dim 128, tiles moved by the load unit, folded softmax
// ===========================================================================
// One 32-query block per wave, like prefill_bf16_kernel, with two changes.
//
// Data movement: tiles go from global memory straight into LDS with
// global_load_lds_dwordx4: no staging registers, no LDS stores, no V
// transposition on the way in.  K and V sit row-major in LDS (256-byte rows)
// with the 16-byte chunks of row r permuted by dma_swz(r); the V^T fragments
// of the PV product come from ds_read_b64_tr_b16.  NS stages: tile kt + NS - 1
// is loaded while tile kt is computed.  Tiles past the last one are never
// loaded, so the stages of the last NS - 1 tiles are intact after the loop;
// every wave's diagonal tile is among them (the launch checks that a
// workgroup's queries span at most NS - 1 tiles) and is processed there,
// which keeps the mask out of the main loop.
//
// Softmax, with less work per score:
//   * q is pre-scaled once, q' = bf16(q * scale * log2 e), and the score MFMA
//     chain starts from -m (a register block holding the running max of each
//     query column), so the MFMA delivers s' = q'.k - m and p = 2^s' needs no
//     multiply or subtract;
//   * no per-tile row max: a lane's 16 p values are summed (bf16 dot products
//     of the packed P that the PV product uses), and only when a sum exceeds
//     2^16, which bounds every p by 2^16, does a slow path compute the row max,
//     raise m (rescaling O and the row sum), and recompute P; the first tile
//     of a wave always takes it (m starts at -inf, the bias at 0);
//   * the row sums use the bf16 P of the PV product, so the normalised
//     weights are the ones applied.
// Measured at L = 8192 (16/8 heads, same box, interleaved): 251 us against
// 258-264 us for the same schedule with a per-tile row max, a scaled fma per
// score and fp32 row sums (34 VALU per half-tile instead of about 75).
// One wave's share of the folded-softmax kernels: the scores of its 32
// queries against the 32-key halves of a K/V tile staged in LDS (K rows
// permuted by dma_swz, V^T read with ds_read_b64_tr_b16), the folded softmax
// with its lazy raise of the running max, and the O^T accumulators.
struct FoldWave {
    static constexpr int NKS = 8;   // k-steps of the score product
    static constexpr int NDB = 4;   // 32-row d blocks of O^T
    int n, hh;                      // this lane's query column in the wave's block, and its half
    int q0;                         // the wave's first query
    bf16x8_t qf[NKS];
    f32x16_t acc[NDB];
    float ms;                       // running max of this query (log2 domain) at the last raise
    float lp;                       // this lane's part of the row sum
    float cap;                      // kSumCap once ms is finite: the first tile always raises
    f32x16_t negm;                  // -ms in every element (0 while ms = -inf): the score chain's start
    int k_off[NKS];
    int v_off[2][NDB];

    // q' = bf16(q * scale * log2 e) for query q_first + n (clamped to the
    // sequence) of the head whose rows start at Q with row stride q_row; the
    // scores then come out in the log2 domain.
    __device__ __forceinline__ void init(const uint16_t* Q, long long q_row, int q_first, int L, float scale,
                                         int lane) {
        n = lane & 31;
        hh = lane >> 5;
        q0 = q_first;
        {
            const float sq = scale * kLog2eP;
            const int qi = min(q0 + n, L - 1);
            const uint16_t* qrow = Q + qi * q_row + 8 * hh;
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) {
                const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(qrow + ks * 16);
                float x[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[2 * i] = bf16_lo(raw[i]) * sq;
                    x[2 * i + 1] = bf16_hi(raw[i]) * sq;
                }
                qf[ks] = pack_bf16x8(x);
            }
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[db] = f32x16_t{};
        ms = -INFINITY;
        lp = 0.f;
        cap = -1.f;
        negm = f32x16_t{};
        {
            const int r = swap_bits23(n);
#pragma unroll
            for (int ks = 0; ks < NKS; ++ks) k_off[ks] = r * kDmaRowBytes + (((2 * ks + hh) ^ dma_swz(r & 15)) << 4);
        }
        {
            const int g = lane >> 4, j = lane & 15;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int r = 8 * hh + 4 * u + j / 4;
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    const int col = 32 * db + 16 * (g & 1) + 4 * (j & 3);
                    v_off[u][db] =
                        kDmaTileBytes + r * kDmaRowBytes + (((col >> 3) ^ dma_swz(r & 15)) << 4) + (col & 7) * 2;
                }
            }
        }
    }

    __device__ __forceinline__ bf16x8_t lds_k(const lds_u8_t* sb, int kb, int ks) const {
        return *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(sb + kb * 32 * kDmaRowBytes +
                                                                                     k_off[ks]);
    }
    __device__ __forceinline__ bf16x8_t lds_vt(const lds_u8_t* sb, int kb, int t, int db) const {
        const lds_u8_t* p = sb + (kb * 32 + t * 16) * kDmaRowBytes;
        const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p + v_off[0][db]));
        const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(p + v_off[1][db]));
        return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }

    // Scores of one 32-key half, biased by -m: element j is key 16 (j/8) +
    // 8 hh + j%8 of the half for query q0 + n.
    __device__ __forceinline__ f32x16_t scores(const bf16x8_t (&kf)[NKS]) const {
        f32x16_t s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[0], qf[0], negm, 0, 0, 0);
#pragma unroll
        for (int ks = 1; ks < NKS; ++ks) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], s, 0, 0, 0);
        return s;
    }
    // P = 2^s as the PV product's B operand, and this lane's sum of it.
    // This lane's sum of the 16 bf16 P values: two independent chains of
    // four dot products each (one chain of eight measured 1 % slower at
    // L = 8192).
    __device__ __forceinline__ static float psum(const bf16x8_t (&pb)[2]) {
        return sum_bf16x8(pb[1], 0.f) + sum_bf16x8(pb[0], 0.f);
    }
    __device__ __forceinline__ static float softmax(const f32x16_t& s, bf16x8_t (&pb)[2]) {
        float p[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) p[j] = __builtin_amdgcn_exp2f(s[j]);
        pb[0] = pack_bf16x8(p);
        pb[1] = pack_bf16x8(p + 8);
        return psum(pb);
    }
    // Raise m to the row max of this half when the sum left the cap (or m is
    // still -inf): O and the row sum are rescaled and P recomputed.
    __device__ __forceinline__ void settle(const f32x16_t& s, bf16x8_t (&pb)[2], float& rs) {
        if (!__any(!(rs <= cap))) return;
        float mt = s[0];
#pragma unroll
        for (int j = 1; j < 16; ++j) mt = fmaxf(mt, s[j]);
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
        const float b = negm[0];
        const float mq = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) - b;   // unbiased row max
        const float m_new = fmaxf(ms, mq);
        const float alpha = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - m_new);
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[db] *= alpha;
        lp *= alpha;
        const float b_new = m_new == -INFINITY ? 0.f : -m_new;
        const float delta = b_new - b;
        float p[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) p[j] = __builtin_amdgcn_exp2f(s[j] + delta);
        pb[0] = pack_bf16x8(p);
        pb[1] = pack_bf16x8(p + 8);
        rs = psum(pb);
        ms = m_new;
        cap = m_new == -INFINITY ? -1.f : kSumCap;
#pragma unroll
        for (int j = 0; j < 16; ++j) negm[j] = b_new;
    }
    __device__ __forceinline__ void pv(const bf16x8_t (&vf)[NDB][2], const bf16x8_t (&pb)[2]) {
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int t = 0; t < 2; ++t) acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[db][t], pb[t], acc[db], 0, 0, 0);
    }

    // Tile kt (keys 64 kt ..) from LDS stage sb, per 32-key half: scores,
    // mask (the diagonal tile only), P, settle, PV.
    template <bool DIAG>
    __device__ __forceinline__ void tile(int kt, const lds_u8_t* sb) {
        bf16x8_t kf[NKS];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) kf[ks] = lds_k(sb, 0, ks);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x16_t s = scores(kf);
            if constexpr (DIAG) {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    if (kt * kKTile + 32 * kb + 16 * (j / 8) + 8 * hh + (j % 8) > q0 + n) s[j] = -INFINITY;
            }
            bf16x8_t vf[NDB][2];
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int t = 0; t < 2; ++t) vf[db][t] = lds_vt(sb, kb, t, db);
            bf16x8_t pb[2];
            float rs = softmax(s, pb);
            settle(s, pb, rs);
            lp += rs;
            if (kb == 0) {
#pragma unroll
                for (int ks = 0; ks < NKS; ++ks) kf[ks] = lds_k(sb, 1, ks);
            }
            pv(vf, pb);
        }
    }

    // O / l for query q0 + n (when inside the sequence), row-major from orow0
    // (the head's first output row) with row stride o_row.
    __device__ __forceinline__ void store(float* orow0, long long o_row, int L) const {
        const float l = lp + __shfl_xor(lp, 32, 64);
        const int qi = q0 + n;
        if (qi >= L) return;
        const float inv = 1.0f / l;
        float* orow = orow0 + qi * o_row + 4 * hh;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                *reinterpret_cast<float4*>(orow + 32 * db + 8 * jj) =
                    make_float4(acc[db][4 * jj] * inv, acc[db][4 * jj + 1] * inv, acc[db][4 * jj + 2] * inv,
                                acc[db][4 * jj + 3] * inv);
    }
};

// Per-lane rows and columns of the tile loads of a W-wave workgroup: load i
// of a wave copies 4 rows x 256 bytes (16 lanes per row), 16 / W loads per
// wave cover a 64-row tile.
template <int W>
struct DmaMap {
    static constexpr int NI = 16 / W;
    int row[NI], col[NI];
    __device__ __forceinline__ DmaMap(int wave, int lane) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int r = 4 * (wave * NI + i) + lane / 16;
            row[i] = r;
            col[i] = 8 * ((lane % 16) ^ dma_swz(r & 15));
        }
    }
    // K and V rows key0 .. key0 + 63 (clamped to the sequence) into the tile
    // slot sb: K at sb, V at sb + kDmaTileBytes.
    __device__ __forceinline__ void load(const uint16_t* K, const uint16_t* V, int kv_row, int key0, int L,
                                         int wave, lds_u8_t* sb) const {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const long long e = (long long)min(key0 + row[i], L - 1) * kv_row + col[i];
            lds_u8_t* dst = sb + (wave * NI + i) * 1024;
            dma16(K + e, dst);
            dma16(V + e, dst + kDmaTileBytes);
        }
    }
};

template <int W, int NS>
__global__ void __launch_bounds__(W * 64)
prefill_bf16_fold_kernel(PrefillArgs pa) {
    constexpr int NDB = FoldWave::NDB;
    constexpr int NI = DmaMap<W>::NI;   // loads per wave, tensor and tile (64 lanes x 16 bytes each)
    extern __shared__ __align__(16) unsigned char smem[];
    lds_u8_t* const lsm = (lds_u8_t*)smem;

    const int L = pa.L;
    const Work wk = map_work(pa, blockIdx.x);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    const int wph = W / pa.gh;
    const int qtile = wph * 32;
    const int h = wk.h0 + wave / wph;
    const uint16_t* Q = static_cast<const uint16_t*>(pa.q) + wk.b * pa.qs[0] + h * pa.qs[1];
    const uint16_t* K = static_cast<const uint16_t*>(pa.k) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const uint16_t* V = static_cast<const uint16_t*>(pa.v) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const int kv_row = static_cast<int>(pa.kvs[2]);

    const int q_wave0 = wk.qt * qtile + (wave % wph) * 32;
    const int n_kt = (min(L, (wk.qt + 1) * qtile) - 1) / kKTile + 1;
    const int wave_kt = q_wave0 < L ? (q_wave0 + 31) / kKTile + 1 : 0;

    const DmaMap<W> dm(wave, lane);
    auto dma_tile = [&](int kt, int stage) {
        dm.load(K, V, kv_row, kt * kKTile, L, wave, lsm + stage * kDmaStageBytes);
    };
#pragma unroll
    for (int s = 0; s < (W == 8 ? NS : NS - 1); ++s) dma_tile(s, s);

    FoldWave fw;
    fw.init(Q, pa.qs[2], q_wave0, L, pa.scale, lane);

    constexpr int VM = (NS - 2) * 2 * NI;
    static_assert(VM == 0 || VM == 4 || VM == 8, "vmcnt literal");
    auto next_tile_ready = [&]() {
        if constexpr (VM == 0) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else if constexpr (VM == 4) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    if constexpr (W == 8) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else next_tile_ready();   // tile 0

    if constexpr (W == 8) {
        // Ping-pong schedule: waves w and w + 4 share a SIMD (read from
        // HW_ID).  Each 32-key half is an MFMA block (the previous half's PV,
        // then this half's scores) and a softmax block.  Waves 4-7 take the
        // half's barrier between their two blocks, waves 0-3 after both, so
        // on every SIMD one wave's softmax runs while the other issues MFMAs.
        // The previous half's P and V^T fragments stay in registers across
        // the barrier.  The loop covers the tiles every wave computes off its
        // diagonal, without per-wave branches; the remaining tiles and each
        // wave's diagonal run one tile per barrier.  Tile kt + 2 loads once
        // every wave is done with tile kt.
        static_assert(NS == 2 && NI == 2, "ping-pong schedule: two stages, two loads per tensor tile");
        const bool late = wave >= W / 2;
        // The early waves' MFMAs go first when both waves of a SIMD have some
        // ready, so the early wave's softmax starts sooner (L = 8192, same
        // box: 1 % faster; the late waves first: 2 % slower).
        if (!late) __builtin_amdgcn_s_setprio(1);
        bf16x8_t pv_v[NDB][2];
        bf16x8_t pv_p[2];
#pragma unroll
        for (int db = 0; db < NDB; ++db) pv_v[db][0] = pv_v[db][1] = bf16x8_t{};
        pv_p[0] = pv_p[1] = bf16x8_t{};
        auto end_tile = [&](int kt, int stage) {
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (kt + NS < n_kt) dma_tile(kt + NS, stage);
        };
        // The second half of a tile takes its first kKPre K fragments from
        // reads issued during the first half's softmax, so its score MFMAs do
        // not wait on them (all eight read there spill at 256 VGPRs; L = 8192,
        // same box: 0.2361-0.2364 against 0.2420 ms, five 0.2400, seven 0.2410).
        constexpr int kKPre = 6;
        bf16x8_t kf_next[kKPre];
        auto half = [&](int kt, int stage, int kb) {
            const lds_u8_t* sb = lsm + stage * kDmaStageBytes;
            bf16x8_t kf[FoldWave::NKS];
#pragma unroll
            for (int ks = 0; ks < FoldWave::NKS; ++ks)
                kf[ks] = kb == 1 && ks < kKPre ? kf_next[ks] : fw.lds_k(sb, kb, ks);
            fw.pv(pv_v, pv_p);
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int t = 0; t < 2; ++t) pv_v[db][t] = fw.lds_vt(sb, kb, t, db);
            const f32x16_t s = fw.scores(kf);
            auto sync = [&]() {
                __builtin_amdgcn_sched_barrier(0);
                if (kb == 0) asm volatile("s_barrier" ::: "memory");
                else end_tile(kt, stage);
                __builtin_amdgcn_sched_barrier(0);
            };
            if (late) sync();
            if (kb == 0) {
#pragma unroll
                for (int ks = 0; ks < kKPre; ++ks) kf_next[ks] = fw.lds_k(sb, 1, ks);
                __builtin_amdgcn_sched_barrier(0);
            }
            float rs = FoldWave::softmax(s, pv_p);
            fw.settle(s, pv_p, rs);
            fw.lp += rs;
            if (!late) sync();
        };
        const int kt_pp = (wk.qt * qtile + 31) / kKTile / NS * NS;
        for (int kt = 0; kt < kt_pp; kt += NS) {
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                half(kt + s, s, 0);
                half(kt + s, s, 1);
            }
        }
        fw.pv(pv_v, pv_p);
        for (int kt = kt_pp; kt < n_kt; ++kt) {
            const int stage = kt % NS;
            if (kt + 1 < wave_kt) fw.tile<false>(kt, lsm + stage * kDmaStageBytes);
            end_tile(kt, stage);
        }
    } else {
        auto step = [&](int kt, int stage) {
            const bool more = kt + NS - 1 < n_kt;
            if (more) dma_tile(kt + NS - 1, (stage + NS - 1) % NS);
            if (kt + 1 < wave_kt) fw.tile<false>(kt, lsm + stage * kDmaStageBytes);
            if (more) next_tile_ready();
            else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        };
        const int n_steps = (n_kt + NS - 1) / NS * NS;
        for (int kt = 0; kt < n_steps; kt += NS) {
#pragma unroll
            for (int s = 0; s < NS; ++s) step(kt + s, s);
        }
    }
    if (wave_kt > 0) fw.tile<true>(wave_kt - 1, lsm + ((wave_kt - 1) % NS) * kDmaStageBytes);

    fw.store(pa.out + wk.b * pa.os[0] + h * pa.os[1], pa.os[2], L);
}


// ===========================================================================
// bf16 kernel, head_dim 128, short prompts: each 32-query tile's key range
// split across wave groups of one workgroup
// ===========================================================================
// When even 4-wave workgroups leave CUs idle, the chain of key tiles that
// one workgroup walks sets the time (about 1.2 us per tile with one wave per
// SIMD, on top of a fixed ~6 us).  A workgroup here serves 32 queries of GH
// query heads of one KV group; its W = KS x GH waves form KS groups, group g
// walking tiles g, g + KS, ... of the shared key range, so a chain is
// ceil(n_kt / KS) tiles long.  One step stages the KS tiles of the groups
// (NS = 2 steps resident, loaded straight into LDS); the diagonal tile, the
// last one, stays in its stage after the loop and its group applies the
// mask there.  The groups' (m, l, O) partials then meet in LDS, where group
// 0 merges them (O = sum 2^(m_g - M) O_g, l likewise, M the largest m_g) and
// writes the output.  No second launch and no global workspace.
template <int KS, int GH>
__global__ void __launch_bounds__(KS * GH * 64)
prefill_bf16_split_kernel(PrefillArgs pa) {
    constexpr int W = KS * GH;
    constexpr int NDB = FoldWave::NDB;
    constexpr int STEP_BYTES = KS * kDmaStageBytes;
    extern __shared__ __align__(16) unsigned char smem[];
    lds_u8_t* const lsm = (lds_u8_t*)smem;

    const int L = pa.L;
    const Work wk = map_work(pa, blockIdx.x);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = wave / GH;                  // key group
    const int hl = wave % GH;                 // head of the workgroup's set
    const int h = wk.h0 + hl;
    const uint16_t* Q = static_cast<const uint16_t*>(pa.q) + wk.b * pa.qs[0] + h * pa.qs[1];
    const uint16_t* K = static_cast<const uint16_t*>(pa.k) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const uint16_t* V = static_cast<const uint16_t*>(pa.v) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const int kv_row = static_cast<int>(pa.kvs[2]);

    const int q0 = wk.qt * 32;
    const int n_kt = (min(L, q0 + 32) - 1) / kKTile + 1;   // tiles through the diagonal
    const int n_steps = (n_kt + KS - 1) / KS;

    const DmaMap<W> dm(wave, lane);
    auto dma_step = [&](int t, int stage) {
        lds_u8_t* sb = lsm + stage * STEP_BYTES;
#pragma unroll
        for (int s = 0; s < KS; ++s)
            if (t * KS + s < n_kt) dm.load(K, V, kv_row, (t * KS + s) * kKTile, L, wave, sb + s * kDmaStageBytes);
    };
    dma_step(0, 0);
    FoldWave fw;
    fw.init(Q, pa.qs[2], q0, L, pa.scale, lane);
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");   // step 0 resident

    // Step t: the loads of step t + 1 go out, then this group's tile of step
    // t unless it is the diagonal; every load has landed at the barrier.
    auto step = [&](int t, int stage) {
        if (t + 1 < n_steps) dma_step(t + 1, stage ^ 1);
        const int kt = t * KS + g;
        if (kt + 1 < n_kt) fw.tile<false>(kt, lsm + stage * STEP_BYTES + g * kDmaStageBytes);
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };
    for (int t = 0; t < n_steps; t += 2) {
        step(t, 0);
        step(t + 1, 1);
    }
    const int kd = n_kt - 1;
    if (g == kd % KS) fw.tile<true>(kd, lsm + ((kd / KS) & 1) * STEP_BYTES + g * kDmaStageBytes);

    // Partials of groups 1 .. KS-1 into LDS, [element][lane] per wave (the
    // stages are free once every wave is past the diagonal tile).
    constexpr int NE = NDB * 16 + 2;
    float* const part = reinterpret_cast<float*>(smem);
    __syncthreads();
    if (g > 0) {
        float* p = part + ((g - 1) * GH + hl) * NE * 64 + lane;
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) p[(db * 16 + j) * 64] = fw.acc[db][j];
        p[(NE - 2) * 64] = fw.ms;
        p[(NE - 1) * 64] = fw.lp;
    }
    __syncthreads();
    if (g != 0) return;
    // Group 0 always holds tile 0, so its m is finite; a group without a
    // tile carries m = -inf and weight 0.
#pragma unroll
    for (int o = 1; o < KS; ++o) {
        const float* p = part + ((o - 1) * GH + hl) * NE * 64 + lane;
        const float mo = p[(NE - 2) * 64], lo = p[(NE - 1) * 64];
        const float m = fmaxf(fw.ms, mo);
        const float a = __builtin_amdgcn_exp2f(fw.ms - m);
        const float b = mo == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - m);
#pragma unroll
        for (int db = 0; db < NDB; ++db)
#pragma unroll
            for (int j = 0; j < 16; ++j) fw.acc[db][j] = fw.acc[db][j] * a + p[(db * 16 + j) * 64] * b;
        fw.lp = fw.lp * a + lo * b;
        fw.ms = m;
    }
    fw.store(pa.out + wk.b * pa.os[0] + h * pa.os[1], pa.os[2], L);
}

// ===========================================================================
// fp32 kernel
// ===========================================================================
constexpr int kFQTile = 128;    // queries per workgroup (4 waves of 32; 64 with 16 per wave)
constexpr int kFThreads = 256;
constexpr int kF32SplitW = 8;   // waves of the short-prompt fp32 kernel

template <int D>
struct F32Lds {
    static constexpr int K_STRIDE = D + 4;           // K row-major [64][D + 4]
    static constexpr int V_STRIDE = D + 4;           // V row-major [64][D + 4]
    static constexpr int K_ELEMS = kKTile * K_STRIDE;
    static constexpr int STAGE = K_ELEMS + kKTile * V_STRIDE;   // floats per stage
    static constexpr int BYTES = 2 * STAGE * 4;
    static constexpr int CPR = D / 4;                // 16-byte chunks per row
};

// Register staging of one K/V tile, spread over the NT threads of a workgroup.
template <int D, int NT = kFThreads>
struct F32Stage {
    static constexpr int NK = kKTile * (D / 4) / NT;
    static_assert(NK >= 1 && NK * NT == kKTile * (D / 4), "tile chunks per thread");
    u32x4_t k[NK];
    u32x4_t v[NK];
};

template <int D, int NT>
__device__ __forceinline__ void f32_load(F32Stage<D, NT>& st, const float* K, const float* V, long long kv_row,
                                         int key0, int L) {
    using Lds = F32Lds<D>;
    const int rmax = L - 1 - key0;
#pragma unroll
    for (int i = 0; i < F32Stage<D, NT>::NK; ++i) {
        const int idx = threadIdx.x + i * NT;
        const long long off = min(idx / Lds::CPR, rmax) * kv_row + (idx % Lds::CPR) * 4;
        st.k[i] = *reinterpret_cast<const u32x4_t*>(K + key0 * kv_row + off);
        st.v[i] = *reinterpret_cast<const u32x4_t*>(V + key0 * kv_row + off);
    }
}

template <int D, int NT>
__device__ __forceinline__ void f32_store(const F32Stage<D, NT>& st, float* sK, float* sV) {
    using Lds = F32Lds<D>;
#pragma unroll
    for (int i = 0; i < F32Stage<D, NT>::NK; ++i) {
        const int idx = threadIdx.x + i * NT;
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

// Four waves of GQ groups of 16 queries: a workgroup serves 64 GQ queries
// of one head (GQ = 2: 128, GQ = 1: 64).
template <int D, int GQ = 2>
__global__ void __launch_bounds__(kFThreads)
prefill_f32_kernel(PrefillArgs pa) {
    using Lds = F32Lds<D>;
    constexpr int NT = kFThreads;
    constexpr int QW = 16 * GQ;            // queries per wave
    constexpr int QT = 4 * QW;             // queries per workgroup
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

    const float* Q = static_cast<const float*>(pa.q) + wk.b * pa.qs[0] + wk.h0 * pa.qs[1];
    const float* K = static_cast<const float*>(pa.k) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const float* V = static_cast<const float*>(pa.v) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const long long q_row = pa.qs[2], kv_row = pa.kvs[2];

    const int q_wave0 = wk.qt * QT + wave * QW;   // first query of this wave
    const int n_kt = (min(L, (wk.qt + 1) * QT) - 1) / kKTile + 1;

    F32Stage<D, NT> next;
    f32_load<D, NT>(next, K, V, kv_row, 0, L);

    // Q^T fragments (B operand) per 16-query group.
    float qf[GQ][QF];
#pragma unroll
    for (int gq = 0; gq < GQ; ++gq) {
        const int qi = min(q_wave0 + gq * 16 + c16, L - 1);
#pragma unroll
        for (int s = 0; s < QF; ++s) qf[gq][s] = Q[qi * q_row + s * 4 + g];
    }

    f32x4_t acc[GQ][NDB];
#pragma unroll
    for (int gq = 0; gq < GQ; ++gq)
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[gq][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run[GQ];
    float l_run[GQ];
#pragma unroll
    for (int gq = 0; gq < GQ; ++gq) { m_run[gq] = -INFINITY; l_run[gq] = 0.f; }

    f32_store<D, NT>(next, stage_base, stage_base + Lds::K_ELEMS);
    __syncthreads();

    for (int kt = 0; kt < n_kt; ++kt) {
        const int key0 = kt * kKTile;
        const float* sK = stage_base + (kt & 1) * Lds::STAGE;
        const float* sV = sK + Lds::K_ELEMS;
        const bool more = kt + 1 < n_kt;
        if (more) f32_load<D, NT>(next, K, V, kv_row, key0 + kKTile, L);

        if (key0 <= q_wave0 + QW - 1 && q_wave0 < L) {   // else the whole wave is above the diagonal
            const bool diag = key0 + kKTile - 1 > q_wave0;
#pragma unroll
            for (int gq = 0; gq < GQ; ++gq) {
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
            f32_store<D, NT>(next, nK, nK + Lds::K_ELEMS);
        }
        __syncthreads();
    }

    // ---- normalise and store: lane holds O^T[d = db*16 + 4g + i][q = c16] ----
#pragma unroll
    for (int gq = 0; gq < GQ; ++gq) {
        const int qi = q_wave0 + gq * 16 + c16;
        if (qi >= L) continue;
        const float inv = 1.0f / l_run[gq];
        float* orow = pa.out + wk.b * pa.os[0] + wk.h0 * pa.os[1] + qi * pa.os[2];
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            float4 o4 = make_float4(acc[gq][db][0] * inv, acc[gq][db][1] * inv, acc[gq][db][2] * inv,
                                    acc[gq][db][3] * inv);
            *reinterpret_cast<float4*>(orow + db * 16 + g * 4) = o4;
        }
    }
}

// ===========================================================================
// fp32 on bf16 MFMA, head_dim 128: exact three-term splits
// ===========================================================================
// An fp32 value x is the exact sum of three bf16 terms, t0 = rne(x),
// t1 = rne(x - t0), t2 = x - t0 - t1 (each difference is exact in fp32 and the
// last fits bf16 exactly).  A product x y of two fp32 operands is taken as
// the six products ti uj with i + j <= 2; the three left out are below
// 2^-24 |x y|, the rounding of an fp32 product.  Every bf16 x bf16 product is
// exact in fp32 and accumulates in fp32 (v_mfma_f32_16x16x32_bf16), so the
// scores q.k and the output sum p.v come out at fp32 accuracy, at 6 bf16
// MFMAs per fp32 product: 16/6 times the fp32 MFMA rate of
// v_mfma_f32_16x16x4f32.
//
// A wave owns 16 queries of one head; a workgroup of W waves serves gh query
// heads of one KV group, W / gh waves per head.  Key tiles of 32 rows are
// loaded as fp32 into registers one tile ahead, split into their three terms
// and stored to LDS (K terms and V terms, 48 KiB per stage, two stages).
// Scores S^T = K Q^T (two 16-key blocks, K rows permuted so that a lane's
// scores are the 8 consecutive keys the B operand of the PV product needs),
// folded softmax as in the bf16 kernels (q pre-scaled by scale log2(e), the
// score chain starting from -m, the running max raised lazily when a lane's
// sum of p exceeds kSumCap), P split into three terms, O^T += V^T P^T with
// the V^T operands read by ds_read_b64_tr_b16.
constexpr int kX3KTile = 32;                          // keys per tile
constexpr int kX3Row = 256;                           // bytes per LDS row: 128 bf16
constexpr int kX3TermBytes = kX3KTile * kX3Row;       // one term of one tensor's tile
constexpr int kX3StageBytes = 6 * kX3TermBytes;       // K terms 0-2, V terms 0-2
// Term pairs (of the first and the second operand) of a product.
constexpr int kX3Pairs = 6;
__host__ __device__ constexpr int x3_pair_a(int pr) { return pr == 2 || pr == 4 ? 1 : pr == 5 ? 2 : 0; }
__host__ __device__ constexpr int x3_pair_b(int pr) { return pr == 1 || pr == 4 ? 1 : pr == 3 ? 2 : 0; }

// 16-byte chunk c of tile row r sits at chunk position c ^ x3_swz(r): the
// rows one K-fragment read touches (8a + 4kb + b, a, b < 4) and the rows one
// V^T read touches (8G + 4u + b) land on distinct positions.
__device__ __forceinline__ int x3_swz(int r) { return ((r & 3) << 2) | ((r >> 3) & 3); }
__device__ __forceinline__ int x3_off(int r, int c16) { return r * kX3Row + ((c16 ^ x3_swz(r)) << 4); }

// x = t0 + t1 + t2 for a pair of fp32 values: three packed bf16 pairs.
__device__ __forceinline__ void x3_split2(float a, float b, uint32_t& t0, uint32_t& t1, uint32_t& t2) {
    t0 = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
    a -= bf16_lo(t0);
    b -= bf16_hi(t0);
    t1 = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
    a -= bf16_lo(t1);
    b -= bf16_hi(t1);
    t2 = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void x3_st(lds_u8_t* p, uint32_t a, uint32_t b) {
    *reinterpret_cast<__attribute__((address_space(3))) u32x2_t*>(p) = u32x2_t{a, b};
}

// Eight fp32 values as three bf16x8 terms.
__device__ __forceinline__ void x3_split8(const float* x, bf16x8_t (&t)[3]) {
    uint32_t w[3][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) x3_split2(x[2 * i], x[2 * i + 1], w[0][i], w[1][i], w[2][i]);
#pragma unroll
    for (int k = 0; k < 3; ++k) t[k] = __builtin_bit_cast(bf16x8_t, u32x4_t{w[k][0], w[k][1], w[k][2], w[k][3]});
}

template <int W, bool PAIRED>
__global__ void __launch_bounds__(W * 64)
prefill_f32x3_kernel(PrefillArgs pa) {
    constexpr int NT = W * 64;
    constexpr int NC = kX3KTile * 32 / NT;   // 16-byte fp32 chunks per thread and tensor of a tile
    static_assert(NC >= 1 && NC * NT == kX3KTile * 32, "tile chunks per thread");
    extern __shared__ __align__(16) unsigned char smem[];
    lds_u8_t* const lsm = (lds_u8_t*)smem;

    const int L = pa.L;
    const Work wk = map_work(pa, blockIdx.x);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, g = lane >> 4;
    const int wph = W / pa.gh;
    const int qtile = wph * 16;
    const int h = wk.h0 + wave / wph;
    const float* Q = static_cast<const float*>(pa.q) + wk.b * pa.qs[0] + h * pa.qs[1];
    const float* K = static_cast<const float*>(pa.k) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const float* V = static_cast<const float*>(pa.v) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const long long kv_row = pa.kvs[2];

    // ---- segments: (query tile, key tiles [k0, k1), output) ----
    const PairSegs sg = PAIRED ? pair_segments(pa, wk.qt, qtile, kX3KTile)
                               : PairSegs{1, {wk.qt, 0}, {0, 0}, {pair_key_tiles(L, qtile, kX3KTile, wk.qt), 0},
                                          {-1, -1}};

    // ---- tile staging: fp32 rows in registers, three bf16 terms in LDS ----
    f32x4_t sk[NC], sv[NC];
    auto load_tile = [&](int kt) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int idx = threadIdx.x + i * NT;
            const long long key = min(kt * kX3KTile + (idx >> 5), L - 1);
            const long long e = key * kv_row + 4 * (idx & 31);
            sk[i] = *reinterpret_cast<const f32x4_t*>(K + e);
            sv[i] = *reinterpret_cast<const f32x4_t*>(V + e);
        }
    };
    auto store_tile = [&](int stage) {
        lds_u8_t* base = lsm + stage * kX3StageBytes;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int idx = threadIdx.x + i * NT;
            const int r = idx >> 5, c4 = idx & 31;
            const int off = x3_off(r, c4 >> 1) + (c4 & 1) * 8;
            uint32_t k0a, k1a, k2a, k0b, k1b, k2b, v0a, v1a, v2a, v0b, v1b, v2b;
            x3_split2(sk[i][0], sk[i][1], k0a, k1a, k2a);
            x3_split2(sk[i][2], sk[i][3], k0b, k1b, k2b);
            x3_split2(sv[i][0], sv[i][1], v0a, v1a, v2a);
            x3_split2(sv[i][2], sv[i][3], v0b, v1b, v2b);
            x3_st(base + 0 * kX3TermBytes + off, k0a, k0b);
            x3_st(base + 1 * kX3TermBytes + off, k1a, k1b);
            x3_st(base + 2 * kX3TermBytes + off, k2a, k2b);
            x3_st(base + 3 * kX3TermBytes + off, v0a, v0b);
            x3_st(base + 4 * kX3TermBytes + off, v1a, v1b);
            x3_st(base + 5 * kX3TermBytes + off, v2a, v2b);
        }
    };

    // K fragment rows: block kb's row r16 is tile key 8 (r16 / 4) + 4 kb + r16 % 4,
    // so score element e of block kb is key 8 g + 4 kb + e of the lane's query.
    int k_off[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        const int r = 8 * (r16 >> 2) + 4 * kb + (r16 & 3);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) k_off[kb][ks] = x3_off(r, 4 * ks + g);
    }
    // V^T reads (ds_read_b64_tr_b16, read u of d block db): source lane s of
    // the lane's 16-group reads row 8 g + 4 u + s / 4, columns 16 db + 4 (s % 4) ..;
    // output lane r16 then holds V[8 g + 4 u + e][16 db + r16], e < 4.
    int v_off[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int r = 8 * g + 4 * u + (r16 >> 2);
#pragma unroll
        for (int db = 0; db < 8; ++db) {
            const int col = 16 * db + 4 * (r16 & 3);
            v_off[u][db] = 3 * kX3TermBytes + x3_off(r, col >> 3) + (col & 7) * 2;
        }
    }

    const int segs = PAIRED ? sg.n : 1;
#pragma unroll 1
    for (int si = 0; si < segs; ++si) {
        const int qt = si ? sg.qt[1] : sg.qt[0], k0 = si ? sg.k0[1] : sg.k0[0], k1 = si ? sg.k1[1] : sg.k1[0];
        const int q0 = qt * qtile + (wave % wph) * 16;   // this wave's first query
        // key tiles this wave computes: up to its last query's
        const int wave_end = min(k1, q0 < L ? min(q0 + 15, L - 1) / kX3KTile + 1 : 0);

        // ---- this wave's queries: q' = q * scale * log2(e), three terms of the
        // B operand per 32-wide d step (lane: query q0 + r16, d 32 ks + 8 g ..) ----
        bf16x8_t qf[4][3];
        {
            const float sq = pa.scale * kLog2eP;
            const float* qrow = Q + (long long)min(q0 + r16, L - 1) * pa.qs[2] + 8 * g;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const f32x4_t a = *reinterpret_cast<const f32x4_t*>(qrow + 32 * ks);
                const f32x4_t b = *reinterpret_cast<const f32x4_t*>(qrow + 32 * ks + 4);
                const float x[8] = {a[0] * sq, a[1] * sq, a[2] * sq, a[3] * sq,
                                    b[0] * sq, b[1] * sq, b[2] * sq, b[3] * sq};
                x3_split8(x, qf[ks]);
            }
        }

        f32x4_t acc[8];
#pragma unroll
        for (int db = 0; db < 8; ++db) acc[db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        float ms = -INFINITY;      // running max of the lane's query (log2 domain) at the last raise
        float b = 0.f;             // -ms once finite: the score chain's start
        float lp = 0.f;            // the lane's part of the row sum
        float cap = -1.f;          // kSumCap once ms is finite: the first tile always raises

        auto compute = [&](int kt, const lds_u8_t* sb) {
            // ---- scores, two independent chains ----
            f32x4_t s[2] = {f32x4_t{b, b, b, b}, f32x4_t{b, b, b, b}};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                bf16x8_t kf[2][3];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int t = 0; t < 3; ++t)
                        kf[kb][t] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8_t*>(
                            sb + t * kX3TermBytes + k_off[kb][ks]);
#pragma unroll
                for (int pr = 0; pr < kX3Pairs; ++pr)
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
                        s[kb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kb][x3_pair_a(pr)],
                                                                        qf[ks][x3_pair_b(pr)], s[kb], 0, 0, 0);
            }
            if (kt * kX3KTile + kX3KTile - 1 > q0) {   // the diagonal: keys past the query
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (kt * kX3KTile + 8 * g + 4 * kb + e > q0 + r16) s[kb][e] = -INFINITY;
            }
            // ---- P = 2^s, its sum; raise the max when the sum left the cap ----
            float p[8];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int e = 0; e < 4; ++e) p[4 * kb + e] = __builtin_amdgcn_exp2f(s[kb][e]);
            float rs = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            if (__any(!(rs <= cap))) {
                float mt = s[0][0];
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) mt = fmaxf(mt, s[kb][e]);
                mt = xmax16_32(mt);                       // the row: lanes r16, r16 + 16, + 32, + 48
                const float mq = mt - b;                  // unbiased row max of this tile
                const float m_new = fmaxf(ms, mq);
                const float alpha = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - m_new);
#pragma unroll
                for (int db = 0; db < 8; ++db) acc[db] *= alpha;
                lp *= alpha;
                const float b_new = m_new == -INFINITY ? 0.f : -m_new;
                const float delta = b_new - b;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                    for (int e = 0; e < 4; ++e) p[4 * kb + e] = __builtin_amdgcn_exp2f(s[kb][e] + delta);
                rs = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
                ms = m_new;
                b = b_new;
                cap = m_new == -INFINITY ? -1.f : kSumCap;
            }
            lp += rs;
            bf16x8_t pt[3];
            x3_split8(p, pt);
            // ---- O^T += V^T P^T, 8 blocks of 16 d ----
#pragma unroll
            for (int db = 0; db < 8; ++db) {
                bf16x8_t vf[3];
#pragma unroll
                for (int t = 0; t < 3; ++t) {
                    const lds_u8_t* p0 = sb + t * kX3TermBytes + v_off[0][db];
                    const lds_u8_t* p1 = sb + t * kX3TermBytes + v_off[1][db];
                    const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p0);
                    const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)p1);
                    vf[t] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                }
#pragma unroll
                for (int pr = 0; pr < kX3Pairs; ++pr)
                    acc[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[x3_pair_a(pr)], pt[x3_pair_b(pr)],
                                                                      acc[db], 0, 0, 0);
            }
        };

        // The previous segment's last iteration ended on a barrier: no wave
        // still reads stage 0.
        load_tile(k0);
        store_tile(0);
        if (k0 + 1 < k1) load_tile(k0 + 1);
        __syncthreads();
        for (int kt = k0; kt < k1; ++kt) {
            if (kt < wave_end) compute(kt, lsm + ((kt - k0) & 1) * kX3StageBytes);
            if (kt + 1 < k1) {
                store_tile((kt - k0 + 1) & 1);
                if (kt + 2 < k1) load_tile(kt + 2);
            }
            __syncthreads();
        }

        // ---- lane holds O[q0 + r16][16 db + 4 g + e] (times l) ----
        const float l = xsum16_32(lp);
        const int qi = q0 + r16;
        const int part = si ? sg.part[1] : sg.part[0];
        if (qi < L && part < 0) {
            const float inv = 1.0f / l;
            float* orow = pa.out + wk.b * pa.os[0] + h * pa.os[1] + (long long)qi * pa.os[2] + 4 * g;
#pragma unroll
            for (int db = 0; db < 8; ++db)
                *reinterpret_cast<float4*>(orow + 16 * db) =
                    make_float4(acc[db][0] * inv, acc[db][1] * inv, acc[db][2] * inv, acc[db][3] * inv);
        } else if (qi < L) {
            const long long row = pair_row(pa, wk.b, h, qt, qi);
            float* po = pa.part + ((long long)part * pa.part_rows + row) * 128 + 4 * g;
#pragma unroll
            for (int db = 0; db < 8; ++db)
                *reinterpret_cast<float4*>(po + 16 * db) = make_float4(acc[db][0], acc[db][1], acc[db][2], acc[db][3]);
            if (g == 0)
                *reinterpret_cast<float2*>(pa.part + 2 * pa.part_rows * 128 + 2 * (part * pa.part_rows + row)) =
                    make_float2(ms, l);
        }
    }
}

// The second launch of a paired three-term launch: the rows of query tiles
// whose key tiles the two workgroups of a pair split: O = (2^(m0-M) O0 + 2^(m1-M) O1) / (2^(m0-M) l0 + 2^(m1-M) l1), M the
// larger m, each partial's O and l taken against its own m (log2 domain).
// One workgroup per (batch, query head, pair); pairs without a split return.
// A thread takes float4 column c of rows r, r + 8, ... (qtile <= 64 rows:
// at most 8); every load is issued before the first use (rows past L load
// the tile's first row and store nothing).
constexpr int kPairMergeRows = 8;
__global__ void __launch_bounds__(256) prefill_pair_merge_kernel(PrefillArgs pa) {
    const int np = pa.n_qt / 2;
    const int pair = blockIdx.x % np;
    const int bh = blockIdx.x / np;   // batch * Hq + query head
    const int qtile = pa.q_tile;
    const int u = pa.n_qt - 1 - pair;
    if (pair_split(pa.L, qtile, pa.k_tile, pair, u) == 0) return;
    const int bi = bh / pa.Hq, h = bh % pa.Hq;
    const long long row0 = ((long long)bh * np + pair) * qtile;
    const float4* o0 = reinterpret_cast<const float4*>(pa.part + row0 * 128);
    const float4* o1 = reinterpret_cast<const float4*>(pa.part + (pa.part_rows + row0) * 128);
    const float2* ml0 = reinterpret_cast<const float2*>(pa.part + 2 * pa.part_rows * 128) + row0;
    const float2* ml1 = ml0 + pa.part_rows;
    const int c = threadIdx.x & 31, r0 = threadIdx.x >> 5;
    const int rows = min(qtile, pa.L - u * qtile);   // rows of the tile below L
    float4 x[kPairMergeRows], y[kPairMergeRows];
    float2 a[kPairMergeRows], b[kPairMergeRows];
#pragma unroll
    for (int i = 0; i < kPairMergeRows; ++i) {
        const int r = r0 + 8 * i < rows ? r0 + 8 * i : 0;
        a[i] = ml0[r];
        b[i] = ml1[r];
        x[i] = o0[r * 32 + c];
        y[i] = o1[r * 32 + c];
    }
    float* out = pa.out + bi * pa.os[0] + h * pa.os[1] + (long long)u * qtile * pa.os[2] + 4 * c;
#pragma unroll
    for (int i = 0; i < kPairMergeRows; ++i) {
        const int r = r0 + 8 * i;
        if (r < rows) {
            const float M = fmaxf(a[i].x, b[i].x);
            const float w0 = a[i].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(a[i].x - M);
            const float w1 = b[i].x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(b[i].x - M);
            const float inv = 1.0f / (w0 * a[i].y + w1 * b[i].y);
            *reinterpret_cast<float4*>(out + (long long)r * pa.os[2]) =
                make_float4((w0 * x[i].x + w1 * y[i].x) * inv, (w0 * x[i].y + w1 * y[i].y) * inv,
                            (w0 * x[i].z + w1 * y[i].z) * inv, (w0 * x[i].w + w1 * y[i].w) * inv);
        }
    }
}

// fp32, short prompts: a workgroup serves 32 queries of one head, and its
// waves split every staged 64-key tile, each taking one 16-key block of it
// (with 128-query workgroups a 512-token prompt of 16 heads fills 64 CUs,
// and one wave's tile of 32 queries x 64 keys is ~7 us of fp32 MFMA work).
// With W = 8 waves, waves 0-3 serve queries 0-15 and waves 4-7 queries
// 16-31 (two waves per SIMD); with W = 4 each wave serves all 32.  Each wave
// keeps its own (m, l, O) over its keys; a block a wave sees fully masked
// leaves m at -inf, so the softmax subtracts 0 in its place.  At the end the
// waves of blocks 1-3 leave their partials in LDS and the wave of block 0
// merges them (O = sum 2^(m_w - M) O_w, l likewise, M the largest m_w) and
// writes the output.
template <int D, int W>
__global__ void __launch_bounds__(W * 64)
prefill_f32_split_kernel(PrefillArgs pa) {
    static_assert(W == 4 || W == 8, "4 or 8 waves");
    using Lds = F32Lds<D>;
    constexpr int NT = W * 64;
    constexpr int GW = 8 / W;               // 16-query groups per wave
    const int L = pa.L;
    const float sl2 = pa.scale * kLog2eP;
    constexpr int NDB = D / 16;
    constexpr int QF = D / 4;
    extern __shared__ __align__(16) unsigned char smem[];
    float* stage_base = reinterpret_cast<float*>(smem);

    const Work wk = map_work(pa, blockIdx.x);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int blk = wave & 3;               // 16-key block of each tile
    const int qset = wave >> 2;             // which 16 queries (W = 8)
    const int g = lane >> 4;
    const int c16 = lane & 15;

    const float* Q = static_cast<const float*>(pa.q) + wk.b * pa.qs[0] + wk.h0 * pa.qs[1];
    const float* K = static_cast<const float*>(pa.k) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const float* V = static_cast<const float*>(pa.v) + wk.b * pa.kvs[0] + wk.kvh * pa.kvs[1];
    const long long q_row = pa.qs[2], kv_row = pa.kvs[2];

    const int q0 = wk.qt * 32;
    const int qw0 = q0 + qset * 16 * GW;    // this wave's first query
    const int n_kt = (min(L, q0 + 32) - 1) / kKTile + 1;

    F32Stage<D, NT> next;
    f32_load<D, NT>(next, K, V, kv_row, 0, L);

    float qf[GW][QF];
#pragma unroll
    for (int gq = 0; gq < GW; ++gq) {
        const int qi = min(qw0 + gq * 16 + c16, L - 1);
#pragma unroll
        for (int s = 0; s < QF; ++s) qf[gq][s] = Q[qi * q_row + s * 4 + g];
    }

    f32x4_t acc[GW][NDB];
    float m_run[GW], l_run[GW];
#pragma unroll
    for (int gq = 0; gq < GW; ++gq) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) acc[gq][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        m_run[gq] = -INFINITY;
        l_run[gq] = 0.f;
    }

    f32_store<D, NT>(next, stage_base, stage_base + Lds::K_ELEMS);
    __syncthreads();

    for (int kt = 0; kt < n_kt; ++kt) {
        const float* sK = stage_base + (kt & 1) * Lds::STAGE;
        const float* sV = sK + Lds::K_ELEMS;
        const bool more = kt + 1 < n_kt;
        if (more) f32_load<D, NT>(next, K, V, kv_row, (kt + 1) * kKTile, L);

        const int kb0 = kt * kKTile + blk * 16;   // this wave's first key
        if (kb0 <= qw0 + 16 * GW - 1) {           // else above every query of the wave
            const bool diag = kb0 + 15 > qw0;
#pragma unroll
            for (int gq = 0; gq < GW; ++gq) {
                const int qi = qw0 + gq * 16 + c16;
                f32x4_t s = {0.f, 0.f, 0.f, 0.f};
                const float* krow = sK + (blk * 16 + c16) * Lds::K_STRIDE;
#pragma unroll
                for (int ks = 0; ks < QF; ++ks) s = __builtin_amdgcn_mfma_f32_16x16x4f32(krow[ks * 4 + g], qf[gq][ks], s, 0, 0, 0);
                float mt = -INFINITY;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float sv = s[i] * sl2;
                    if (diag && kb0 + g * 4 + i > qi) sv = -INFINITY;
                    s[i] = sv;
                    mt = fmaxf(mt, sv);
                }
                mt = xmax16_32(mt);
                const float m_new = fmaxf(m_run[gq], mt);
                const float m_use = m_new == -INFINITY ? 0.f : m_new;
                const float alpha = __builtin_amdgcn_exp2f(m_run[gq] - m_use);
                float rs = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = __builtin_amdgcn_exp2f(s[i] - m_use);
                    s[i] = p;
                    rs += p;
                }
                rs = xsum16_32(rs);
                l_run[gq] = l_run[gq] * alpha + rs;
                m_run[gq] = m_new;
#pragma unroll
                for (int db = 0; db < NDB; ++db) acc[gq][db] *= alpha;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float* vrow = sV + (blk * 16 + g * 4 + i) * Lds::V_STRIDE;
#pragma unroll
                    for (int db = 0; db < NDB; ++db)
                        acc[gq][db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[db * 16 + c16], s[i], acc[gq][db], 0, 0, 0);
                }
            }
        }
        if (more) {
            // The other stage was last read before the previous iteration's barrier.
            float* nK = stage_base + ((kt + 1) & 1) * Lds::STAGE;
            f32_store<D, NT>(next, nK, nK + Lds::K_ELEMS);
        }
        __syncthreads();
    }

    // Partials of the waves of blocks 1-3 into LDS, [element][lane] per wave.
    constexpr int NE = GW * (NDB * 4 + 2);
    float* const part = stage_base;
    if (blk > 0) {
        float* p = part + (qset * 3 + blk - 1) * NE * 64 + lane;
#pragma unroll
        for (int gq = 0; gq < GW; ++gq) {
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i) p[((gq * NDB + db) * 4 + i) * 64] = acc[gq][db][i];
            p[(GW * NDB * 4 + gq) * 64] = m_run[gq];
            p[(GW * NDB * 4 + GW + gq) * 64] = l_run[gq];
        }
    }
    __syncthreads();
    if (blk != 0) return;
    // Block 0 holds key 0, so this wave's m is finite.
#pragma unroll
    for (int o = 0; o < 3; ++o) {
        const float* p = part + (qset * 3 + o) * NE * 64 + lane;
#pragma unroll
        for (int gq = 0; gq < GW; ++gq) {
            const float mo = p[(GW * NDB * 4 + gq) * 64], lo = p[(GW * NDB * 4 + GW + gq) * 64];
            const float m = fmaxf(m_run[gq], mo);
            const float a = __builtin_amdgcn_exp2f(m_run[gq] - m);
            const float b = mo == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mo - m);
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[gq][db][i] = acc[gq][db][i] * a + p[((gq * NDB + db) * 4 + i) * 64] * b;
            l_run[gq] = l_run[gq] * a + lo * b;
            m_run[gq] = m;
        }
    }
#pragma unroll
    for (int gq = 0; gq < GW; ++gq) {
        const int qi = qw0 + gq * 16 + c16;
        if (qi >= L) continue;
        const float inv = 1.0f / l_run[gq];
        float* orow = pa.out + wk.b * pa.os[0] + wk.h0 * pa.os[1] + qi * pa.os[2];
#pragma unroll
        for (int db = 0; db < NDB; ++db)
            *reinterpret_cast<float4*>(orow + db * 16 + g * 4) =
                make_float4(acc[gq][db][0] * inv, acc[gq][db][1] * inv, acc[gq][db][2] * inv, acc[gq][db][3] * inv);
    }
}

// ===========================================================================
// Launch
// ===========================================================================

// bf16 shape: W waves of QB 32-query blocks each.  Measured at L = 8192
// (16/8 heads) on MI355X, steady-state clocks, with the register-staged
// kernel: 8 waves x 32 queries (two waves per SIMD, both query heads of a KV
// group per workgroup) 0.281 ms.  Slower there: 4 waves x 64 queries (also
// with the O accumulators in AGPRs); a phase-locked schedule in which the two
// waves of a SIMD alternate between MFMA and softmax phases at workgroup
// barriers (the load-to-LDS kernel's ping-pong schedule is that idea without
// the register spills); the next half's score MFMAs software-pipelined under
// the current half's softmax (sched_group_barrier interleaving, three LDS
// stages); the score product split into two independent MFMA chains.  With
// the load-to-LDS tiles and the folded softmax, 4 waves x 64 queries (one
// wave per SIMD, O and q in AGPRs, four stages, each K and V^T fragment
// feeding two MFMAs) measured 272-275 us at L = 8192 against 261-273 us for
// the 8-wave ping-pong kernel on the same box: its dependency stalls fell
// (28 % of wave cycles waiting against 43 %) but the single wave spent 45 %
// of its cycles issuing VALU, AGPR reads of the scores included.  With the
// accumulators and scores in VGPRs instead (one wave per SIMD holding 32
// queries of both heads of a KV group, the two heads' blocks pipelined so
// that one head's softmax runs under the other's MFMAs, K and V^T fragments
// read right before each MFMA): bit-exact with the ping-pong kernel, but
// 372 us at L = 8192 and 175 us at L = 4096 against 246 and 106 us.  The
// O accumulators and q of two heads (192 registers) left no room to read
// fragments ahead, so every MFMA waited for its own LDS read.
constexpr int kBfQB = 1;
constexpr int kBfW = 8;
constexpr int kBfWSmall = 4;

template <int D, int QB, int W>
sa_status launch_bf16(const PrefillArgs& pa, dim3 grid, hipStream_t st) {
    constexpr int bytes = BfLds<D, W>::BYTES;
    sa_status s = opt_in_lds<&prefill_bf16_kernel<D, QB, W>>(bytes);
    if (s != SA_OK) return s;
    hipLaunchKernelGGL((prefill_bf16_kernel<D, QB, W>), grid, dim3(W * 64), bytes, st, pa);
    return SA_OK;
}

// LDS stages of the load-unit kernel: two (with 4 waves, two workgroups per
// CU fit in LDS; with 8, the ping-pong schedule loads tile kt + 2 once tile kt
// is done, and three stages measured 1 % slower).
template <int W>
constexpr int dma_stages() { return 2; }

template <int W>
sa_status launch_bf16_dma(const PrefillArgs& pa, dim3 grid, hipStream_t st) {
    constexpr int NS = dma_stages<W>();
    constexpr int bytes = NS * kDmaStageBytes;
    sa_status s = opt_in_lds<&prefill_bf16_fold_kernel<W, NS>>(bytes);
    if (s != SA_OK) return s;
    hipLaunchKernelGGL((prefill_bf16_fold_kernel<W, NS>), grid, dim3(W * 64), bytes, st, pa);
    return SA_OK;
}

// The split kernel: KS = 2 key groups of GH = 2 heads, 2 stages of 2 tiles
// (128 KiB of LDS, one workgroup per CU).  Measured against an 8-wave
// variant whose four groups take 32-key halves of the same tiles (2 waves per
// SIMD): equal at L = 1024, slower below; per CU both are bound by the
// heaviest query tile's tile count at one tile per ~1.2 us per SIMD.
constexpr int kSplitKS = 2;
constexpr int kSplitGH = 2;

// The second launch of a paired launch: one workgroup per (batch, query
// head, pair).
void launch_pair_merge(const PrefillArgs& pa, hipStream_t st) {
    const long long n_merge = pa.part_rows / pa.q_tile;
    hipLaunchKernelGGL(prefill_pair_merge_kernel, dim3(static_cast<unsigned>(n_merge)), dim3(256), 0, st, pa);
}

sa_status launch_bf16_split(const PrefillArgs& pa, dim3 grid, hipStream_t st) {
    constexpr int bytes = 2 * kSplitKS * kDmaStageBytes;
    sa_status s = opt_in_lds<&prefill_bf16_split_kernel<kSplitKS, kSplitGH>>(bytes);
    if (s != SA_OK) return s;
    hipLaunchKernelGGL((prefill_bf16_split_kernel<kSplitKS, kSplitGH>), grid, dim3(kSplitKS * kSplitGH * 64), bytes,
                       st, pa);
    return SA_OK;
}

template <int D, int GQ = 2>
sa_status launch_f32(const PrefillArgs& pa, dim3 grid, hipStream_t st) {
    sa_status s = opt_in_lds<&prefill_f32_kernel<D, GQ>>(F32Lds<D>::BYTES);
    if (s == SA_OK)
        hipLaunchKernelGGL((prefill_f32_kernel<D, GQ>), grid, dim3(kFThreads), F32Lds<D>::BYTES, st, pa);
    return s;
}

// 8 waves (two per SIMD) where the tile's chunks cover 512 threads, else 4.
template <int D>
sa_status launch_f32_split(const PrefillArgs& pa, dim3 grid, hipStream_t st) {
    constexpr int W = D >= 32 ? kF32SplitW : 4;
    sa_status s = opt_in_lds<&prefill_f32_split_kernel<D, W>>(F32Lds<D>::BYTES);
    if (s == SA_OK)
        hipLaunchKernelGGL((prefill_f32_split_kernel<D, W>), grid, dim3(W * 64), F32Lds<D>::BYTES, st, pa);
    return s;
}

// Workgroups of W waves serve gh = gcd(Hq / Hkv, W) query heads, W / gh
// waves of 32 queries per head.
long long bf16_grid(const PrefillArgs& pa, int B, int W) {
    const int gh = std::gcd(pa.Hq / pa.Hkv, W);
    const int q_tile = (W / gh) * kBfQB * 32;
    return (long long)B * (pa.Hq / gh) * ((pa.L + q_tile - 1) / q_tile);
}

template <int W>
sa_status launch_f32x3(const PrefillArgs& pa, dim3 grid, bool paired, hipStream_t st) {
    constexpr int bytes = 2 * kX3StageBytes;
    if (paired) {
        SA_TRY((opt_in_lds<&prefill_f32x3_kernel<W, true>>(bytes)));
        hipLaunchKernelGGL((prefill_f32x3_kernel<W, true>), grid, dim3(W * 64), bytes, st, pa);
        SA_CHECK_LAUNCH();
        launch_pair_merge(pa, st);
        return SA_OK;
    }
    SA_TRY((opt_in_lds<&prefill_f32x3_kernel<W, false>>(bytes)));
    hipLaunchKernelGGL((prefill_f32x3_kernel<W, false>), grid, dim3(W * 64), bytes, st, pa);
    return SA_OK;
}

// Workgroups of the three-term fp32 kernel: W waves of 16 queries serve
// gcd(Hq / Hkv, W) query heads.
long long x3_grid(const PrefillArgs& pa, int B, int W) {
    const int gh = std::gcd(pa.Hq / pa.Hkv, W);
    const int q_tile = (W / gh) * 16;
    return (long long)B * (pa.Hq / gh) * ((pa.L + q_tile - 1) / q_tile);
}

// The kernel a prefill launch takes and its query tile.
enum class PfKind { BfSplit, Bf, F32Split, F32, F32x3 };
struct PfPlan {
    PfKind kind;
    int W;        // Bf: waves per workgroup (kBfWSmall or kBfW)
    int gh;       // query heads per workgroup
    int q_tile;   // query rows per workgroup and head
    bool pair;    // F32x3: the shape takes paired key ranges when given a workspace
};

// Paired three-term launches: one round of workgroups (96 KiB of LDS each,
// so one per CU) and at least this many query tiles per head.
constexpr int kPairMinTiles = 8;

// Rows of partials a paired launch of this plan writes: (batch, query head,
// pair, query of the tile).
long long pair_part_rows(const PrefillArgs& pa, int B, const PfPlan& plan) {
    const int n_qt = (pa.L + plan.q_tile - 1) / plan.q_tile;
    return (long long)B * pa.Hq * (n_qt / 2) * plan.q_tile;
}

size_t pair_ws_bytes(const PrefillArgs& pa, int B, const PfPlan& plan) {
    return plan.pair ? (size_t)pair_part_rows(pa, B, plan) * 2 * (128 + 2) * sizeof(float) : 0;
}

PfPlan plan_prefill(const PrefillArgs& pa, int B, bool bf16, int D) {
    const int G = pa.Hq / pa.Hkv;
    const bool split_shape = bf16 && D == 128 && G % kSplitGH == 0;
    // A query tile set through sa_set_attention_blocks (the reference's
    // g_q_block_size): fp32 32 (the split kernel), 64 or 128 (16 or 32
    // queries per wave); bf16 32 (the split kernel, head_dim 128 and even
    // GQA groups) or the unsplit workgroup width whose per-head tile it is
    // (16/8 heads: 64 with 4 waves, 128 with 8).  A bf16 shape with no
    // kernel of that tile takes the launch's own choice.
    const int want = attn_q_block();
    if (want > 0) {
        if (!bf16) return {want == 32 ? PfKind::F32Split : PfKind::F32, 0, 1, want, false};
        if (want == 32 && split_shape) return {PfKind::BfSplit, 0, kSplitGH, 32, false};
        for (int W : {kBfWSmall, kBfW}) {
            const int gh = std::gcd(G, W);
            if ((W / gh) * kBfQB * 32 == want) return {PfKind::Bf, W, gh, want, false};
        }
    }
    // bf16: 8-wave workgroups while they give every CU two of them; below
    // that, 4-wave workgroups (one wave per SIMD) spread the same waves over
    // twice as many CUs.  Measured (16/8 heads, D = 128): 4 waves are faster
    // for L = 128 .. 4096 (1.06x .. 1.40x), 8 waves at L = 8192.
    // SA_PREFILL_WAVES=4 or 8 forces the workgroup size (tests cover both).
    const char* forced = std::getenv("SA_PREFILL_WAVES");
    const int fw = forced ? std::atoi(forced) : 0;
    // Shorter prompts still (the 4-wave grid has at most one workgroup per
    // CU), head_dim 128, GQA groups of an even size: the split kernel, whose
    // 32-query workgroups walk each half of their key range in one of two
    // wave groups.  Measured (16/8 heads, graph-replayed calls): L = 512 /
    // 1024 / 2048 take 12.1 / 18.5 / 37.6 us against 15.4 / 24.8 / 43.5 us
    // with 4-wave workgroups; L = 128 8.3 us either way.
    // SA_PREFILL_SPLIT=1 / 0 forces it on (where the shape allows) / off.
    const char* fsplit = std::getenv("SA_PREFILL_SPLIT");
    const bool split = split_shape && (fsplit ? std::atoi(fsplit) != 0
                                              : !forced && bf16_grid(pa, B, kBfWSmall) <= device_cu_count());
    // Paired key ranges (see the three-term kernel below) measured slower
    // here: at ~1.45 us per step of two 64-key tiles, the second segment's
    // prologue and epilogue in workgroup A and the merge launch cost more
    // than the steps they save (16/8 heads, graph-replayed: L = 1024 17.9
    // against 23.5 us, L = 256 9.3 against 15.5 us).
    if (split) return {PfKind::BfSplit, 0, kSplitGH, 32, false};
    // fp32: 32-query workgroups whose waves split each tile's keys while
    // 128-query ones would give fewer than two workgroups per CU.  Measured
    // (16/8 heads, D = 128, graph-replayed calls): L = 128 / 512 / 1024 /
    // 2048 take 16.0 / 35.3 / 72.4 / 245.7 us against 29.0 / 86.9 / 164.3 /
    // 319.5 us with 128-query workgroups (4 waves per 32-query workgroup
    // instead of 8: 17.3 / 38.3 / 78.4 / 266.6 us); L = 4096 896 against
    // 681 us.
    // fp32 at head_dim 128: the three-term kernel on bf16 MFMA, 8 waves
    // while that grid fills the CUs, else 4.  SA_PREFILL_F32X3=0 (or a
    // SA_PREFILL_SPLIT setting) selects the fp32-MFMA kernels below.
    const char* fx3 = std::getenv("SA_PREFILL_F32X3");
    if (!bf16 && D == 128 && !fsplit && (!fx3 || std::atoi(fx3) != 0)) {
        const int W = x3_grid(pa, B, 8) >= device_cu_count() ? 8 : 4;
        const int gh = std::gcd(G, W);
        const int q_tile = (W / gh) * 16;
        // Paired key ranges where the grid is one round: the longest query
        // tile no longer sets the launch's time (its keys are split with the
        // shortest tile's workgroup).  SA_PREFILL_PAIR=0 / 1 turns them off /
        // on regardless of the size rules (one round of workgroups still required).
        const char* fpair = std::getenv("SA_PREFILL_PAIR");
        const int n_qt = (pa.L + q_tile - 1) / q_tile;
        const bool one_round = x3_grid(pa, B, W) <= device_cu_count();
        const bool pair = one_round && n_qt >= 2 && q_tile <= 8 * kPairMergeRows &&
                          (fpair ? std::atoi(fpair) != 0 : n_qt >= kPairMinTiles);
        return {PfKind::F32x3, W, gh, q_tile, pair};
    }
    if (!bf16) {
        const bool fsp = fsplit ? std::atoi(fsplit) != 0
                                : (long long)B * pa.Hq * ((pa.L + kFQTile - 1) / kFQTile) < 2LL * device_cu_count();
        return fsp ? PfPlan{PfKind::F32Split, 0, 1, 32, false} : PfPlan{PfKind::F32, 0, 1, kFQTile, false};
    }
    const int W = fw == kBfW || fw == kBfWSmall ? fw
                  : bf16_grid(pa, B, kBfW) < 2LL * device_cu_count() ? kBfWSmall : kBfW;
    const int gh = std::gcd(G, W);
    return {PfKind::Bf, W, gh, (W / gh) * kBfQB * 32, false};
}

// ws / ws_bytes: the caller's workspace, or null / 0.  A paired shape (see
// PfPlan::pair) with a workspace of at least pair_ws_bytes takes paired key
// ranges; without one, the single launch.
sa_status launch(PrefillArgs pa, int B, bool bf16, int D, void* ws, size_t ws_bytes, hipStream_t st) {
    const PfPlan plan = plan_prefill(pa, B, bf16, D);
    pa.gh = plan.gh;
    pa.q_tile = plan.q_tile;
    pa.n_qt = (pa.L + plan.q_tile - 1) / plan.q_tile;
    pa.k_tile = plan.kind == PfKind::F32x3 ? kX3KTile : kKTile;
    const bool paired = plan.pair && ws != nullptr;
    if (paired) {
        if (ws_bytes < pair_ws_bytes(pa, B, plan)) return fail(SA_ENOMEM, "workspace too small for prefill partials");
        pa.part = static_cast<float*>(ws);
        pa.part_rows = pair_part_rows(pa, B, plan);
    }
    const int groups = B * pa.Hkv;
    pa.xcd_groups = groups % 8 == 0 ? groups / 8 : 0;
    const long long n_wg = (long long)B * (pa.Hq / pa.gh) * pa.n_qt;
    if (n_wg > 0x7fffffffLL) return fail(SA_ERANGE, "prefill grid too large");
    const dim3 grid(static_cast<unsigned>(n_wg));
    sa_status s = SA_OK;
    switch (plan.kind) {
        case PfKind::BfSplit:
            s = launch_bf16_split(pa, grid, st);
            break;
        case PfKind::F32x3:
            s = plan.W == 8 ? launch_f32x3<8>(pa, grid, paired, st) : launch_f32x3<4>(pa, grid, paired, st);
            break;
        case PfKind::F32Split:
            switch (D) {
                case 16: s = launch_f32_split<16>(pa, grid, st); break;
                case 32: s = launch_f32_split<32>(pa, grid, st); break;
                case 64: s = launch_f32_split<64>(pa, grid, st); break;
                default: s = launch_f32_split<128>(pa, grid, st); break;
            }
            break;
        case PfKind::F32:
            if (plan.q_tile == 64) {
                switch (D) {
                    case 16: s = launch_f32<16, 1>(pa, grid, st); break;
                    case 32: s = launch_f32<32, 1>(pa, grid, st); break;
                    case 64: s = launch_f32<64, 1>(pa, grid, st); break;
                    default: s = launch_f32<128, 1>(pa, grid, st); break;
                }
            } else {
                switch (D) {
                    case 16: s = launch_f32<16>(pa, grid, st); break;
                    case 32: s = launch_f32<32>(pa, grid, st); break;
                    case 64: s = launch_f32<64>(pa, grid, st); break;
                    default: s = launch_f32<128>(pa, grid, st); break;
                }
            }
            break;
        case PfKind::Bf: {
            // head_dim 128 in bf16 uses the load-unit kernel when a
            // workgroup's queries end within the tiles its schedule keeps
            // resident (two with 8 waves, one with 4), so every wave's
            // diagonal tile is still in LDS after the loop: GQA groups of 2 or
            // more.  Measured against the register-staged kernel (16/8 heads):
            // 1.04x at L = 8192, 1.08x .. 1.14x at L = 1024 .. 4096.
            const int W = plan.W;
            const bool dma = D == 128 && plan.q_tile <= (W == kBfW ? 2 : 1) * kKTile;
            if (dma) {
                s = W == kBfW ? launch_bf16_dma<kBfW>(pa, grid, st) : launch_bf16_dma<kBfWSmall>(pa, grid, st);
            } else if (W == kBfW) {
                s = D == 64 ? launch_bf16<64, kBfQB, kBfW>(pa, grid, st) : launch_bf16<128, kBfQB, kBfW>(pa, grid, st);
            } else {
                s = D == 64 ? launch_bf16<64, kBfQB, kBfWSmall>(pa, grid, st)
                            : launch_bf16<128, kBfQB, kBfWSmall>(pa, grid, st);
            }
            break;
        }
    }
    if (s != SA_OK) return s;
    SA_CHECK_LAUNCH();
    return SA_OK;
}

sa_status prefill(const void* q, const void* k, const void* v, sa_dtype dtype, int batch, int n_q_heads,
                  int n_kv_heads, int L, int D, const int64_t* qs, const int64_t* kvs, const int64_t* os,
                  float scale, float* out, void* ws, size_t ws_bytes, hipStream_t st) {
    if (!q || !k || !v || !out || !qs || !kvs || !os) return fail(SA_EINVAL, "null pointer");
    if (ws && !aligned16(ws)) return fail(SA_EINVAL, "workspace must be 16-byte aligned");
    if (batch <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads)
        return fail(SA_EINVAL, "bad head counts");
    if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16) return fail(SA_EINVAL, "dtype must be F32 or BF16");
    if (dtype == SA_DTYPE_BF16 ? D != 64 && D != 128 : D != 16 && D != 32 && D != 64 && D != 128)
        return fail(SA_EINVAL, dtype == SA_DTYPE_BF16 ? "bf16 prefill head_dim must be 64 or 128"
                                                      : "fp32 prefill head_dim must be 16, 32, 64 or 128");
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
    return launch(pa, batch, dtype == SA_DTYPE_BF16, D, ws, ws_bytes, st);
}

}  // namespace
}  // namespace sa

extern "C" int sa_prefill_query_tile(sa_dtype dtype, int batch, int n_q_heads, int n_kv_heads, int L, int D) {
    sa::clear_error();
    if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16) return sa::fail(SA_EINVAL, "dtype must be F32 or BF16");
    if (batch <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads || L <= 0)
        return sa::fail(SA_EINVAL, "bad prefill shape");
    if (dtype == SA_DTYPE_BF16 ? D != 64 && D != 128 : D != 16 && D != 32 && D != 64 && D != 128)
        return sa::fail(SA_EINVAL, "unsupported head_dim");
    sa::PrefillArgs pa{};
    pa.Hq = n_q_heads; pa.Hkv = n_kv_heads; pa.L = L;
    return sa::plan_prefill(pa, batch, dtype == SA_DTYPE_BF16, D).q_tile;
}

extern "C" size_t sa_prefill_causal_ws_bytes(sa_dtype dtype, int batch, int n_q_heads, int n_kv_heads, int L,
                                             int D) {
    if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16) return 0;
    if (batch <= 0 || n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads || L <= 0) return 0;
    if (dtype == SA_DTYPE_BF16 ? D != 64 && D != 128 : D != 16 && D != 32 && D != 64 && D != 128) return 0;
    sa::PrefillArgs pa{};
    pa.Hq = n_q_heads; pa.Hkv = n_kv_heads; pa.L = L;
    const sa::PfPlan plan = sa::plan_prefill(pa, batch, dtype == SA_DTYPE_BF16, D);
    return sa::pair_ws_bytes(pa, batch, plan);
}

extern "C" sa_status sa_prefill_causal(const void* q, const void* k, const void* v, sa_dtype dtype,
                                       int batch, int n_q_heads, int n_kv_heads, int L, int D,
                                       float scale, float* out, sa_stream_t stream) {
    return sa_prefill_causal_ws(q, k, v, dtype, batch, n_q_heads, n_kv_heads, L, D, scale, out, nullptr, 0, stream);
}

extern "C" sa_status sa_prefill_causal_ws(const void* q, const void* k, const void* v, sa_dtype dtype,
                                          int batch, int n_q_heads, int n_kv_heads, int L, int D,
                                          float scale, float* out, void* ws, size_t ws_bytes,
                                          sa_stream_t stream) {
    sa::clear_error();
    const int64_t Ld = (int64_t)L * D;
    const int64_t qs[3] = {n_q_heads * Ld, Ld, D};
    const int64_t kvs[3] = {n_kv_heads * Ld, Ld, D};
    return sa::prefill(q, k, v, dtype, batch, n_q_heads, n_kv_heads, L, D, qs, kvs, qs, scale, out, ws, ws_bytes,
                       sa::as_stream(stream));
}

extern "C" sa_status sa_prefill_causal_strided(const void* q, const void* k, const void* v, sa_dtype dtype,
                                               int batch, int n_q_heads, int n_kv_heads, int L, int D,
                                               const int64_t q_strides[3], const int64_t kv_strides[3],
                                               const int64_t out_strides[3], float scale, float* out,
                                               sa_stream_t stream) {
    return sa_prefill_causal_strided_ws(q, k, v, dtype, batch, n_q_heads, n_kv_heads, L, D, q_strides, kv_strides,
                                        out_strides, scale, out, nullptr, 0, stream);
}

extern "C" sa_status sa_prefill_causal_strided_ws(const void* q, const void* k, const void* v, sa_dtype dtype,
                                                  int batch, int n_q_heads, int n_kv_heads, int L, int D,
                                                  const int64_t q_strides[3], const int64_t kv_strides[3],
                                                  const int64_t out_strides[3], float scale, float* out, void* ws,
                                                  size_t ws_bytes, sa_stream_t stream) {
    sa::clear_error();
    return sa::prefill(q, k, v, dtype, batch, n_q_heads, n_kv_heads, L, D, q_strides, kv_strides, out_strides,
                       scale, out, ws, ws_bytes, sa::as_stream(stream));
}
