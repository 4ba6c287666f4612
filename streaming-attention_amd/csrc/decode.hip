// Split-KV single-query attention for gfx950: one kernel body serves the
// single-head streaming attention of attention.h, dense multi-head GQA decode
// and paged GQA decode.
//
// Algorithm (the reference's online softmax, reference utils/softmax_online.h:40-87,
// plus its chunk merge, attention/src/streaming_omp.cpp:27-48):
//   * the KV sequence of each (sequence, KV head) is cut into chunks; one
//     workgroup (4 or 8 waves) owns a chunk and all query heads of the GQA
//     group, so every K/V byte is read from HBM once;
//   * a wave walks 16..64-token tiles of its chunk; each lane issues 16-byte
//     loads so one wave-load covers 1 KiB of consecutive rows (coalesced), and
//     the next tile's loads are in flight while the current tile is reduced;
//   * scores are reduced across the lanes of a row with DPP / swizzle, the
//     running max m and normaliser l are wave-uniform, and the output O is
//     kept unnormalised (O = sum p_i V_i with p relative to m);
//   * the waves merge through LDS; a chunk's (m, l, O) goes to the workspace
//     and a second launch applies the log-sum-exp merge
//     O = sum_c e^{m_c-M} O_c / sum_c e^{m_c-M} l_c; a sequence that fits one
//     chunk is written directly and needs no merge.
//
// Workspace: [(m, l) per (sequence, q head, chunk)][O per (sequence, q head,
// chunk)], fp32; nothing in it survives from one call to the next.
#include "sa_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <mutex>
#include <vector>

namespace sa {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kSplitCap = 1024;     // hard cap on chunks per (sequence, KV head)
constexpr int kSplitTarget = 256;   // default cap: keeps the final merge short
constexpr int kMaxChunkPages = 256; // paged chunks stage their page ids in LDS

template <int D, bool BF16>
struct Geo {
    static constexpr int kElemBytes = BF16 ? 2 : 4;
    static constexpr int E = 16 / kElemBytes;       // elements per lane per load
    static constexpr int LPR = D / E;               // lanes per K/V row
    static constexpr int RPW = kWave / LPR;         // rows per wave-load
    static constexpr int R = (RPW * 8 <= 64) ? 8 : 64 / RPW;  // loads per lane per tile
    static constexpr int TILE = R * RPW;            // tokens per wave tile (divides 64)
    static_assert(LPR >= 1 && LPR <= kWave, "unsupported head_dim");
    static_assert(64 % TILE == 0, "tile must divide a page");
};

// Waves per workgroup.  Four: two workgroups fit a CU at the kernels'
// register use, so one's prologue and merge overlap the other's streaming
// (measured: 5.86 TB/s against 4.9 TB/s with eight-wave groups on batched
// paged decode).  A dense single-head launch whose chunks do not outnumber
// the CUs uses eight (one workgroup per CU either way; twice the loads in
// flight): T = 262144, d = 128, fp32: 47.1 against 47.8 us per call.
template <int D, int NREP>
constexpr int waves_for() { return 4; }
constexpr int kWavesOneRound = 8;

struct DecodeArgs {
    const float* q;          // [n_seq][n_q_heads][D]
    const void* k;           // dense: [n_seq][n_kv][T][D]; paged: pool [pages][n_kv][64][D]
    const void* v;
    float* out;              // [n_seq][n_q_heads][D]
    float* part_ml;          // [n_seq*n_q_heads][n_split][2]
    float* part_o;           // [n_seq*n_q_heads][n_split][D]
    const int32_t* block_table;  // paged only: [max_seqs][max_pages]
    const int32_t* seq_lens;     // paged only: committed lengths
    RowList rows;                // paged only: cache row of each sequence of the launch
    int n_kv;
    int n_q;
    int T;                   // dense length
    int max_pages;
    int num_pages;           // paged only: pages in the pool
    int n_pending;
    int chunk;               // tokens per workgroup, multiple of 64
    int n_split;             // chunks per (sequence, kv head) in the grid
    float scale;
    // Fused append step (FUSED kernels only): q above is the raw q; the new
    // token's K/V, norm weights, RoPE tables, optional q output, and its
    // position in each sequence (the committed length, from the host).
    const float* k_new;      // [n_seq][n_kv][D]
    const float* v_new;
    const float* wq;
    const float* wk;
    const float* cos_t;
    const float* sin_t;
    float* q_out;            // [n_seq][n_q_heads][D] or NULL
    int32_t* lens_out;       // the cache's device lengths, written on commit
    // Or q, k_new and v_new as the sum of part_S split-K partials: row seq of
    // an [.][part_N] projection (q columns, then k, then v), partial t at
    // part + t * part_split.
    const float* part;
    size_t part_split;
    int part_S;
    int part_N;
    RowList pos;
    float eps;
    int rope_max_pos;
    int commit;
    // Compact grid (paged launches): blockIdx.y runs over the chunks that
    // hold tokens, sequence i's at cstart[i] .. cstart[i + 1] - 1 (entries
    // past the launch's sequences hold INT_MAX), and blockIdx.z is 0.
    int compact;
    // Paged, not FUSED: the committed lengths come from pos (host values)
    // instead of seq_lens.
    int host_lens;
    int32_t cstart[kRowsPerLaunch + 1];
};

// Widen one 16-byte slice of a K/V row to fp32.
template <bool BF16, class V4>
__device__ __forceinline__ void widen(const V4& raw, float* out) {
    if constexpr (BF16) {
        out[0] = bf16_lo(raw.x); out[1] = bf16_hi(raw.x);
        out[2] = bf16_lo(raw.y); out[3] = bf16_hi(raw.y);
        out[4] = bf16_lo(raw.z); out[5] = bf16_hi(raw.z);
        out[6] = bf16_lo(raw.w); out[7] = bf16_hi(raw.w);
    } else {
        out[0] = __uint_as_float(raw.x); out[1] = __uint_as_float(raw.y);
        out[2] = __uint_as_float(raw.z); out[3] = __uint_as_float(raw.w);
    }
}

// Reduction over the whole workgroup of W waves; every thread gets the result.
template <class Op, int W>
__device__ __forceinline__ float block_reduce(float v, float* scratch) {
    v = group_reduce<Op, 1, kWave>(v);
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if ((threadIdx.x & (kWave - 1)) == 0) scratch[wave] = v;
    __syncthreads();
    float r = scratch[0];
#pragma unroll
    for (int w = 1; w < W; ++w) r = Op::apply(r, scratch[w]);
    return r;
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// One tile of K/V rows in registers: R 16-byte loads of K and of V per lane.
template <int R>
struct TileRegs {
    u32x4 k[R];
    u32x4 v[R];
};

template <int D, int NREP, bool BF16, bool PAGED>
struct TileWalker {
    using G = Geo<D, BF16>;
    static constexpr int ROW_BYTES = D * G::kElemBytes;

    const DecodeArgs& a;
    const char* kbase;
    const char* vbase;
    const int* pages;   // paged: LDS copy of the chunk's page ids, from page0
    int page0, g, t_end, grp, col;

    // Issue the loads of tile t0 (rows past t_end re-read the last valid
    // row).  No branch and no global index load sits between the loads of
    // two tiles, so a second tile's loads stay in flight behind the first's.
    __device__ __forceinline__ void load(int t0, TileRegs<G::R>& regs) const {
        const char* kt;
        const char* vt;
        if constexpr (PAGED) {
            const int page = pages[(t0 >> 6) - page0];
            const size_t off = (((size_t)page * a.n_kv + g) * 64 + (t0 & 63)) * (size_t)ROW_BYTES;
            kt = static_cast<const char*>(a.k) + off;
            vt = static_cast<const char*>(a.v) + off;
        } else {
            kt = kbase + (size_t)t0 * ROW_BYTES;
            vt = vbase + (size_t)t0 * ROW_BYTES;
        }
        const int last = t_end - t0 - 1;
#pragma unroll
        for (int r = 0; r < G::R; ++r) {
            const int rr = min(r * G::RPW + grp, last);
            regs.k[r] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(kt + (size_t)rr * ROW_BYTES + col * 16));
            regs.v[r] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(vt + (size_t)rr * ROW_BYTES + col * 16));
        }
    }
};

// Fold one loaded tile into the running (m, l, O) of every head of the group.
template <int D, int NREP, bool BF16>
__device__ __forceinline__ void consume(const TileRegs<Geo<D, BF16>::R>& regs, int n_valid, int grp,
                                        const float (&qv)[NREP][Geo<D, BF16>::E], float (&m)[NREP],
                                        float (&l)[NREP], float (&o)[NREP][Geo<D, BF16>::E]) {
    using G = Geo<D, BF16>;
    constexpr int E = G::E, LPR = G::LPR, RPW = G::RPW, R = G::R, TILE = G::TILE;
    float s[R][NREP];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float kf[E];
        widen<BF16>(regs.k[r], kf);
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
            float acc = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) acc = fmaf(qv[h][e], kf[e], acc);
            s[r][h] = group_reduce<OpSum, 1, LPR>(acc);
        }
    }
    if (n_valid < TILE) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r * RPW + grp >= n_valid) {
#pragma unroll
                for (int h = 0; h < NREP; ++h) s[r][h] = -INFINITY;
            }
        }
    }
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        float mt = s[0][h];
#pragma unroll
        for (int r = 1; r < R; ++r) mt = fmaxf(mt, s[r][h]);
        mt = group_reduce<OpMax, LPR, kWave>(mt);
        const float m_new = fmaxf(m[h], mt);
        const float alpha = __builtin_amdgcn_exp2f((m[h] - m_new) * kLog2e);
        float lsum = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            s[r][h] = __builtin_amdgcn_exp2f((s[r][h] - m_new) * kLog2e);
            lsum += s[r][h];
        }
        l[h] = l[h] * alpha + lsum;
        m[h] = m_new;
#pragma unroll
        for (int e = 0; e < E; ++e) o[h][e] *= alpha;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float vf[E];
        widen<BF16>(regs.v[r], vf);
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
#pragma unroll
            for (int e = 0; e < E; ++e) o[h][e] = fmaf(s[r][h], vf[e], o[h][e]);
        }
    }
}

// FUSED (paged only): the decode step's append runs in the same launch.  Each
// workgroup normalises and rotates the q heads of its group into LDS; the
// workgroup whose chunk holds the new token's position also normalises and
// rotates its K, writes K and V into the cache there (and q to q_out), and,
// on commit, sets the sequence's device length to pos + 1.  Lengths come
// from the launch arguments, so no workgroup reads the device length another
// one writes.
// PF: each wave keeps the next tile's loads in flight while it reduces the
// current one (two register tiles).  One-round launches whose waves walk at
// most two tiles take PF = false: one register tile (100 VGPRs against 199
// at fp32 d = 128), bit-identical; dense single-head calls graph-replayed
// T = 65536 16.21 against 16.50 us, T = 8192 8.34 against 8.65 us; at
// T = 262144 (eight tiles per wave) the prefetch keeps 45.1 against 46.1 us.
template <int D, int NREP, bool BF16, bool PAGED, int W, bool FUSED = false, bool PF = true>
__global__ void __launch_bounds__(W * kWave)
split_kv_decode_kernel(DecodeArgs a) {
    static_assert(!FUSED || PAGED, "the fused step appends to a paged cache");
    using G = Geo<D, BF16>;
    constexpr int E = G::E, LPR = G::LPR, TILE = G::TILE;
    constexpr int THREADS = W * kWave;
    constexpr bool kPrefetch = PF && NREP <= 2;

    // The KV head varies fastest in the grid: workgroups go to the XCDs
    // round-robin by linear id, so with 8 KV heads each XCD serves one head's
    // chunks of every sequence (equal work).  With the chunk index fastest, a
    // chunk count that is a multiple of 8 gave each XCD fixed chunk indices,
    // and the late chunks only long sequences have (B = 64, 979-31,078
    // tokens, 16 chunks of 2048: 0.844 against 0.686 ms at 2112 tokens).
    const int g = blockIdx.x;      // kv head
    int split = blockIdx.y;
    int seq = blockIdx.z;          // batch row
    if constexpr (PAGED) {
        if (a.compact) {
            // the last sequence whose first chunk is at or before blockIdx.y
            int lo = 0, hi = kRowsPerLaunch;
            while (hi - lo > 1) {
                const int mid = (lo + hi) >> 1;
                if (a.cstart[mid] <= (int)blockIdx.y) lo = mid;
                else hi = mid;
            }
            seq = lo;
            split = blockIdx.y - a.cstart[lo];
        }
    }
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int col = lane % LPR;    // 16-byte column slice of a row
    const int grp = lane / LPR;    // row inside a wave-load

    int len;
    int cache_row = seq;
    int pos = 0;                   // FUSED: position of the new token
    if constexpr (PAGED) {
        cache_row = a.rows.row[seq];
        // Never walk past the block-table row or the chunks of the grid,
        // whatever the device lengths say (the host has checked them).
        if constexpr (FUSED) {
            pos = a.pos.row[seq];
            len = min(min(pos + 1, a.max_pages * 64), a.n_split * a.chunk);
        } else {
            const int committed = a.host_lens ? a.pos.row[seq] : a.seq_lens[cache_row];
            len = min(min(committed + a.n_pending, a.max_pages * 64), a.n_split * a.chunk);
        }
        if (len <= 0) {
            // An empty sequence attends to nothing: its output is zero.
            if (split == 0) {
                for (int i = threadIdx.x; i < NREP * D; i += THREADS)
                    a.out[((size_t)seq * a.n_q + g * NREP) * D + i] = 0.f;
            }
            return;
        }
    } else {
        len = a.T;
    }
    const int t_begin = split * a.chunk;
    if (t_begin >= len) return;    // whole workgroup: uniform exit
    const int t_end = min(len, t_begin + a.chunk);
    const int n_active = (len - 1) / a.chunk + 1;   // chunks holding tokens

    TileWalker<D, NREP, BF16, PAGED> walk{a, nullptr, nullptr, nullptr, 0, g, t_end, grp, col};
    __shared__ int sh_pages[kMaxChunkPages];
    auto setup_walk = [&]() {
        if constexpr (PAGED) {
            // The chunk's page ids, once per workgroup; an id outside the pool (a
            // table the caller left unassigned) is clamped so no load can fault.
            const int p0 = t_begin >> 6, np = ((t_end - 1) >> 6) - p0 + 1;
            const int32_t* row = a.block_table + (size_t)cache_row * a.max_pages + p0;
            for (int i = threadIdx.x; i < np; i += THREADS) sh_pages[i] = min(max(row[i], 0), a.num_pages - 1);
            __syncthreads();
            walk.pages = sh_pages;
            walk.page0 = p0;
        } else {
            const size_t off = ((size_t)seq * a.n_kv + g) * (size_t)a.T * TileWalker<D, NREP, BF16, PAGED>::ROW_BYTES;
            walk.kbase = static_cast<const char*>(a.k) + off;
            walk.vbase = static_cast<const char*>(a.v) + off;
        }
    };
    constexpr int STRIDE = W * TILE;
    const int first = t_begin + wave * TILE;
    const int n_tiles = first < t_end ? (t_end - first + STRIDE - 1) / STRIDE : 0;   // wave-uniform
    TileRegs<G::R> ra, rb;
    bool first_loaded = false;

    // FUSED prologue.  Every global load of the step's own data (q, k, v,
    // norm weights, cos/sin) is issued first, so their latency overlaps the
    // page-id load; the first K/V tile is then in flight while q and k are
    // normalised and rotated.  The new K/V row goes to the cache and, encoded
    // as stored, to LDS: the tile that holds it takes the row from LDS, so
    // nothing waits for the stores.  (Measured: each wave computing every q
    // head itself, with the K/V row computed by the wave whose tile holds it
    // and no barrier, was slower: 7.6 against 7.3 us per fp32 step.)
    constexpr int KV_SLICES = D * G::kElemBytes / 16;                 // 16-byte slices of a row
    __shared__ __align__(16) float sh_q[FUSED ? NREP : 1][FUSED ? D : 4];
    __shared__ u32x4 sh_knew[FUSED ? KV_SLICES : 1];
    __shared__ u32x4 sh_vnew[FUSED ? KV_SLICES : 1];
    const bool owner = FUSED && t_begin <= pos && pos < t_end;   // this chunk holds the new token
    if constexpr (FUSED) {
        using RP = RowPairs<D>;
        constexpr int NP = RP::NP;
        constexpr int QPW = (NREP + W - 1) / W;                   // q heads per wave
        const bool writer = owner && wave == W - 1;
        const bool rope_on = a.cos_t && pos < a.rope_max_pos;
        RP qr[QPW], kr;
        float vl[NP], vh[NP], wql[NP], wqh[NP], wkl[NP], wkh[NP], cs[NP], sn[NP];
        const float* prow = a.part ? a.part + (size_t)seq * a.part_N : nullptr;   // uniform
#pragma unroll
        for (int j = 0; j < QPW; ++j) {
            const int h = wave + j * W;
            if (h < NREP) {
                if (prow) qr[j].load_sum(prow + (g * NREP + h) * D, a.part_split, a.part_S, lane);
                else qr[j].load(a.q + ((size_t)seq * a.n_q + g * NREP + h) * D, lane);
            }
        }
        const size_t kv_src = ((size_t)seq * a.n_kv + g) * D;
        if (writer) {
            if (prow) {
                const float* kp = prow + (a.n_q + g) * D;
                RP vr;
                kr.load_sum(kp, a.part_split, a.part_S, lane);
                vr.load_sum(kp + a.n_kv * D, a.part_split, a.part_S, lane);
#pragma unroll
                for (int c = 0; c < NP; ++c) { vl[c] = vr.lo[c]; vh[c] = vr.hi[c]; }
            } else {
                kr.load(a.k_new + kv_src, lane);
                RP::load_pairs(a.v_new + kv_src, lane, vl, vh);
            }
            if (a.wk) RP::load_pairs(a.wk, lane, wkl, wkh);
        }
        if (a.wq) RP::load_pairs(a.wq, lane, wql, wqh);
        if (rope_on) {
            RP::load_row(a.cos_t + (size_t)pos * (D / 2), lane, cs);
            RP::load_row(a.sin_t + (size_t)pos * (D / 2), lane, sn);
        }
        int page = -1;
        if (writer) page = a.block_table[(size_t)cache_row * a.max_pages + (pos >> 6)];
        setup_walk();                         // its barrier also waits for the loads above
        if constexpr (kPrefetch) {
            if (n_tiles > 0) {
                walk.load(first, ra);
                first_loaded = true;
            }
        }
        // q of every head of the group: RMSNorm + RoPE at pos, into LDS.
#pragma unroll
        for (int j = 0; j < QPW; ++j) {
            const int h = wave + j * W;
            if (h < NREP) {
                if (a.wq) qr[j].rms_norm_with(wql, wqh, a.eps);
                if (rope_on) qr[j].rope_with(cs, sn);
                qr[j].store(&sh_q[h][0], lane);
                if (a.q_out && owner) qr[j].store(a.q_out + ((size_t)seq * a.n_q + g * NREP + h) * D, lane);
            }
        }
        if (writer) {
            // K (normed, rotated) and V (as given) of the new token at pos; the
            // host has checked that the row has a page there.
            if (a.wk) kr.rms_norm_with(wkl, wkh, a.eps);
            if (rope_on) kr.rope_with(cs, sn);
            constexpr int H = D / 2;
            const bool paged_ok = page >= 0 && page < a.num_pages;
            const size_t row = (((size_t)(paged_ok ? page : 0) * a.n_kv + g) * 64 + (pos & 63)) * D;
#pragma unroll
            for (int c = 0; c < NP; ++c) {
                const int i = lane + c * kWave;
                if (i < H) {
                    if constexpr (BF16) {
                        const uint16_t k0 = f32_to_bf16_rne(kr.lo[c]), k1 = f32_to_bf16_rne(kr.hi[c]);
                        const uint16_t v0 = f32_to_bf16_rne(vl[c]), v1 = f32_to_bf16_rne(vh[c]);
                        uint16_t* lk = reinterpret_cast<uint16_t*>(sh_knew);
                        uint16_t* lv = reinterpret_cast<uint16_t*>(sh_vnew);
                        lk[i] = k0; lk[i + H] = k1; lv[i] = v0; lv[i + H] = v1;
                        if (paged_ok) {
                            uint16_t* kd = const_cast<uint16_t*>(static_cast<const uint16_t*>(a.k)) + row;
                            uint16_t* vd = const_cast<uint16_t*>(static_cast<const uint16_t*>(a.v)) + row;
                            kd[i] = k0; kd[i + H] = k1; vd[i] = v0; vd[i + H] = v1;
                        }
                    } else {
                        float* lk = reinterpret_cast<float*>(sh_knew);
                        float* lv = reinterpret_cast<float*>(sh_vnew);
                        lk[i] = kr.lo[c]; lk[i + H] = kr.hi[c]; lv[i] = vl[c]; lv[i + H] = vh[c];
                        if (paged_ok) {
                            float* kd = const_cast<float*>(static_cast<const float*>(a.k)) + row;
                            float* vd = const_cast<float*>(static_cast<const float*>(a.v)) + row;
                            kd[i] = kr.lo[c]; kd[i + H] = kr.hi[c]; vd[i] = vl[c]; vd[i + H] = vh[c];
                        }
                    }
                }
            }
        }
        // LDS only: the tile loads and the cache stores stay in flight.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    // The tile at t0 that holds the new token takes its row from LDS (rows past
    // the end re-read that row too).
    auto patch = [&](TileRegs<G::R>& regs, int t0) {
        if constexpr (FUSED) {
            if (t0 <= pos && pos < t0 + TILE) {      // wave-uniform
                const int last = t_end - t0 - 1;
#pragma unroll
                for (int r = 0; r < G::R; ++r) {
                    if (t0 + min(r * G::RPW + grp, last) == pos) {
                        regs.k[r] = sh_knew[col];
                        regs.v[r] = sh_vnew[col];
                    }
                }
            }
        }
    };

    // q slice of every head of the group, pre-multiplied by scale.
    float qv[NREP][E];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        const float* qp;
        if constexpr (FUSED) qp = &sh_q[h][col * E];
        else qp = a.q + ((size_t)seq * a.n_q + g * NREP + h) * D + col * E;
#pragma unroll
        for (int e = 0; e < E; e += 4) {
            float4 t = *reinterpret_cast<const float4*>(qp + e);
            qv[h][e] = t.x * a.scale; qv[h][e + 1] = t.y * a.scale;
            qv[h][e + 2] = t.z * a.scale; qv[h][e + 3] = t.w * a.scale;
        }
    }

    float m[NREP], l[NREP], o[NREP][E];
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        m[h] = -INFINITY; l[h] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) o[h][e] = 0.f;
    }

    if constexpr (!FUSED) setup_walk();

    if (n_tiles > 0) {
        if constexpr (kPrefetch) {
            // Two register tiles, alternating: the loads of tile i+1 are issued
            // before tile i is reduced.  No tile is loaded twice (a repeated
            // non-temporal load misses the cache and costs HBM bytes).
            if (!first_loaded) walk.load(first, ra);
            if constexpr (PAGED) {
                // Loads behind wave-uniform branches.  The compiler's wait
                // before reducing tile i then covers the path without tile
                // i+1's loads, so it waits for them too (vmcnt(0)); the dense
                // loop below avoids that, but here it measured no faster
                // (64 sequences, same process: 6.18-6.23 against 6.23-6.34
                // TB/s; 244 against 228 VGPRs).
                for (int i = 0; i < n_tiles; i += 2) {
                    const int ta = first + i * STRIDE;
                    if (i + 1 < n_tiles) walk.load(ta + STRIDE, rb);
                    patch(ra, ta);
                    consume<D, NREP, BF16>(ra, t_end - ta, grp, qv, m, l, o);
                    if (i + 1 >= n_tiles) break;
                    if (i + 2 < n_tiles) walk.load(ta + 2 * STRIDE, ra);
                    patch(rb, ta + STRIDE);
                    consume<D, NREP, BF16>(rb, t_end - ta - STRIDE, grp, qv, m, l, o);
                }
            } else {
                // The steady-state loop issues its loads unconditionally, so
                // tile i+1's loads stay in flight while tile i is reduced
                // (T = 262144, d = 128, fp32: 5.69 -> 5.79 TB/s per call).
                int i = 0;
                for (; i + 2 < n_tiles; i += 2) {
                    const int ta = first + i * STRIDE;
                    walk.load(ta + STRIDE, rb);
                    consume<D, NREP, BF16>(ra, t_end - ta, grp, qv, m, l, o);
                    walk.load(ta + 2 * STRIDE, ra);
                    consume<D, NREP, BF16>(rb, t_end - ta - STRIDE, grp, qv, m, l, o);
                }
                const int ta = first + i * STRIDE;
                if (i + 1 < n_tiles) {
                    walk.load(ta + STRIDE, rb);
                    consume<D, NREP, BF16>(ra, t_end - ta, grp, qv, m, l, o);
                    consume<D, NREP, BF16>(rb, t_end - ta - STRIDE, grp, qv, m, l, o);
                } else {
                    consume<D, NREP, BF16>(ra, t_end - ta, grp, qv, m, l, o);
                }
            }
        } else {
            for (int i = 0; i < n_tiles; ++i) {
                TileRegs<G::R> rt;
                walk.load(first + i * STRIDE, rt);
                patch(rt, first + i * STRIDE);
                consume<D, NREP, BF16>(rt, t_end - first - i * STRIDE, grp, qv, m, l, o);
            }
        }
    }

    // Sum the row groups of this wave: l and O were accumulated per group.
    // l is uniform inside a group; O holds a different column slice in each
    // lane of a group, so its sum pairs lanes by xor only (the mirror steps of
    // group_reduce would mix columns when a row spans fewer than 16 lanes:
    // fp32 D <= 32, bf16 D <= 64).
#pragma unroll
    for (int h = 0; h < NREP; ++h) {
        l[h] = group_reduce<OpSum, LPR, kWave>(l[h]);
#pragma unroll
        for (int e = 0; e < E; ++e) o[h][e] = group_reduce_xor<OpSum, LPR, kWave>(o[h][e]);
    }

    __shared__ float sh_m[W][NREP];
    __shared__ float sh_l[W][NREP];
    __shared__ float sh_o[W][NREP][D];
    if (lane < LPR) {
#pragma unroll
        for (int h = 0; h < NREP; ++h) {
#pragma unroll
            for (int e = 0; e < E; ++e) sh_o[wave][h][col * E + e] = o[h][e];
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < NREP; ++h) { sh_m[wave][h] = m[h]; sh_l[wave][h] = l[h]; }
    }
    __syncthreads();

    // Merge the waves: this chunk's (m, l, O).
    for (int i = threadIdx.x; i < NREP * D; i += THREADS) {
        const int h = i / D, d = i % D;
        float mm = sh_m[0][h];
#pragma unroll
        for (int w = 1; w < W; ++w) mm = fmaxf(mm, sh_m[w][h]);
        float acc = 0.f, lsum = 0.f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            // A wave that saw no tile has m = -inf and contributes nothing.
            const float c = (sh_m[w][h] == -INFINITY) ? 0.f
                          : __builtin_amdgcn_exp2f((sh_m[w][h] - mm) * kLog2e);
            acc = fmaf(c, sh_o[w][h][d], acc);
            lsum = fmaf(c, sh_l[w][h], lsum);
        }
        const size_t bh = (size_t)seq * a.n_q + g * NREP + h;
        if (n_active == 1) {
            a.out[bh * D + d] = acc / lsum;
        } else {
            a.part_o[(bh * a.n_split + split) * D + d] = acc;
            if (d == 0) {
                a.part_ml[(bh * a.n_split + split) * 2 + 0] = mm;
                a.part_ml[(bh * a.n_split + split) * 2 + 1] = lsum;
            }
        }
    }
    if constexpr (FUSED) {
        // Commit: one workgroup per sequence; no workgroup of this launch
        // reads the device length.
        if (a.commit && owner && g == 0 && threadIdx.x == 0) a.lens_out[cache_row] = pos + 1;
    }
}

// Log-sum-exp merge of the chunk partials of one (sequence, query head):
// O = sum_c e^{m_c-M} O_c / sum_c e^{m_c-M} l_c.  A separate launch: the
// kernel boundary publishes the partials, where an in-kernel hand-off would
// need a device-scope fence per workgroup (measured at ~57 ns each,
// serialised across the device).  A row's DS workgroups each take D/DS of
// its columns; MT threads read the partials as float4 columns, PARTS chunks
// at a time, so one round trip covers up to MT/(D/4/DS) chunks.
template <int D, bool PAGED, int MT, bool FUSED = false, int DS = 1>
__global__ void __launch_bounds__(MT)
lse_merge_kernel(DecodeArgs a) {
    constexpr int V4 = D / 4 / DS;    // float4 columns of this workgroup: slice blockIdx.y of DS
    constexpr int PARTS = MT / V4;
    static_assert(PARTS >= 1 && PARTS * V4 == MT, "threads per column");
    const int bh = blockIdx.x;
    const int seq = bh / a.n_q;
    int len;
    if constexpr (FUSED) {
        len = min(min(a.pos.row[seq] + 1, a.max_pages * 64), a.n_split * a.chunk);
    } else if constexpr (PAGED) {
        const int row = a.rows.row[seq];
        const int committed = a.host_lens ? a.pos.row[seq] : a.seq_lens[row];
        len = min(min(committed + a.n_pending, a.max_pages * 64), a.n_split * a.chunk);
    } else {
        len = a.T;
    }
    const int n_active = len > 0 ? (len - 1) / a.chunk + 1 : 0;
    if (n_active <= 1) return;     // written directly by the split kernel
    __shared__ float sh_w[kSplitCap];
    __shared__ float4 sh_red[PARTS][V4];
    __shared__ float sh_scr[MT / kWave];
    const float* ml = a.part_ml + (size_t)bh * a.n_split * 2;
    const float4* po = reinterpret_cast<const float4*>(a.part_o + (size_t)bh * a.n_split * D) + blockIdx.y * V4;
    const int j = threadIdx.x % V4;
    const int part = threadIdx.x / V4;
    // The first NPRE partial rows of this thread are loaded before the
    // reductions, so their latency overlaps that of the (m, l) loads.
    constexpr int NPRE = 8;
    float4 pre[NPRE];
#pragma unroll
    for (int k = 0; k < NPRE; ++k) {
        const int c = part + k * PARTS;
        pre[k] = c < n_active ? po[(size_t)c * (D / 4) + j] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mx = -INFINITY;
    for (int c = threadIdx.x; c < n_active; c += MT) mx = fmaxf(mx, ml[2 * c]);
    mx = block_reduce<OpMax, MT / kWave>(mx, sh_scr);
    float ls = 0.f;
    for (int c = threadIdx.x; c < n_active; c += MT) {
        const float w = __builtin_amdgcn_exp2f((ml[2 * c] - mx) * kLog2e);
        sh_w[c] = w;
        ls = fmaf(w, ml[2 * c + 1], ls);
    }
    ls = block_reduce<OpSum, MT / kWave>(ls, sh_scr);   // also orders the sh_w writes
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < NPRE; ++k) {
        const int c = part + k * PARTS;
        if (c < n_active) {
            const float w = sh_w[c];
            acc.x = fmaf(w, pre[k].x, acc.x); acc.y = fmaf(w, pre[k].y, acc.y);
            acc.z = fmaf(w, pre[k].z, acc.z); acc.w = fmaf(w, pre[k].w, acc.w);
        }
    }
#pragma unroll 4
    for (int c = part + NPRE * PARTS; c < n_active; c += PARTS) {
        const float4 x = po[(size_t)c * (D / 4) + j];
        const float w = sh_w[c];
        acc.x = fmaf(w, x.x, acc.x); acc.y = fmaf(w, x.y, acc.y);
        acc.z = fmaf(w, x.z, acc.z); acc.w = fmaf(w, x.w, acc.w);
    }
    sh_red[part][j] = acc;
    __syncthreads();
    if (threadIdx.x < V4) {
        float4 t = sh_red[0][j];
#pragma unroll
        for (int pp = 1; pp < PARTS; ++pp) {
            const float4 u = sh_red[pp][j];
            t.x += u.x; t.y += u.y; t.z += u.z; t.w += u.w;
        }
        const float inv = 1.0f / ls;
        reinterpret_cast<float4*>(a.out + (size_t)bh * D)[blockIdx.y * V4 + j] =
            make_float4(t.x * inv, t.y * inv, t.z * inv, t.w * inv);
    }
}

__global__ void zero_kernel(float* p, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0.f;
}

int env_int(const char* name, int dflt) {
    const char* s = std::getenv(name);
    return s ? std::atoi(s) : dflt;
}

long long round64(long long c) { return (c + 63) / 64 * 64; }

// Smallest chunk ever used: every wave of a workgroup gets a tile.
constexpr int kMinChunk = 128;
// Default chunks stay within [256, 4096] tokens: small enough for many
// workgroups per CU (a ragged last round of a few large workgroups costs more
// than their merge), large enough to amortise a workgroup's prologue.  About
// 16 workgroups per CU of total work, in multiples of 128 tokens (every wave
// of a 4-wave workgroup then walks the same number of 32-token bf16 tiles).
// Measured (B = 64 paged bf16, 979-31,078 tokens, chunks 1088 .. 3072):
// 2048 tokens 0.676 ms, 2112 0.690, 1088 0.700.
constexpr int kChunkLo = 256;
constexpr int kChunkHi = 4096;
constexpr int kGroupsPerCu = 16;
constexpr int kChunkAlign = 128;

// Tokens per workgroup for a launch over total_rows (sequence x KV head x
// token) rows whose longest sequence may reach max_len tokens: about
// kGroupsPerCu workgroups per CU within [kChunkLo, kChunkHi], at most
// kSplitTarget chunks per sequence, a multiple of kChunkAlign tokens.
// SA_DECODE_CHUNK overrides those rules (still at most kSplitCap chunks).
// max_chunk bounds the result (paged chunks: kMaxChunkPages pages) unless
// kSplitCap forbids it.
// A chunk the caller fixed: sa_set_attention_blocks' kv block, else
// SA_DECODE_CHUNK; 0 when neither is set.
int forced_chunk() {
    const int set = attn_kv_block();
    return set > 0 ? set : env_int("SA_DECODE_CHUNK", 0);
}

int pick_chunk(long long total_rows, long long max_len, long long max_chunk = 1LL << 30) {
    const long long cap_floor = round64((max_len + kSplitCap - 1) / kSplitCap);
    const int forced = forced_chunk();
    long long c;
    if (forced > 0) {
        // A fixed chunk may be a single page: the waves past its tiles see
        // none and contribute nothing to the chunk's merge.
        c = std::max<long long>(round64(forced), 64);
    } else {
        const long long target = (long long)kGroupsPerCu * device_cu_count();
        c = std::min<long long>(std::max<long long>((total_rows + target - 1) / target, kChunkLo), kChunkHi);
        c = std::max<long long>(c, (max_len + kSplitTarget - 1) / kSplitTarget);
        c = (c + kChunkAlign - 1) / kChunkAlign * kChunkAlign;
        // Above 1024 tokens, the nearest multiple of 512 (still within the
        // split caps below).  B = 64 paged bf16 (979-31,078 tokens), same
        // box: 2048-token chunks 0.680 ms per call and 20.47 ms per 28-layer
        // model step, against 0.689 / 20.71 at the 2176 of 128-alignment,
        // 0.685 / 20.69 at 1792 and 0.683 / 20.64 at 2304.
        if (c > 1024) c = (c + 256) / 512 * 512;
    }
    return (int)std::max<long long>(std::min<long long>(c, max_chunk), cap_floor);
}

// Upper bound of the split count any call may use for sequences up to max_len.
long long max_splits_for(long long max_len) {
    // Fixed chunks may be as short as one 64-token page.
    const long long c = std::max<long long>(64, round64((max_len + kSplitCap - 1) / kSplitCap));
    return (max_len + c - 1) / c;
}

size_t ws_bytes_for(long long bh, long long n_split, int d) {
    if (n_split <= 1) return 0;
    return (size_t)(bh * n_split * (2 + d)) * sizeof(float);
}

void carve_ws(DecodeArgs& a, void* ws, long long bh) {
    a.part_ml = static_cast<float*>(ws);
    a.part_o = a.part_ml + (size_t)bh * a.n_split * 2;
}

template <int D, int NREP, bool BF16, bool PAGED, bool FUSED>
sa_status launch_decode(const DecodeArgs& a, int n_seq, hipStream_t st) {
    constexpr int W = waves_for<D, NREP>();
    dim3 grid(a.n_kv, a.n_split, n_seq);
    if (PAGED && a.compact) grid = dim3(a.n_kv, a.cstart[n_seq], 1);
    if constexpr (NREP == 1 && !PAGED) {
        if ((long long)a.n_split * a.n_kv * n_seq <= device_cu_count()) {
            if (a.chunk <= 2 * kWavesOneRound * Geo<D, BF16>::TILE)
                hipLaunchKernelGGL((split_kv_decode_kernel<D, NREP, BF16, PAGED, kWavesOneRound, false, false>), grid,
                                   dim3(kWavesOneRound * kWave), 0, st, a);
            else
                hipLaunchKernelGGL((split_kv_decode_kernel<D, NREP, BF16, PAGED, kWavesOneRound>), grid,
                                   dim3(kWavesOneRound * kWave), 0, st, a);
        } else {
            hipLaunchKernelGGL((split_kv_decode_kernel<D, NREP, BF16, PAGED, W>), grid, dim3(W * kWave), 0, st, a);
        }
    } else if constexpr (PAGED && NREP <= 4 && NREP * D <= 512) {
        // Paged launches that fit one round of workgroups (short sequences, a
        // decode step of a few rows) use eight waves: half the tiles per
        // wave, so fewer dependent load round trips.
        if ((long long)a.n_split * a.n_kv * n_seq <= device_cu_count()) {
            // One register tile when every wave walks at most two tiles
            // (config-3 loop, graph-replayed: fp32 fused step 7.31-7.36 ->
            // 6.51-6.54 us, bf16 6.71-6.76 -> 6.60 us, same box).
            if (a.chunk <= 2 * kWavesOneRound * Geo<D, BF16>::TILE)
                hipLaunchKernelGGL((split_kv_decode_kernel<D, NREP, BF16, PAGED, kWavesOneRound, FUSED, false>), grid,
                                   dim3(kWavesOneRound * kWave), 0, st, a);
            else
                hipLaunchKernelGGL((split_kv_decode_kernel<D, NREP, BF16, PAGED, kWavesOneRound, FUSED>), grid,
                                   dim3(kWavesOneRound * kWave), 0, st, a);
        } else {
            hipLaunchKernelGGL((split_kv_decode_kernel<D, NREP, BF16, PAGED, W, FUSED>), grid, dim3(W * kWave), 0, st,
                               a);
        }
    } else {
        hipLaunchKernelGGL((split_kv_decode_kernel<D, NREP, BF16, PAGED, W, FUSED>), grid, dim3(W * kWave), 0, st, a);
    }
    SA_CHECK_LAUNCH();
    if (a.n_split > 1) {
        const dim3 mgrid(n_seq * a.n_q);
        // Rows with many chunks: four 256-thread workgroups per row, each
        // merging a quarter of head_dim (their block reductions span 4
        // waves).  Measured on the T = 262144 single-query call (256 chunks,
        // same box, interleaved): 44.7 us per call against 45.9 us with one
        // 1024-thread workgroup per row; 2 or 8 slices, or 128 threads,
        // 45.2-45.5 us.
        if (a.n_split >= 64) {
            if constexpr (D % 16 == 0)
                hipLaunchKernelGGL((lse_merge_kernel<D, PAGED, 256, FUSED, 4>), dim3(n_seq * a.n_q, 4), dim3(256), 0,
                                   st, a);
            else
                hipLaunchKernelGGL((lse_merge_kernel<D, PAGED, 1024, FUSED>), mgrid, dim3(1024), 0, st, a);
        } else
            hipLaunchKernelGGL((lse_merge_kernel<D, PAGED, 256, FUSED>), mgrid, dim3(256), 0, st, a);
        SA_CHECK_LAUNCH();
    }
    return SA_OK;
}

template <int D, bool BF16, bool PAGED, bool FUSED>
sa_status dispatch_nrep(const DecodeArgs& a, int n_seq, int nrep, hipStream_t st) {
    switch (nrep) {
        case 1: return launch_decode<D, 1, BF16, PAGED, FUSED>(a, n_seq, st);
        case 2: return launch_decode<D, 2, BF16, PAGED, FUSED>(a, n_seq, st);
        case 4: return launch_decode<D, 4, BF16, PAGED, FUSED>(a, n_seq, st);
        case 8: return launch_decode<D, 8, BF16, PAGED, FUSED>(a, n_seq, st);
        default: return fail(SA_EINVAL, "n_q_heads / n_kv_heads must be 1, 2, 4 or 8");
    }
}

// Head sizes 8 .. 256 (powers of two): a K/V row is D / E lanes of 16-byte
// loads, 64 / (D / E) rows per wave-load.  The fused decode step takes the
// sizes of the model path, 64 .. 256.
template <bool BF16, bool PAGED, bool FUSED = false>
sa_status dispatch_decode(const DecodeArgs& a, int n_seq, int d, int nrep, hipStream_t st) {
    if constexpr (!FUSED) {
        switch (d) {
            case 8: return dispatch_nrep<8, BF16, PAGED, false>(a, n_seq, nrep, st);
            case 16: return dispatch_nrep<16, BF16, PAGED, false>(a, n_seq, nrep, st);
            case 32: return dispatch_nrep<32, BF16, PAGED, false>(a, n_seq, nrep, st);
            default: break;
        }
    }
    switch (d) {
        case 64: return dispatch_nrep<64, BF16, PAGED, FUSED>(a, n_seq, nrep, st);
        case 128: return dispatch_nrep<128, BF16, PAGED, FUSED>(a, n_seq, nrep, st);
        case 256: return dispatch_nrep<256, BF16, PAGED, FUSED>(a, n_seq, nrep, st);
        default:
            return fail(SA_EINVAL, FUSED ? "head_dim must be 64, 128 or 256"
                                         : "head_dim must be 8, 16, 32, 64, 128 or 256");
    }
}

bool supported_d(int d) { return d == 8 || d == 16 || d == 32 || d == 64 || d == 128 || d == 256; }

}  // namespace

// ----- dense -----------------------------------------------------------------

sa_status decode_dense(const float* q, const float* k, const float* v, int batch, int n_q,
                       int n_kv, int T, int d, float scale, float* out, void* ws,
                       size_t ws_bytes, hipStream_t st) {
    if (!q || !out || (T > 0 && (!k || !v))) return fail(SA_EINVAL, "null pointer");
    if (batch <= 0 || n_q <= 0 || n_kv <= 0 || n_q % n_kv)
        return fail(SA_EINVAL, "bad head counts");
    if (!supported_d(d)) return fail(SA_EINVAL, "head_dim must be 8, 16, 32, 64, 128 or 256");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
        return fail(SA_EINVAL, "q, k, v and out must be 16-byte aligned");
    if (T <= 0) {
        size_t n = (size_t)batch * n_q * d;
        hipLaunchKernelGGL(zero_kernel, dim3((n + 255) / 256), dim3(256), 0, st, out, n);
        SA_CHECK_LAUNCH();
        return SA_OK;
    }
    DecodeArgs a{};
    a.q = q; a.k = k; a.v = v; a.out = out;
    a.n_kv = n_kv; a.n_q = n_q; a.T = T; a.scale = scale;
    const long long rows = (long long)batch * n_kv * T;
    a.chunk = pick_chunk(rows, T);
    // Dense launches of at most 64 rows per CU (one head of up to 16,384
    // tokens on 256 CUs) take the smallest chunk: one tile per wave, still
    // one round of workgroups.  Measured per single-head call: T = 1024
    // 8.0-8.4 against 9.9 us, T = 8192 9.4-9.7 against 10.8-11.0 us; at
    // T = 65536 it would mean two rounds (17.6 against 16.5 us).
    if (forced_chunk() <= 0 && rows <= 64LL * device_cu_count()) a.chunk = kMinChunk;
    a.n_split = (T + a.chunk - 1) / a.chunk;
    const long long bh = (long long)batch * n_q;
    const size_t need = ws_bytes_for(bh, a.n_split, d);
    if (need > 0) {
        if (!ws || ws_bytes < need) return fail(SA_ENOMEM, "workspace too small for split-KV partials");
        carve_ws(a, ws, bh);
    }
    return dispatch_decode<false, false>(a, batch, d, n_q / n_kv, st);
}

size_t decode_dense_ws(int batch, int n_q, int T, int d) {
    if (batch <= 0 || n_q <= 0 || T <= 0 || !supported_d(d)) return 0;
    // n_kv <= n_q: sized for the most groups and the most chunks.
    return ws_bytes_for((long long)batch * n_q, max_splits_for(T), d);
}

// ----- paged -----------------------------------------------------------------

size_t paged_ws(int n_seq, int n_q, int n_kv, int d, int max_pages) {
    const long long max_tokens = (long long)max_pages * 64;
    (void)n_kv;
    // Launches take up to kRowsPerLaunch sequences and reuse the workspace.
    return ws_bytes_for((long long)std::min(n_seq, kRowsPerLaunch) * n_q, max_splits_for(max_tokens), d);
}

sa_status decode_paged(const PagedView& c, const float* q, int n_seq, const int32_t* seq_ids,
                       const int32_t* lens, int n_q, int n_pending, int max_len, long long total_len,
                       float scale, float* out, void* ws, size_t ws_bytes, hipStream_t st) {
    if (!q || !out) return fail(SA_EINVAL, "null pointer");
    if (n_seq <= 0 || n_q <= 0 || n_q % c.n_kv) return fail(SA_EINVAL, "bad head counts");
    if (!aligned16(q) || !aligned16(out)) return fail(SA_EINVAL, "q and out must be 16-byte aligned");
    if (max_len <= 0) max_len = 1;
    DecodeArgs a{};
    a.q = q; a.k = c.k_pool; a.v = c.v_pool; a.out = out;
    a.block_table = c.block_table; a.seq_lens = c.seq_lens;
    a.n_kv = c.n_kv; a.n_q = n_q; a.max_pages = c.max_pages; a.n_pending = n_pending;
    a.num_pages = c.num_pages;
    a.scale = scale;
    // The chunk bound uses the table capacity so the workspace size holds.
    a.chunk = pick_chunk(total_len * c.n_kv, (long long)c.max_pages * 64, (long long)kMaxChunkPages * 64);
    if (a.chunk > kMaxChunkPages * 64) return fail(SA_EINVAL, "max_pages_per_seq too large for the split cap");
    a.n_split = (max_len + a.chunk - 1) / a.chunk;
    const long long bh = (long long)std::min(n_seq, kRowsPerLaunch) * n_q;
    const size_t need = ws_bytes_for(bh, a.n_split, c.d);
    if (need > 0) {
        if (!ws || ws_bytes < need) return fail(SA_ENOMEM, "workspace too small for split-KV partials");
        carve_ws(a, ws, bh);
    }
    // Up to kRowsPerLaunch sequences per launch, their cache rows by value;
    // the workspace is reused launch after launch in stream order.
    for (int i0 = 0; i0 < n_seq; i0 += kRowsPerLaunch) {
        const int m = std::min(kRowsPerLaunch, n_seq - i0);
        for (int i = 0; i < m; ++i) a.rows.row[i] = seq_ids ? seq_ids[i0 + i] : i0 + i;
        if (lens) {
            a.host_lens = 1;
            a.cstart[0] = 0;
            for (int i = 0; i < m; ++i) {
                a.pos.row[i] = lens[i0 + i];
                const int len = std::min(std::min(lens[i0 + i] + n_pending, c.max_pages * 64), a.n_split * a.chunk);
                a.cstart[i + 1] = a.cstart[i] + std::max(1, (len + a.chunk - 1) / a.chunk);
            }
            for (int i = m; i < kRowsPerLaunch; ++i) a.cstart[i + 1] = 0x7fffffff;
            a.compact = env_int("SA_DECODE_COMPACT", 1) != 0 && a.cstart[m] <= 65535 ? 1 : 0;
        }
        a.q = q + (size_t)i0 * n_q * c.d;
        a.out = out + (size_t)i0 * n_q * c.d;
        if (c.bf16) {
            SA_TRY((dispatch_decode<true, true>(a, m, c.d, n_q / c.n_kv, st)));
        } else {
            SA_TRY((dispatch_decode<false, true>(a, m, c.d, n_q / c.n_kv, st)));
        }
    }
    return SA_OK;
}

sa_status decode_paged_fused(const PagedView& c, const float* q, int n_seq, const int32_t* seq_ids, int n_q,
                             const FusedAppend& f, int max_len, long long total_len, float scale, float* out,
                             void* ws, size_t ws_bytes, hipStream_t st) {
    if (!out || !f.pos || !f.lens || (!f.part && (!q || !f.k || !f.v))) return fail(SA_EINVAL, "null pointer");
    if (f.part && (f.part_S <= 0 || f.part_M < n_seq)) return fail(SA_EINVAL, "bad projection partials");
    if (n_seq <= 0 || n_q <= 0 || n_q % c.n_kv) return fail(SA_EINVAL, "bad head counts");
    if (!aligned16(q) || !aligned16(out)) return fail(SA_EINVAL, "q and out must be 16-byte aligned");
    if (max_len <= 0) max_len = 1;
    DecodeArgs a{};
    a.k = c.k_pool; a.v = c.v_pool;
    a.part_N = (n_q + 2 * c.n_kv) * c.d;
    a.part_S = f.part_S;
    a.part_split = (size_t)f.part_M * a.part_N;
    a.block_table = c.block_table; a.seq_lens = c.seq_lens;
    a.n_kv = c.n_kv; a.n_q = n_q; a.max_pages = c.max_pages; a.n_pending = 1;
    a.num_pages = c.num_pages;
    a.scale = scale;
    a.wq = f.wq; a.wk = f.wk; a.eps = f.eps; a.cos_t = f.cos_t; a.sin_t = f.sin_t;
    a.rope_max_pos = f.rope_max_pos; a.lens_out = f.lens; a.commit = f.commit ? 1 : 0;
    // The same chunking as decode_paged with one pending token.
    a.chunk = pick_chunk(total_len * c.n_kv, (long long)c.max_pages * 64, (long long)kMaxChunkPages * 64);
    if (a.chunk > kMaxChunkPages * 64) return fail(SA_EINVAL, "max_pages_per_seq too large for the split cap");
    a.n_split = (max_len + a.chunk - 1) / a.chunk;
    const long long bh = (long long)std::min(n_seq, kRowsPerLaunch) * n_q;
    const size_t need = ws_bytes_for(bh, a.n_split, c.d);
    if (need > 0) {
        if (!ws || ws_bytes < need) return fail(SA_ENOMEM, "workspace too small for split-KV partials");
        carve_ws(a, ws, bh);
    }
    for (int i0 = 0; i0 < n_seq; i0 += kRowsPerLaunch) {
        const int m = std::min(kRowsPerLaunch, n_seq - i0);
        // The grid covers only the chunks that hold tokens (with chunks sized
        // for the longest sequence, the short ones' empty workgroups took
        // about 2 % of the 28-layer, 64-sequence step: 19.28 against
        // 19.63-19.88 ms, same box).  SA_DECODE_COMPACT=0 keeps the full
        // (KV head, chunk, sequence) grid.
        a.cstart[0] = 0;
        for (int i = 0; i < m; ++i) {
            a.rows.row[i] = seq_ids ? seq_ids[i0 + i] : i0 + i;
            a.pos.row[i] = f.pos[i0 + i];
            const int len = std::min(std::min(f.pos[i0 + i] + 1, c.max_pages * 64), a.n_split * a.chunk);
            a.cstart[i + 1] = a.cstart[i] + std::max(1, (len + a.chunk - 1) / a.chunk);
        }
        for (int i = m; i < kRowsPerLaunch; ++i) a.cstart[i + 1] = 0x7fffffff;
        a.compact = env_int("SA_DECODE_COMPACT", 1) != 0 && a.cstart[m] <= 65535 ? 1 : 0;
        a.out = out + (size_t)i0 * n_q * c.d;
        a.q_out = f.q_out ? f.q_out + (size_t)i0 * n_q * c.d : nullptr;
        if (f.part) {
            a.part = f.part + (size_t)i0 * a.part_N;
        } else {
            a.q = q + (size_t)i0 * n_q * c.d;
            a.k_new = f.k + (size_t)i0 * c.n_kv * c.d;
            a.v_new = f.v + (size_t)i0 * c.n_kv * c.d;
        }
        if (c.bf16) {
            SA_TRY((dispatch_decode<true, true, true>(a, m, c.d, n_q / c.n_kv, st)));
        } else {
            SA_TRY((dispatch_decode<false, true, true>(a, m, c.d, n_q / c.n_kv, st)));
        }
    }
    return SA_OK;
}

// ----- allocation-free single-query entry --------------------------------------

namespace {

// Split-KV partials of sa_stream_attn_f32_noalloc: (m, l) and O per chunk,
// for the most chunks any call can use (kSplitCap) at the widest head
// (SA_MAX_HEAD_DIM): 1,056,768 bytes, held by each GPU the library runs on
// until the process ends.  Nothing in it needs clearing: a call writes every
// partial it reads.
constexpr size_t kScratchBytes = (size_t)kSplitCap * (2 + SA_MAX_HEAD_DIM) * sizeof(float);
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

// The device address of this GPU's copy of `scratch`, looked up once per
// device with that device current.  Host code never passes the array's name
// itself to a kernel: on the host it is only a stand-in for the symbol.
sa_status scratch_address(void** out) {
    static std::mutex mu;
    static std::vector<void*> per_device;
    int dev = 0;
    SA_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(mu);
    if ((int)per_device.size() <= dev) per_device.resize(dev + 1, nullptr);
    if (!per_device[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                   "hipGetSymbolAddress(scratch)");
        per_device[dev] = p;
    }
    *out = per_device[dev];
    return SA_OK;
}

}  // namespace

sa_status stream_attn_noalloc(const float* Q, const float* K, const float* V, int T, int d, float scale,
                              float* O, hipStream_t st) {
    const size_t need = decode_dense_ws(1, 1, T, d);
    if (need > kScratchBytes) return fail(SA_EINVAL, "T and d need more split-KV scratch than the 1 MiB maximum");
    void* ws = nullptr;
    SA_TRY(scratch_address(&ws));
    return decode_dense(Q, K, V, 1, 1, 1, T, d, scale, O, ws, kScratchBytes, st);
}

}  // namespace sa

// ----- C ABI -------------------------------------------------------------------

extern "C" size_t sa_stream_attn_ws_bytes(int T, int d) { return sa::decode_dense_ws(1, 1, T, d); }

extern "C" sa_status sa_stream_attn_f32(const float* Q, const float* K, const float* V, int T,
                                        int d, int block_size, float scale, float* O, void* ws,
                                        size_t ws_bytes, sa_stream_t stream) {
    sa::clear_error();
    if (block_size <= 0) return sa::fail(SA_EINVAL, "block_size must be positive");
    return sa::decode_dense(Q, K, V, 1, 1, 1, T, d, scale, O, ws, ws_bytes, sa::as_stream(stream));
}

extern "C" sa_status sa_stream_attn_f32_noalloc(const float* Q, const float* K, const float* V, int T,
                                                int d, int block_size, float scale, float* O,
                                                sa_stream_t stream) {
    sa::clear_error();
    if (block_size <= 0) return sa::fail(SA_EINVAL, "block_size must be positive");
    return sa::stream_attn_noalloc(Q, K, V, T, d, scale, O, sa::as_stream(stream));
}

extern "C" size_t sa_decode_dense_ws_bytes(int batch, int n_q_heads, int T, int d) {
    return sa::decode_dense_ws(batch, n_q_heads, T, d);
}

extern "C" sa_status sa_decode_dense_f32(const float* q, const float* k, const float* v, int batch,
                                         int n_q_heads, int n_kv_heads, int T, int d, float scale,
                                         float* out, void* ws, size_t ws_bytes, sa_stream_t stream) {
    sa::clear_error();
    return sa::decode_dense(q, k, v, batch, n_q_heads, n_kv_heads, T, d, scale, out, ws, ws_bytes,
                            sa::as_stream(stream));
}
