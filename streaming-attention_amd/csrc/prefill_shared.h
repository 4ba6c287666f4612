// Types and device helpers of the causal prefill kernels: launch arguments,
// the work mapping, the load-to-LDS tile movement, and the folded-softmax
// helpers.
#pragma once

#include <cstdlib>

#include "sa_internal.h"

namespace sa {
namespace pf {

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
    int gh;             // query heads per workgroup (divides Hq / Hkv)
    float sl2;          // |scale| * log2(e)
    uint32_t q_sign;    // 0x80008000 to negate bf16 q pairs (negative scale), else 0
    float scale;        // signed scale (fp32 kernel)
    int q_tile;         // query rows per workgroup and head
    int k_tile;         // keys per tile of the kernel's loop (paired launches)
    float* part;        // paired launches: the split tiles' partials
    long long part_rows;
};

// Work mapping shared by both kernels.  A KV group is one (batch, kv head);
// its G = Hq/Hkv query heads read the same K/V, and a workgroup serves gh of
// them (so G/gh workgroups share each query tile).  When the number of groups
// is a multiple of 8, hardware workgroup i (dispatched to XCD i % 8) takes
// work slot i / 8 of the groups owned by that XCD, so each XCD's L2 holds the
// K/V of its own groups only.  Inside an XCD (or the whole grid otherwise)
// slots run heaviest query tile first, which balances the causal triangle.
struct Work { int b, h0, kvh, qt; };
__device__ __forceinline__ Work map_work(const PrefillArgs& pa, int i) {
    const int G = pa.Hq / pa.Hkv;
    const int HS = G / pa.gh;                         // head sets per group
    int x = 0, j = i, span = gridDim.x / (HS * pa.n_qt);   // groups in this slot range
    if (pa.xcd_groups) { x = i & 7; j = i >> 3; span = pa.xcd_groups; }
    const int per_qt = span * HS;
    Work w;
    w.qt = pa.n_qt - 1 - j / per_qt;
    const int rem = j % per_qt;
    const int group = x * span + rem / HS;
    w.b = group / pa.Hkv;
    w.kvh = group % pa.Hkv;
    w.h0 = w.kvh * G + (rem % HS) * pa.gh;
    return w;
}

// Paired launches (short prompts, one round of workgroups): query tile t and
// tile u = n_qt - 1 - t form a pair whose key tiles add up to about the same
// count for every t.  Workgroup A computes tile t whole and the first s key
// tiles of u; workgroup B the rest of u's; so every workgroup walks about
// half the longest tile's keys instead of up to all of them.  u's two
// partials meet in the merge launch.  s = 0: no split, B writes u.

// Key tiles (ktile keys each) of query tile t (qtile rows) under the causal mask.
__host__ __device__ constexpr int pair_key_tiles(int L, int qtile, int ktile, int t) {
    return ((L < (t + 1) * qtile ? L : (t + 1) * qtile) - 1) / ktile + 1;
}
__host__ __device__ constexpr int pair_split(int L, int qtile, int ktile, int t, int u) {
    return (pair_key_tiles(L, qtile, ktile, u) - pair_key_tiles(L, qtile, ktile, t)) / 2;
}

// A workgroup's segments: query tile qt[i], key tiles [k0[i], k1[i]); part[i]
// < 0 writes the output rows, else partial slot part[i] of the pair.
struct PairSegs {
    int n;
    int qt[2], k0[2], k1[2], part[2];
};

// The segments of the workgroup map_work gave query tile slot wk_qt (slot
// n_qt - 1 - wk_qt is dispatched in that order: B of each pair, then A).
__device__ __forceinline__ PairSegs pair_segments(const PrefillArgs& pa, int wk_qt, int qtile, int ktile) {
    const int L = pa.L;
    const int slot = pa.n_qt - 1 - wk_qt;
    const int np = pa.n_qt / 2;
    PairSegs sg{1, {0, 0}, {0, 0}, {0, 0}, {-1, -1}};
    if (slot >= 2 * np) {                     // the middle tile of an odd count
        sg.qt[0] = np;
        sg.k1[0] = pair_key_tiles(L, qtile, ktile, np);
        return sg;
    }
    const int t = slot >> 1, u = pa.n_qt - 1 - t;
    const int s = pair_split(L, qtile, ktile, t, u);
    if (slot & 1) {                           // A: tile t whole, then u's first s key tiles
        sg.qt[0] = t;
        sg.k1[0] = pair_key_tiles(L, qtile, ktile, t);
        if (s > 0) {
            sg.qt[1] = u;
            sg.k1[1] = s;
            sg.part[1] = 0;
            sg.n = 2;
        }
    } else {                                  // B: the rest of u's key tiles
        sg.qt[0] = u;
        sg.k0[0] = s;
        sg.k1[0] = pair_key_tiles(L, qtile, ktile, u);
        sg.part[0] = s > 0 ? 1 : -1;
    }
    return sg;
}

// Partial rows of a paired launch: [2][part_rows][128] O, then [2][part_rows]
// (m, l); row ((b Hq + h) n_pairs + pair) qtile + query within the tile,
// pair = n_qt - 1 - (the long tile).
__device__ __forceinline__ long long pair_row(const PrefillArgs& pa, int b, int h, int qt, int qi) {
    return (((long long)b * pa.Hq + h) * (pa.n_qt / 2) + (pa.n_qt - 1 - qt)) * pa.q_tile + (qi - qt * pa.q_tile);
}

// The K rows a lane feeds to the score MFMA are permuted within each 32-key
// block (bits 2 and 3 of the row swapped).  With the 32x32 output layout
// (lane l: column l%32, rows 8*(j/4) + 4*(l/32) + j%4 for element j) this
// makes element j of lane l the score of key 16*(j/8) + 8*(l/32) + j%8: each
// lane's 8-element groups are 8 consecutive keys, exactly what the B operand
// of the 32x32x16 PV step needs, and what one 16-byte read of V^T supplies.
__device__ __forceinline__ int swap_bits23(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

constexpr int kDmaRowBytes = 256;                     // one row of 128 bf16
constexpr int kDmaTileBytes = kKTile * kDmaRowBytes;  // one tensor's tile
constexpr int kDmaStageBytes = 2 * kDmaTileBytes;     // K, then V

// Chunk c (16 bytes) of tile row r sits at chunk position c ^ dma_swz(r) of
// the row.  Exhaustive check over the lane patterns: the K fragment reads (16
// lanes, 16 rows, one chunk) and the V transpose reads (32 lanes, 2 x 4 rows,
// 4 chunks) touch 64 distinct banks per cycle.
__device__ __forceinline__ int dma_swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) unsigned char lds_u8_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

// One global_load_lds_dwordx4: lane l copies 16 bytes from g into LDS at dst
// + 16 l.  Issued as inline assembly so that the compiler does not track it:
// its wait-count pass makes every LDS read after a load-to-LDS wait for all
// of them (vmcnt(0)), which would drain the tile prefetched NS - 1 tiles ahead
// in the middle of each tile.  The kernel waits for these loads itself
// (s_waitcnt vmcnt before each tile barrier).  m0 holds the LDS address; the
// s_nop covers the m0-write-to-load-to-LDS hazard.  hipcc warns that m0 in a
// clobber list is reserved; no code it generates for these kernels reads or
// writes m0 (every m0 access in their ISA is this block's), so nothing it
// holds there is lost.
__device__ __forceinline__ void dma16(const uint16_t* g, lds_u8_t* dst) {
    const uint32_t m = static_cast<uint32_t>(reinterpret_cast<size_t>(dst));
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(m) : "memory", "m0");
}

constexpr float kSumCap = 65536.f;

// acc + the sum of the 8 bf16 values of v (v_dot2c_f32_bf16 against 1.0).
// The pairs are taken with shufflevector: bit-casting the 32-bit elements of
// the vector to bf16 pairs made hipcc (ROCm 7.2) feed the first pair to all
// four dot products.
__device__ __forceinline__ float sum_bf16x8(const bf16x8_t& v, float acc) {
    const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 0, 1), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 2, 3), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 4, 5), one, acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_shufflevector(v, v, 6, 7), one, acc, false);
    return acc;
}

__device__ __forceinline__ bf16x8_t pack_bf16x8(const float* p) {
    const bf16x2_t p01 = __builtin_convertvector(f32x2_t{p[0], p[1]}, bf16x2_t);
    const bf16x2_t p23 = __builtin_convertvector(f32x2_t{p[2], p[3]}, bf16x2_t);
    const bf16x2_t p45 = __builtin_convertvector(f32x2_t{p[4], p[5]}, bf16x2_t);
    const bf16x2_t p67 = __builtin_convertvector(f32x2_t{p[6], p[7]}, bf16x2_t);
    return __builtin_bit_cast(bf16x8_t, make_uint4(__builtin_bit_cast(uint32_t, p01), __builtin_bit_cast(uint32_t, p23),
                                                   __builtin_bit_cast(uint32_t, p45), __builtin_bit_cast(uint32_t, p67)));
}

// Dynamic LDS above 64 KiB needs a per-kernel, per-device opt-in.
template <auto KERNEL>
sa_status opt_in_lds(int bytes) {
    if (bytes <= 65536) return SA_OK;
    static thread_local int opted_device = -1;
    int dev = 0;
    SA_HIP_TRY(hipGetDevice(&dev));
    if (opted_device != dev) {
        SA_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(KERNEL),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
        opted_device = dev;
    }
    return SA_OK;
}

}  // namespace pf
}  // namespace sa
