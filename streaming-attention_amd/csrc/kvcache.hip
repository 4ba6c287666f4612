// Paged KV cache for gfx950 and the fused q/k RMSNorm + RoPE + K/V append.
//
// Storage: one device allocation holding, per layer, a K pool and a V pool of
// [num_pages][n_kv_heads][64][head_dim] elements (fp32 or bf16).  A page of one
// head is 64 consecutive rows, so the decode kernel streams 8-32 KiB of
// contiguous memory per page.  Pages are handed out from a host free list;
// block_table[seq][j] names the page holding tokens 64j..64j+63 (-1: none).
//
// The reference keeps a dense [B, Hkv, max_seq, D] fp32 tensor per layer and
// copies it out on every step (reference tensor_cpp/include/tensor_cpp/kv_cache.h:27-238);
// here the cache stays resident and the decode kernel reads it in place.
//
// Ordering: the host decides (page_table.cpp) and publishes the table rows and
// lengths with small kernels on the stream the caller passes, so a reset,
// reserve, set_pages, append, decode and commit issued on one stream run in
// the order they were called.
#include "sa_internal.h"
#include "page_table.h"

#include <algorithm>
#include <cmath>
#include <vector>

struct sa_kvcache {
    sa_kv_desc desc{};
    int device = 0;
    char* pool = nullptr;          // [layers][2][num_pages][n_kv][64][D]
    size_t elem_bytes = 4;
    size_t page_bytes = 0;         // one page of one of K / V: n_kv * 64 * D * elem
    size_t layer_bytes = 0;        // K pool + V pool of one layer
    size_t total_bytes = 0;
    int32_t* d_table = nullptr;    // [max_seqs][max_pages_per_seq]
    int32_t* d_lens = nullptr;     // [max_seqs]
    sa::PageTable pt;              // host decisions; the device arrays follow them
};

namespace sa {
namespace {

__global__ void fill_i32_kernel(int32_t* p, size_t n, int32_t v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void fill_zero_u128_kernel(uint4* p, size_t n) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        p[i] = make_uint4(0, 0, 0, 0);
}

// Row [first, first + n) of the block table, values passed by value.
struct TableRow {
    int32_t v[64];
};

__global__ void write_table_kernel(int32_t* dst, TableRow row, int n) {
    if ((int)threadIdx.x < n) dst[threadIdx.x] = row.v[threadIdx.x];
}

// seq_lens[rows[i]] = add ? seq_lens[rows[i]] + val : val
__global__ void update_lens_kernel(int32_t* lens, RowList rows, int n, int val, int add) {
    int i = threadIdx.x;
    if (i < n) lens[rows.row[i]] = add ? lens[rows.row[i]] + val : val;
}

__global__ void add_lens_range_kernel(int32_t* lens, int n, int val) {
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) lens[i] += val;
}

// Publish entries [0, n) of seq's host table row (the rest of the device row
// already holds -1 or is overwritten here).
sa_status write_table_row(sa_kvcache* c, int seq, int n, hipStream_t st) {
    const int mp = c->desc.max_pages_per_seq;
    const int32_t* src = c->pt.row(seq);
    for (int j0 = 0; j0 < n; j0 += 64) {
        TableRow row;
        const int m = std::min(64, n - j0);
        for (int j = 0; j < m; ++j) row.v[j] = src[j0 + j];
        hipLaunchKernelGGL(write_table_kernel, dim3(1), dim3(64), 0, st,
                           c->d_table + (size_t)seq * mp + j0, row, m);
        SA_CHECK_LAUNCH();
    }
    return SA_OK;
}

// Set (add = 0) or add to (add = 1) the device lengths of rows[0, n)
// (rows == NULL: 0 .. n-1).
sa_status publish_lens(sa_kvcache* c, const int32_t* rows, int n, int val, int add, hipStream_t st) {
    for (int i0 = 0; i0 < n; i0 += kRowsPerLaunch) {
        RowList rl;
        const int m = std::min(kRowsPerLaunch, n - i0);
        for (int i = 0; i < m; ++i) rl.row[i] = rows ? rows[i0 + i] : i0 + i;
        hipLaunchKernelGGL(update_lens_kernel, dim3(1), dim3(kRowsPerLaunch), 0, st, c->d_lens, rl, m, val, add);
        SA_CHECK_LAUNCH();
    }
    return SA_OK;
}

sa_status refused(const Verdict& v) { return fail(v.status, v.msg); }

// ---------------------------------------------------------------------------
// Fused QK-norm + RoPE + append.  One wave per (token, head row): waves
// [0, n_q) handle query heads, [n_q, n_q + n_kv) handle a key head and its
// value head.  Lane j holds the rotate-half pairs (i, i + D/2) for
// i = j, j + 64, ... so RoPE needs no lane exchange.
// ---------------------------------------------------------------------------
struct AppendArgs {
    const float* q; const float* k; const float* v;
    float* q_out;
    float* k_out;              // optional: K normed and rotated, as q_out
    // Optional: q, k and v are the sum of part_S split-K partials of rows
    // [part_row0 + i_seq * S + s] of a [part_M][(n_q + 2 n_kv) * D] projection;
    // v also goes to v_out.
    const float* part;
    int part_S, part_M, part_row0;
    float* v_out;
    const float* wq; const float* wk;
    const float* cos_t; const float* sin_t;
    RowList rows;              // cache row of each sequence of this launch
    const int32_t* seq_lens;
    const int32_t* table;
    char* k_pool; char* v_pool;
    int n_q, n_kv, S, max_pages, rope_max_pos;
    float eps;
};

template <int D>
__global__ void __launch_bounds__(256)
qk_norm_rope_kernel(const float* x, int n_rows, const int32_t* pos, const float* w, float eps,
                    bool eps_outside, const float* cos_t, const float* sin_t, int max_pos, float* y) {
    const int lane = threadIdx.x & (kWave - 1);
    const int row = blockIdx.x * 4 + threadIdx.x / kWave;
    if (row >= n_rows) return;
    RowPairs<D> r;
    r.load(x + (size_t)row * D, lane);
    if (w) r.rms_norm(w, eps, lane, eps_outside);
    const int p = pos ? pos[row] : 0;
    if (cos_t && p >= 0 && p < max_pos) r.rope(cos_t, sin_t, p, lane);
    r.store(y + (size_t)row * D, lane);
}

template <int D, bool BF16>
__global__ void __launch_bounds__(256)
qknorm_rope_append_kernel(AppendArgs a) {
    constexpr int H = D / 2;
    constexpr int NP = (H + kWave - 1) / kWave;   // pairs per lane
    const int lane = threadIdx.x & (kWave - 1);
    const int row_id = blockIdx.x * 4 + threadIdx.x / kWave;
    const int s = blockIdx.y;
    const int i_seq = blockIdx.z;
    const int n_rows = a.n_q + a.n_kv;
    if (row_id >= n_rows) return;
    const bool is_q = row_id < a.n_q;
    if (is_q && !a.q && !a.part) return;
    const int head = is_q ? row_id : row_id - a.n_q;
    const int cache_row = a.rows.row[i_seq];
    const int pos = a.seq_lens[cache_row] + s;

    const int nh = is_q ? a.n_q : a.n_kv;
    const size_t src = (((size_t)i_seq * a.S + s) * nh + head) * D;
    const float* x = (is_q ? a.q : a.k) + src;
    const float* w = is_q ? a.wq : a.wk;

    const int part_cols = (a.n_q + 2 * a.n_kv) * D;
    const size_t part_row = (size_t)(a.part_row0 + i_seq * a.S + s) * part_cols;
    const size_t part_split = (size_t)a.part_M * part_cols;
    RowPairs<D> r;
    if (a.part) r.load_sum(a.part + part_row + (is_q ? head : a.n_q + head) * D, part_split, a.part_S, lane);
    else r.load(x, lane);
    if (w) r.rms_norm(w, a.eps, lane);
    if (a.cos_t && pos < a.rope_max_pos) r.rope(a.cos_t, a.sin_t, pos, lane);
    if (is_q) {
        r.store(a.q_out + src, lane);
        return;
    }
    if (a.k_out) r.store(a.k_out + src, lane);
    const float* lo = r.lo;
    const float* hi = r.hi;
    // V as given, or summed from the partials (and written to v_out).
    RowPairs<D> vr;
    if (a.part) {
        vr.load_sum(a.part + part_row + (a.n_q + a.n_kv + head) * D, part_split, a.part_S, lane);
        if (a.v_out) vr.store(a.v_out + src, lane);
    } else {
        vr.load(a.v + src, lane);
    }
    // Append K (normed, rotated) and V (as given) at pos.  The host has
    // checked that every row has a page there; these tests only keep a
    // device length that disagrees with the host from writing out of bounds.
    if (pos >= a.max_pages * 64) return;
    const int page = a.table[(size_t)cache_row * a.max_pages + (pos >> 6)];
    if (page < 0) return;
    const size_t row = (((size_t)page * a.n_kv + head) * 64 + (pos & 63)) * D;
#pragma unroll
    for (int c = 0; c < NP; ++c) {
        const int i = lane + c * kWave;
        if (i < H) {
            if constexpr (BF16) {
                uint16_t* kd = reinterpret_cast<uint16_t*>(a.k_pool) + row;
                uint16_t* vd = reinterpret_cast<uint16_t*>(a.v_pool) + row;
                kd[i] = f32_to_bf16_rne(lo[c]);
                kd[i + H] = f32_to_bf16_rne(hi[c]);
                vd[i] = f32_to_bf16_rne(vr.lo[c]);
                vd[i + H] = f32_to_bf16_rne(vr.hi[c]);
            } else {
                float* kd = reinterpret_cast<float*>(a.k_pool) + row;
                float* vd = reinterpret_cast<float*>(a.v_pool) + row;
                kd[i] = lo[c];
                kd[i + H] = hi[c];
                vd[i] = vr.lo[c];
                vd[i + H] = vr.hi[c];
            }
        }
    }
}

// Dense copy [n_kv][len][D] of one sequence (fp32 out).
template <bool BF16>
__global__ void gather_kernel(const char* k_pool, const char* v_pool, const int32_t* table_row,
                              int n_kv, int D, int len, float* k_out, float* v_out) {
    const int t = blockIdx.x;
    const int h = blockIdx.y;
    const int page = table_row[t >> 6];
    const size_t row = (((size_t)page * n_kv + h) * 64 + (t & 63)) * D;
    const size_t dst = ((size_t)h * len + t) * D;
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        float kv, vv;
        if constexpr (BF16) {
            kv = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(k_pool)[row + i] << 16);
            vv = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(v_pool)[row + i] << 16);
        } else {
            kv = reinterpret_cast<const float*>(k_pool)[row + i];
            vv = reinterpret_cast<const float*>(v_pool)[row + i];
        }
        if (k_out) k_out[dst + i] = kv;
        if (v_out) v_out[dst + i] = vv;
    }
}

bool valid_cache(const sa_kvcache* c) { return c && c->pool; }

char* k_pool_of(const sa_kvcache* c, int layer) { return c->pool + (size_t)layer * c->layer_bytes; }
char* v_pool_of(const sa_kvcache* c, int layer) {
    return c->pool + (size_t)layer * c->layer_bytes + c->layer_bytes / 2;
}

}  // namespace
}  // namespace sa

using namespace sa;

extern "C" sa_status sa_kvcache_create(const sa_kv_desc* d, sa_kvcache** out) {
    clear_error();
    if (!d || !out) return fail(SA_EINVAL, "null pointer");
    *out = nullptr;
    if (d->num_layers <= 0 || d->num_kv_heads <= 0 || d->max_seqs <= 0 ||
        d->max_pages_per_seq <= 0 || d->num_pages <= 0)
        return fail(SA_EINVAL, "cache dimensions must be positive");
    if (d->max_pages_per_seq > (1 << 18))
        return fail(SA_EINVAL, "max_pages_per_seq must be at most 262144 (16M tokens)");
    if (d->head_dim != 8 && d->head_dim != 16 && d->head_dim != 32 && d->head_dim != 64 && d->head_dim != 128 &&
        d->head_dim != 256)
        return fail(SA_EINVAL, "head_dim must be 8, 16, 32, 64, 128 or 256");
    if (d->kv_dtype != SA_DTYPE_F32 && d->kv_dtype != SA_DTYPE_BF16)
        return fail(SA_EINVAL, "kv_dtype must be F32 or BF16");
    int device = 0;
    const hipError_t de = hipGetDevice(&device);
    if (de != hipSuccess) return hip_fail(de, "hipGetDevice");
    auto* c = new sa_kvcache();
    c->desc = *d;
    c->device = device;
    c->elem_bytes = d->kv_dtype == SA_DTYPE_BF16 ? 2 : 4;
    c->page_bytes = (size_t)d->num_kv_heads * 64 * d->head_dim * c->elem_bytes;
    c->layer_bytes = 2 * c->page_bytes * (size_t)d->num_pages;
    c->total_bytes = c->layer_bytes * (size_t)d->num_layers;
    const size_t n_table = (size_t)d->max_seqs * d->max_pages_per_seq;
    hipError_t e = hipMalloc(&c->pool, c->total_bytes);
    if (e != hipSuccess) {
        delete c;
        return fail(SA_ENOMEM, "KV pool allocation failed");
    }
    e = hipMalloc(&c->d_table, n_table * sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc(&c->d_lens, (size_t)d->max_seqs * sizeof(int32_t));
    if (e != hipSuccess) {
        (void)hipFree(c->pool);
        (void)hipFree(c->d_table);
        (void)hipFree(c->d_lens);
        delete c;
        return fail(SA_ENOMEM, "KV table allocation failed");
    }
    c->pt.init(d->max_seqs, d->max_pages_per_seq, d->num_pages);
    *out = c;
    sa_status st = sa_kvcache_reset(c, nullptr);
    if (st == SA_OK) {
        hipError_t se = hipStreamSynchronize(nullptr);
        if (se != hipSuccess) st = hip_fail(se, "hipStreamSynchronize");
    }
    if (st != SA_OK) {
        sa_kvcache_destroy(c);
        *out = nullptr;
    }
    return st;
}

extern "C" sa_status sa_kvcache_destroy(sa_kvcache* c) {
    clear_error();
    if (!c) return SA_OK;
    // Best effort: work still queued on the cache must finish before its
    // memory goes; a failure here leaves nothing else to do.
    (void)hipDeviceSynchronize();
    (void)hipFree(c->pool);
    (void)hipFree(c->d_table);
    (void)hipFree(c->d_lens);
    delete c;
    return SA_OK;
}

extern "C" sa_status sa_kvcache_reset(sa_kvcache* c, sa_stream_t stream) {
    clear_error();
    if (!valid_cache(c)) return fail(SA_EINVAL, "invalid cache");
    hipStream_t st = as_stream(stream);
    const size_t n_table = (size_t)c->desc.max_seqs * c->desc.max_pages_per_seq;
    c->pt.reset();
    hipLaunchKernelGGL(fill_i32_kernel, dim3((n_table + 255) / 256), dim3(256), 0, st, c->d_table,
                       n_table, -1);
    SA_CHECK_LAUNCH();
    hipLaunchKernelGGL(fill_i32_kernel, dim3((c->desc.max_seqs + 255) / 256), dim3(256), 0, st,
                       c->d_lens, (size_t)c->desc.max_seqs, 0);
    SA_CHECK_LAUNCH();
    const size_t n16 = c->total_bytes / 16;
    hipLaunchKernelGGL(fill_zero_u128_kernel, dim3(4096), dim3(256), 0, st,
                       reinterpret_cast<uint4*>(c->pool), n16);
    SA_CHECK_LAUNCH();
    return SA_OK;
}

extern "C" sa_status sa_kvcache_reserve(sa_kvcache* c, int seq, int n_tokens, sa_stream_t stream) {
    clear_error();
    if (!valid_cache(c)) return fail(SA_EINVAL, "invalid cache");
    const int before = c->pt.valid_seq(seq) ? c->pt.npages(seq) : 0;
    const Verdict v = c->pt.reserve(seq, n_tokens);
    if (!v.ok()) return refused(v);
    if (c->pt.npages(seq) == before) return SA_OK;
    return write_table_row(c, seq, c->pt.npages(seq), as_stream(stream));
}

extern "C" sa_status sa_kvcache_set_pages(sa_kvcache* c, int seq, const int32_t* pages, int n_pages,
                                          sa_stream_t stream) {
    clear_error();
    if (!valid_cache(c)) return fail(SA_EINVAL, "invalid cache");
    const int before = c->pt.valid_seq(seq) ? c->pt.npages(seq) : 0;
    bool len_cut = false;
    const Verdict v = c->pt.set_pages(seq, pages, n_pages, &len_cut);
    if (!v.ok()) return refused(v);
    hipStream_t st = as_stream(stream);
    // Entries past the new list become -1 on the device too.
    SA_TRY(write_table_row(c, seq, std::max(before, n_pages), st));
    if (len_cut) {
        const int32_t row = seq;
        SA_TRY(publish_lens(c, &row, 1, c->pt.len(seq), 0, st));
    }
    return SA_OK;
}

extern "C" sa_status sa_kvcache_set_len(sa_kvcache* c, int seq, int len, sa_stream_t stream) {
    clear_error();
    if (!valid_cache(c)) return fail(SA_EINVAL, "invalid cache");
    const Verdict v = c->pt.set_len(seq, len);
    if (!v.ok()) return refused(v);
    const int32_t row = seq;
    return publish_lens(c, &row, 1, len, 0, as_stream(stream));
}

extern "C" int sa_kvcache_len(const sa_kvcache* c, int seq) {
    if (!valid_cache(c) || !c->pt.valid_seq(seq)) return -1;
    return c->pt.len(seq);
}

extern "C" int sa_kvcache_capacity(const sa_kvcache* c, int seq) {
    if (!valid_cache(c) || !c->pt.valid_seq(seq)) return -1;
    return c->pt.capacity(seq);
}

extern "C" sa_status sa_kvcache_commit(sa_kvcache* c, const int32_t* seqs, int n_seqs, int n,
                                       sa_stream_t stream) {
    clear_error();
    if (!valid_cache(c)) return fail(SA_EINVAL, "invalid cache");
    const Verdict v = c->pt.commit(seqs, n_seqs, n);
    if (!v.ok()) return refused(v);
    hipStream_t st = as_stream(stream);
    if (!seqs) {
        hipLaunchKernelGGL(add_lens_range_kernel, dim3((n_seqs + 255) / 256), dim3(256), 0, st,
                           c->d_lens, n_seqs, n);
        SA_CHECK_LAUNCH();
        return SA_OK;
    }
    return publish_lens(c, seqs, n_seqs, n, 1, st);
}

extern "C" sa_status sa_kvcache_get_desc(const sa_kvcache* c, sa_kv_desc* out) {
    clear_error();
    if (!valid_cache(c) || !out) return fail(SA_EINVAL, "invalid cache or null output");
    *out = c->desc;
    return SA_OK;
}

extern "C" void* sa_kvcache_k_pool(sa_kvcache* c, int layer) {
    if (!valid_cache(c) || layer < 0 || layer >= c->desc.num_layers) return nullptr;
    return k_pool_of(c, layer);
}
extern "C" void* sa_kvcache_v_pool(sa_kvcache* c, int layer) {
    if (!valid_cache(c) || layer < 0 || layer >= c->desc.num_layers) return nullptr;
    return v_pool_of(c, layer);
}
extern "C" int32_t* sa_kvcache_block_table(sa_kvcache* c) { return valid_cache(c) ? c->d_table : nullptr; }
extern "C" int32_t* sa_kvcache_seq_lens(sa_kvcache* c) { return valid_cache(c) ? c->d_lens : nullptr; }
extern "C" size_t sa_kvcache_bytes(const sa_kvcache* c) { return valid_cache(c) ? c->total_bytes : 0; }

extern "C" sa_status sa_rope_table_init(float* d_cos, float* d_sin, int max_pos, int head_dim,
                                        float theta, sa_stream_t stream) {
    clear_error();
    if (!d_cos || !d_sin) return fail(SA_EINVAL, "null pointer");
    if (max_pos <= 0 || head_dim <= 0 || head_dim % 2) return fail(SA_EINVAL, "bad table size");
    const int half = head_dim / 2;
    // Same fp32 arithmetic as the reference (powf, then cosf / sinf of the
    // fp32 angle), evaluated once on the host with the C library.
    std::vector<float> inv(half), cs((size_t)max_pos * half), sn((size_t)max_pos * half);
    for (int i = 0; i < half; ++i)
        inv[i] = 1.0f / std::pow(theta, static_cast<float>(i) / static_cast<float>(head_dim));
    for (int p = 0; p < max_pos; ++p) {
        for (int i = 0; i < half; ++i) {
            const float ang = static_cast<float>(p) * inv[i];
            cs[(size_t)p * half + i] = std::cos(ang);
            sn[(size_t)p * half + i] = std::sin(ang);
        }
    }
    hipStream_t st = as_stream(stream);
    SA_HIP_TRY(hipMemcpyAsync(d_cos, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice, st));
    SA_HIP_TRY(hipMemcpyAsync(d_sin, sn.data(), sn.size() * sizeof(float), hipMemcpyHostToDevice, st));
    SA_HIP_TRY(hipStreamSynchronize(st));
    return SA_OK;
}

namespace sa {

namespace {

// Shared by the entry points below: q/k/v given (part == NULL), or summed from
// the n_part split-K partials of the projection at part (q, k, v NULL).
sa_status append_impl(sa_kvcache* c, int layer, const float* q, const float* k, const float* v, const float* part,
                      int n_part, int n_seq, int S, const int32_t* seq_ids, int n_q_heads, const float* q_norm_w,
                      const float* k_norm_w, float eps, const float* rope_cos, const float* rope_sin,
                      int rope_max_pos, float* q_out, float* k_out, float* v_out, hipStream_t st) {
    if (!valid_cache(c)) return fail(SA_EINVAL, "invalid cache");
    if (layer < 0 || layer >= c->desc.num_layers) return fail(SA_ERANGE, "Layer index out of range");
    if (part ? n_part <= 0 : (!k || !v)) return fail(SA_EINVAL, "null k or v");
    if ((q || part) && (!q_out || n_q_heads <= 0)) return fail(SA_EINVAL, "q needs q_out and n_q_heads > 0");
    if (n_seq <= 0 || S <= 0) return fail(SA_EINVAL, "n_seq and S must be positive");
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) return fail(SA_EINVAL, "cos and sin go together");
    if (rope_cos && rope_max_pos <= 0) return fail(SA_EINVAL, "RoPE table needs rope_max_pos > 0");
    const Verdict vd = c->pt.check_append(seq_ids, n_seq, S, rope_cos ? rope_max_pos : 0);
    if (!vd.ok()) return refused(vd);
    AppendArgs a{};
    a.q_out = q_out;
    a.part = part; a.part_S = n_part; a.part_M = n_seq * S;
    a.wq = q_norm_w; a.wk = k_norm_w; a.cos_t = rope_cos; a.sin_t = rope_sin;
    a.seq_lens = c->d_lens; a.table = c->d_table;
    a.k_pool = k_pool_of(c, layer); a.v_pool = v_pool_of(c, layer);
    a.n_q = q || part ? n_q_heads : 0; a.n_kv = c->desc.num_kv_heads; a.S = S;
    a.max_pages = c->desc.max_pages_per_seq; a.rope_max_pos = rope_max_pos; a.eps = eps;
    const int rows = a.n_q + a.n_kv;
    const int D = c->desc.head_dim;
    const bool bf = c->desc.kv_dtype == SA_DTYPE_BF16;
    // Up to kRowsPerLaunch sequences per launch, their cache rows by value.
    for (int i0 = 0; i0 < n_seq; i0 += kRowsPerLaunch) {
        const int m = std::min(kRowsPerLaunch, n_seq - i0);
        for (int i = 0; i < m; ++i) a.rows.row[i] = seq_ids ? seq_ids[i0 + i] : i0 + i;
        a.q = q ? q + (size_t)i0 * S * n_q_heads * D : nullptr;
        a.q_out = a.n_q ? q_out + (size_t)i0 * S * n_q_heads * D : nullptr;
        a.k = k ? k + (size_t)i0 * S * a.n_kv * D : nullptr;
        a.k_out = k_out ? k_out + (size_t)i0 * S * a.n_kv * D : nullptr;
        a.v = v ? v + (size_t)i0 * S * a.n_kv * D : nullptr;
        a.v_out = v_out ? v_out + (size_t)i0 * S * a.n_kv * D : nullptr;
        a.part_row0 = i0 * S;
        dim3 grid((rows + 3) / 4, S, m);
        switch (D) {
#define SA_APPEND_CASE(DD)                                                                        \
    case DD:                                                                                      \
        if (bf) hipLaunchKernelGGL((qknorm_rope_append_kernel<DD, true>), grid, dim3(256), 0, st, a); \
        else hipLaunchKernelGGL((qknorm_rope_append_kernel<DD, false>), grid, dim3(256), 0, st, a); \
        break;
            SA_APPEND_CASE(8)
            SA_APPEND_CASE(16)
            SA_APPEND_CASE(32)
            SA_APPEND_CASE(64)
            SA_APPEND_CASE(128)
            SA_APPEND_CASE(256)
#undef SA_APPEND_CASE
            default: return fail(SA_EINVAL, "head_dim");
        }
        SA_CHECK_LAUNCH();
    }
    return SA_OK;
}

}  // namespace

sa_status qknorm_rope_append(sa_kvcache* c, int layer, const float* q, const float* k, const float* v, int n_seq,
                             int S, const int32_t* seq_ids, int n_q_heads, const float* q_norm_w,
                             const float* k_norm_w, float eps, const float* rope_cos, const float* rope_sin,
                             int rope_max_pos, float* q_out, float* k_out, hipStream_t st) {
    return append_impl(c, layer, q, k, v, nullptr, 0, n_seq, S, seq_ids, n_q_heads, q_norm_w, k_norm_w, eps, rope_cos,
                       rope_sin, rope_max_pos, q_out, k_out, nullptr, st);
}

sa_status qknorm_rope_append_partials(sa_kvcache* c, int layer, const float* part, int n_part, int n_seq, int S,
                                      int n_q_heads, const float* q_norm_w, const float* k_norm_w, float eps,
                                      const float* rope_cos, const float* rope_sin, int rope_max_pos, float* q_out,
                                      float* k_out, float* v_out, hipStream_t st) {
    if (!part) return fail(SA_EINVAL, "null partials");
    return append_impl(c, layer, nullptr, nullptr, nullptr, part, n_part, n_seq, S, nullptr, n_q_heads, q_norm_w,
                       k_norm_w, eps, rope_cos, rope_sin, rope_max_pos, q_out, k_out, v_out, st);
}

}  // namespace sa

extern "C" sa_status sa_qknorm_rope_append(sa_kvcache* c, int layer, const float* q, const float* k,
                                           const float* v, int n_seq, int S, const int32_t* seq_ids,
                                           int n_q_heads, const float* q_norm_w,
                                           const float* k_norm_w, float eps, const float* rope_cos,
                                           const float* rope_sin, int rope_max_pos, float* q_out,
                                           sa_stream_t stream) {
    clear_error();
    return qknorm_rope_append(c, layer, q, k, v, n_seq, S, seq_ids, n_q_heads, q_norm_w, k_norm_w, eps, rope_cos,
                              rope_sin, rope_max_pos, q_out, nullptr, as_stream(stream));
}

extern "C" size_t sa_paged_decode_ws_bytes(const sa_kvcache* c, int n_seq, int n_q_heads) {
    if (!valid_cache(c) || n_seq <= 0 || n_q_heads <= 0) return 0;
    return paged_ws(n_seq, n_q_heads, c->desc.num_kv_heads, c->desc.head_dim, c->desc.max_pages_per_seq);
}

extern "C" sa_status sa_paged_decode(const sa_kvcache* c, int layer, const float* q, int n_seq,
                                     const int32_t* seq_ids, int n_q_heads, int n_pending, float scale,
                                     float* out, void* ws, size_t ws_bytes, sa_stream_t stream) {
    clear_error();
    if (!valid_cache(c)) return fail(SA_EINVAL, "invalid cache");
    if (layer < 0 || layer >= c->desc.num_layers) return fail(SA_ERANGE, "Layer index out of range");
    if (n_seq <= 0) return fail(SA_EINVAL, "n_seq must be positive");
    int max_len = 0;
    long long total = 0;
    const Verdict vd = c->pt.check_decode(seq_ids, n_seq, n_pending, &max_len, &total);
    if (!vd.ok()) return refused(vd);
    PagedView pv;
    pv.k_pool = k_pool_of(c, layer); pv.v_pool = v_pool_of(c, layer);
    pv.block_table = c->d_table; pv.seq_lens = c->d_lens;
    pv.n_kv = c->desc.num_kv_heads; pv.d = c->desc.head_dim;
    pv.max_pages = c->desc.max_pages_per_seq; pv.num_pages = c->desc.num_pages;
    pv.bf16 = c->desc.kv_dtype == SA_DTYPE_BF16;
    std::vector<int32_t> lens(n_seq);
    for (int i = 0; i < n_seq; ++i) lens[i] = c->pt.len(seq_ids ? seq_ids[i] : i);
    return decode_paged(pv, q, n_seq, seq_ids, lens.data(), n_q_heads, n_pending, max_len, total, scale, out, ws,
                        ws_bytes, as_stream(stream));
}

namespace sa {
namespace {

// sa_append_decode; with part set, q, k and v come from the projection's
// split-K partials instead (FusedAppend::part).
sa_status append_decode_impl(sa_kvcache* c, int layer, const float* q, const float* k, const float* v,
                             const float* part, int n_part, int n_seq, const int32_t* seq_ids, int n_q_heads,
                             const float* q_norm_w, const float* k_norm_w, float eps, const float* rope_cos,
                             const float* rope_sin, int rope_max_pos, float scale, float* out, float* q_out,
                             void* ws, size_t ws_bytes, int commit, hipStream_t stream) {
    if (!valid_cache(c)) return fail(SA_EINVAL, "invalid cache");
    if (layer < 0 || layer >= c->desc.num_layers) return fail(SA_ERANGE, "Layer index out of range");
    if (!out || (part ? n_part <= 0 : (!q || !k || !v))) return fail(SA_EINVAL, "null q, k, v or out");
    if (n_seq <= 0) return fail(SA_EINVAL, "n_seq must be positive");
    if (n_q_heads <= 0 || n_q_heads % c->desc.num_kv_heads) return fail(SA_EINVAL, "bad head counts");
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) return fail(SA_EINVAL, "cos and sin go together");
    if (rope_cos && rope_max_pos <= 0) return fail(SA_EINVAL, "RoPE table needs rope_max_pos > 0");
    if (c->desc.head_dim < 64) return fail(SA_EINVAL, "the fused decode step takes head_dim 64, 128 or 256");
    Verdict vd = c->pt.check_append(seq_ids, n_seq, 1, rope_cos ? rope_max_pos : 0);
    if (!vd.ok()) return refused(vd);
    int max_len = 0;
    long long total = 0;
    vd = c->pt.check_decode(seq_ids, n_seq, 1, &max_len, &total);
    if (!vd.ok()) return refused(vd);
    std::vector<int32_t> pos(n_seq);
    for (int i = 0; i < n_seq; ++i) pos[i] = c->pt.len(seq_ids ? seq_ids[i] : i);
    PagedView pv;
    pv.k_pool = k_pool_of(c, layer); pv.v_pool = v_pool_of(c, layer);
    pv.block_table = c->d_table; pv.seq_lens = c->d_lens;
    pv.n_kv = c->desc.num_kv_heads; pv.d = c->desc.head_dim;
    pv.max_pages = c->desc.max_pages_per_seq; pv.num_pages = c->desc.num_pages;
    pv.bf16 = c->desc.kv_dtype == SA_DTYPE_BF16;
    FusedAppend f{};
    f.k = k; f.v = v; f.wq = q_norm_w; f.wk = k_norm_w; f.eps = eps;
    f.cos_t = rope_cos; f.sin_t = rope_sin; f.rope_max_pos = rope_max_pos;
    // One launch (up to kRowsPerLaunch rows) commits inside the kernel.  A
    // call of more rows takes several launches; their lengths are published
    // by one pass after the last launch is enqueued, so a launch that fails
    // leaves every device length as it was.
    const bool in_kernel_commit = commit && n_seq <= kRowsPerLaunch;
    f.q_out = q_out; f.lens = c->d_lens; f.pos = pos.data(); f.commit = in_kernel_commit;
    f.part = part; f.part_S = n_part; f.part_M = n_seq;
    SA_TRY(decode_paged_fused(pv, q, n_seq, seq_ids, n_q_heads, f, max_len, total, scale, out, ws, ws_bytes,
                              stream));
    if (commit) {
        if (!in_kernel_commit) SA_TRY(publish_lens(c, seq_ids, n_seq, 1, 1, stream));
        vd = c->pt.commit(seq_ids, n_seq, 1);   // checked above: cannot be refused
        if (!vd.ok()) return refused(vd);
    }
    return SA_OK;
}

}  // namespace

sa_status append_decode_partials(sa_kvcache* c, int layer, const float* part, int n_part, int n_seq,
                                 const int32_t* seq_ids, int n_q_heads, const float* q_norm_w,
                                 const float* k_norm_w, float eps, const float* rope_cos, const float* rope_sin,
                                 int rope_max_pos, float scale, float* out, float* q_out, void* ws,
                                 size_t ws_bytes, int commit, hipStream_t st) {
    if (!part) return fail(SA_EINVAL, "null projection partials");
    return append_decode_impl(c, layer, nullptr, nullptr, nullptr, part, n_part, n_seq, seq_ids, n_q_heads,
                              q_norm_w, k_norm_w, eps, rope_cos, rope_sin, rope_max_pos, scale, out, q_out, ws,
                              ws_bytes, commit, st);
}

}  // namespace sa

extern "C" sa_status sa_append_decode(sa_kvcache* c, int layer, const float* q, const float* k, const float* v,
                                      int n_seq, const int32_t* seq_ids, int n_q_heads, const float* q_norm_w,
                                      const float* k_norm_w, float eps, const float* rope_cos,
                                      const float* rope_sin, int rope_max_pos, float scale, float* out,
                                      float* q_out, void* ws, size_t ws_bytes, int commit, sa_stream_t stream) {
    clear_error();
    if (!q || !k || !v) return fail(SA_EINVAL, "null q, k, v or out");
    return append_decode_impl(c, layer, q, k, v, nullptr, 0, n_seq, seq_ids, n_q_heads, q_norm_w, k_norm_w, eps,
                              rope_cos, rope_sin, rope_max_pos, scale, out, q_out, ws, ws_bytes, commit,
                              as_stream(stream));
}

extern "C" sa_status sa_append_decode_partials(sa_kvcache* c, int layer, const float* part, int n_part,
                                               int n_seq, const int32_t* seq_ids, int n_q_heads,
                                               const float* q_norm_w, const float* k_norm_w, float eps,
                                               const float* rope_cos, const float* rope_sin, int rope_max_pos,
                                               float scale, float* out, float* q_out, void* ws, size_t ws_bytes,
                                               int commit, sa_stream_t stream) {
    clear_error();
    return append_decode_partials(c, layer, part, n_part, n_seq, seq_ids, n_q_heads, q_norm_w, k_norm_w, eps,
                                  rope_cos, rope_sin, rope_max_pos, scale, out, q_out, ws, ws_bytes, commit,
                                  as_stream(stream));
}

extern "C" sa_status sa_kvcache_gather(const sa_kvcache* c, int layer, int seq, int len, float* k_out,
                                       float* v_out, sa_stream_t stream) {
    clear_error();
    if (!valid_cache(c)) return fail(SA_EINVAL, "invalid cache");
    if (layer < 0 || layer >= c->desc.num_layers) return fail(SA_ERANGE, "Layer index out of range");
    if (seq < 0 || seq >= c->desc.max_seqs) return fail(SA_ERANGE, "sequence index out of range");
    if (len < 0 || len > c->pt.len(seq)) return fail(SA_ERANGE, "Requested seq_len exceeds cached length");
    if (len == 0) return SA_OK;
    if (!k_out && !v_out) return fail(SA_EINVAL, "null outputs");
    dim3 grid(len, c->desc.num_kv_heads);
    const int32_t* row = c->d_table + (size_t)seq * c->desc.max_pages_per_seq;
    hipStream_t st = as_stream(stream);
    if (c->desc.kv_dtype == SA_DTYPE_BF16)
        hipLaunchKernelGGL(gather_kernel<true>, grid, dim3(128), 0, st, k_pool_of(c, layer),
                           v_pool_of(c, layer), row, c->desc.num_kv_heads, c->desc.head_dim, len,
                           k_out, v_out);
    else
        hipLaunchKernelGGL(gather_kernel<false>, grid, dim3(128), 0, st, k_pool_of(c, layer),
                           v_pool_of(c, layer), row, c->desc.num_kv_heads, c->desc.head_dim, len,
                           k_out, v_out);
    SA_CHECK_LAUNCH();
    return SA_OK;
}

extern "C" sa_status sa_qk_norm_rope_ex(const float* x, int n_rows, int D, const int32_t* pos,
                                        const float* norm_w, float eps, sa_norm_mode mode,
                                        const float* rope_cos, const float* rope_sin, int rope_max_pos,
                                        float* y, sa_stream_t stream) {
    clear_error();
    if (!x || !y) return fail(SA_EINVAL, "null pointer");
    if (n_rows < 0) return fail(SA_EINVAL, "n_rows must be >= 0");
    if (mode != SA_NORM_EPS_INSIDE && mode != SA_NORM_EPS_OUTSIDE) return fail(SA_EINVAL, "unknown norm mode");
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) return fail(SA_EINVAL, "cos and sin go together");
    if (rope_cos && !pos) return fail(SA_EINVAL, "RoPE needs positions");
    if (n_rows == 0) return SA_OK;
    hipStream_t st = as_stream(stream);
    const dim3 grid((n_rows + 3) / 4);
    const bool outside = mode == SA_NORM_EPS_OUTSIDE;
    switch (D) {
#define SA_NORM_ROPE_CASE(DD)                                                                          \
    case DD:                                                                                           \
        hipLaunchKernelGGL(qk_norm_rope_kernel<DD>, grid, dim3(256), 0, st, x, n_rows, pos, norm_w, eps, \
                           outside, rope_cos, rope_sin, rope_max_pos, y);                              \
        break;
        SA_NORM_ROPE_CASE(8)
        SA_NORM_ROPE_CASE(16)
        SA_NORM_ROPE_CASE(32)
        SA_NORM_ROPE_CASE(64)
        SA_NORM_ROPE_CASE(128)
        SA_NORM_ROPE_CASE(256)
#undef SA_NORM_ROPE_CASE
        default:
            return fail(SA_EINVAL, "head_dim must be 8, 16, 32, 64, 128 or 256");
    }
    SA_CHECK_LAUNCH();
    return SA_OK;
}

extern "C" sa_status sa_qk_norm_rope(const float* x, int n_rows, int D, const int32_t* pos,
                                     const float* norm_w, float eps, const float* rope_cos,
                                     const float* rope_sin, int rope_max_pos, float* y,
                                     sa_stream_t stream) {
    return sa_qk_norm_rope_ex(x, n_rows, D, pos, norm_w, eps, SA_NORM_EPS_INSIDE, rope_cos, rope_sin,
                              rope_max_pos, y, stream);
}
