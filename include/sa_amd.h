/*
 * sa_amd.h - C ABI of the MI355X (gfx950) streaming-attention library.
 *
 * Every entry point takes plain device pointers and sizes, runs asynchronously
 * on the HIP stream it is given (NULL = the default stream), and returns an
 * sa_status.  No C++ type and no exception crosses this boundary.  The C++
 * mirror of the reference API (attention.h, tensor_cpp/kv_cache.h,
 * tensor_cpp/ops.h, tensor_cpp/qwen3_ops.h) is built on top of these calls.
 *
 * Layouts are row-major.  "token-major" means [seq][token][head][head_dim],
 * which is what a Q/K/V projection writes before any transpose.
 *
 * Head sizes (head_dim, d, D): 8, 16, 32, 64, 128 or 256 for single-query
 * attention, decode, the KV cache and QK-norm/RoPE; the fused decode step
 * (sa_append_decode) takes 64, 128 or 256; causal prefill 16, 32, 64 or 128
 * in fp32 and 64 or 128 in bf16.  Other sizes return SA_EINVAL.
 */
#ifndef SA_AMD_H
#define SA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SA_PAGE_TOKENS 64      /* tokens per KV-cache page */
#define SA_MAX_HEAD_DIM 256

typedef enum sa_status {
    SA_OK = 0,
    SA_EINVAL = -1,   /* bad argument (null pointer, unsupported size, ...) */
    SA_ENOMEM = -2,   /* device allocation failed / workspace too small      */
    SA_EFULL = -3,    /* KV cache has no room for the requested tokens       */
    SA_EHIP = -4,     /* a HIP runtime call failed                           */
    SA_ERANGE = -5,   /* index (layer, sequence, length) out of range        */
    SA_EIO = -6       /* a file could not be read or is malformed            */
} sa_status;

typedef enum sa_dtype {
    SA_DTYPE_F32 = 0,
    SA_DTYPE_BF16 = 1
} sa_dtype;

typedef void* sa_stream_t;   /* a hipStream_t */

/* Message describing the last failure on the calling thread ("" if none). */
const char* sa_last_error(void);

/* ------------------------------------------------------------------------
 * Single-query streaming attention (split-KV online softmax + LSE merge).
 *
 * Replaces the compute of streaming_attention_serial / _omp / _mpi_simple and
 * naive_attention_serial / _omp (reference attention/src/attention.h:27-208,
 * attention/src/streaming_serial.cpp:20-71, attention/src/streaming_omp.cpp:99-154).
 * O = softmax(scale * Q K^T) V with Q [d], K and V [T][d], O [d], all fp32 on
 * the device.  The reference API is unscaled: pass scale = 1.
 * block_size must be > 0; it is the reference's streaming block and does not
 * change the result beyond rounding.  T <= 0 writes a zero output.
 * ws must hold sa_stream_attn_ws_bytes(T, d) bytes (NULL allowed when that is 0).
 * ------------------------------------------------------------------------ */
size_t sa_stream_attn_ws_bytes(int T, int d);
sa_status sa_stream_attn_f32(const float* Q, const float* K, const float* V,
                             int T, int d, int block_size, float scale,
                             float* O, void* ws, size_t ws_bytes,
                             sa_stream_t stream);

/* The same computation with no workspace argument and no allocation: the
 * split-KV partials live in a 1 MiB device array of the library (one per GPU,
 * held until the process ends), which covers every valid T for d <= 256.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The entry point calls no hipMalloc,
 * hipFree or allocating library routine.  All calls on one GPU share that
 * array, so calls that overlap on one GPU (concurrent streams or threads)
 * race; serialise them.  Results equal sa_stream_attn_f32's bit for bit. */
sa_status sa_stream_attn_f32_noalloc(const float* Q, const float* K, const float* V,
                                     int T, int d, int block_size, float scale,
                                     float* O, sa_stream_t stream);

/* ------------------------------------------------------------------------
 * Dense multi-head single-query (decode) attention with grouped KV heads.
 *
 * Replaces the compute of ops::self_attention_streaming and of the decode
 * (q_len = 1) case of ops::self_attention (reference tensor_cpp/src/ops.cpp:964-1017
 * and :514-641), without materialising repeat_kv (qwen3_ops.cpp:194-234):
 * query head h reads KV head h / (n_q_heads / n_kv_heads).
 * q [batch][n_q_heads][d], k and v [batch][n_kv_heads][T][d], out like q; fp32.
 * out = softmax(scale * q k^T) v  (the mathematically correct decode; the
 * reference's streaming decode multiplies the output by scale instead, see
 * compat_scale_on_output in tensor_cpp/ops.h).
 * ------------------------------------------------------------------------ */
size_t sa_decode_dense_ws_bytes(int batch, int n_q_heads, int T, int d);
sa_status sa_decode_dense_f32(const float* q, const float* k, const float* v,
                              int batch, int n_q_heads, int n_kv_heads, int T, int d,
                              float scale, float* out, void* ws, size_t ws_bytes,
                              sa_stream_t stream);

/* ------------------------------------------------------------------------
 * Paged KV cache (64-token pages, int32 block tables, fp32 or bf16 storage).
 *
 * Replaces tensor_cpp::qwen3::KVCache (reference
 * tensor_cpp/include/tensor_cpp/kv_cache.h:27-238).  Storage per layer:
 * K pool and V pool of [num_pages][num_kv_heads][64][head_dim].
 * Sequence s owns pages block_table[s][0..]; token t of s lives in page
 * block_table[s][t / 64], row t % 64.  seq_len[s] is the committed length:
 * appends write at positions seq_len[s] + i and become visible to later
 * steps only after sa_kvcache_commit (append-then-commit, as the reference's
 * update()/increment_seq_len()).
 *
 * Ordering: the page table and the lengths are decided on the host and
 * published to the device by small kernels on the stream each call is given.
 * Calls that change or read a cache (reset, reserve, set_pages, set_len,
 * append, decode, commit, gather) are ordered when they are issued on one
 * stream; a caller that spreads them over streams orders them itself.
 * Every capacity, index and page check runs on the host before anything is
 * enqueued: an append or decode that would overflow a sequence's pages
 * returns SA_EFULL / SA_ERANGE and enqueues nothing.
 * ------------------------------------------------------------------------ */
typedef struct sa_kv_desc {
    int num_layers;
    int num_kv_heads;
    int head_dim;           /* 8, 16, 32, 64, 128 or 256 */
    int max_seqs;
    int max_pages_per_seq;
    int num_pages;          /* pages in the pool shared by all sequences */
    sa_dtype kv_dtype;
} sa_kv_desc;

typedef struct sa_kvcache sa_kvcache;

sa_status sa_kvcache_create(const sa_kv_desc* desc, sa_kvcache** out);
sa_status sa_kvcache_destroy(sa_kvcache* cache);
/* All sequences back to length 0, pages returned to the pool, storage zeroed. */
sa_status sa_kvcache_reset(sa_kvcache* cache, sa_stream_t stream);
/* Make room for n_tokens tokens in total in sequence seq, taking pages from
 * the free list in order.  SA_EFULL if the pool or the table row is exhausted. */
sa_status sa_kvcache_reserve(sa_kvcache* cache, int seq, int n_tokens, sa_stream_t stream);
/* Give sequence seq an explicit page list (host array; replaces its current
 * pages).  Each page must be in the pool, listed once, and free or already
 * seq's (SA_ERANGE / SA_EINVAL otherwise).  A committed length beyond the new
 * capacity is cut to it. */
sa_status sa_kvcache_set_pages(sa_kvcache* cache, int seq, const int32_t* pages,
                               int n_pages, sa_stream_t stream);
/* Set the committed length of seq (host and device), within its reserved pages. */
sa_status sa_kvcache_set_len(sa_kvcache* cache, int seq, int len, sa_stream_t stream);
/* Committed length of seq as tracked on the host, or -1. */
int sa_kvcache_len(const sa_kvcache* cache, int seq);
/* Tokens the pages assigned to seq can hold (64 per page), or -1.  No
 * counterpart in the reference, whose dense cache has one fixed capacity
 * (tensor_cpp/include/tensor_cpp/kv_cache.h:47-86). */
int sa_kvcache_capacity(const sa_kvcache* cache, int seq);
/* Add n to the committed length of seqs[0..n_seqs) (host ids, each at most
 * once; NULL = 0..n_seqs-1). */
sa_status sa_kvcache_commit(sa_kvcache* cache, const int32_t* seqs, int n_seqs, int n,
                            sa_stream_t stream);
/* Device pointers into the cache, for callers that drive kernels themselves. */
void* sa_kvcache_k_pool(sa_kvcache* cache, int layer);
void* sa_kvcache_v_pool(sa_kvcache* cache, int layer);
int32_t* sa_kvcache_block_table(sa_kvcache* cache);   /* [max_seqs][max_pages_per_seq] */
int32_t* sa_kvcache_seq_lens(sa_kvcache* cache);      /* [max_seqs] committed lengths */
size_t sa_kvcache_bytes(const sa_kvcache* cache);
/* The geometry the cache was created with (an accessor with no counterpart in
 * the reference; the model driver checks its shapes against it). */
sa_status sa_kvcache_get_desc(const sa_kvcache* cache, sa_kv_desc* out);

/* ------------------------------------------------------------------------
 * RoPE tables, built exactly as the reference: inv_freq[i] = 1/theta^(i/D),
 * cos/sin[pos][i] = cos/sin(float(pos) * inv_freq[i]) in fp32
 * (reference tensor_cpp/src/qwen3_ops.cpp:70-104).  d_cos and d_sin are
 * device buffers of max_pos * head_dim/2 floats.
 * ------------------------------------------------------------------------ */
sa_status sa_rope_table_init(float* d_cos, float* d_sin, int max_pos, int head_dim,
                             float theta, sa_stream_t stream);

/* ------------------------------------------------------------------------
 * Fused per-head q/k RMSNorm + rotate-half RoPE + K/V append.
 *
 * Replaces the QK-norm loops, the RoPE at position current_seq_len + s, the
 * concat and KVCache::update of the reference decoder layer (reference
 * tensor_cpp/src/qwen3_ops.cpp:697-861, kv_cache.h:94-130).
 * q [n_seq][S][n_q_heads][D], k and v [n_seq][S][n_kv_heads][D], fp32,
 * token-major.  seq_ids: host array [n_seq] of distinct cache rows, or NULL
 * for 0..n_seq-1.  Token s of sequence i is written at position
 * seq_len[seq_ids[i]] + s; every row must have pages for seq_len + S tokens
 * (SA_EFULL otherwise) and, with RoPE, seq_len + S <= rope_max_pos.
 * q_norm_w / k_norm_w: [D] RMSNorm weights, or NULL to skip the norm
 * (y = x / sqrt(mean(x^2) + eps) * w).  rope_cos / rope_sin: tables from
 * sa_rope_table_init with rope_max_pos rows, or NULL to skip RoPE.
 * q may be NULL (K/V append only); otherwise q_out receives the normed and
 * rotated q in q's layout.  The caller must have reserved the pages.
 * ------------------------------------------------------------------------ */
sa_status sa_qknorm_rope_append(sa_kvcache* cache, int layer,
                                const float* q, const float* k, const float* v,
                                int n_seq, int S, const int32_t* seq_ids, int n_q_heads,
                                const float* q_norm_w, const float* k_norm_w, float eps,
                                const float* rope_cos, const float* rope_sin, int rope_max_pos,
                                float* q_out, sa_stream_t stream);

/* ------------------------------------------------------------------------
 * Per-row RMSNorm + rotate-half RoPE without a cache.
 *
 * Replaces apply_rotary_pos_emb and the QK-norm loops when no cache is
 * involved (reference tensor_cpp/src/qwen3_ops.cpp:110-188, :697-753).
 * x and y: [n_rows][D] fp32 (y may alias x); pos: device int32 [n_rows].
 * norm_w: [D] or NULL (no norm); rope_cos / rope_sin: sa_rope_table_init
 * tables with rope_max_pos rows, or NULL (no RoPE).  Rows whose position is
 * outside the table are left unrotated.
 * ------------------------------------------------------------------------ */
sa_status sa_qk_norm_rope(const float* x, int n_rows, int D, const int32_t* pos,
                          const float* norm_w, float eps, const float* rope_cos,
                          const float* rope_sin, int rope_max_pos, float* y,
                          sa_stream_t stream);

/* Where eps enters the per-row RMSNorm: inside the sqrt,
 * x / sqrt(mean(x^2) + eps) (reference tensor_cpp/src/qwen3_ops.cpp:716-717),
 * or added to it, x / (sqrt(mean(x^2)) + eps), as the reference's AVX2 layer
 * normalises q and k (tensor_cpp/src/qwen3_ops_avx.cpp:537, :566). */
typedef enum { SA_NORM_EPS_INSIDE = 0, SA_NORM_EPS_OUTSIDE = 1 } sa_norm_mode;

/* sa_qk_norm_rope with the placement of eps chosen by mode. */
sa_status sa_qk_norm_rope_ex(const float* x, int n_rows, int D, const int32_t* pos,
                             const float* norm_w, float eps, sa_norm_mode mode,
                             const float* rope_cos, const float* rope_sin, int rope_max_pos,
                             float* y, sa_stream_t stream);

/* ------------------------------------------------------------------------
 * Paged GQA decode attention (split-KV online softmax + LSE merge).
 *
 * Replaces repeat_kv + ops::self_attention_streaming / self_attention on the
 * cache path (reference tensor_cpp/src/qwen3_ops.cpp:863-909).  Each sequence
 * i attends over its first seq_len[seq_ids[i]] + n_pending tokens, where
 * n_pending counts tokens appended but not yet committed (1 in a decode
 * step).  seq_ids: host array [n_seq] of cache rows, or NULL for
 * 0..n_seq-1; every row must have pages for seq_len + n_pending tokens
 * (SA_ERANGE otherwise).  A sequence of length 0 gets a zero output.
 * seq_len is the cache's committed length as the library's calls have set
 * it (the host copy the launch is sized from, published to the device in
 * stream order); lengths written into sa_kvcache_seq_lens by other code are
 * not read.  q [n_seq][n_q_heads][D] fp32, out likewise.
 * ws must hold sa_paged_decode_ws_bytes(...) bytes.
 * ------------------------------------------------------------------------ */
size_t sa_paged_decode_ws_bytes(const sa_kvcache* cache, int n_seq, int n_q_heads);
sa_status sa_paged_decode(const sa_kvcache* cache, int layer, const float* q,
                          int n_seq, const int32_t* seq_ids, int n_q_heads, int n_pending,
                          float scale, float* out, void* ws, size_t ws_bytes,
                          sa_stream_t stream);

/* ------------------------------------------------------------------------
 * One decode step of a layer in one call: sa_qknorm_rope_append with S = 1,
 * sa_paged_decode with n_pending = 1 and, when commit != 0,
 * sa_kvcache_commit(cache, seq_ids, n_seq, 1).
 *
 * Replaces the per-token body of the reference decoder layer's attention
 * block: QK-norm, RoPE at current_seq_len, KVCache::update, attention over
 * the cache plus the new token (reference tensor_cpp/src/qwen3_ops.cpp:697-909),
 * and, for the last layer, increment_seq_len(1) (qwen3_ops.cpp:986-991).
 * q [n_seq][n_q_heads][D] (before norm and RoPE), k and v [n_seq][n_kv_heads][D];
 * out [n_seq][n_q_heads][D]; q_out, when not NULL, receives the normed and
 * rotated q.  Other arguments as in sa_qknorm_rope_append and
 * sa_paged_decode (ws: sa_paged_decode_ws_bytes bytes).  Sequences whose
 * cache plus the new token fit one chunk take a single kernel launch per 64
 * sequences; longer ones add the LSE merge launch.  Rows are checked as for
 * an append of one token; a refused call enqueues nothing.
 * ------------------------------------------------------------------------ */
sa_status sa_append_decode(sa_kvcache* cache, int layer, const float* q, const float* k,
                           const float* v, int n_seq, const int32_t* seq_ids, int n_q_heads,
                           const float* q_norm_w, const float* k_norm_w, float eps,
                           const float* rope_cos, const float* rope_sin, int rope_max_pos,
                           float scale, float* out, float* q_out, void* ws, size_t ws_bytes,
                           int commit, sa_stream_t stream);

/* sa_append_decode with q, k and v given as the sum of n_part split-K partial
 * products of the layer's fused qkv projection, summed in order 0 .. n_part-1
 * from zero: part [n_part][n_seq][(n_q_heads + 2 n_kv_heads) D] fp32, each row
 * its q columns, then k, then v (the q/k/v split of qwen3_ops.cpp:652-688).
 * The device decoder's step calls this form; a caller whose projection ends
 * in split-K partials saves the pass that sums them. */
sa_status sa_append_decode_partials(sa_kvcache* cache, int layer, const float* part, int n_part,
                                    int n_seq, const int32_t* seq_ids, int n_q_heads,
                                    const float* q_norm_w, const float* k_norm_w, float eps,
                                    const float* rope_cos, const float* rope_sin, int rope_max_pos,
                                    float scale, float* out, float* q_out, void* ws, size_t ws_bytes,
                                    int commit, sa_stream_t stream);

/* Dense copy of a sequence's first len tokens: k_out, v_out [n_kv_heads][len][D]
 * fp32 (serves KVCache::get_cached_keys / get_cached_values, kv_cache.h:161-237). */
sa_status sa_kvcache_gather(const sa_kvcache* cache, int layer, int seq, int len,
                            float* k_out, float* v_out, sa_stream_t stream);

/* ------------------------------------------------------------------------
 * Causal prefill attention on MFMA.
 *
 * Replaces ops::self_attention_streaming_blockwise[_avx2] (reference
 * tensor_cpp/src/ops.cpp:1027-1112, :1383-1599) without repeat_kv.
 * q [batch][n_q_heads][L][D], k and v [batch][n_kv_heads][L][D] in dtype
 * (fp32 or bf16); out [batch][n_q_heads][L][D] fp32.  Query i attends to keys
 * 0..i with scores scale * q.k; accumulation is fp32.
 * ------------------------------------------------------------------------ */
sa_status sa_prefill_causal(const void* q, const void* k, const void* v, sa_dtype dtype,
                            int batch, int n_q_heads, int n_kv_heads, int L, int D,
                            float scale, float* out, sa_stream_t stream);

/* The same with explicit element strides {batch, head, row} for q, for k and
 * v (shared), and for out; rows of D elements must be contiguous and start
 * 16-byte aligned.  Token-major [B][L][H][D] tensors use {L*H*D, D, H*D}. */
sa_status sa_prefill_causal_strided(const void* q, const void* k, const void* v, sa_dtype dtype,
                                    int batch, int n_q_heads, int n_kv_heads, int L, int D,
                                    const int64_t q_strides[3], const int64_t kv_strides[3],
                                    const int64_t out_strides[3], float scale, float* out,
                                    sa_stream_t stream);

/* The same two calls with a caller workspace (they replace the same
 * reference functions, ops.cpp:1027-1112 and :1383-1599, whose per-call
 * std::vector state, :1040-1041 and :1075, the workspace stands for).
 * fp32 at head_dim 128 on a grid
 * of one round of workgroups (short prompts: 16/8 heads up to L = 2048)
 * pairs the longest query tiles with the shortest and splits the pair's key
 * tiles evenly between two workgroups, whose partials a second launch merges;
 * every other shape ignores the workspace.  ws_bytes at least
 * sa_prefill_causal_ws_bytes of the shape (0 where the shape takes no
 * partials), else SA_ENOMEM; ws = NULL takes the single launch.  Results
 * agree with the single launch to fp32 rounding.  Calls that overlap on one
 * workspace race. */
size_t sa_prefill_causal_ws_bytes(sa_dtype dtype, int batch, int n_q_heads, int n_kv_heads, int L, int D);
sa_status sa_prefill_causal_ws(const void* q, const void* k, const void* v, sa_dtype dtype,
                               int batch, int n_q_heads, int n_kv_heads, int L, int D,
                               float scale, float* out, void* ws, size_t ws_bytes, sa_stream_t stream);
sa_status sa_prefill_causal_strided_ws(const void* q, const void* k, const void* v, sa_dtype dtype,
                                       int batch, int n_q_heads, int n_kv_heads, int L, int D,
                                       const int64_t q_strides[3], const int64_t kv_strides[3],
                                       const int64_t out_strides[3], float scale, float* out,
                                       void* ws, size_t ws_bytes, sa_stream_t stream);

/* ------------------------------------------------------------------------
 * Tile sizes of the attention kernels, for the whole process: the
 * counterpart of the reference's tensor_cpp::g_q_block_size and
 * g_kv_block_size (tensor_cpp/src/ops.cpp:1630-1631), which benchmark_qwen3
 * sets from --q-block-size and --kv-block-size (benchmark_qwen3.cpp:1072-1073).
 *
 * q_block: query rows per prefill workgroup and head.  fp32: 32 (workgroups
 * whose waves split each key tile), 64 or 128.  bf16: 32 (the split-key
 * kernel; head_dim 128 and even GQA groups) or the workgroup width whose
 * per-head tile it is (16/8 heads: 64 or 128); a bf16 shape with no kernel of
 * that tile keeps the launch's own choice.  The key tile stays 64 rows.
 * kv_block: tokens per split-KV chunk of decode attention (the range one
 * workgroup streams before the log-sum-exp merge), a multiple of 64 in
 * [64, 16384]; raised where a sequence would need more than 1,024 chunks.
 * 0 selects the launch's own choice.  Other values return SA_EINVAL and
 * change nothing.  Results agree across settings up to fp32 rounding.
 * ------------------------------------------------------------------------ */
sa_status sa_set_attention_blocks(int q_block, int kv_block);
sa_status sa_get_attention_blocks(int* q_block, int* kv_block);

/* The query rows per workgroup and head a prefill launch of this shape takes
 * under the current settings, or a negative sa_status for a shape the
 * prefill refuses. */
int sa_prefill_query_tile(sa_dtype dtype, int batch, int n_q_heads, int n_kv_heads, int L, int D);

/* ------------------------------------------------------------------------
 * Dense fp32 operators of the decoder layer (projections, norms, MLP,
 * residuals), for callers whose weights are fp32.  All pointers are device
 * pointers; rows are contiguous.
 * ------------------------------------------------------------------------ */

/* y[M][N] = x[M][K] . w[N][K]^T (+ bias[N] when bias is not NULL), fp32 MFMA
 * with fp32 accumulation: ops::linear with nn.Linear's weight layout
 * (reference tensor_cpp/src/ops.cpp:315-369).  y must not overlap x or w; x
 * and w may be NULL when K = 0 (then y = bias, or 0). */
sa_status sa_linear_f32(const float* x, int M, int K, const float* w, int N, const float* bias,
                        float* y, sa_stream_t stream);

/* y[r] = (x[r] / sqrt(sum(x[r]^2) / n + eps)) * w over rows of n floats; w may
 * be NULL (no gain); y may alias x (ops::rms_norm, reference
 * tensor_cpp/src/ops.cpp:375-418). */
sa_status sa_rms_norm_f32(const float* x, int rows, int n, const float* w, float eps, float* y,
                          sa_stream_t stream);

/* out[i] = up[i] * gate[i] * sigmoid(gate[i]): the SwiGLU of qwen3_mlp and
 * ops::swiglu(up, gate) (reference tensor_cpp/src/qwen3_ops.cpp:282-290,
 * tensor_cpp/src/ops.cpp:493-509).  out may alias either input. */
sa_status sa_swiglu_f32(const float* gate, const float* up, size_t n, float* out, sa_stream_t stream);

/* out[i] = a x[i] + b y[i], or a x[i] when y is NULL; out may alias x or y.
 * With a = 1 it is ops::add(x, y, b) (reference tensor_cpp/src/ops.cpp:194-207)
 * and, with b = 1, the residual add of the decoder layer. */
sa_status sa_axpby_f32(const float* x, float a, const float* y, float b, size_t n, float* out,
                       sa_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SA_AMD_H */
