/*
 * oracle.c - CPU restatement of the reference's streaming-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker / baseline; the product (streaming-attention_amd) never calls it.
 *
 * Every function restates one reference routine (cited file:line relative to
 * the reference repository root) in plain C, fp32 arithmetic in the same
 * order as the reference unless stated.  Functions suffixed _f64 are fp64
 * brute-force forms used to pin the fp32 ones.
 *
 * Parity pins (see tests/test_oracle.py):
 *   or_streaming_serial, or_naive_serial, or_streaming_omp, or_l2_error,
 *   or_max_error, or_rope_tables, or_apply_rope, or_rms_norm_rows,
 *   or_decode_gqa, or_decode_streaming_compat, or_prefill_blockwise:
 *   each is checked against the reference compiled from its own sources
 *   (oracle/_ref) on committed golden vectors, and against the fp64 forms
 *   and closed-form invariants.
 *   or_sequence_np1 (timing only: the reference's MPI path cannot be built
 *   here, mpi.h is absent) is checked against its closed form in fp64.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Online-softmax state (reference utils/softmax_online.h:22-28): m = -inf, l = 1. */
typedef struct { float m, l; } or_state;

/* One block update (reference utils/softmax_online.h:40-87). O stays normalised. */
static void or_process_block(const float* scores, const float* values, or_state* st,
                             float* out, int bs, int d) {
    float m_new = st->m;
    for (int i = 0; i < bs; ++i) m_new = scores[i] > m_new ? scores[i] : m_new;
    float sum_exp = 0.0f;
    for (int i = 0; i < bs; ++i) sum_exp += expf(scores[i] - m_new);
    const float scale_old = expf(st->m - m_new);
    const float l_new = st->l * scale_old + sum_exp;
    const float alpha_old = (st->l * scale_old) / l_new;
    const float alpha_new = 1.0f / l_new;
    for (int j = 0; j < d; ++j) out[j] *= alpha_old;
    for (int i = 0; i < bs; ++i) {
        const float w = alpha_new * expf(scores[i] - m_new);
        const float* vr = values + (size_t)i * d;
        for (int j = 0; j < d; ++j) out[j] += w * vr[j];
    }
    st->m = m_new;
    st->l = l_new;
}

/* Blocks of [t0, t1) into (state, out) (reference attention/src/streaming_omp.cpp:53-89). */
static void or_process_range(const float* Q, const float* K, const float* V, int t0, int t1,
                             int d, int block, or_state* st, float* out) {
    float* scores = (float*)malloc(sizeof(float) * (size_t)(block > 0 ? block : 1));
    for (int b0 = t0; b0 < t1; b0 += block) {
        const int b1 = b0 + block < t1 ? b0 + block : t1;
        for (int i = b0; i < b1; ++i) {
            float s = 0.0f;
            const float* kr = K + (size_t)i * d;
            for (int j = 0; j < d; ++j) s += Q[j] * kr[j];
            scores[i - b0] = s;
        }
        or_process_block(scores, V + (size_t)b0 * d, st, out, b1 - b0, d);
    }
    free(scores);
}

/* streaming_attention_serial (reference attention/src/streaming_serial.cpp:20-71):
 * unscaled softmax(Q K^T) V, processed in blocks of `block`. */
void or_streaming_serial(const float* Q, const float* K, const float* V, int T, int d, int block,
                         float* O) {
    or_state st = {-INFINITY, 1.0f};
    memset(O, 0, sizeof(float) * (size_t)d);
    if (T <= 0) return;
    or_process_range(Q, K, V, 0, T, d, block, &st, O);
}

/* naive_attention_serial (reference attention/src/naive_serial.cpp:18-72). */
void or_naive_serial(const float* Q, const float* K, const float* V, int T, int d, float* O) {
    memset(O, 0, sizeof(float) * (size_t)d);
    if (T <= 0) return;
    float* s = (float*)malloc(sizeof(float) * (size_t)T);
    for (int i = 0; i < T; ++i) {
        float a = 0.0f;
        for (int j = 0; j < d; ++j) a += Q[j] * K[(size_t)i * d + j];
        s[i] = a;
    }
    float mx = -INFINITY;
    for (int i = 0; i < T; ++i) mx = s[i] > mx ? s[i] : mx;
    float sum = 0.0f;
    for (int i = 0; i < T; ++i) { s[i] = expf(s[i] - mx); sum += s[i]; }
    for (int i = 0; i < T; ++i) s[i] /= sum;
    for (int i = 0; i < T; ++i)
        for (int j = 0; j < d; ++j) O[j] += s[i] * V[(size_t)i * d + j];
    free(s);
}

/* merge_partial_results (reference attention/src/streaming_omp.cpp:27-48). */
static void or_merge(or_state* a, float* Oa, const or_state* b, const float* Ob, int d) {
    const float m_new = a->m > b->m ? a->m : b->m;
    const float sa = expf(a->m - m_new), sb = expf(b->m - m_new);
    const float l_new = a->l * sa + b->l * sb;
    const float wa = (a->l * sa) / l_new, wb = (b->l * sb) / l_new;
    for (int j = 0; j < d; ++j) Oa[j] = Oa[j] * wa + Ob[j] * wb;
    a->m = m_new;
    a->l = l_new;
}

/* streaming_attention_omp (reference attention/src/streaming_omp.cpp:99-154):
 * n_chunks = max(1, min(threads, ceil(T / (2 block)))) contiguous chunks, each
 * processed serially, then merged left to right.  nthreads <= 0 uses the
 * OpenMP default.  T <= 0 returns zeros (the reference returns NaN there). */
void or_streaming_omp(const float* Q, const float* K, const float* V, int T, int d, int block,
                      int nthreads, float* O) {
    memset(O, 0, sizeof(float) * (size_t)d);
    if (T <= 0) return;
    int nt = 1;
#ifdef _OPENMP
    nt = nthreads > 0 ? nthreads : omp_get_max_threads();
#else
    (void)nthreads;
#endif
    int n_chunks = (T + block * 2 - 1) / (block * 2);
    if (nt < n_chunks) n_chunks = nt;
    if (n_chunks < 1) n_chunks = 1;
    const int chunk = (T + n_chunks - 1) / n_chunks;
    or_state* st = (or_state*)malloc(sizeof(or_state) * (size_t)n_chunks);
    float* po = (float*)calloc((size_t)n_chunks * d, sizeof(float));
#pragma omp parallel for num_threads(nt) schedule(static, 1)
    for (int c = 0; c < n_chunks; ++c) {
        const int t0 = c * chunk;
        const int t1 = t0 + chunk < T ? t0 + chunk : T;
        st[c].m = -INFINITY;
        st[c].l = 1.0f;
        if (t0 < t1) or_process_range(Q, K, V, t0, t1, d, block, &st[c], po + (size_t)c * d);
    }
    or_state acc = {-INFINITY, 1.0f};
    for (int c = 0; c < n_chunks; ++c) or_merge(&acc, O, &st[c], po + (size_t)c * d, d);
    free(st);
    free(po);
}

/* compute_l2_error: relative L2, absolute when |b| < 1e-10
 * (reference attention/src/naive_serial.cpp:75-90). */
float or_l2_error(const float* a, const float* b, int n) {
    float sq = 0.0f, ref = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float df = a[i] - b[i];
        sq += df * df;
        ref += b[i] * b[i];
    }
    const float rn = sqrtf(ref);
    return rn < 1e-10f ? sqrtf(sq) : sqrtf(sq) / rn;
}

/* compute_max_error (reference attention/src/naive_serial.cpp:92-98). */
float or_max_error(const float* a, const float* b, int n) {
    float mx = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float e = fabsf(a[i] - b[i]);
        mx = e > mx ? e : mx;
    }
    return mx;
}

/* Per-row RMSNorm of q/k heads, eps inside the sqrt
 * (reference tensor_cpp/src/qwen3_ops.cpp:697-753):
 * y = (x / sqrt(sum(x^2)/D + eps)) * w.  eps_outside != 0 gives the AVX2
 * path's sqrt(mean) + eps (reference tensor_cpp/src/qwen3_ops_avx.cpp:537). */
void or_rms_norm_rows(const float* x, const float* w, int rows, int D, float eps, int eps_outside,
                      float* y) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * D;
        float ss = 0.0f;
        for (int i = 0; i < D; ++i) ss += xr[i] * xr[i];
        const float rms = eps_outside ? sqrtf(ss / (float)D) + eps : sqrtf(ss / (float)D + eps);
        for (int i = 0; i < D; ++i) y[(size_t)r * D + i] = (xr[i] / rms) * w[i];
    }
}

/* compute_rope_freqs (reference tensor_cpp/src/qwen3_ops.cpp:70-104):
 * inv_freq[i] = 1 / theta^(i / D) (not HF's 2i/D), cos/sin of float(pos)*inv_freq. */
void or_rope_tables(int max_pos, int D, float theta, float* cos_t, float* sin_t) {
    const int h = D / 2;
    float* inv = (float*)malloc(sizeof(float) * (size_t)h);
    for (int i = 0; i < h; ++i) inv[i] = 1.0f / powf(theta, (float)i / (float)D);
    for (int p = 0; p < max_pos; ++p)
        for (int i = 0; i < h; ++i) {
            const float a = (float)p * inv[i];
            cos_t[(size_t)p * h + i] = cosf(a);
            sin_t[(size_t)p * h + i] = sinf(a);
        }
    free(inv);
}

/* rotate_half + apply_rotary_pos_emb on rows (reference
 * tensor_cpp/src/qwen3_ops.cpp:30-64, 110-188): for i < D/2,
 * y_i = x_i cos - x_{i+D/2} sin, y_{i+D/2} = x_{i+D/2} cos + x_i sin,
 * with cos/sin taken at row pos[r] of the tables. */
void or_apply_rope(const float* x, int rows, int D, const int* pos, const float* cos_t,
                   const float* sin_t, float* y) {
    const int h = D / 2;
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * D;
        float* yr = y + (size_t)r * D;
        const float* c = cos_t + (size_t)pos[r] * h;
        const float* s = sin_t + (size_t)pos[r] * h;
        for (int i = 0; i < h; ++i) {
            const float lo = xr[i], hi = xr[i + h];
            yr[i] = lo * c[i] + (-hi) * s[i];
            yr[i + h] = hi * c[i] + lo * s[i];
        }
    }
}

/* Decode attention, q_len = 1, over a dense cache, as the reference's
 * STANDARD path computes it: repeat_kv head map h -> h / (Hq/Hkv)
 * (reference tensor_cpp/src/qwen3_ops.cpp:194-234) then self_attention with an
 * all-zero mask (reference tensor_cpp/src/ops.cpp:514-641):
 * out = softmax(scale * q k^T) v.
 * q [B][Hq][D], k/v [B][Hkv][L][D], out [B][Hq][D]. */
void or_decode_gqa(const float* q, const float* k, const float* v, int B, int Hq, int Hkv, int L,
                   int D, float scale, float* out) {
    const int rep = Hq / Hkv;
#pragma omp parallel for collapse(2)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < Hq; ++h) {
            const float* qr = q + ((size_t)b * Hq + h) * D;
            const float* kb = k + ((size_t)b * Hkv + h / rep) * (size_t)L * D;
            const float* vb = v + ((size_t)b * Hkv + h / rep) * (size_t)L * D;
            float* o = out + ((size_t)b * Hq + h) * D;
            float* s = (float*)malloc(sizeof(float) * (size_t)(L > 0 ? L : 1));
            float mx = -INFINITY;
            for (int j = 0; j < L; ++j) {
                float a = 0.0f;
                for (int i = 0; i < D; ++i) a += qr[i] * kb[(size_t)j * D + i];
                s[j] = a * scale;
                mx = s[j] > mx ? s[j] : mx;
            }
            float sum = 0.0f;
            for (int j = 0; j < L; ++j) { s[j] = expf(s[j] - mx); sum += s[j]; }
            for (int j = 0; j < L; ++j) s[j] /= sum;
            for (int i = 0; i < D; ++i) {
                float a = 0.0f;
                for (int j = 0; j < L; ++j) a += s[j] * vb[(size_t)j * D + i];
                o[i] = L > 0 ? a : 0.0f;
            }
            free(s);
        }
}

/* self_attention_streaming as the reference writes it (reference
 * tensor_cpp/src/ops.cpp:964-1017): unscaled streaming attention per head,
 * then the output multiplied by scale (the reference's decode-scale quirk).
 * Heads are given already repeated: k/v [B][H][L][D]. */
void or_decode_streaming_compat(const float* q, const float* k, const float* v, int B, int H, int L,
                                int D, float scale, int block, float* out) {
#pragma omp parallel for collapse(2)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const size_t qo = ((size_t)b * H + h) * D;
            const size_t ko = ((size_t)b * H + h) * (size_t)L * D;
            or_streaming_omp(q + qo, k + ko, v + ko, L, D, block, 1, out + qo);
            for (int i = 0; i < D; ++i) out[qo + i] *= scale;
        }
}

/* self_attention_streaming_blockwise, causal prefill from position 0
 * (reference tensor_cpp/src/ops.cpp:1027-1112): query i keeps its own
 * online-softmax state over kv blocks restricted to keys 0..i, with
 * scores = (q.k) * scale.  GQA through the repeat_kv head map.
 * q [B][Hq][L][D], k/v [B][Hkv][L][D], out [B][Hq][L][D].
 * rows: optional list of n_rows query positions to compute (others untouched);
 * NULL computes all L rows. */
void or_prefill_blockwise(const float* q, const float* k, const float* v, int B, int Hq, int Hkv,
                          int L, int D, float scale, int kv_block, const int* rows, int n_rows,
                          float* out) {
    const int rep = Hq / Hkv;
    const int nr = rows ? n_rows : L;
#pragma omp parallel for collapse(3) schedule(dynamic, 4)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < Hq; ++h)
            for (int ri = 0; ri < nr; ++ri) {
                const int qi = rows ? rows[ri] : ri;
                const float* qr = q + (((size_t)b * Hq + h) * L + qi) * D;
                const float* kb = k + ((size_t)b * Hkv + h / rep) * (size_t)L * D;
                const float* vb = v + ((size_t)b * Hkv + h / rep) * (size_t)L * D;
                float* o = out + (((size_t)b * Hq + h) * L + qi) * D;
                or_state st = {-INFINITY, 1.0f};
                float* sc = (float*)malloc(sizeof(float) * (size_t)kv_block);
                memset(o, 0, sizeof(float) * (size_t)D);
                for (int k0 = 0; k0 <= qi; k0 += kv_block) {
                    int k1 = k0 + kv_block < L ? k0 + kv_block : L;
                    if (k1 > qi + 1) k1 = qi + 1;
                    for (int j = k0; j < k1; ++j) {
                        float a = 0.0f;
                        for (int i = 0; i < D; ++i) a += qr[i] * kb[(size_t)j * D + i];
                        sc[j - k0] = a * scale;
                    }
                    or_process_block(sc, vb + (size_t)k0 * D, &st, o, k1 - k0, D);
                }
                free(sc);
            }
}

/* fp64 brute force: out_i = sum_j softmax_j(scale q_i.k_j) v_j over keys
 * j < L (causal: j <= pos0 + i).  q [nq][D], k/v [L][D], out fp64 [nq][D]. */
void or_sdpa_f64(const float* q, const float* k, const float* v, int nq, int L, int D, double scale,
                 int causal, int pos0, double* out) {
#pragma omp parallel for
    for (int i = 0; i < nq; ++i) {
        const int lim = causal ? (pos0 + i + 1 < L ? pos0 + i + 1 : L) : L;
        double* s = (double*)malloc(sizeof(double) * (size_t)(lim > 0 ? lim : 1));
        double mx = -INFINITY;
        for (int j = 0; j < lim; ++j) {
            double a = 0.0;
            for (int t = 0; t < D; ++t) a += (double)q[(size_t)i * D + t] * (double)k[(size_t)j * D + t];
            s[j] = a * scale;
            if (s[j] > mx) mx = s[j];
        }
        double sum = 0.0;
        for (int j = 0; j < lim; ++j) { s[j] = exp(s[j] - mx); sum += s[j]; }
        for (int t = 0; t < D; ++t) {
            double a = 0.0;
            for (int j = 0; j < lim; ++j) a += s[j] * (double)v[(size_t)j * D + t];
            out[(size_t)i * D + t] = lim > 0 ? a / sum : 0.0;
        }
        free(s);
    }
}

/* TIMING ONLY, never a checker.  The np = 1 loop of the MPI sequence-parallel
 * prefill attention (reference tensor_cpp/src/ops_mpi.cpp:1216-1454,
 * attention_sequence_online_softmax_avx2, the `mpi+avx2
 * --parallel-strategy sequence` path) for query heads [h0, h0 + nh) of every
 * batch row: the same per-query work in the same order, AVX2/FMA like the
 * reference's build, one thread (the reference's OpenMP loop runs over the
 * batch, which is 1 in the prefill benchmark).  Per query i (q scaled
 * first, :1257-1270) and per 64-key block holding a key j <= i (:1274-1290):
 * fresh zeroed block buffers (:1293-1294); for each such key the score
 * s_j = q'.k_j (8-lane FMA then a horizontal sum, :1303-1320) and s_j v_j
 * (:1325-1339); the block max over every slot, the masked ones holding 0
 * (:1343-1345); e_j = exp(s_j - m) over the valid keys (:1348-1360); the
 * running sum and the O row rescaled by exp(m_old - m) (:1363-1381), then
 * O += e_j (s_j v_j) (:1384-1407).  With one rank the Allreduce is skipped
 * and the correction factor is exp(0) = 1 (:1414-1438): out = O / l.
 *
 * Its numerics are the reference's, which are wrong: the weights multiply
 * s_j v_j, not v_j, so out_i = sum_{j<=i} e^{s_j} s_j v_j / sum_{j<=i} e^{s_j}
 * (the maxima cancel).  tests/test_oracle.py pins it to that closed form in
 * fp64.  q [B][Hq][L][D], k/v [B][Hkv][L][D], out [B][Hq][L][D] (heads
 * outside the range untouched). */
#include <immintrin.h>

__attribute__((target("avx2,fma"))) static float or_hsum8(__m256 x) {
    const __m128 s4 = _mm_add_ps(_mm256_castps256_ps128(x), _mm256_extractf128_ps(x, 1));
    const __m128 s2 = _mm_add_ps(s4, _mm_movehl_ps(s4, s4));
    return _mm_cvtss_f32(_mm_add_ss(s2, _mm_shuffle_ps(s2, s2, 1)));
}

__attribute__((target("avx2,fma"))) void or_sequence_np1(const float* q, const float* k, const float* v, int B,
                                                         int Hq, int Hkv, int L, int D, float scale, int h0,
                                                         int nh, float* out) {
    const int rep = Hq / Hkv;
    const int KB = 64;
    const size_t nstat = (size_t)B * Hq * L;
    float* m_all = (float*)malloc(sizeof(float) * nstat);
    float* l_all = (float*)malloc(sizeof(float) * nstat);
    for (size_t i = 0; i < nstat; ++i) { m_all[i] = -INFINITY; l_all[i] = 0.0f; }
    for (int b = 0; b < B; ++b)
        for (int h = h0; h < h0 + nh; ++h) {
            const float* kb = k + ((size_t)b * Hkv + h / rep) * (size_t)L * D;
            const float* vb = v + ((size_t)b * Hkv + h / rep) * (size_t)L * D;
            for (int i = 0; i < L; ++i) {
                const size_t row = ((size_t)b * Hq + h) * L + i;
                float* o = out + row * D;
                memset(o, 0, sizeof(float) * (size_t)D);
                float* qs = (float*)malloc(sizeof(float) * (size_t)D);
                const float* qr = q + row * D;
                const __m256 vs = _mm256_set1_ps(scale);
                int d = 0;
                for (; d + 8 <= D; d += 8) _mm256_storeu_ps(qs + d, _mm256_mul_ps(_mm256_loadu_ps(qr + d), vs));
                for (; d < D; ++d) qs[d] = qr[d] * scale;
                for (int j0 = 0; j0 < L; j0 += KB) {
                    const int j1 = j0 + KB < L ? j0 + KB : L;
                    int any = 0;                   /* a key of the block is <= i */
                    for (int j = j0; j < j1; ++j)
                        if (j <= i) { any = 1; break; }
                    if (!any) continue;
                    const int n = j1 - j0;
                    float* sc = (float*)calloc((size_t)n, sizeof(float));
                    float* wv = (float*)calloc((size_t)n * D, sizeof(float));
                    for (int j = j0; j < j1 && j <= i; ++j) {
                        const float* kr = kb + (size_t)j * D;
                        __m256 acc = _mm256_setzero_ps();
                        d = 0;
                        for (; d + 8 <= D; d += 8)
                            acc = _mm256_fmadd_ps(_mm256_loadu_ps(qs + d), _mm256_loadu_ps(kr + d), acc);
                        float s = d > 0 ? or_hsum8(acc) : 0.0f;
                        for (; d < D; ++d) s += qs[d] * kr[d];
                        sc[j - j0] = s;
                        const float* vr = vb + (size_t)j * D;
                        float* w = wv + (size_t)(j - j0) * D;
                        const __m256 sv = _mm256_set1_ps(s);
                        d = 0;
                        for (; d + 8 <= D; d += 8) _mm256_storeu_ps(w + d, _mm256_mul_ps(sv, _mm256_loadu_ps(vr + d)));
                        for (; d < D; ++d) w[d] = s * vr[d];
                    }
                    float bm = sc[0];
                    for (int t = 1; t < n; ++t) bm = sc[t] > bm ? sc[t] : bm;
                    const float m_old = m_all[row];
                    const float m_new = m_old > bm ? m_old : bm;
                    m_all[row] = m_new;
                    float* e = (float*)calloc((size_t)n, sizeof(float));
                    float esum = 0.0f;
                    for (int j = j0; j < j1 && j <= i; ++j) {
                        e[j - j0] = expf(sc[j - j0] - m_new);
                        esum += e[j - j0];
                    }
                    const float f = expf(m_old - m_new);
                    l_all[row] = l_all[row] * f + esum;
                    const __m256 vf = _mm256_set1_ps(f);
                    d = 0;
                    for (; d + 8 <= D; d += 8) _mm256_storeu_ps(o + d, _mm256_mul_ps(_mm256_loadu_ps(o + d), vf));
                    for (; d < D; ++d) o[d] *= f;
                    for (int j = j0; j < j1 && j <= i; ++j) {
                        const float* w = wv + (size_t)(j - j0) * D;
                        const __m256 ve = _mm256_set1_ps(e[j - j0]);
                        d = 0;
                        for (; d + 8 <= D; d += 8)
                            _mm256_storeu_ps(o + d, _mm256_fmadd_ps(ve, _mm256_loadu_ps(w + d), _mm256_loadu_ps(o + d)));
                        for (; d < D; ++d) o[d] += e[j - j0] * w[d];
                    }
                    free(e);
                    free(wv);
                    free(sc);
                }
                free(qs);
            }
        }
    /* the normalisation pass; with one rank the global statistics are the local ones */
    for (int b = 0; b < B; ++b)
        for (int h = h0; h < h0 + nh; ++h)
            for (int i = 0; i < L; ++i) {
                const size_t row = ((size_t)b * Hq + h) * L + i;
                const float corr = expf(m_all[row] - m_all[row]);
                for (int d = 0; d < D; ++d) out[row * D + d] = out[row * D + d] * corr / l_all[row];
            }
    free(l_all);
    free(m_all);
}
