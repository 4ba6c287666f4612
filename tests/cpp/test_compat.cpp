// C++ tests of the reference-shaped API (attention.h, tensor_cpp/kv_cache.h,
// tensor_cpp/ops.h, tensor_cpp/qwen3_ops.h) running on the GPU, checked
// against the CPU oracle (oracle/oracle.c).  Structure follows the
// reference's tensor_cpp/tests/unit/test_streaming_attention.cpp: a
// correctness grid T x d with U(-1,1) inputs and a 1e-5 max-abs bar, thread
// variants against serial at 1e-4, plus the KV cache and Qwen3 attention path.
// Prints one line per check; exit status is the number of failures.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <functional>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

#include "attention.h"
#include "tensor_cpp/kv_cache.h"
#include "tensor_cpp/ops.h"
#include "tensor_cpp/qwen3_ops.h"

extern "C" {
void or_streaming_serial(const float*, const float*, const float*, int, int, int, float*);
void or_naive_serial(const float*, const float*, const float*, int, int, float*);
void or_rms_norm_rows(const float*, const float*, int, int, float, int, float*);
void or_rope_tables(int, int, float, float*, float*);
void or_apply_rope(const float*, int, int, const int*, const float*, const float*, float*);
void or_decode_gqa(const float*, const float*, const float*, int, int, int, int, int, float, float*);
void or_prefill_blockwise(const float*, const float*, const float*, int, int, int, int, int, float, int,
                          const int*, int, float*);
}

using tensor_cpp::Shape;
using tensor_cpp::Tensor;
namespace q3 = tensor_cpp::qwen3;

static int g_fail = 0;

static void report(const std::string& name, bool ok, const std::string& detail = "") {
    std::printf("%s %s %s\n", ok ? "PASS" : "FAIL", name.c_str(), detail.c_str());
    std::fflush(stdout);
    if (!ok) ++g_fail;
}

// splitmix64-based uniform stream, independent of any C++ library distribution.
struct Rng {
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed) {}
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    float uniform(float lo, float hi) { return lo + (hi - lo) * (float)((next() >> 40) * (1.0 / 16777216.0)); }
    std::vector<float> vec(size_t n, float lo = -1.f, float hi = 1.f) {
        std::vector<float> v(n);
        for (auto& x : v) x = uniform(lo, hi);
        return v;
    }
};

static float max_abs(const std::vector<float>& a, const std::vector<float>& b) {
    return compute_max_error(a.data(), b.data(), (int)a.size());
}

template <class E>
static bool throws(const std::function<void()>& f) {
    try {
        f();
    } catch (const E&) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

static void test_correctness() {
    Rng rng(42);
    for (int T : {512, 1024, 2048, 4096})
        for (int d : {64, 128, 256}) {
            auto Q = rng.vec(d), K = rng.vec((size_t)T * d), V = rng.vec((size_t)T * d);
            std::vector<float> naive(d), oracle_s(d);
            or_naive_serial(Q.data(), K.data(), V.data(), T, d, naive.data());
            or_streaming_serial(Q.data(), K.data(), V.data(), T, d, 64, oracle_s.data());
            auto gpu = streaming_attention_serial(Q.data(), K.data(), V.data(), T, d, 64);
            const float e = max_abs(gpu, naive);
            report("correctness T=" + std::to_string(T) + " d=" + std::to_string(d), e <= 1e-5f,
                   "max_err=" + std::to_string(e));
            auto gn = naive_attention_serial(Q.data(), K.data(), V.data(), T, d);
            report("naive T=" + std::to_string(T) + " d=" + std::to_string(d), max_abs(gn, oracle_s) <= 1e-5f);
        }
}

static void test_thread_variants() {
    Rng rng(7);
    const int T = 8192, d = 128;
    auto Q = rng.vec(d), K = rng.vec((size_t)T * d), V = rng.vec((size_t)T * d);
    auto serial = streaming_attention_serial(Q.data(), K.data(), V.data(), T, d, 64);
    for (int threads : {2, 4, 8}) {
        auto o = streaming_attention_omp(Q.data(), K.data(), V.data(), T, d, 64, threads);
        report("omp threads=" + std::to_string(threads), max_abs(o, serial) <= 1e-4f);
    }
    report("omp_numa", max_abs(streaming_attention_omp_numa(Q.data(), K.data(), V.data(), T, d, 128), serial) <= 1e-4f);
    report("naive_omp", max_abs(naive_attention_omp(Q.data(), K.data(), V.data(), T, d, 4), serial) <= 1e-4f);
    MPI_Comm comm = nullptr;
    report("streaming_mpi_simple single rank",
           max_abs(streaming_attention_mpi_simple(Q.data(), K.data(), V.data(), T, T, d, 64, comm), serial) <= 1e-4f);
    report("naive_mpi single rank",
           max_abs(naive_attention_mpi(Q.data(), K.data(), V.data(), T, T, d, 4, comm), serial) <= 1e-4f);
    report("naive_mpi_simple single rank",
           max_abs(naive_attention_mpi_simple(Q.data(), K.data(), V.data(), T, T, d, comm), serial) <= 1e-4f);
    report("mpi rejects a partial sequence", throws<std::invalid_argument>([&] {
               streaming_attention_mpi_simple(Q.data(), K.data(), V.data(), T / 2, T, d, 64, comm);
           }));
    auto ns = tensor_cpp::ops::streaming_attention_serial(Q.data(), K.data(), V.data(), T, d, 128);
    report("ops::streaming_attention_serial", max_abs(ns, serial) <= 1e-5f);
}

static void test_edges() {
    std::vector<float> Q(128, 1.0f), K(128 * 10, 0.5f);
    auto z = streaming_attention_serial(Q.data(), K.data(), K.data(), 0, 128, 64);
    bool zeros = true;
    for (float x : z) zeros &= x == 0.0f;
    report("T=0 gives zeros", zeros && z.size() == 128);
    report("d=100 rejected", throws<std::invalid_argument>([&] {
               streaming_attention_serial(Q.data(), K.data(), K.data(), 10, 100, 64);
           }));
    report("block 0 rejected", throws<std::invalid_argument>([&] {
               streaming_attention_serial(Q.data(), K.data(), K.data(), 10, 128, 0);
           }));
    std::vector<float> a = {1, 2, 2}, b = {0, 2, 0};
    report("compute_l2_error relative", std::fabs(compute_l2_error(a.data(), b.data(), 3) - std::sqrt(5.0f) / 2) < 1e-6f);
    report("compute_max_error", compute_max_error(a.data(), b.data(), 3) == 2.0f);
}

static Tensor rand_tensor(Rng& rng, Shape s) { return Tensor(rng.vec(s.total()), s); }

static void test_kv_cache() {
    Rng rng(11);
    const size_t L = 2, B = 2, H = 8, D = 128, MAX = 300;
    q3::KVCache cache(L, B, H, D, MAX);
    Tensor k1 = rand_tensor(rng, {B, H, 5, D}), v1 = rand_tensor(rng, {B, H, 5, D});
    cache.update(0, k1, v1);
    report("get before increment throws", throws<std::runtime_error>([&] { cache.get_cached_keys(0, 5); }));
    cache.increment_seq_len(5);
    Tensor gk = cache.get_cached_keys(0, 5), gv = cache.get_cached_values(0, 5);
    bool same = gk.shape() == k1.shape() && gv.shape() == v1.shape();
    for (size_t i = 0; same && i < k1.size(); ++i) same = gk[i] == k1[i] && gv[i] == v1[i];
    report("update/get round trip", same);
    Tensor k2 = rand_tensor(rng, {B, H, 3, D}), v2 = rand_tensor(rng, {B, H, 3, D});
    cache.update(0, k2, v2);
    cache.increment_seq_len(3);
    Tensor g8 = cache.get_cached_keys(0, 8);
    bool cat = true;
    for (size_t b = 0; b < B; ++b)
        for (size_t h = 0; h < H; ++h)
            for (size_t s = 0; s < 8; ++s)
                for (size_t x = 0; x < D; ++x) {
                    const float want = s < 5 ? k1[((b * H + h) * 5 + s) * D + x] : k2[((b * H + h) * 3 + s - 5) * D + x];
                    cat &= g8[((b * H + h) * 8 + s) * D + x] == want;
                }
    report("append continues at current_seq_len", cat && cache.current_seq_len == 8);
    report("layer 1 untouched", cache.get_cached_values(1, 8)[17] == 0.0f);
    report("bad layer -> out_of_range", throws<std::out_of_range>([&] { cache.get_cached_keys(2, 1); }));
    report("update bad layer -> out_of_range", throws<std::out_of_range>([&] { cache.update(7, k2, v2); }));
    report("overflow -> runtime_error", throws<std::runtime_error>([&] {
               Tensor big = rand_tensor(rng, {B, H, MAX, D});
               cache.update(0, big, big);
           }));
    cache.reset();
    report("reset", cache.current_seq_len == 0 && cache.get_cached_keys(0, 0).size() == 0);
    q3::KVCache bf(1, 1, H, D, 128, SA_DTYPE_BF16);
    Tensor kb = rand_tensor(rng, {1, H, 4, D});
    bf.update(0, kb, kb);
    bf.increment_seq_len(4);
    Tensor gb = bf.get_cached_keys(0, 4);
    float err = 0;
    for (size_t i = 0; i < kb.size(); ++i) err = std::max(err, std::fabs(gb[i] - kb[i]) / std::max(std::fabs(kb[i]), 1e-3f));
    report("bf16 cache stores to bf16 precision", err <= 1.0f / 256, "rel=" + std::to_string(err));
}

static void test_ops() {
    Rng rng(13);
    const size_t B = 2, Hq = 16, Hkv = 8, D = 128, Lk = 300, Lp = 200;
    const float scale = 1.0f / std::sqrt((float)D);
    // decode through self_attention (zero mask) and self_attention_streaming
    Tensor q = rand_tensor(rng, {B, Hq, 1, D}), k = rand_tensor(rng, {B, Hkv, Lk, D}), v = rand_tensor(rng, {B, Hkv, Lk, D});
    std::vector<float> want(B * Hq * D);
    or_decode_gqa(q.data(), k.data(), v.data(), (int)B, (int)Hq, (int)Hkv, (int)Lk, (int)D, scale, want.data());
    Tensor zero_mask(std::vector<float>(Lk, 0.0f), Shape({1, 1, 1, Lk}));
    Tensor sd = tensor_cpp::ops::self_attention(q, k, v, &zero_mask, scale);
    report("self_attention decode", max_abs(std::vector<float>(sd.data(), sd.data() + sd.size()), want) <= 1e-5f);
    Tensor ss = tensor_cpp::ops::self_attention_streaming(q, k, v, scale);
    report("self_attention_streaming", max_abs(std::vector<float>(ss.data(), ss.data() + ss.size()), want) <= 1e-5f);
    tensor_cpp::ops::g_streaming_scale_on_output = true;
    Tensor sc = tensor_cpp::ops::self_attention_streaming(q, k, v, scale);
    tensor_cpp::ops::g_streaming_scale_on_output = false;
    std::vector<float> want_compat(B * Hq * D);
    or_decode_gqa(q.data(), k.data(), v.data(), (int)B, (int)Hq, (int)Hkv, (int)Lk, (int)D, 1.0f, want_compat.data());
    for (auto& x : want_compat) x *= scale;
    report("self_attention_streaming scale-on-output compat",
           max_abs(std::vector<float>(sc.data(), sc.data() + sc.size()), want_compat) <= 1e-5f);
    // with repeat_kv the same answer
    Tensor kr = q3::repeat_kv(k, 2), vr = q3::repeat_kv(v, 2);
    Tensor sr = tensor_cpp::ops::self_attention_streaming(q, kr, vr, scale);
    report("repeat_kv heads give the same decode", max_abs(std::vector<float>(sr.data(), sr.data() + sr.size()), want) <= 1e-5f);
    // causal prefill through self_attention (causal mask) and blockwise
    Tensor qp = rand_tensor(rng, {1, Hq, Lp, D}), kp = rand_tensor(rng, {1, Hkv, Lp, D}), vp = rand_tensor(rng, {1, Hkv, Lp, D});
    std::vector<float> pw(qp.size());
    or_prefill_blockwise(qp.data(), kp.data(), vp.data(), 1, (int)Hq, (int)Hkv, (int)Lp, (int)D, scale, 64, nullptr, 0,
                         pw.data());
    Tensor cm = q3::create_causal_mask(Lp).view({1, 1, Lp, Lp});
    Tensor sp = tensor_cpp::ops::self_attention(qp, kp, vp, &cm, scale);
    report("self_attention causal prefill", max_abs(std::vector<float>(sp.data(), sp.data() + sp.size()), pw) <= 1e-4f);
    Tensor bw = tensor_cpp::ops::self_attention_streaming_blockwise(qp, kp, vp, scale, 32, 64);
    report("self_attention_streaming_blockwise", max_abs(std::vector<float>(bw.data(), bw.data() + bw.size()), pw) <= 1e-4f);
    Tensor bw2 = tensor_cpp::ops::self_attention_streaming_blockwise_avx2(qp, kp, vp, scale, 128, 128);
    report("blockwise_avx2 entry point", max_abs(std::vector<float>(bw2.data(), bw2.data() + bw2.size()), pw) <= 1e-4f);
    Tensor odd(std::vector<float>(Lp * Lp, 1.0f), Shape({Lp, Lp}));
    report("arbitrary mask rejected", throws<std::invalid_argument>([&] { tensor_cpp::ops::self_attention(qp, kp, vp, &odd, scale); }));
}

static void test_rope() {
    Rng rng(17);
    const size_t D = 128, S = 40;
    auto cs = q3::compute_rope_freqs(4096, D, 1e6f);
    std::vector<float> oc(4096 * D / 2), os(4096 * D / 2);
    or_rope_tables(4096, (int)D, 1e6f, oc.data(), os.data());
    bool same = true;
    for (size_t i = 0; i < oc.size(); ++i) same &= cs.first[i] == oc[i] && cs.second[i] == os[i];
    report("compute_rope_freqs bit-exact", same);
    Tensor q = rand_tensor(rng, {1, 4, S, D}), k = rand_tensor(rng, {1, 2, S, D});
    auto r = q3::apply_rotary_pos_emb(q, k, cs.first, cs.second);
    std::vector<int> pq(4 * S), pk(2 * S);
    for (size_t i = 0; i < pq.size(); ++i) pq[i] = (int)(i % S);
    for (size_t i = 0; i < pk.size(); ++i) pk[i] = (int)(i % S);
    std::vector<float> wq(q.size()), wk(k.size());
    or_apply_rope(q.data(), (int)(4 * S), (int)D, pq.data(), oc.data(), os.data(), wq.data());
    or_apply_rope(k.data(), (int)(2 * S), (int)D, pk.data(), oc.data(), os.data(), wk.data());
    report("apply_rotary_pos_emb q", max_abs(std::vector<float>(r.first.data(), r.first.data() + q.size()), wq) <= 1e-6f);
    report("apply_rotary_pos_emb k", max_abs(std::vector<float>(r.second.data(), r.second.data() + k.size()), wk) <= 1e-6f);
}

static void test_qwen3_attention() {
    Rng rng(19);
    const size_t B = 2, Hq = 16, Hkv = 8, D = 128, P = 9, STEPS = 5, N = P + STEPS;
    const float scale = 1.0f / std::sqrt((float)D), eps = 1e-6f;
    q3::KVCache cache(1, B, Hkv, D, 64);
    Tensor wq(rng.vec(D, 0.9f, 1.1f), Shape({D})), wk(rng.vec(D, 0.9f, 1.1f), Shape({D}));
    // token streams [B][N][H][D]
    auto qa = rng.vec(B * N * Hq * D), ka = rng.vec(B * N * Hkv * D), va = rng.vec(B * N * Hkv * D);
    auto slice = [&](const std::vector<float>& src, size_t H, size_t t0, size_t n) {
        std::vector<float> out(B * n * H * D);
        for (size_t b = 0; b < B; ++b)
            std::copy(src.begin() + ((b * N + t0) * H) * D, src.begin() + ((b * N + t0 + n) * H) * D,
                      out.begin() + b * n * H * D);
        return Tensor(std::move(out), Shape({B, n, H * D}));
    };
    // oracle: normed + roped q and k at their positions, raw v
    std::vector<float> oc(64 * D / 2), os(64 * D / 2);
    or_rope_tables(64, (int)D, 1e6f, oc.data(), os.data());
    auto prep = [&](const std::vector<float>& x, size_t H, const Tensor& w) {
        std::vector<float> n(x.size()), r(x.size());
        or_rms_norm_rows(x.data(), w.data(), (int)(x.size() / D), (int)D, eps, 0, n.data());
        std::vector<int> pos(x.size() / D);
        for (size_t i = 0; i < pos.size(); ++i) pos[i] = (int)((i / H) % N);
        or_apply_rope(n.data(), (int)pos.size(), (int)D, pos.data(), oc.data(), os.data(), r.data());
        return r;   // [B][N][H][D]
    };
    auto qr = prep(qa, Hq, wq), kr = prep(ka, Hkv, wk);
    auto head_major = [&](const std::vector<float>& x, size_t H, size_t n) {   // [B][H][n][D]
        std::vector<float> out(B * H * n * D);
        for (size_t b = 0; b < B; ++b)
            for (size_t t = 0; t < n; ++t)
                for (size_t h = 0; h < H; ++h)
                    std::copy(x.begin() + ((b * N + t) * H + h) * D, x.begin() + ((b * N + t) * H + h + 1) * D,
                              out.begin() + ((b * H + h) * n + t) * D);
        return out;
    };
    // prompt
    Tensor got = q3::qwen3_attention_with_cache(slice(qa, Hq, 0, P), slice(ka, Hkv, 0, P), slice(va, Hkv, 0, P), &cache,
                                                0, Hq, Hkv, D, eps, wq, wk);
    cache.increment_seq_len(P);
    {
        auto qh = head_major(qr, Hq, P), kh = head_major(kr, Hkv, P), vh = head_major(va, Hkv, P);
        std::vector<float> want(qh.size());
        or_prefill_blockwise(qh.data(), kh.data(), vh.data(), (int)B, (int)Hq, (int)Hkv, (int)P, (int)D, scale, 64,
                             nullptr, 0, want.data());
        report("qwen3_attention_with_cache prefill",
               max_abs(std::vector<float>(got.data(), got.data() + got.size()), want) <= 1e-4f);
    }
    for (size_t t = P; t < N; ++t) {
        Tensor o = q3::qwen3_attention_with_cache(slice(qa, Hq, t, 1), slice(ka, Hkv, t, 1), slice(va, Hkv, t, 1), &cache,
                                                  0, Hq, Hkv, D, eps, wq, wk, q3::AttentionType::STREAMING);
        cache.increment_seq_len(1);
        auto kh = head_major(kr, Hkv, t + 1), vh = head_major(va, Hkv, t + 1);
        std::vector<float> qt(B * Hq * D), want(B * Hq * D);
        for (size_t b = 0; b < B; ++b)
            std::copy(qr.begin() + ((b * N + t) * Hq) * D, qr.begin() + ((b * N + t + 1) * Hq) * D, qt.begin() + b * Hq * D);
        or_decode_gqa(qt.data(), kh.data(), vh.data(), (int)B, (int)Hq, (int)Hkv, (int)(t + 1), (int)D, scale, want.data());
        report("qwen3_attention_with_cache decode step " + std::to_string(t - P),
               max_abs(std::vector<float>(o.data(), o.data() + o.size()), want) <= 1e-4f);
    }
    report("two tokens at once after the prompt rejected", throws<std::invalid_argument>([&] {
               q3::qwen3_attention_with_cache(slice(qa, Hq, 0, 2), slice(ka, Hkv, 0, 2), slice(va, Hkv, 0, 2), &cache, 0,
                                              Hq, Hkv, D, eps, wq, wk);
           }));
}

// The Tensor members of the reference's tensor.h (tensor_cpp/src/tensor.cpp):
// element-wise arithmetic, reductions, shapes, factories, and matmul (GPU)
// against a double-precision host product.
static void test_tensor() {
    Rng rng(7);
    Tensor a(rng.vec(6), Shape({2, 3})), b(rng.vec(6), Shape({2, 3}));
    bool ok = true;
    const Tensor s = a + b, d = a - b, m = a * b, q = a / b, sc = a * 2.0f + 1.0f;
    for (size_t i = 0; i < 6; ++i)
        ok = ok && s[i] == a[i] + b[i] && d[i] == a[i] - b[i] && m[i] == a[i] * b[i] && q[i] == a[i] / b[i] &&
             sc[i] == a[i] * 2.0f + 1.0f;
    report("tensor element-wise", ok);
    report("tensor shape mismatch throws", throws<std::invalid_argument>([&] { (void)(a + Tensor(Shape({3, 2}))); }));
    Tensor acc = a;
    acc += b;
    acc *= 0.5f;
    ok = true;
    for (size_t i = 0; i < 6; ++i) ok = ok && acc[i] == (a[i] + b[i]) * 0.5f;
    report("tensor in-place", ok);
    double sum = 0;
    for (size_t i = 0; i < 6; ++i) sum += a[i];
    report("tensor reductions", std::fabs(a.sum() - sum) < 1e-6 && std::fabs(a.mean() - sum / 6) < 1e-6 &&
                                    a.max() == *std::max_element(a.data(), a.data() + 6) &&
                                    a.min() == *std::min_element(a.data(), a.data() + 6));
    const Tensor t = a.transpose();
    report("tensor transpose / index", t.shape() == Shape({3, 2}) && t({2, 1}) == a({1, 2}) && t({0, 1}) == a[3]);
    const Tensor u = a.unsqueeze(0);
    report("tensor squeeze / unsqueeze", u.shape() == Shape({1, 2, 3}) && u.squeeze().shape() == Shape({2, 3}));
    const Tensor e = Tensor::eye(3, 4);
    report("tensor eye / ones", e({2, 2}) == 1.0f && e({2, 3}) == 0.0f && e.sum() == 3.0f &&
                                    Tensor::ones(Shape({2, 2})).sum() == 4.0f);
    const size_t M = 37, K = 130, N = 67;
    Tensor x(rng.vec(M * K), Shape({M, K})), w(rng.vec(K * N), Shape({K, N}));
    const Tensor y = x.matmul(w);
    double err = 0, ref_max = 0;
    for (size_t i = 0; i < M; ++i)
        for (size_t j = 0; j < N; ++j) {
            double r = 0;
            for (size_t k = 0; k < K; ++k) r += (double)x[i * K + k] * w[k * N + j];
            err = std::max(err, std::fabs(r - y[i * N + j]));
            ref_max = std::max(ref_max, std::fabs(r));
        }
    report("tensor matmul on the GPU", y.shape() == Shape({M, N}) && err <= 1e-5 * ref_max,
           "max err " + std::to_string(err));
}

int main() {
    const struct {
        const char* name;
        void (*fn)();
    } suites[] = {{"correctness", test_correctness}, {"thread variants", test_thread_variants}, {"edges", test_edges},
                  {"kv cache", test_kv_cache},       {"ops", test_ops},                       {"rope", test_rope},
                  {"qwen3 attention", test_qwen3_attention}, {"tensor", test_tensor}};
    for (const auto& s : suites) {
        std::printf("== %s\n", s.name);
        std::fflush(stdout);
        try {
            s.fn();
        } catch (const std::exception& e) {
            report(std::string(s.name) + " threw", false, e.what());
        }
    }
    std::printf("%d failure(s)\n", g_fail);
    return g_fail;
}
