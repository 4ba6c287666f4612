// benchmark_qwen3 - the reference's Qwen3 prefill / decode benchmark command
// line (reference tensor_cpp/tests/benchmark/benchmark_qwen3.cpp:43-220, main
// :1061-1155) over the MI355X library: the same options, phases and result
// lines, with every forward on the GPU through the C ABI (include/sa_qwen3.h).
//
//   benchmark_qwen3 --model model.safetensors --phase prefill --prompt-len 128 --iters 10
//   benchmark_qwen3 --model model.safetensors --phase decode --gen-len 100 --use-kv-cache
//   benchmark_qwen3 --synthetic --phase decode --batch-size 8 --gen-len 64
//   benchmark_qwen3 --model model.safetensors --compare-kv-cache --gen-len 10
//   benchmark_qwen3 --model model.safetensors --verify 151644,872,198
//
// Options the GPU path has no use for are accepted and reported: --mode,
// --method, --parallel-strategy, --attention-algo and --attention all select
// the same kernels (the online-softmax kernels are exact attention) and
// --threads sets nothing.  --q-block-size and --kv-block-size set the
// attention tiles, as the reference sets g_q_block_size / g_kv_block_size
// from them (benchmark_qwen3.cpp:1072-1073): the prefill's query rows per
// workgroup and head (32, 64 or 128) and the decode's split-KV chunk (a
// multiple of 64 tokens); unset, each launch picks its own, and the header
// prints the query tile the prefill launch takes.  --synthetic replaces --model
// with seeded random weights of the Qwen3-0.6B shape; --synthetic-shape,
// --seed and --std (not in the reference) pick another shape and draw, and
// --logits-out writes --verify's logits, so the command line can be checked
// against a host forward of the same weights.
//
// Phases, as the reference times them:
//  prefill: iters forwards of batch x prompt-len tokens (after warmup ones),
//           tokens = batch * prompt_len * iters.
//  decode with KV cache: a 16-token prompt, warmup steps, the cache reset and
//           the prompt run again, then gen-len greedy steps timed,
//           tokens = batch * gen_len.
//  decode without KV cache: from a 4-token prompt, each of gen-len steps
//           runs the whole sequence so far again.
// The result lines keep the reference's labels (总时间, 处理token数,
// 平均时间/token, 吞吐量) because its experiment scripts read them.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <iomanip>
#include <iostream>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "sa_qwen3.h"

namespace {

struct Config {
    std::string model_path;
    bool synthetic = false;
    std::string phase = "prefill";
    std::string mode = "omp", method = "baseline", parallel_strategy = "headwise";
    std::string attention_algo = "standard", attention = "standard";
    int batch_size = 1, prompt_len = 128, gen_len = 100, iters = 10, num_threads = 16, warmup = 2;
    int q_block_size = 0, kv_block_size = 0;     // 0: each launch picks its tile
    bool verbose = false, use_kv_cache = true, compare_kv_cache = false, verify_mode = false;
    bool kv_bf16 = false;
    std::vector<int> shape;                 // layers, hidden, intermediate, vocab, q heads, kv heads, head_dim
    unsigned long long seed = 42;
    float init_std = 0.02f;
    std::string logits_out;
    std::vector<int32_t> verify_tokens = {151644, 872, 198, 35127, 752, 264, 2805, 16800, 311,
                                          3460, 4128, 1614, 13, 151645, 198, 151644, 77091, 198};
};

void usage(const char* prog) {
    std::cout << "usage: " << prog << " [options]\n"
              << "  --model PATH              safetensors checkpoint (Hugging Face Qwen3 names)\n"
              << "  --synthetic               seeded random weights of the Qwen3-0.6B shape instead\n"
              << "  --phase prefill|decode    [prefill]\n"
              << "  --batch-size N            [1]\n"
              << "  --prompt-len N            prefill prompt length [128]\n"
              << "  --gen-len N               decode tokens [100]\n"
              << "  --iters N                 prefill iterations [10]\n"
              << "  --warmup N                [2]\n"
              << "  --use-kv-cache | --no-kv-cache   decode with or without the cache [with]\n"
              << "  --compare-kv-cache        decode both ways and print the speedup\n"
              << "  --verify [T1,T2,...]      prefill vs token-by-token decode on these tokens\n"
              << "  --kv-bf16                 bf16 KV cache (default fp32, as the reference)\n"
              << "  --synthetic-shape L,H,I,V,Hq,Hkv,D   shape of the synthetic model [28,1024,3072,151936,16,8,128]\n"
              << "  --seed N, --std X         synthetic draw: seed [42], N(0, X) matrices, 1 + N(0, X) norms [0.02]\n"
              << "  --logits-out PATH         --verify writes both paths' last logits there (fp32 [2][batch][vocab])\n"
              << "  --q-block-size N          prefill query rows per workgroup and head: 32, 64, 128 [auto]\n"
              << "  --kv-block-size N         decode split-KV chunk, tokens: multiple of 64 in [64, 16384] [auto]\n"
              << "  --mode, --method, --parallel-strategy, --attention-algo, --attention,\n"
              << "  --threads: accepted for compatibility\n"
              << "  --verbose, --help\n";
}

int to_int(const char* s, const char* what) {
    char* end = nullptr;
    const long v = std::strtol(s, &end, 10);
    if (!end || *end || v < 0 || v > 1 << 30) {
        std::cerr << "error: bad value for " << what << ": " << s << "\n";
        std::exit(1);
    }
    return static_cast<int>(v);
}

Config parse(int argc, char** argv) {
    Config c;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto val = [&](const char* what) -> const char* {
            if (i + 1 >= argc) {
                std::cerr << "error: " << what << " needs a value\n";
                std::exit(1);
            }
            return argv[++i];
        };
        if (a == "--model") c.model_path = val("--model");
        else if (a == "--synthetic") c.synthetic = true;
        else if (a == "--phase") c.phase = val("--phase");
        else if (a == "--mode") c.mode = val("--mode");
        else if (a == "--method") c.method = val("--method");
        else if (a == "--parallel-strategy") c.parallel_strategy = val("--parallel-strategy");
        else if (a == "--attention-algo") c.attention_algo = val("--attention-algo");
        else if (a == "--attention") c.attention = val("--attention");
        else if (a == "--batch-size") c.batch_size = to_int(val("--batch-size"), "--batch-size");
        else if (a == "--prompt-len") c.prompt_len = to_int(val("--prompt-len"), "--prompt-len");
        else if (a == "--gen-len") c.gen_len = to_int(val("--gen-len"), "--gen-len");
        else if (a == "--iters") c.iters = to_int(val("--iters"), "--iters");
        else if (a == "--threads") c.num_threads = to_int(val("--threads"), "--threads");
        else if (a == "--warmup") c.warmup = to_int(val("--warmup"), "--warmup");
        else if (a == "--q-block-size") c.q_block_size = to_int(val("--q-block-size"), "--q-block-size");
        else if (a == "--kv-block-size") c.kv_block_size = to_int(val("--kv-block-size"), "--kv-block-size");
        else if (a == "--use-kv-cache") c.use_kv_cache = true;
        else if (a == "--no-kv-cache") c.use_kv_cache = false;
        else if (a == "--compare-kv-cache") c.compare_kv_cache = true;
        else if (a == "--kv-bf16") c.kv_bf16 = true;
        else if (a == "--synthetic-shape") {
            std::stringstream ss(val("--synthetic-shape"));
            std::string t;
            while (std::getline(ss, t, ',')) c.shape.push_back(to_int(t.c_str(), "--synthetic-shape"));
            if (c.shape.size() != 7) {
                std::cerr << "error: --synthetic-shape takes 7 integers L,H,I,V,Hq,Hkv,D\n";
                std::exit(1);
            }
        } else if (a == "--seed") c.seed = (unsigned long long)to_int(val("--seed"), "--seed");
        else if (a == "--std") {
            const char* v = val("--std");
            char* end = nullptr;
            c.init_std = std::strtof(v, &end);
            if (!end || *end || !(c.init_std > 0.0f)) {
                std::cerr << "error: bad value for --std: " << v << "\n";
                std::exit(1);
            }
        } else if (a == "--logits-out") c.logits_out = val("--logits-out");
        else if (a == "--verify") {
            c.verify_mode = true;
            if (i + 1 < argc && argv[i + 1][0] != '-') {
                std::stringstream ss(argv[++i]);
                std::string t;
                c.verify_tokens.clear();
                while (std::getline(ss, t, ',')) c.verify_tokens.push_back(to_int(t.c_str(), "--verify token"));
                if (c.verify_tokens.empty()) {
                    std::cerr << "error: --verify needs at least one token id\n";
                    std::exit(1);
                }
            }
        } else if (a == "--verbose") c.verbose = true;
        else if (a == "--help") {
            usage(argv[0]);
            std::exit(0);
        } else {
            std::cerr << "unknown option: " << a << "\n";
            usage(argv[0]);
            std::exit(1);
        }
    }
    if (c.attention == "streaming") c.attention_algo = "online_softmax";
    if (c.batch_size < 1 || c.batch_size > 1024) {
        std::cerr << "error: --batch-size must be in [1, 1024]\n";
        std::exit(1);
    }
    if (c.prompt_len < 1 || c.gen_len < 1 || c.iters < 1) {
        std::cerr << "error: --prompt-len, --gen-len and --iters must be at least 1\n";
        std::exit(1);
    }
    // The tiles are process-wide settings of the library (host state only).
    if (sa_set_attention_blocks(c.q_block_size, c.kv_block_size) != SA_OK) {
        std::cerr << "error: --q-block-size " << c.q_block_size << " / --kv-block-size " << c.kv_block_size
                  << ": " << sa_last_error() << "\n";
        std::exit(1);
    }
    return c;
}

void check(sa_status s, const char* what) {
    if (s != SA_OK) throw std::runtime_error(std::string(what) + ": " + sa_last_error());
}
void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Device buffers freed at scope exit.
template <class T>
struct DevBuf {
    T* p = nullptr;
    explicit DevBuf(size_t n) { hip_check(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)), "hipMalloc"); }
    ~DevBuf() { (void)hipFree(p); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
};

struct Runner {
    const Config& cfg;
    sa_qwen3_desc desc{};
    sa_qwen3* model = nullptr;
    sa_kvcache* cache = nullptr;
    int max_tokens = 0;

    Runner(const Config& c, int max_tokens_) : cfg(c), max_tokens(max_tokens_) {
        if (c.synthetic && !c.shape.empty()) {
            const auto& s = c.shape;
            desc = sa_qwen3_desc{s[0], s[1], s[2], s[3], s[4], s[5], s[6], 0, 1e-6f, 1e6f};
        } else if (c.synthetic) {
            desc = sa_qwen3_desc{28, 1024, 3072, 151936, 16, 8, 128, 0, 1e-6f, 1e6f};
        } else {
            if (c.model_path.empty()) throw std::runtime_error("--model PATH or --synthetic is required");
            check(sa_qwen3_desc_from_safetensors(c.model_path.c_str(), &desc), "reading the checkpoint header");
        }
        desc.max_pos = max_tokens + 1;
        check(sa_qwen3_create(&desc, c.batch_size, &model), "sa_qwen3_create");
        if (c.synthetic) {
            check(sa_qwen3_init_random(model, c.seed, c.init_std, nullptr), "sa_qwen3_init_random");
        } else {
            check(sa_qwen3_load_safetensors(model, c.model_path.c_str()), "loading the checkpoint");
        }
        const int pages = (max_tokens + 1 + 63) / 64;
        sa_kv_desc kd{desc.num_layers, desc.n_kv_heads, desc.head_dim, c.batch_size, pages, pages * c.batch_size,
                      c.kv_bf16 ? SA_DTYPE_BF16 : SA_DTYPE_F32};
        check(sa_kvcache_create(&kd, &cache), "sa_kvcache_create");
        hip_check(hipDeviceSynchronize(), "loading");
    }
    ~Runner() {
        if (cache) sa_kvcache_destroy(cache);
        if (model) sa_qwen3_destroy(model);
    }

    void reset(int tokens) {
        check(sa_kvcache_reset(cache, nullptr), "sa_kvcache_reset");
        for (int s = 0; s < cfg.batch_size; ++s) check(sa_kvcache_reserve(cache, s, tokens, nullptr), "sa_kvcache_reserve");
    }
    // Prefill prompt [L] replicated over the batch; returns the next token of sequence 0.
    int32_t prefill(const std::vector<int32_t>& prompt, float* logits = nullptr) {
        const int B = cfg.batch_size, L = static_cast<int>(prompt.size());
        std::vector<int32_t> h((size_t)B * L);
        for (int b = 0; b < B; ++b) std::copy(prompt.begin(), prompt.end(), h.begin() + (size_t)b * L);
        DevBuf<int32_t> d_tok(h.size()), d_next(B);
        hip_check(hipMemcpy(d_tok.p, h.data(), h.size() * sizeof(int32_t), hipMemcpyHostToDevice), "tokens");
        check(sa_qwen3_prefill(model, cache, d_tok.p, B, L, d_next.p, logits, nullptr), "sa_qwen3_prefill");
        int32_t next = 0;
        hip_check(hipMemcpy(&next, d_next.p, sizeof(int32_t), hipMemcpyDeviceToHost), "next token");
        return next;
    }
    // One decode step feeding token to every sequence; returns sequence 0's next token.
    int32_t step(int32_t token, int32_t* d_tok, int32_t* d_next, float* logits = nullptr) {
        std::vector<int32_t> h(cfg.batch_size, token);
        hip_check(hipMemcpy(d_tok, h.data(), h.size() * sizeof(int32_t), hipMemcpyHostToDevice), "token");
        check(sa_qwen3_decode_step(model, cache, d_tok, cfg.batch_size, d_next, logits, nullptr), "decode step");
        int32_t next = 0;
        hip_check(hipMemcpy(&next, d_next, sizeof(int32_t), hipMemcpyDeviceToHost), "next token");
        return next;
    }
};

using Clock = std::chrono::steady_clock;
double ms_since(Clock::time_point t0) { return std::chrono::duration<double, std::milli>(Clock::now() - t0).count(); }

std::vector<int32_t> random_tokens(int n, int vocab) {
    std::mt19937 gen(42);
    std::vector<int32_t> t(n);
    for (auto& x : t) x = static_cast<int32_t>(gen() % static_cast<uint32_t>(vocab));
    return t;
}

double bench_prefill(Runner& r) {
    const auto prompt = random_tokens(r.cfg.prompt_len, r.desc.vocab);
    for (int i = 0; i < r.cfg.warmup; ++i) {
        r.reset(r.cfg.prompt_len);
        r.prefill(prompt);
    }
    double total = 0.0;
    for (int i = 0; i < r.cfg.iters; ++i) {
        r.reset(r.cfg.prompt_len);
        hip_check(hipDeviceSynchronize(), "sync");
        const auto t0 = Clock::now();
        r.prefill(prompt);
        hip_check(hipDeviceSynchronize(), "sync");
        total += ms_since(t0);
    }
    return total;
}

double bench_decode_cache(Runner& r) {
    const auto prompt = random_tokens(16, r.desc.vocab);
    DevBuf<int32_t> d_tok(r.cfg.batch_size), d_next(r.cfg.batch_size);
    r.reset(16 + std::max(r.cfg.warmup, r.cfg.gen_len));
    int32_t next = r.prefill(prompt);
    for (int i = 0; i < r.cfg.warmup; ++i) next = r.step(next, d_tok.p, d_next.p);
    r.reset(16 + r.cfg.gen_len);
    next = r.prefill(prompt);
    hip_check(hipDeviceSynchronize(), "sync");
    const auto t0 = Clock::now();
    for (int s = 0; s < r.cfg.gen_len; ++s) next = r.step(next, d_tok.p, d_next.p);
    hip_check(hipDeviceSynchronize(), "sync");
    return ms_since(t0);
}

double bench_decode_no_cache(Runner& r) {
    auto seq = random_tokens(4, r.desc.vocab);
    r.reset((int)seq.size());
    seq.push_back(r.prefill(seq));
    hip_check(hipDeviceSynchronize(), "sync");
    const auto t0 = Clock::now();
    for (int s = 0; s < r.cfg.gen_len; ++s) {
        r.reset((int)seq.size());
        seq.push_back(r.prefill(seq));
    }
    hip_check(hipDeviceSynchronize(), "sync");
    return ms_since(t0);
}

std::string block_name(int b) { return b ? std::to_string(b) : std::string("auto"); }

// The query tile the model's prefill attention (fp32, token-major q/k/v)
// takes for this benchmark's shape.
int prefill_tile(const Config& c, const Runner& r) {
    const int L = c.phase == "prefill" ? c.prompt_len : 16;
    return sa_prefill_query_tile(SA_DTYPE_F32, c.batch_size, r.desc.n_q_heads, r.desc.n_kv_heads, L,
                                 r.desc.head_dim);
}

void print_header(const Config& c, const Runner& r) {
    std::cout << "\n==================================================\n"
              << "         Qwen3 Performance Benchmark (MI355X)\n"
              << "==================================================\n"
              << "model:           "
              << (c.synthetic ? "synthetic (seed " + std::to_string(c.seed) + ", N(0, " + std::to_string(c.init_std) + "))"
                              : c.model_path)
              << "\n"
              << "phase:           " << c.phase << "\n"
              << "method:          " << c.method << " / " << c.attention_algo << " (one GPU path for all)\n";
    if (c.phase == "prefill")
        std::cout << "prompt length:   " << c.prompt_len << "\n";
    else
        std::cout << "gen length:      " << c.gen_len << "\nKV cache:        " << (c.use_kv_cache ? "yes" : "no")
                  << "\n";
    std::cout << "batch size:      " << c.batch_size << "\n"
              << "iterations:      " << c.iters << "\n"
              << "KV cache dtype:  " << (c.kv_bf16 ? "bf16" : "fp32") << "\n"
              << "block sizes:     q " << block_name(c.q_block_size) << ", kv " << block_name(c.kv_block_size) << "\n"
              << "attention tiles: prefill " << prefill_tile(c, r) << " queries per workgroup and head, 64-key tiles; "
              << "decode split-KV chunk "
              << (c.kv_block_size ? std::to_string(c.kv_block_size) + " tokens" : std::string("per launch"))
              << "\n"
              << "model config:    layers " << r.desc.num_layers << ", heads " << r.desc.n_q_heads << "/"
              << r.desc.n_kv_heads << " x " << r.desc.head_dim << ", hidden " << r.desc.hidden << ", vocab "
              << r.desc.vocab << "\n"
              << "==================================================\n\n";
}

void print_results(double total_ms, int n_tokens) {
    std::cout << "\n==================================================\n"
              << "              Benchmark Results\n"
              << "==================================================\n"
              << "总时间:         " << std::fixed << std::setprecision(2) << total_ms << " ms\n"
              << "处理token数:    " << n_tokens << "\n"
              << "平均时间/token: " << std::fixed << std::setprecision(4) << total_ms / n_tokens << " ms\n"
              << "吞吐量:         " << std::fixed << std::setprecision(2) << n_tokens * 1000.0 / total_ms
              << " tokens/sec\n"
              << "==================================================\n\n";
}

// Last-position logits of the verify tokens two ways: one prefill of the whole
// sequence, and a one-token prefill followed by decode steps.
int verify(Runner& r) {
    const auto& toks = r.cfg.verify_tokens;
    for (int32_t t : toks)
        if (t < 0 || t >= r.desc.vocab) throw std::runtime_error("verify token outside the vocabulary");
    const int V = r.desc.vocab, B = r.cfg.batch_size, n = static_cast<int>(toks.size());
    DevBuf<float> la((size_t)B * V), lb((size_t)B * V);
    DevBuf<int32_t> d_tok(B), d_next(B);
    r.reset(n);
    const int32_t next_a = r.prefill(toks, la.p);
    r.reset(n);
    int32_t next_b = r.prefill(std::vector<int32_t>(toks.begin(), toks.begin() + 1), n == 1 ? lb.p : nullptr);
    for (int i = 1; i < n; ++i) next_b = r.step(toks[i], d_tok.p, d_next.p, i + 1 == n ? lb.p : nullptr);
    std::vector<float> a((size_t)B * V), b((size_t)B * V);
    hip_check(hipMemcpy(a.data(), la.p, a.size() * sizeof(float), hipMemcpyDeviceToHost), "logits");
    hip_check(hipMemcpy(b.data(), lb.p, b.size() * sizeof(float), hipMemcpyDeviceToHost), "logits");
    float max_diff = 0.f, max_rel = 0.f;
    for (size_t i = 0; i < a.size(); ++i) {
        const float d = std::fabs(a[i] - b[i]);
        max_diff = std::max(max_diff, d);
        const float m = std::max(std::fabs(a[i]), std::fabs(b[i]));
        max_rel = std::max(max_rel, m > 1e-6f ? d / m : d);
    }
    std::cout << "verify: " << n << " tokens, batch " << B << ", block sizes q " << block_name(r.cfg.q_block_size)
              << ", kv " << block_name(r.cfg.kv_block_size) << "\n"
              << "  prefill of the whole sequence -> next token " << next_a << "\n"
              << "  prefill of 1 + " << n - 1 << " decode steps   -> next token " << next_b << "\n"
              << "  last-position logits: max abs diff " << max_diff << ", max rel diff " << max_rel * 100.f
              << "%\n";
    if (!r.cfg.logits_out.empty()) {
        FILE* f = std::fopen(r.cfg.logits_out.c_str(), "wb");
        if (!f) throw std::runtime_error("cannot write " + r.cfg.logits_out);
        const bool wrote = std::fwrite(a.data(), sizeof(float), a.size(), f) == a.size() &&
                           std::fwrite(b.data(), sizeof(float), b.size(), f) == b.size();
        if (std::fclose(f) != 0 || !wrote) throw std::runtime_error("cannot write " + r.cfg.logits_out);
    }
    const bool ok = next_a == next_b && max_diff <= 1e-3f;
    std::cout << "  result: " << (ok ? "MATCH" : "MISMATCH") << "\n";
    return ok ? 0 : 2;
}

}  // namespace

int main(int argc, char** argv) {
    const Config cfg = parse(argc, argv);
    try {
        int max_tokens = cfg.prompt_len;
        if (cfg.phase == "decode" || cfg.compare_kv_cache)
            max_tokens = std::max(max_tokens, 16 + std::max(cfg.gen_len, cfg.warmup) + 1);
        if (cfg.verify_mode) max_tokens = std::max<int>(max_tokens, (int)cfg.verify_tokens.size());
        std::cout << "\nloading model...\n";
        Runner r(cfg, max_tokens);
        if (cfg.verify_mode) return verify(r);
        if (cfg.compare_kv_cache) {
            const double without = bench_decode_no_cache(r);
            const double with = bench_decode_cache(r);
            std::cout << "decode " << cfg.gen_len << " tokens: without KV cache " << without << " ms, with "
                      << with << " ms, speedup " << std::setprecision(2) << without / with << "x\n";
            return 0;
        }
        print_header(cfg, r);
        double total = 0.0;
        int n_tokens = 0;
        if (cfg.phase == "prefill") {
            std::cout << "running the prefill benchmark...\n";
            n_tokens = cfg.batch_size * cfg.prompt_len * cfg.iters;
            total = bench_prefill(r);
        } else if (cfg.phase == "decode") {
            std::cout << "running the decode benchmark...\n";
            n_tokens = cfg.batch_size * cfg.gen_len;
            total = cfg.use_kv_cache ? bench_decode_cache(r) : bench_decode_no_cache(r);
        } else {
            std::cerr << "error: unknown phase '" << cfg.phase << "' (prefill, decode)\n";
            return 1;
        }
        print_results(total, n_tokens);
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << "\n";
        return 1;
    }
}
