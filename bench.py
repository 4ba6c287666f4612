"""Benchmark of the streaming-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only headline|all]

Headline (`value`): single-query streaming attention over a long context,
T = 262144 tokens, d = 128, fp32 (0.5 N(0,1) with 1% of K rows x8), as HBM
GB/s of algorithmic traffic (K and V read once, Q read, O written).  Inputs
are resident in HBM before the timed region; K/V are rotated over replicas
whose footprint exceeds the 256 MB Infinity Cache, so every call streams from
HBM.  A step is a batch of CALLS_PER_STEP back-to-back calls of the library
(each a split-KV launch and its merge) over the replicas in turn, so even
--steps 20 times a steady stream of calls rather than the first call's
submission latency.

`roofline` is computed for that kernel from its average duration measured
with HIP events on the launch stream.  `cpu_baseline` times the reference's
streaming_attention_omp (compiled from its own sources into oracle/_ref, or
the oracle's restatement when that is absent) on this host's cores over a
bounded sample of the same workload.  `extra` carries the other measured
configurations (single-head T=1024, one-layer Qwen3 decode loop, causal
prefill, batched paged decode, the 28-layer decode step) with their own
roofline fractions, and each with the reference's own CPU path timed on this
host beside it (the decoder layer, the AVX2 blockwise prefill).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBS = 8000.0
CALLS_PER_STEP = 25      # one headline step: 25 calls, 5 rounds over the 5 replicas
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
METRIC = "decode attn HBM GB/s (% of peak); prefill TFLOP/s; Qwen3-0.6B-shape tok/s"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


PROFILE_SUMMARY = ROOT / "profiles" / "split_kv_decode_T262144_d128_f32.md"


def profiled_traffic(T: int):
    """HBM bytes per launch of the headline kernel from the committed
    rocprofv3 counter summary (FETCH_SIZE and WRITE_SIZE, calibrated against a
    plain copy), when it covers this workload; otherwise None."""
    if T != 262144 or not PROFILE_SUMMARY.exists():
        return None
    for line in PROFILE_SUMMARY.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch"):
            return int(line.split("=")[1])
    return None


def load_pkg():
    from util import load_pkg as lp, load_synth
    return lp(), load_synth()


def time_launches(torch, fn, steps: int, warmup: int):
    """Run fn(i) warmup + steps times; return (per-launch ms from HIP events on
    the current stream, wall ms per step between two synchronisations)."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        starts[i].record()
        fn(warmup + i)
        ends[i].record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    per = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return per, wall


def time_batch(torch, fn, steps: int, warmup: int, warm_s: float = 0.0):
    """Run fn(i) warmup times (and for warm_s more seconds, synchronising every
    64 calls), then time steps calls enqueued back to back: return (ms per call
    from two HIP events around the batch on the current stream, wall ms per
    call between two synchronisations)."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t_end = time.perf_counter() + warm_s
    i = warmup
    while time.perf_counter() < t_end:
        for _ in range(64):
            fn(i)
            i += 1
        torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for j in range(steps):
        fn(warmup + j)
    end.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return start.elapsed_time(end) / steps, wall


# ---------------------------------------------------------------- headline

def bench_stream(torch, sa, synth, T: int, steps: int, warmup: int, min_footprint: float = 1.1e9,
                 calls_per_step: int = 1, graph: bool = False):
    log(f"[bench] single-head streaming attention T={T} d=128 fp32: generating inputs")
    Q, K, V = synth.stream_inputs(T, 128, seed=2, scale=0.5, outlier_frac=0.01)
    per_rep = K.nbytes + V.nbytes
    n_rep = max(1, int(np.ceil(min_footprint / per_rep)))
    dQ = torch.from_numpy(Q).cuda()
    reps = []
    dK0, dV0 = torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda()
    for _ in range(n_rep):
        reps.append((dK0.clone(), dV0.clone()))
    del dK0, dV0
    out = torch.empty(128, device="cuda")
    ws = torch.zeros(max(sa.lib().sa_stream_attn_ws_bytes(T, 128), 1), dtype=torch.uint8, device="cuda")

    # A serving caller holds device pointers and calls the C ABI directly; the
    # arguments of each replica are bound once, outside the timed region.
    call = sa.lib().sa_stream_attn_f32
    stream = torch.cuda.current_stream().cuda_stream
    bound = [(dQ.data_ptr(), k.data_ptr(), v.data_ptr(), T, 128, 128, 1.0, out.data_ptr(), ws.data_ptr(),
              ws.numel(), stream) for k, v in reps]

    def one_call(i):
        sa.check(call(*bound[i % n_rep]))

    n_calls = steps * calls_per_step
    kern_ms, wall = time_batch(torch, one_call, n_calls, warmup * calls_per_step, warm_s=0.5)
    bytes_per = bytes_per_call(T)
    got = out.cpu().numpy()
    graph_res = {}
    if graph:
        # A short call's kernels finish before the ctypes call that launches
        # them returns; one call per replica replayed from a HIP graph gives
        # the device-side time per call (every replica once per replay, so the
        # footprint stays above the caches).
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cap = torch.cuda.current_stream().cuda_stream
            for b in bound:
                sa.check(call(*b[:-1], cap))
        g.replay()
        torch.cuda.synchronize()
        g_per, _ = time_launches(torch, lambda i: g.replay(), 20, 2)
        g_ms = statistics.mean(g_per) / n_rep
        del g
        graph_res = {"graph_kernel_ms": g_ms, "graph_gbs": bytes_per_call(T) / (g_ms * 1e-3) / 1e9,
                     "graph_equals_eager": bool(np.array_equal(out.cpu().numpy(), got))}
    from oracle import Oracle
    want = Oracle().streaming_serial(Q, K, V, 128)
    err = float(np.abs(got - want).max())
    rl2 = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    del reps
    torch.cuda.empty_cache()
    return {"T": T, "bytes_per_launch": bytes_per, "kernel_ms": kern_ms, "wall_ms_per_call": wall,
            "wall_ms_per_step": wall * calls_per_step, "calls_per_step": calls_per_step,
            "gbs": bytes_per / (kern_ms * 1e-3) / 1e9, "wall_gbs": bytes_per / (wall * 1e-3) / 1e9,
            "replicas": n_rep, "max_abs_err": err, "rel_l2_err": rl2, "gpu_out": got, **graph_res}, (Q, K, V)


def bytes_per_call(T: int) -> int:
    """Bytes one single-query call must move: K and V, q in, out."""
    return (2 * T * 128 + 2 * 128) * 4


def graph_fields(c: dict) -> dict:
    """The graph-replayed timing of a bench_stream result, rounded."""
    return {"graph_kernel_ms": round(c["graph_kernel_ms"], 5), "graph_gbs": round(c["graph_gbs"], 1),
            "graph_hbm_frac": round(c["graph_gbs"] / HBM_PEAK_GBS, 4),
            "graph_equals_eager": c["graph_equals_eager"]}


def fp64_errors(Q, K, V, gpu_out):
    """Config-2 errors against fp64 brute force: the GPU output, and the
    reference's own streaming_attention_serial (block 128) when its build is
    present (relative L2 and max-abs, as compute_l2_error / compute_max_error
    define them)."""
    from oracle import Oracle, Reference
    exact = Oracle().sdpa_f64(Q[None], K, V, 1.0)[0]

    def errs(x):
        d = np.asarray(x, np.float64) - exact
        return {"rel_l2_err": float(np.linalg.norm(d) / np.linalg.norm(exact)), "max_abs_err": float(np.abs(d).max())}

    res = {"gpu_vs_fp64": errs(gpu_out)}
    if Reference.available():
        res["reference_vs_fp64"] = errs(Reference().streaming_serial(Q, K, V, 128))
    return res


def host_cpu() -> dict:
    """The host the CPU baselines run on: model, sockets x cores x threads as
    lscpu reports them, the CPUs this process may use, and the OpenMP thread
    count the baselines run with."""
    info = {}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = dict(line.split(":", 1) for line in out.splitlines() if ":" in line)
        kv = {k.strip(): v.strip() for k, v in kv.items()}
        info = {"model": kv.get("Model name"), "sockets": int(kv.get("Socket(s)", 0) or 0),
                "cores_per_socket": int(kv.get("Core(s) per socket", 0) or 0),
                "threads_per_core": int(kv.get("Thread(s) per core", 0) or 0),
                "logical_cpus": int(kv.get("CPU(s)", 0) or 0)}
    except Exception as e:      # lscpu absent: report what Python knows
        info = {"model": None, "error": str(e)}
    try:
        info["cpus_allowed"] = len(os.sched_getaffinity(0))
    except AttributeError:
        info["cpus_allowed"] = os.cpu_count()
    info["omp_threads"] = _cpu_threads()
    return info


def cpu_baseline(Q, K, V, budget_s: float = 10.0):
    """The reference's streaming_attention_omp on this host, bounded sample."""
    from oracle import Oracle, Reference
    threads = _cpu_threads()
    if Reference.available():
        impl, kind = Reference(), "reference"
    else:
        impl, kind = Oracle(), "port"
    T = K.shape[0]
    for _ in range(2):
        impl.streaming_omp(Q, K, V, 128, threads)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        impl.streaming_omp(Q, K, V, 128, threads)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    gbs = (2 * T * 128 + 2 * 128) * 4 / med / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": kind,
            "sample": f"streaming_attention_omp, T={T}, d=128, block 128, {len(times)} timed calls "
                      f"(median {med * 1e3:.2f} ms) after 2 warmups, {threads} OpenMP threads",
            "host": host_cpu()}


def _cpu_threads() -> int:
    """OpenMP threads for the CPU baselines: OMP_NUM_THREADS when set (the
    process's CPU share on a shared host), else every CPU this process may
    use."""
    omp = os.environ.get("OMP_NUM_THREADS")
    if omp and omp.isdigit():
        return int(omp)
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_layer_decode(steps: int = 100, warm: int = 2):
    """The one-layer decode loop on the CPU: the reference's qwen3_decoder_layer_avx_with_cache
    (STREAMING) for 100 one-token steps after a 128-token cache, 16/8 heads,
    D=128.  Hidden size and MLP width are 8, so the projections are negligible
    and the call is the attention path: q/k norm, RoPE, the cache read + concat
    + update, repeat_kv and self_attention_streaming."""
    from oracle import Reference
    threads = _cpu_threads()
    secs = Reference().time_decode_layer(8, 8, 16, 8, 128, 1, 128 - warm, steps + warm, threads)[warm:]
    total = float(secs.sum())
    return {"value": round(steps / total, 1), "unit": "steps/s", "cores": threads, "kind": "reference", "host": host_cpu(),
            "sample": f"qwen3_decoder_layer_avx_with_cache STREAMING, hidden 8, {steps} steps over "
                      f"cached lengths 128..{127 + steps} after {warm} warmup steps; median "
                      f"{float(np.median(secs)) * 1e6:.0f} us/step"}


def cpu_prefill(L: int):
    """Causal prefill on the CPU: the reference's
    self_attention_streaming_blockwise_avx2 with q and kv blocks of 128 (the
    benchmark's setting), 16 heads over repeat_kv'd K/V, fp32."""
    from oracle import Reference
    threads = _cpu_threads()
    ref = Reference()
    ref.set_threads(threads)
    HQ, D = 16, 128
    rng = np.random.default_rng(61)       # timing inputs only: N(0,1), results unchecked
    q, k, v = (rng.standard_normal((1, HQ, L, D), dtype=np.float32) for _ in range(3))
    sc = float(1 / np.sqrt(D))
    # 2 warmups and the median of 10 timed calls (the reference benchmark's
    # defaults) up to L = 2048; at longer prompts one call takes seconds, so
    # 1 warmup and the median of 3.
    warm, reps = (2, 10) if L <= 2048 else (1, 3)
    for _ in range(warm):
        ref.blockwise(q, k, v, sc, 128, 128, 1)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        ref.blockwise(q, k, v, sc, 128, 128, 1)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    tf = 2.0 * HQ * D * L * (L + 1) / med / 1e12
    return {"value": round(tf, 4), "unit": "TFLOP/s", "cores": threads, "kind": "reference", "host": host_cpu(),
            "sample": f"self_attention_streaming_blockwise_avx2, L={L}, 16 heads, blocks 128/128, "
                      f"{warm} warmup call(s), median of {reps} timed calls: {med:.4f} s"}


def cpu_prefill_sequence(L: int):
    """Causal prefill on the CPU along the reference's `mpi+avx2
    --parallel-strategy sequence` path at one rank: the oracle's restatement of
    attention_sequence_online_softmax_avx2's loop (AVX2/FMA, one thread: the
    reference's OpenMP loop runs over the batch of 1).  Timing only: that path's
    numerics are wrong (its weights multiply s_j v_j), so nothing is checked."""
    from oracle import Oracle
    oracle = Oracle()
    HQ, HKV, D = 16, 8, 128
    rng = np.random.default_rng(61)       # timing inputs only: N(0,1), results unchecked
    q = rng.standard_normal((1, HQ, L, D), dtype=np.float32)
    k, v = (rng.standard_normal((1, HKV, L, D), dtype=np.float32) for _ in range(2))
    sc = float(1 / np.sqrt(D))
    # Every head does the same work, so above L = 1024 one head of the 16 is
    # timed and the call time scaled by 16 (a few seconds of CPU per call).
    heads = HQ if L <= 1024 else 1
    warm, reps = (2, 10) if L <= 1024 else (1, 3)
    for _ in range(warm):
        oracle.sequence_np1(q, k, v, sc, heads=(0, heads))
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        oracle.sequence_np1(q, k, v, sc, heads=(0, heads))
        times.append(time.perf_counter() - t0)
    med = statistics.median(times) * HQ / heads
    tf = 2.0 * HQ * D * L * (L + 1) / med / 1e12
    return {"value": round(tf, 5), "unit": "TFLOP/s", "cores": 1, "kind": "port", "host": host_cpu(),
            "sample": f"np=1 sequence-parallel online-softmax loop (mpi+avx2 --parallel-strategy sequence), "
                      f"L={L}, {heads} of 16 heads timed, {warm} warmup call(s), median of {reps} timed calls, "
                      f"scaled to 16 heads: {med:.4f} s per call; timing only (the path's numerics are wrong)"}


def cpu_model_decode(sum_len: int, B: int = 64, layers: int = 28, steps: int = 3):
    """The 28-layer batched decode on the CPU, extrapolated: one reference decoder layer
    (qwen3_decoder_layer_avx_with_cache, STREAMING, Qwen3-0.6B shapes) on one
    sequence at the batch's mean context length, times 28 layers.  The
    reference's cache has one length for the whole batch, so the batch of
    ragged sequences is priced as B such calls per layer.  Embedding, final
    norm and lm_head are left out, which favours the CPU."""
    from oracle import Reference
    threads = _cpu_threads()
    L = sum_len // B
    secs = Reference().time_decode_layer(1024, 3072, 16, 8, 128, 1, L, steps + 1, threads)[1:]
    med = float(np.median(secs))
    return {"value": round(1.0 / (layers * med), 4), "unit": "tok/s", "cores": threads, "kind": "reference",
            "host": host_cpu(),
            "sample": f"qwen3_decoder_layer_avx_with_cache STREAMING at hidden 1024, one sequence of "
                      f"{L} cached tokens (the mean of the batch), {steps} timed calls after 1 warmup, "
                      f"median {med * 1e3:.1f} ms per layer; tok/s = 1 / (28 x that), lm_head excluded"}


# ---------------------------------------------------------------- extra configs

def bench_layer_decode_loop(torch, sa, synth, steps_timed: int = 3):
    """One layer, B=1, 16 q / 8 KV heads, D=128: 128-token prompt, 100 decode
    steps, each q/k norm + RoPE + append, paged decode and commit: one
    sa_append_decode call (a single kernel launch while the sequence fits one
    chunk), and, under "three_calls", as sa_qknorm_rope_append +
    sa_paged_decode + sa_kvcache_commit.  Eager: every step's launches issued
    from the host.  Graph: the 100 steps captured once into a HIP graph (each
    step's launch parameters are the ones the eager loop uses) and replayed
    from the 128-token cache; every replay's per-step outputs must equal the
    eager ones bit for bit."""
    res = {}
    for name, dt in (("fp32", sa.SA_DTYPE_F32), ("bf16", sa.SA_DTYPE_BF16)):
        res[name] = _layer_decode_loop(torch, sa, synth, dt, True, steps_timed)
        res[name]["three_calls"] = _layer_decode_loop(torch, sa, synth, dt, False, steps_timed)
    return res


def _layer_decode_loop(torch, sa, synth, dt, fused: bool, steps_timed: int):
    HQ, HKV, D, P, N = 16, 8, 128, 128, 100
    cache = sa.KVCache(1, HKV, D, 1, 4, 4, dt)
    cos, sin = sa.rope_tables(P + N, D, 1e6)
    wq = torch.from_numpy(1 + synth.normal(40, 1, D, 0.02)).cuda()
    wk = torch.from_numpy(1 + synth.normal(40, 2, D, 0.02)).cuda()
    q = torch.from_numpy(synth.normal(40, 5, (N, 1, 1, HQ, D))).cuda()
    k = torch.from_numpy(synth.normal(40, 6, (N, 1, 1, HKV, D))).cuda()
    v = torch.from_numpy(synth.normal(40, 7, (N, 1, 1, HKV, D))).cuda()
    kp = torch.from_numpy(synth.normal(40, 3, (1, P, HKV, D))).cuda()
    vp = torch.from_numpy(synth.normal(40, 4, (1, P, HKV, D))).cuda()
    ws = torch.zeros(max(cache.decode_ws_bytes(1, HQ), 1), dtype=torch.uint8, device="cuda")
    outs_e = torch.empty(N, 1, HQ, D, device="cuda")
    outs_g = torch.empty(N, 1, HQ, D, device="cuda")
    qo = torch.empty(1, 1, HQ, D, device="cuda")
    sc = float(1 / np.sqrt(D))

    def prompt():
        cache.reset()
        cache.reserve(0, P + N)
        cache.append(0, None, kp, vp, None, wk, 1e-6, rope=(cos, sin))
        cache.commit(P, n_seqs=1)

    def steps(outs):
        for t in range(N):
            if fused:
                cache.append_decode(0, q[t].view(1, HQ, D), k[t].view(1, HKV, D), v[t].view(1, HKV, D), sc,
                                    wq, wk, 1e-6, rope=(cos, sin), out=outs[t], ws=ws, commit=True)
            else:
                cache.append(0, q[t], k[t], v[t], wq, wk, 1e-6, rope=(cos, sin), q_out=qo)
                cache.decode(0, qo.view(1, HQ, D), sc, n_pending=1, out=outs[t], ws=ws)
                cache.commit(1, n_seqs=1)

    walls = []
    for rep in range(steps_timed + 1):
        prompt()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        steps(outs_e)
        torch.cuda.synchronize()
        if rep:
            walls.append(time.perf_counter() - t0)
    wall = statistics.median(walls)

    prompt()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        steps(outs_g)
    g_walls, exact = [], True
    for rep in range(steps_timed + 1):
        outs_g.zero_()
        cache.set_len(0, P)          # the captured steps start from the prompt
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        graph.replay()
        torch.cuda.synchronize()
        if rep:
            g_walls.append(time.perf_counter() - t0)
        exact = exact and bool(torch.equal(outs_g, outs_e))
    del graph
    cache.close()
    g_wall = statistics.median(g_walls)
    kv_bytes = sum(HKV * (P + t + 1) * D * 2 * (4 if dt == sa.SA_DTYPE_F32 else 2) for t in range(N))
    return {"steps_per_s": round(N / wall, 1), "us_per_step": round(wall / N * 1e6, 2),
            "graph_steps_per_s": round(N / g_wall, 1), "graph_us_per_step": round(g_wall / N * 1e6, 2),
            "graph_equals_eager": exact,
            "kv_read_bytes_100_steps": kv_bytes,
            "hbm_frac": round(kv_bytes / g_wall / 1e9 / HBM_PEAK_GBS, 5)}


def batch_lengths(synth, B: int = 64, lo: int = 512, hi: int = 32768, seed: int = 70):
    """Per-sequence context lengths ~ U[lo, hi] (seeded)."""
    return synth.batch_lengths(B, lo, hi, seed)


def bench_paged_batch(torch, sa, synth, steps: int = 10, bf16: bool = True):
    """Batched paged GQA decode, one layer: B=64 sequences, lengths U[512, 32768],
    16 q / 8 KV heads, D=128, 64-token pages assigned from a seeded shuffle of
    the pool, KV synthesised as N(0,1) (no prefill run)."""
    HQ, HKV, D, B = 16, 8, 128, 64
    lens = batch_lengths(synth, B)
    pages_per = [(L + 1 + 63) // 64 for L in lens]            # room for the step's new token
    n_pages = sum(pages_per)
    max_pages = max(pages_per)
    cache = sa.KVCache(1, HKV, D, B, max_pages, n_pages, sa.SA_DTYPE_BF16 if bf16 else sa.SA_DTYPE_F32)
    perm = synth.permutation(70, 2, n_pages)
    off = 0
    gen = torch.Generator(device="cuda")
    gen.manual_seed(70)
    for s, L in enumerate(lens):
        cache.set_pages(s, perm[off:off + pages_per[s]])
        off += pages_per[s]
        ids = [s]
        for t0 in range(0, L, 4096):
            n = min(4096, L - t0)
            k = torch.randn(1, n, HKV, D, device="cuda", generator=gen)
            v = torch.randn(1, n, HKV, D, device="cuda", generator=gen)
            cache.append(0, None, k, v, seq_ids=ids)
            cache.commit(n, seqs=[s])
    torch.cuda.synchronize()
    q = torch.randn(B, HQ, D, device="cuda", generator=gen)
    out = torch.empty_like(q)
    ws = torch.zeros(max(cache.decode_ws_bytes(B, HQ), 1), dtype=torch.uint8, device="cuda")
    sc = float(1 / np.sqrt(D))
    per, _ = time_launches(torch, lambda i: cache.decode(0, q, sc, out=out, ws=ws), steps, 3)
    ms = statistics.mean(per)
    elem = 2 if bf16 else 4
    kv_bytes = sum(lens) * HKV * D * 2 * elem
    total = kv_bytes + 2 * B * HQ * D * 4
    # Outside the timed region: the last timed call's output for the shortest,
    # the longest and 8 seeded random sequences against the oracle's STANDARD
    # decode on the K/V the cache holds (gathered as fp32).
    from oracle import Oracle
    oracle = Oracle()
    got, qh = out.cpu().numpy(), q.cpu().numpy()
    order = np.argsort(lens)
    check = [int(order[0]), int(order[-1])] + [int(x) for x in synth.permutation(70, 3, B)
                                               if x not in (order[0], order[-1])][:8]
    errs, rl2s = [], []
    for s in check:
        gk, gv = cache.gather(0, s, lens[s])
        want = oracle.decode_gqa(qh[s][None], gk.cpu().numpy()[None], gv.cpu().numpy()[None], np.float32(sc))[0]
        errs.append(float(np.abs(got[s] - want).max()))
        rl2s.append(float(np.linalg.norm((got[s] - want).astype(np.float64)) / np.linalg.norm(want.astype(np.float64))))
    cache.close()
    return {"batch": B, "sum_len": sum(lens), "min_len": min(lens), "max_len": max(lens),
            "kv": "bf16" if bf16 else "f32", "ms": round(ms, 4), "bytes_per_call": total,
            "gbs": round(total / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "parity": {"sequences_checked": len(check), "max_abs_err": max(errs), "max_rel_l2_err": max(rl2s),
                       "against": "oracle STANDARD decode on the cached bf16 K/V (fp32 bar 1e-4 / 1e-5)"}}


def bench_model_decode(torch, sa, synth, steps: int = 128, warmup: int = 2, B: int = 64):
    """Greedy decode through the whole Qwen3-0.6B-shape model (28 layers,
    hidden 1024, 16/8 heads, vocab 151936, weights N(0, 0.02) in bf16):
    B=64 sequences with context lengths U[512, 32768], 64-token pages from a
    seeded shuffle of the pool, bf16 KV synthesised as N(0,1) (no prefill
    run).  Timed: `steps` consecutive greedy steps; tok/s = B * steps / wall."""
    cfg = sa.QWEN3_0_6B
    NL, HKV, D = cfg["num_layers"], cfg["n_kv_heads"], cfg["head_dim"]
    lens = batch_lengths(synth, B)
    check_steps = 2                       # untimed steps checked against the oracle
    pages_per = [(L + warmup + steps + check_steps + 63) // 64 for L in lens]
    n_pages = sum(pages_per)
    cache = sa.KVCache(NL, HKV, D, B, max(pages_per), n_pages, sa.SA_DTYPE_BF16)
    log(f"[bench] model decode: KV pool {cache.nbytes() / 1e9:.1f} GB, {n_pages} pages")
    perm = synth.permutation(71, 2, n_pages)
    off = 0
    for s, (L, n) in enumerate(zip(lens, pages_per)):
        cache.set_pages(s, perm[off:off + n])
        cache.set_len(s, L)
        off += n
    gen = torch.Generator(device="cuda")
    gen.manual_seed(71)
    t0 = time.perf_counter()
    for l in range(NL):
        for pool in sa.kv_pool_views(cache, l):
            pool.normal_(generator=gen)
    torch.cuda.synchronize()
    log(f"[bench] model decode: KV synthesised in {time.perf_counter() - t0:.1f} s")
    model = sa.Qwen3(B, max(lens) + warmup + steps + check_steps + 1)
    model.init_random(71, 0.02)
    tokens = torch.tensor([int(x * cfg["vocab"]) % cfg["vocab"] for x in synth.uniform(71, 3, B)],
                          dtype=torch.int32, device="cuda")
    cur = tokens
    for _ in range(warmup):
        cur = model.decode_step(cache, cur)
    torch.cuda.synchronize()
    for s, L in enumerate(lens):          # the timed steps start from the stated lengths
        cache.set_len(s, L)
    cur = tokens
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record()
    for _ in range(steps):
        cur = model.decode_step(cache, cur)
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = ev0.elapsed_time(ev1) * 1e-3
    # HBM bytes the step cannot avoid: every K/V element of every layer once
    # (committed tokens plus the new one), the projection weights and lm_head
    # once, the appended K/V written once.
    kv_token = NL * HKV * D * 2 * 2
    kv_bytes = sum((L + t + 1) * kv_token for L in lens for t in range(steps))
    H, I, V, HQ = cfg["hidden"], cfg["intermediate"], cfg["vocab"], cfg["n_q_heads"]
    w_layer = 2 * ((HQ + 2 * HKV) * D * H + H * HQ * D + 2 * I * H + H * I)
    w_bytes = steps * (NL * w_layer + 2 * V * H)
    total = kv_bytes + w_bytes + steps * B * kv_token
    parity = model_decode_parity(torch, sa, model, cache, cfg, lens, cur, check_steps)
    cache.close()
    model.close()
    gbs = total / wall / 1e9
    return {"batch": B, "steps": steps, "sum_len": sum(lens), "min_len": min(lens), "max_len": max(lens),
            "kv": "bf16", "weights": "bf16", "wall_s": round(wall, 4), "gpu_s": round(gpu_s, 4),
            "ms_per_step": round(wall * 1e3 / steps, 3), "tok_per_s": round(B * steps / wall, 1),
            "bytes_per_step": int(total / steps), "gbs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
            "roofline_tok_per_s": round(B * steps / (total / (HBM_PEAK_GBS * 1e9)), 1), "parity": parity}


def model_decode_parity(torch, sa, model, cache, cfg, lens, tokens, n_steps: int):
    """Outside the timed region, after the timed steps: n_steps more greedy
    steps of the whole batch, with the longest sequence, the shortest and two
    of at least three 2,048-token chunks checked against the oracle decoder on
    the device's weights and the gathered cache (each row's logits within
    relative L2 2e-2, greedy tokens identical)."""
    from oracle import Oracle
    from model_parity import SubsetChecker
    from util import load_synth
    synth = load_synth()
    B = len(lens)
    order = np.argsort(lens)
    multi = [int(s) for s in synth.permutation(70, 3, B) if lens[s] > 3 * 2048 and s != order[-1]][:2]
    seqs = [int(order[-1]), int(order[0])] + multi
    t0 = time.perf_counter()
    chk = SubsetChecker(sa, Oracle(), model, cache, dict(cfg), seqs, n_steps, True)
    logits = torch.empty(B, cfg["vocab"], dtype=torch.float32, device="cuda")
    worst, max_abs, same = 0.0, 0.0, True
    for _ in range(n_steps):
        want = chk.want(tokens.cpu().numpy())
        tokens = model.decode_step(cache, tokens, logits=logits)
        res = chk.compare(want, logits.cpu().numpy(), tokens.cpu().numpy())
        worst, max_abs = max(worst, res["worst_row_rel_l2"]), max(max_abs, res["max_abs_err"])
        same = same and res["tokens_identical"]
    log(f"[bench] model decode parity: rows {seqs}, worst row rel-L2 {worst:.2e}, tokens identical {same} "
        f"({time.perf_counter() - t0:.1f} s)")
    return {"sequences": seqs, "context_lens": [int(cache.length(s)) - n_steps for s in seqs], "steps": n_steps,
            "worst_row_rel_l2": worst, "max_abs_err": max_abs, "tokens_identical": same,
            "ok": bool(same and worst <= 2e-2),
            "against": "oracle decoder (oracle/qwen3_model.py) on the device weights and gathered bf16 KV; "
                       "bar: rel-L2 <= 2e-2 per row, identical greedy tokens"}


def bench_prefill(torch, sa, synth, L: int, bf16: bool, steps: int = 5):
    HQ, HKV, D = 16, 8, 128
    dt = torch.bfloat16 if bf16 else torch.float32
    # q, k ~ N(0,1) rotated at positions 0 .. L-1 (theta 1e6), v ~ N(0,1)
    rope = sa.rope_tables(L, D, 1e6)

    def roped(x):
        pos = torch.arange(x.numel() // D, dtype=torch.int32, device="cuda") % L
        return sa.qk_norm_rope(x, pos, rope=rope)

    q = roped(torch.from_numpy(synth.normal(60, 1, (1, HQ, L, D))).cuda()).to(dt)
    k = roped(torch.from_numpy(synth.normal(60, 2, (1, HKV, L, D))).cuda()).to(dt)
    v = torch.from_numpy(synth.normal(60, 3, (1, HKV, L, D))).cuda().to(dt)
    out = torch.empty(1, HQ, L, D, device="cuda")
    sc = float(1 / np.sqrt(D))
    # The clocks settle only after about a second of MFMA load; the untimed
    # warmup runs that long so the timed launches see steady-state clocks.
    # fp32 short prompts pair their query tiles through a workspace
    # (sa_prefill_causal_ws); other shapes ask for none.
    ws_n = sa.prefill_ws_bytes(sa.SA_DTYPE_BF16 if bf16 else sa.SA_DTYPE_F32, 1, HQ, HKV, L, D)
    ws = torch.empty(ws_n, dtype=torch.uint8, device="cuda") if ws_n else None
    call = lambda i: sa.prefill_causal(q, k, v, sc, out=out, ws=ws)
    t_end = time.perf_counter() + 1.0
    while time.perf_counter() < t_end:
        for i in range(10):
            call(i)
        torch.cuda.synchronize()
    per, _ = time_launches(torch, call, steps, 2)
    ms = statistics.mean(per)
    flops = 2.0 * HQ * D * L * (L + 1)
    tf = flops / (ms * 1e-3) / 1e12
    peak = BF16_PEAK_TFLOPS if bf16 else FP32_PEAK_TFLOPS
    res = {"L": L, "dtype": "bf16" if bf16 else "f32", "ms": round(ms, 4), "tflops": round(tf, 2),
           "mfma_frac": round(tf / peak, 4), "paired_workspace_bytes": ws_n}
    if L <= 1024:
        # A short prompt's kernel runs for less time than the ctypes call that
        # launches it takes on the host; 32 calls replayed from a HIP graph give
        # the device-side time per call.
        n_calls = 32
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n_calls):
                call(i)
        graph.replay()
        torch.cuda.synchronize()
        g_per, _ = time_launches(torch, lambda i: graph.replay(), max(steps, 3), 1)
        g_ms = statistics.mean(g_per) / n_calls
        del graph
        res.update({"graph_ms": round(g_ms, 4), "graph_tflops": round(flops / (g_ms * 1e-3) / 1e12, 2)})
    return res


def copy_calibration(torch, nbytes: int = 1 << 30, steps: int = 5):
    """A plain device-to-device copy of nbytes (reads nbytes, writes nbytes):
    the reference kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE, and the
    bandwidth HBM sustains for a streaming read+write on this device."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    per, _ = time_launches(torch, lambda i: dst.copy_(src), steps, 2)
    ms = statistics.mean(per)
    del src, dst
    torch.cuda.empty_cache()
    return {"bytes_read": nbytes, "bytes_written": nbytes, "ms": round(ms, 4),
            "gbs_read_plus_write": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=["headline", "all", "single", "layer", "paged", "prefill", "model"],
                    default="all",
                    help="headline only, everything, or the headline plus one section")
    ap.add_argument("--T", type=int, default=262144)
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU-baseline sampling for the headline; below 1 also skips the "
                         "per-configuration CPU baselines")
    ap.add_argument("--prefill-lens", default="128,1024,8192",
                    help="prompt lengths of the prefill section (comma-separated)")
    ap.add_argument("--prefill-dtypes", default="bf16,f32", help="bf16, f32 or both (comma-separated)")
    ap.add_argument("--profile-copy", action="store_true",
                    help="also run a 1 GiB device copy (counter calibration for rocprofv3 --pmc)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every configuration of this path runs on a single "
              f"MI355X (got --gpus {args.gpus}); the multi-GPU split is a design note, not a run.",
              file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    sa, synth = load_pkg()
    sa.lib()

    calib = None
    if args.profile_copy:
        log("[bench] 1 GiB device copy (counter calibration)")
        calib = copy_calibration(torch)
    head, (Q, K, V) = bench_stream(torch, sa, synth, args.T, args.steps, args.warmup,
                                   calls_per_step=CALLS_PER_STEP)
    head_fp64 = fp64_errors(Q, K, V, head["gpu_out"])
    log(f"[bench] headline: {head['gbs']:.1f} GB/s kernel, {head['wall_gbs']:.1f} GB/s wall, "
        f"err {head['max_abs_err']:.2e}")
    extra = {}
    run = (lambda name: True) if args.only == "all" else (lambda name: name == args.only)
    if run("single"):
        log("[bench] single-head T=1024")
        c1, _ = bench_stream(torch, sa, synth, 1024, 200, 20, min_footprint=1.1e9, graph=True)
        extra["single_head_T1024"] = {k: c1[k] for k in ("kernel_ms", "gbs", "max_abs_err", "rel_l2_err")}
        extra["single_head_T1024"]["hbm_frac"] = round(c1["gbs"] / HBM_PEAK_GBS, 5)
        extra["single_head_T1024"].update(graph_fields(c1))
        for T in (8192, 65536):
            log(f"[bench] single-head T={T}")
            c2, (q2, k2, v2) = bench_stream(torch, sa, synth, T, 200, 5, graph=True)
            extra[f"single_head_T{T}"] = {"kernel_ms": c2["kernel_ms"], "gbs": round(c2["gbs"], 1),
                                          "hbm_frac": round(c2["gbs"] / HBM_PEAK_GBS, 4),
                                          "rel_l2_err": c2["rel_l2_err"], "max_abs_err": c2["max_abs_err"],
                                          **graph_fields(c2), **fp64_errors(q2, k2, v2, c2["gpu_out"])}
    from oracle import Reference
    cpu_extra = args.cpu_budget >= 1.0 and Reference.available()
    if run("layer"):
        log("[bench] one-layer Qwen3 decode loop")
        extra["qwen3_layer_decode_loop"] = bench_layer_decode_loop(torch, sa, synth)
        if cpu_extra:
            log("[bench] CPU: reference decoder layer, attention path, 100 steps")
            extra["qwen3_layer_decode_loop"]["cpu_baseline"] = cpu_layer_decode()
    if run("paged"):
        log("[bench] batched paged GQA decode, 64 sequences, bf16 KV")
        extra["paged_decode_b64_bf16"] = bench_paged_batch(torch, sa, synth)
    if run("prefill"):
        for L in (int(x) for x in args.prefill_lens.split(",")):
            for bf in (d == "bf16" for d in args.prefill_dtypes.split(",")):
                log(f"[bench] causal prefill L={L} {'bf16' if bf else 'fp32'}, 16/8 heads, D=128")
                extra[f"prefill_L{L}_{'bf16' if bf else 'f32'}"] = bench_prefill(torch, sa, synth, L, bf)
            if cpu_extra:
                log(f"[bench] CPU: reference blockwise AVX2 prefill L={L}")
                extra[f"prefill_L{L}_cpu_baseline"] = cpu_prefill(L)
            if args.cpu_budget >= 1.0:
                log(f"[bench] CPU: np=1 sequence-parallel prefill loop L={L} (timing only)")
                extra[f"prefill_L{L}_cpu_sequence_np1"] = cpu_prefill_sequence(L)
    if run("model"):
        torch.cuda.empty_cache()
        log("[bench] 28-layer Qwen3-0.6B-shape greedy decode, 64 sequences, bf16 KV")
        extra["qwen3_model_decode_b64"] = bench_model_decode(torch, sa, synth)
        if cpu_extra:
            log("[bench] CPU: reference decoder layer at the mean context length")
            extra["qwen3_model_decode_b64"]["cpu_baseline"] = cpu_model_decode(sum(batch_lengths(synth, 64)))
    log("[bench] CPU baseline (reference streaming_attention_omp)")
    cpu = cpu_baseline(Q, K, V, args.cpu_budget)

    gbs = head["gbs"]
    line = {
        "metric": METRIC,
        "value": round(head["wall_gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["wall_ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded splitmix64 + Box-Muller, 0.5 N(0,1), 1% K rows x8)",
        "config": {"workload": f"single-query streaming attention, T={args.T}, d=128, block 128, fp32",
                   "T": args.T, "head_dim": 128, "block": 128, "replicas": head["replicas"],
                   "calls_per_step": CALLS_PER_STEP},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(args.T),
                     "kernel": "decode call = split_kv_decode_kernel<128,1,f32,dense> + lse_merge_kernel",
                     "kernel_ms": round(head["kernel_ms"], 5),
                     "algorithmic_bytes_per_launch": head["bytes_per_launch"]},
        "cpu_baseline": cpu,
        "parity": {"max_abs_err": head["max_abs_err"], "rel_l2_err": head["rel_l2_err"],
                   "against": "oracle streaming_attention_serial, fp32, block 128", **head_fp64},
        "extra": extra,
    }
    if calib:
        line["extra"]["copy_calibration"] = calib
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
