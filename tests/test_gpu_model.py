"""GPU parity: the whole-model greedy decode step (include/sa_qwen3.h) against
the CPU decoder oracle (oracle/qwen3_model.py, pinned to the reference's
qwen3_forward_with_cache by tests/test_oracle.py).

The oracle runs on the model's own weights (read back from the device) and on
the cache's own contents (gathered), so the comparison isolates the step.
fp32 KV: logits max-abs <= 1e-4 and relative L2 <= 1e-5 per step, tokens
identical.  bf16 KV at the Qwen3-0.6B shape: relative L2 <= 2e-2 per step and
greedy tokens identical over 32 steps.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from model_parity import SubsetChecker, host_weights, rel_l2

pytestmark = pytest.mark.gpu

SMALL = dict(num_layers=2, hidden=256, intermediate=512, vocab=1024, n_q_heads=4, n_kv_heads=2,
             head_dim=64, rms_eps=1e-6, rope_theta=1e6)
SHAPE_KEYS = ("num_layers", "hidden", "intermediate", "vocab", "n_q_heads", "n_kv_heads", "head_dim",
              "rms_eps", "rope_theta")


def make_cache(sa, synth, cfg, lens, steps, kv_dtype, seed):
    """Pages from a seeded shuffle of the pool, room for `steps` more tokens,
    committed lengths `lens`, every pool element N(0,1)."""
    pages_per = [(L + steps + 63) // 64 for L in lens]
    n_pages = sum(pages_per)
    cache = sa.KVCache(cfg["num_layers"], cfg["n_kv_heads"], cfg["head_dim"], len(lens), max(pages_per),
                       n_pages, kv_dtype)
    perm = synth.permutation(seed, 2, n_pages)
    off = 0
    for s, (L, n) in enumerate(zip(lens, pages_per)):
        cache.set_pages(s, perm[off:off + n])
        cache.set_len(s, L)
        off += n
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    for l in range(cfg["num_layers"]):
        for pool in sa.kv_pool_views(cache, l):
            pool.normal_(generator=gen)
    torch.cuda.synchronize()
    return cache


def oracle_store(cache, cfg, lens, steps, kv_bf16):
    from oracle.qwen3_model import KvStore
    st = KvStore(cfg["num_layers"], len(lens), cfg["n_kv_heads"], cfg["head_dim"], max(lens) + steps, kv_bf16)
    for l in range(cfg["num_layers"]):
        for b, L in enumerate(lens):
            k, v = cache.gather(l, b, L)
            st.K[l][b][:, :L] = k.cpu().numpy()
            st.V[l][b][:, :L] = v.cpu().numpy()
    st.lens[:] = lens
    return st


def run_parity(sa, oracle, synth, cfg, std, lens, steps, kv_dtype, seed, first_tokens, check):
    from oracle.qwen3_model import Qwen3Decoder
    max_pos = max(lens) + steps + 1
    model = sa.Qwen3(len(lens), max_pos, **{k: cfg[k] for k in SHAPE_KEYS})
    model.init_random(seed, std)
    cache = make_cache(sa, synth, cfg, lens, steps, kv_dtype, seed)
    dec = Qwen3Decoder(host_weights(sa, model, cfg), dict(cfg, max_pos=max_pos), oracle)
    store = oracle_store(cache, cfg, lens, steps, kv_dtype == sa.SA_DTYPE_BF16)
    tokens = torch.tensor(first_tokens, dtype=torch.int32, device="cuda")
    logits = torch.empty(len(lens), cfg["vocab"], dtype=torch.float32, device="cuda")
    for t in range(steps):
        want = dec.step(tokens.cpu().numpy(), store)
        nxt = model.decode_step(cache, tokens, logits=logits)
        got = logits.cpu().numpy()
        check(t, got, want)
        g_tok, w_tok = nxt.cpu().numpy(), want.argmax(-1)
        for b in np.nonzero(g_tok != w_tok)[0]:
            top2 = np.sort(want[b])[-2:]
            raise AssertionError(
                f"step {t} seq {b}: gpu token {g_tok[b]} (oracle logit {want[b, g_tok[b]]:.6f}, gpu "
                f"{got[b, g_tok[b]]:.6f}) vs oracle token {w_tok[b]} (oracle {want[b, w_tok[b]]:.6f}, gpu "
                f"{got[b, w_tok[b]]:.6f}); oracle top-2 gap {top2[1] - top2[0]:.2e}, logits rel-L2 "
                f"{rel_l2(got, want):.2e}")
        assert [cache.length(s) for s in range(len(lens))] == [L + t + 1 for L in lens]
        tokens = nxt
    cache.close()
    model.close()


def test_model_init_matches_generator(sa, synth):
    """sa_qwen3_init_random draws what oracle.qwen3_model.synth_weights draws."""
    from oracle.qwen3_model import synth_weights
    model = sa.Qwen3(2, 64, **{k: SMALL[k] for k in SHAPE_KEYS})
    model.init_random(5, 0.1)
    torch.cuda.synchronize()
    got = host_weights(sa, model, SMALL)
    want = synth_weights(synth, SMALL, 5, 0.1)
    pairs = [(got[t], want[t]) for t in ("embed", "final_norm", "lm_head")]
    pairs += [(g[t], w[t]) for g, w in zip(got["layers"], want["layers"]) for t in g]
    for g, w in pairs:
        # fp64 log/cos may differ by an ulp between device and host libm; after
        # rounding to fp32 / bf16 that can flip at most a rare element by one ulp
        diff = g != w
        assert diff.sum() <= 2
        if diff.any():
            assert np.abs(g[diff] - w[diff]).max() <= np.abs(w[diff]).max() * 2 ** -7
    model.close()


@pytest.fixture(params=["auto", "interleaved"])
def interleave(request, monkeypatch):
    """The decode step as the launch chooses (one stream at these sizes), or
    forced to run its two half-batches on two streams."""
    if request.param == "interleaved":
        monkeypatch.setenv("SA_DECODE_INTERLEAVE", "1")
    else:
        monkeypatch.delenv("SA_DECODE_INTERLEAVE", raising=False)
    return request.param


def test_model_decode_fp32_kv(sa, oracle, synth, interleave):
    """Small model, fp32 KV, three sequences of different lengths (one of a
    single token), 8 greedy steps at the fp32 bar."""

    def check(t, got, want):
        assert np.abs(got - want).max() <= 1e-4, f"step {t}"
        assert rel_l2(got, want) <= 1e-5, f"step {t}"

    run_parity(sa, oracle, synth, SMALL, 0.1, [70, 130, 1], 8, sa.SA_DTYPE_F32, 31, [5, 17, 900], check)


def test_model_decode_qwen3_shape_bf16_kv(sa, oracle, synth, interleave):
    """The Qwen3-0.6B shape (28 layers, 16/8 heads, vocab 151936), bf16 KV on
    shuffled pages, 4 sequences with lengths in [512, 2048], 32 greedy steps:
    identical tokens, logits within the bf16-KV tolerance."""
    lens = [int(x) for x in 512 + (synth.uniform(77, 1, 4) * 1536).astype(np.int64)]
    cfg = dict(sa.QWEN3_0_6B)
    worst = []

    def check(t, got, want):
        worst.append(rel_l2(got, want))
        assert worst[-1] <= 2e-2, f"step {t}"

    run_parity(sa, oracle, synth, cfg, 0.02, lens, 32, sa.SA_DTYPE_BF16, 41, [11, 222, 3333, 44444], check)
    print(f"lens {lens}: worst logits rel-L2 {max(worst):.2e}")


def test_model_decode_beyond_64_rows(sa, oracle, synth, interleave):
    """A decode batch above one 64-row projection tile: 150 sequences of 1 ..
    300 cached tokens (three row tiles of every projection; the fused
    attention in launches of 64 sequences; interleaved, two half-batches of
    more than 64 each), small model, fp32 KV, 3 greedy steps at the fp32 bar
    against the oracle decoder."""
    B = 150
    lens = [1 + int(x * 299) for x in synth.uniform(90, 1, B)]
    first = [int(x) for x in (synth.uniform(90, 2, B) * SMALL["vocab"]).astype(np.int64)]

    def check(t, got, want):
        assert np.abs(got - want).max() <= 1e-4, f"step {t}"
        assert rel_l2(got, want) <= 1e-5, f"step {t}"

    run_parity(sa, oracle, synth, SMALL, 0.1, lens, 3, sa.SA_DTYPE_F32, 33, first, check)


def test_model_batch_limit(sa):
    """max_batch 1 .. 1024 is accepted, 0 and 1025 refused with SA_ERANGE."""
    import ctypes as C
    d = sa.Qwen3Desc(1, 256, 512, 1024, 4, 2, 64, 64, 1e-6, 1e6)
    for n, want in ((0, sa.SA_ERANGE), (1025, sa.SA_ERANGE)):
        h = C.c_void_p()
        assert sa.lib().sa_qwen3_create(C.byref(d), n, C.byref(h)) == want
    model = sa.Qwen3(1024, 64, **{k: SMALL[k] for k in SHAPE_KEYS})
    model.close()


def test_model_rejects_bad_calls(sa):
    import ctypes as C
    model = sa.Qwen3(2, 64, **{k: SMALL[k] for k in SHAPE_KEYS})
    cache = sa.KVCache(SMALL["num_layers"], SMALL["n_kv_heads"], 128, 2, 2, 4)   # wrong head_dim
    tok = torch.zeros(2, dtype=torch.int32, device="cuda")
    with pytest.raises(sa.SaError, match="geometry"):
        model.decode_step(cache, tok)
    with pytest.raises(sa.SaError):
        sa.check(sa.lib().sa_qwen3_decode_step(model.handle, cache.handle, None, 2, None, None, None))
    big = torch.zeros(3, dtype=torch.int32, device="cuda")
    good = sa.KVCache(SMALL["num_layers"], SMALL["n_kv_heads"], SMALL["head_dim"], 4, 2, 8)
    with pytest.raises(sa.SaError, match="batch"):
        model.decode_step(good, big)
    good.reserve(0, 64)                                    # seq 1 has no page for its token
    with pytest.raises(sa.SaError, match="full") as e:
        model.decode_step(good, tok)
    assert e.value.status == sa.SA_EFULL and good.length(0) == 0 and good.length(1) == 0
    d = sa.Qwen3Desc(1, 100, 64, 64, 2, 1, 64, 16, 1e-6, 1e6)   # hidden not a multiple of 64
    h = C.c_void_p()
    assert sa.lib().sa_qwen3_create(C.byref(d), 1, C.byref(h)) == sa.SA_EINVAL
    cache.close()
    good.close()
    model.close()


def test_model_decode_b64_workload_rows(sa, oracle, synth):
    """The 64-sequence workload of the decode benchmark as it runs: the
    Qwen3-0.6B shape (weights N(0, 0.02), seed 71), context lengths
    U[512, 32768] (seed 70), 64-token pages from a seeded shuffle, bf16 KV
    N(0,1).  Its launches are the 4-wave fused step on 8 x 16 x 64
    workgroups.  Two greedy steps; the longest sequence, the shortest and
    two of at least three 2,048-token chunks against the oracle on the
    device's weights and the gathered cache: each row's logits within
    relative L2 2e-2, greedy tokens identical."""
    cfg = dict(sa.QWEN3_0_6B)
    B, steps = 64, 2
    lens = synth.batch_lengths(B, 512, 32768, 70)
    order = np.argsort(lens)
    multi = [int(s) for s in synth.permutation(70, 3, B) if lens[s] > 3 * 2048 and s != order[-1]][:2]
    seqs = [int(order[-1]), int(order[0])] + multi
    model = sa.Qwen3(B, max(lens) + steps + 1)
    model.init_random(71, 0.02)
    cache = make_cache(sa, synth, cfg, lens, steps, sa.SA_DTYPE_BF16, 71)
    chk = SubsetChecker(sa, oracle, model, cache, cfg, seqs, steps, True)
    tokens = torch.tensor([int(x * cfg["vocab"]) % cfg["vocab"] for x in synth.uniform(71, 3, B)],
                          dtype=torch.int32, device="cuda")
    logits = torch.empty(B, cfg["vocab"], dtype=torch.float32, device="cuda")
    for t in range(steps):
        want = chk.want(tokens.cpu().numpy())
        nxt = model.decode_step(cache, tokens, logits=logits)
        res = chk.compare(want, logits.cpu().numpy(), nxt.cpu().numpy())
        print(f"step {t} rows {seqs} (lens {[lens[s] for s in seqs]}): worst row rel-L2 "
              f"{res['worst_row_rel_l2']:.2e}, max-abs {res['max_abs_err']:.2e}")
        assert res["worst_row_rel_l2"] <= 2e-2, (t, res["row_rel_l2"])
        assert res["tokens_identical"], t
        tokens = nxt
    assert [cache.length(s) for s in range(B)] == [L + steps for L in lens]
    cache.close()
    model.close()


def test_model_decode_interleaved_graph_replay(sa, synth, monkeypatch):
    """An interleaved decode step (two half-batches on two streams, attention
    launches ordered by events) captured into a HIP graph: every replay, with
    eager work between replays, reproduces the eager step's logits and
    tokens bit for bit."""
    monkeypatch.setenv("SA_DECODE_INTERLEAVE", "1")
    lens = [300, 17, 129, 64, 1, 500]
    model = sa.Qwen3(len(lens), 600, **{k: SMALL[k] for k in SHAPE_KEYS})
    model.init_random(12, 0.1)
    cache = make_cache(sa, synth, SMALL, lens, 2, sa.SA_DTYPE_BF16, 12)
    tokens = torch.tensor([3, 5, 7, 11, 13, 17], dtype=torch.int32, device="cuda")
    logits = torch.empty(len(lens), SMALL["vocab"], dtype=torch.float32, device="cuda")
    nxt = torch.empty_like(tokens)
    model.decode_step(cache, tokens, next_tokens=nxt, logits=logits)   # eager; also sizes the buffers
    torch.cuda.synchronize()
    want_l, want_t = logits.clone(), nxt.clone()
    for s, L in enumerate(lens):
        cache.set_len(s, L)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        model.decode_step(cache, tokens, next_tokens=nxt, logits=logits)
    for rep in range(3):
        logits.fill_(float("nan"))
        nxt.fill_(-1)
        (torch.randn(1 << 20, device="cuda") * 2).sum().item()
        for s, L in enumerate(lens):
            cache.set_len(s, L)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, want_l), f"replay {rep}"
        assert torch.equal(nxt, want_t), f"replay {rep}"
    del graph
    cache.close()
    model.close()
