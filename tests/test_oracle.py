"""Pins of the CPU oracle: golden vectors from the reference, the reference
itself where it is built, fp64 brute force, and closed-form invariants.

Each check is chosen so that a plausible mistake in the oracle (wrong RoPE
frequency convention, scale on the output instead of the scores, eps outside
the sqrt, off-by-one causal mask, wrong GQA head map) fails at least one of
them; the `mistake_*` tests show that the checks do catch such mistakes.
"""
from __future__ import annotations

import numpy as np
import pytest

import golden_inputs as gi

SCALE128 = np.float32(1.0 / np.sqrt(128.0))


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# ------------------------------------------------------------------ golden

def test_golden_inputs_unchanged():
    """The generator still produces the inputs the fixtures were made from."""
    import hashlib

    def dg(*arrs):
        h = hashlib.sha256()
        for a in arrs:
            h.update(np.ascontiguousarray(a).tobytes())
        return h.hexdigest()

    meta, _ = gi.load("stream_t1024")
    assert dg(*gi.t1024_inputs()) == meta["inputs_sha256"]
    meta, _ = gi.load("stream_long")
    assert dg(*gi.long_inputs(8192)) == meta["inputs_sha256"]["8192"]
    meta, _ = gi.load("decode")
    assert dg(*gi.decode_inputs()) == meta["inputs_sha256"]
    meta, _ = gi.load("layer")
    assert dg(*gi.layer_inputs()) == meta["inputs_sha256"]
    meta, _ = gi.load("qwen3_forward")
    for case, sha in zip(gi.MODEL_CASES, meta["inputs_sha256"]):
        w, tokens = gi.model_inputs(case)
        assert dg(tokens, w["embed"], w["lm_head"], *[v for L in w["layers"] for v in L.values()]) == sha


def test_oracle_streaming_golden_t1024(oracle):
    _, g = gi.load("stream_t1024")
    Q, K, V = gi.t1024_inputs()
    for blk in (64, 128):
        np.testing.assert_allclose(oracle.streaming_serial(Q, K, V, blk), g[f"serial_b{blk}"], atol=2e-6)
        np.testing.assert_allclose(oracle.streaming_serial(Q * SCALE128, K, V, blk),
                                   g[f"serial_scaled_b{blk}"], atol=2e-6)
    np.testing.assert_allclose(oracle.naive_serial(Q, K, V), g["naive"], atol=2e-6)
    np.testing.assert_allclose(oracle.streaming_omp(Q, K, V, 64, 4), g["omp_b64_t4"], atol=2e-6)


def test_oracle_streaming_golden_unit_grid(oracle):
    _, g = gi.load("stream_unit")
    for T, d in gi.UNIT_GRID:
        Q, K, V = gi.unit_inputs(T, d)
        np.testing.assert_allclose(oracle.streaming_serial(Q, K, V, 64), g[f"serial_T{T}_d{d}"], atol=1e-6)


def test_oracle_streaming_golden_long(oracle):
    _, g = gi.load("stream_long")
    for T in (8192, 65536):
        Q, K, V = gi.long_inputs(T)
        for blk in (64, 128):
            out = oracle.streaming_serial(Q, K, V, blk)
            assert rel_l2(out, g[f"serial_T{T}_b{blk}"]) < 2e-6


def test_oracle_rope_golden(oracle):
    meta, g = gi.load("rope")
    cos, sin = oracle.rope_tables(meta["max_pos"], 128, 1e6)
    rows = np.array(meta["rows"])
    np.testing.assert_array_equal(cos[rows], g["cos"])
    np.testing.assert_array_equal(sin[rows], g["sin"])
    q, k = gi.rope_inputs()
    S = q.shape[2]
    qpos = np.tile(np.arange(S), q.shape[1])
    kpos = np.tile(np.arange(S), k.shape[1])
    np.testing.assert_allclose(oracle.apply_rope(q, qpos, cos, sin), g["q_rope"], atol=1e-6)
    np.testing.assert_allclose(oracle.apply_rope(k, kpos, cos, sin), g["k_rope"], atol=1e-6)


def test_oracle_decode_golden(oracle):
    _, g = gi.load("decode")
    q, k, v = gi.decode_inputs()
    sc = np.float32(1.0 / np.sqrt(128))
    np.testing.assert_allclose(oracle.decode_gqa(q, k, v, sc), g["standard"], atol=2e-6)
    rep = q.shape[1] // k.shape[1]
    kr, vr = np.repeat(k, rep, axis=1), np.repeat(v, rep, axis=1)
    np.testing.assert_allclose(oracle.decode_streaming_compat(q, kr, vr, sc), g["streaming"], atol=2e-6)


def test_reference_nested_omp_quirk(oracle):
    """With 8 OpenMP threads the reference's self_attention_streaming runs the
    inner streaming_attention_omp on one thread inside its head loop, yet still
    cuts T into min(8, ceil(T/128)) chunks: only chunk 0 enters the result
    (reference tensor_cpp/src/ops.cpp:987-1005 calling :910-958).  The golden
    made with 8 threads equals scale * attention over the first chunk only."""
    _, g = gi.load("decode")
    q, k, v = gi.decode_inputs()
    sc = np.float32(1.0 / np.sqrt(128))
    T = k.shape[2]
    n_chunks = max(1, min(8, (T + 127) // 128))
    first = (T + n_chunks - 1) // n_chunks
    want = np.stack([np.stack([oracle.streaming_serial(q[b, h], k[b, h // 2, :first], v[b, h // 2, :first], 64)
                               for h in range(4)]) for b in range(2)]) * sc
    np.testing.assert_allclose(g["streaming_nested_t8"], want, atol=2e-6)
    assert np.abs(g["streaming_nested_t8"] - g["streaming"]).max() > 1e-2


def test_oracle_prefill_golden(oracle):
    meta, g = gi.load("prefill")
    q, k, v = gi.prefill_inputs()
    sc = np.float32(1.0 / np.sqrt(128))
    rows = np.array(meta["rows"])
    out = oracle.prefill_blockwise(q, k, v, sc, 64, rows=rows)[:, :, rows, :]
    np.testing.assert_allclose(out, g["blockwise"], atol=2e-6)
    np.testing.assert_allclose(out, g["blockwise_avx2"], atol=5e-6)


def layer_oracle(oracle, eff, wq, wk, Hq, Hkv, prompt, eps_outside=False, streaming=False):
    """The reference decoder layer's attention, restated with oracle pieces."""
    D = 128
    N = eff.shape[0]
    q = eff[:, : Hq * D].reshape(N, Hq, D)
    k = eff[:, Hq * D: (Hq + Hkv) * D].reshape(N, Hkv, D)
    v = eff[:, (Hq + Hkv) * D:].reshape(N, Hkv, D)
    qn = oracle.rms_norm_rows(q, wq, 1e-6, eps_outside)
    kn = oracle.rms_norm_rows(k, wk, 1e-6, eps_outside)
    cos, sin = oracle.rope_tables(N, D, 1e6)
    pos = np.arange(N)
    qr = oracle.apply_rope(qn, np.repeat(pos, Hq), cos, sin)
    kr = oracle.apply_rope(kn, np.repeat(pos, Hkv), cos, sin)
    sc = np.float32(1.0 / np.sqrt(D))
    out = np.empty_like(qr)
    # prompt: causal prefill from position 0
    pq = qr[:prompt].transpose(1, 0, 2)[None]
    pk = kr[:prompt].transpose(1, 0, 2)[None]
    pv = v[:prompt].transpose(1, 0, 2)[None]
    out[:prompt] = oracle.prefill_blockwise(pq, pk, pv, sc, 64)[0].transpose(1, 0, 2)
    for t in range(prompt, N):
        kk = kr[: t + 1].transpose(1, 0, 2)[None]
        vv = v[: t + 1].transpose(1, 0, 2)[None]
        if streaming:
            rep = Hq // Hkv
            out[t] = oracle.decode_streaming_compat(qr[t][None], np.repeat(kk, rep, 1),
                                                    np.repeat(vv, rep, 1), sc)[0]
        else:
            out[t] = oracle.decode_gqa(qr[t][None], kk, vv, sc)[0]
    return out


@pytest.mark.parametrize("avx2", [0, 1])
@pytest.mark.parametrize("streaming", [0, 1])
def test_oracle_layer_golden(oracle, avx2, streaming):
    meta, g = gi.load("layer")
    _, _, _, wq, wk = gi.layer_inputs()
    out = layer_oracle(oracle, g["qkv_eff"], wq, wk, 4, 2, meta["prompt"], eps_outside=bool(avx2),
                       streaming=bool(streaming))
    want = g[f"attn_avx{avx2}_str{streaming}"]
    assert np.abs(out - want).max() < 1e-5
    assert rel_l2(out, want) < 1e-6


# ------------------------------------------------------------------ the reference directly

def test_oracle_matches_reference_random(oracle, ref, synth):
    for T, d, blk in ((1, 64, 64), (63, 128, 64), (1000, 128, 128), (4097, 256, 64)):
        Q, K, V = synth.stream_inputs(T, d, seed=T + d)
        np.testing.assert_allclose(oracle.streaming_serial(Q, K, V, blk), ref.streaming_serial(Q, K, V, blk),
                                   atol=2e-6)
        np.testing.assert_allclose(oracle.streaming_omp(Q, K, V, blk, 3), ref.streaming_omp(Q, K, V, blk, 3),
                                   atol=2e-6)
        a, b = oracle.naive_serial(Q, K, V), ref.naive_serial(Q, K, V)
        assert oracle.l2_error(a, b) == pytest.approx(ref.l2_error(a, b), rel=1e-5, abs=1e-12)
        assert oracle.max_error(a, b) == ref.max_error(a, b)


# ------------------------------------------------------------------ fp64 and closed forms

def test_streaming_vs_fp64(oracle, synth):
    Q, K, V = gi.t1024_inputs()
    f = oracle.sdpa_f64(Q[None] * SCALE128, K, V, 1.0)[0]
    out = oracle.streaming_serial(Q * SCALE128, K, V, 64)
    assert rel_l2(out, f) < 1e-6
    Q, K, V = gi.long_inputs(8192)
    f = oracle.sdpa_f64(Q[None], K, V, 1.0)[0]
    assert rel_l2(oracle.streaming_serial(Q, K, V, 128), f) < 5e-6


def test_streaming_invariants(oracle, synth):
    T, d = 777, 128
    Q, K, V = synth.stream_inputs(T, d, seed=9)
    c = synth.normal(9, 7, d)
    # constant V rows -> O equals that row
    np.testing.assert_allclose(oracle.streaming_serial(Q, K, np.tile(c, (T, 1)), 64), c, atol=2e-6)
    # T = 1 -> O = V[0]
    np.testing.assert_allclose(oracle.streaming_serial(Q, K[:1], V[:1], 64), V[0], atol=0)
    # Q = 0 -> mean of V
    np.testing.assert_allclose(oracle.streaming_serial(np.zeros(d, np.float32), K, V, 64), V.mean(0), atol=2e-6)
    # block size and split count do not matter beyond rounding
    base = oracle.streaming_serial(Q, K, V, 64)
    for blk in (1, 7, 128, 1000):
        np.testing.assert_allclose(oracle.streaming_serial(Q, K, V, blk), base, atol=2e-6)
    for nt in (1, 2, 5, 8):
        np.testing.assert_allclose(oracle.streaming_omp(Q, K, V, 16, nt), base, atol=2e-6)
    # permuting the (K, V) rows together
    p = synth.permutation(9, 8, T)
    np.testing.assert_allclose(oracle.streaming_serial(Q, K[p], V[p], 64), base, atol=2e-6)
    # T = 0 -> zeros
    np.testing.assert_array_equal(oracle.streaming_serial(Q, np.zeros((0, d), np.float32),
                                                          np.zeros((0, d), np.float32), 64), 0)


def test_l2_error_definition(oracle):
    a = np.array([1.0, 2.0, 2.0], np.float32)
    b = np.array([0.0, 2.0, 0.0], np.float32)
    assert oracle.l2_error(a, b) == pytest.approx(np.sqrt(5.0) / 2.0, rel=1e-6)
    # absolute when the reference norm is ~0
    assert oracle.l2_error(a, np.zeros(3, np.float32)) == pytest.approx(3.0, rel=1e-6)
    assert oracle.max_error(a, b) == 2.0


def test_rms_norm_closed_form(oracle, synth):
    D, eps = 128, 1e-6
    x = synth.normal(10, 1, (5, D))
    y = oracle.rms_norm_rows(x, np.ones(D, np.float32), eps)
    mu = (x.astype(np.float64) ** 2).mean(1)
    np.testing.assert_allclose((y.astype(np.float64) ** 2).sum(1), D * mu / (mu + eps), rtol=1e-5)
    # scale invariance up to eps; weight multiplies elementwise
    w = 1 + synth.normal(10, 2, D, 0.02)
    np.testing.assert_allclose(oracle.rms_norm_rows(3 * x, w, 0.0), oracle.rms_norm_rows(x, w, 0.0), rtol=1e-5)


def test_rope_closed_form(oracle, synth):
    D = 128
    cos, sin = oracle.rope_tables(5000, D, 1e6)
    i = np.arange(D // 2)
    # fp64 evaluation of the same formula; one ulp of inv_freq moves the angle
    # by ~p * 6e-8, hence the position-scaled tolerance (the golden pins the
    # exact fp32 tables).
    inv64 = 1.0 / np.power(1e6, i / D)
    for p in (0, 1, 17, 300, 4999):
        tol = 1e-6 + 2e-7 * p
        np.testing.assert_allclose(cos[p], np.cos(p * inv64), atol=tol)
        np.testing.assert_allclose(sin[p], np.sin(p * inv64), atol=tol)
    x = synth.normal(11, 1, (3, D))
    np.testing.assert_array_equal(oracle.apply_rope(x, np.zeros(3, int), cos, sin), x)   # pos 0 = identity
    y = oracle.apply_rope(x, np.array([5, 100, 4000]), cos, sin)
    h = D // 2
    np.testing.assert_allclose(y[:, :h] ** 2 + y[:, h:] ** 2, x[:, :h] ** 2 + x[:, h:] ** 2, rtol=1e-5, atol=1e-6)
    # q(p).k(p') depends only on p - p'
    q, k = synth.normal(11, 2, (1, D)), synth.normal(11, 3, (1, D))
    d1 = (oracle.apply_rope(q, [50], cos, sin) @ oracle.apply_rope(k, [20], cos, sin).T).item()
    d2 = (oracle.apply_rope(q, [1030], cos, sin) @ oracle.apply_rope(k, [1000], cos, sin).T).item()
    assert d1 == pytest.approx(d2, rel=1e-4, abs=1e-4)


def test_decode_gqa_equals_repeat_kv(oracle, ref, synth):
    q = synth.normal(12, 1, (2, 8, 128))
    k = synth.normal(12, 2, (2, 2, 90, 128))
    v = synth.normal(12, 3, (2, 2, 90, 128))
    sc = np.float32(0.1)
    kr, vr = ref.repeat_kv(k, 4), ref.repeat_kv(v, 4)
    np.testing.assert_array_equal(kr, np.repeat(k, 4, axis=1))
    mha = oracle.decode_gqa(q, kr, vr, sc)
    np.testing.assert_allclose(oracle.decode_gqa(q, k, v, sc), mha, atol=1e-6)
    # equals streaming attention on the pre-scaled query, per head
    for b in range(2):
        for h in range(8):
            np.testing.assert_allclose(oracle.streaming_serial(q[b, h] * sc, k[b, h // 4], v[b, h // 4], 64),
                                       mha[b, h], atol=2e-6)


def test_prefill_rows_are_prefix_attention(oracle, synth):
    L, D = 150, 128
    q = synth.normal(13, 1, (1, 2, L, D))
    k = synth.normal(13, 2, (1, 1, L, D))
    v = synth.normal(13, 3, (1, 1, L, D))
    sc = np.float32(1 / np.sqrt(D))
    out = oracle.prefill_blockwise(q, k, v, sc, 64)
    for h in range(2):
        for i in (0, 1, 63, 64, 65, 149):
            f = oracle.sdpa_f64(q[0, h, i:i + 1], k[0, 0, : i + 1], v[0, 0, : i + 1], float(sc))[0]
            np.testing.assert_allclose(out[0, h, i], f, atol=2e-6)
    # the last row equals a decode step over the whole prefix
    dec = oracle.decode_gqa(q[0, :, L - 1][None], k[:, :, :L], v[:, :, :L], sc)
    np.testing.assert_allclose(out[0, :, L - 1], dec[0], atol=2e-6)


def _sequence_np1_closed_form(q, k, v, sc):
    """fp64: out_i = sum_{j<=i} e^{s_j} s_j v_j / sum_{j<=i} e^{s_j}, s_j = (q_i sc).k_j,
    the value the np = 1 sequence-parallel loop computes (its weights multiply
    s_j v_j)."""
    B, Hq, L, D = q.shape
    rep = Hq // k.shape[1]
    qs = (q * np.float32(sc)).astype(np.float32).astype(np.float64)
    out = np.zeros(q.shape)
    for b in range(B):
        for h in range(Hq):
            kk = k[b, h // rep].astype(np.float64)
            vv = v[b, h // rep].astype(np.float64)
            s = qs[b, h] @ kk.T
            for i in range(L):
                si = s[i, : i + 1]
                e = np.exp(si - si.max())
                out[b, h, i] = (e[:, None] * si[:, None] * vv[: i + 1]).sum(0) / e.sum()
    return out


@pytest.mark.parametrize("D", [32, 36])
def test_sequence_np1_closed_form(oracle, synth, D):
    """The timing-only restatement of the np = 1 sequence-parallel loop
    (reference ops_mpi.cpp:1216-1454) against its closed form in fp64, at a
    ragged length (150 keys: blocks of 64, 64, 22), GQA 2, a head size with and
    without a scalar tail, batch 2; a head range leaves the other heads zero."""
    B, Hq, Hkv, L = 2, 4, 2, 150
    q = synth.normal(71, 1, (B, Hq, L, D))
    k = synth.normal(71, 2, (B, Hkv, L, D))
    v = synth.normal(71, 3, (B, Hkv, L, D))
    sc = float(1 / np.sqrt(D))
    want = _sequence_np1_closed_form(q, k, v, sc)
    got = oracle.sequence_np1(q, k, v, sc)
    assert rel_l2(got, want) < 1e-5
    assert np.abs(got - want).max() < 1e-4
    part = oracle.sequence_np1(q, k, v, sc, heads=(1, 2))
    np.testing.assert_array_equal(part[:, 1:3], got[:, 1:3])
    assert not part[:, 0].any() and not part[:, 3].any()
    # the path's known-wrong numerics: it is not causal attention
    true = oracle.prefill_blockwise(q, k, v, np.float32(sc), 64)
    assert rel_l2(got, true) > 0.5


# ------------------------------------------------------------------ the checks catch mistakes

def test_mistake_hf_rope_convention_is_caught(oracle):
    """theta^(-2i/D) (HF) instead of the reference's theta^(-i/D) fails the golden."""
    meta, g = gi.load("rope")
    rows = np.array(meta["rows"])
    i = np.arange(64, dtype=np.float32)
    inv = np.float32(1.0) / np.power(np.float32(1e6), np.float32(2.0) * i / np.float32(128))
    wrong = np.cos(rows[:, None].astype(np.float32) * inv[None])
    assert np.abs(wrong - g["cos"]).max() > 1e-2


def test_mistake_scale_on_output_is_caught(oracle):
    """The reference STREAMING decode (scale on the output) differs from STANDARD."""
    _, g = gi.load("decode")
    assert np.abs(g["standard"] - g["streaming"]).max() > 1e-2
    q, k, v = gi.decode_inputs()
    sc = np.float32(1.0 / np.sqrt(128))
    wrong = oracle.decode_gqa(q, k, v, np.float32(1.0)) * sc
    assert np.abs(wrong - g["standard"]).max() > 1e-2


def test_mistake_causal_off_by_one_is_caught(oracle):
    """Excluding the diagonal key (j < i instead of j <= i) fails the golden."""
    meta, g = gi.load("prefill")
    q, k, v = gi.prefill_inputs()
    sc = np.float32(1.0 / np.sqrt(128))
    i = 150
    wrong = oracle.sdpa_f64(q[0, 0, i:i + 1], k[0, 0, :i], v[0, 0, :i], float(sc))[0]
    r = meta["rows"].index(i)
    assert np.abs(wrong - g["blockwise"][0, 0, r]).max() > 1e-3


def test_mistake_gqa_head_map_is_caught(oracle):
    """Mapping q head h to kv head h % Hkv (instead of h // rep) fails the golden."""
    _, g = gi.load("decode")
    q, k, v = gi.decode_inputs()
    sc = np.float32(1.0 / np.sqrt(128))
    kw = np.stack([k[:, h % 2] for h in range(4)], 1)
    vw = np.stack([v[:, h % 2] for h in range(4)], 1)
    assert np.abs(oracle.decode_gqa(q, kw, vw, sc) - g["standard"]).max() > 1e-2


# ---------------------------------------------------------------- Qwen3 decoder

def _decode_teacher_forced(oracle, case, w, tokens, mutate=None, qk_eps_outside=False):
    """The oracle decoder fed the case's tokens one at a time; logits at the
    positions the reference golden stores (last prompt token, then each step)."""
    from oracle.qwen3_model import KvStore, Qwen3Decoder
    c = case["cfg"]
    dec = Qwen3Decoder(w, c, oracle, qk_eps_outside=qk_eps_outside)
    if mutate:
        mutate(dec)
    B = tokens.shape[0]
    kv = KvStore(c["num_layers"], B, c["n_kv_heads"], c["head_dim"], tokens.shape[1])
    out = []
    for t in range(tokens.shape[1]):
        lg = dec.step(tokens[:, t], kv)
        if t >= case["prompt"] - 1:
            out.append(lg)
    return np.stack(out)


@pytest.mark.parametrize("avx2", [False, True])
@pytest.mark.parametrize("i", range(len(gi.MODEL_CASES)))
def test_oracle_qwen3_decoder_golden(oracle, i, avx2):
    """The oracle's decode step, token by token, equals the reference's
    qwen3_forward_with_cache (avx2: qwen3_forward_avx_with_cache, whose q/k
    RMSNorm adds eps to the root) golden logits: prompt, then single-token
    steps."""
    case = gi.MODEL_CASES[i]
    _, g = gi.load("qwen3_forward")
    w, tokens = gi.model_inputs(case)
    got = _decode_teacher_forced(oracle, case, w, tokens, qk_eps_outside=avx2)
    want = g[f"logits_avx{i}" if avx2 else f"logits{i}"]
    assert np.abs(got - want).max() <= 1e-4
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-5
    assert (got.argmax(-1) == want.argmax(-1)).all()


def test_oracle_qwen3_decoder_matches_reference_random(oracle, ref, synth):
    """A fresh weight draw, GQA 4:1, against the compiled reference."""
    from oracle.qwen3_model import synth_weights
    cfg = dict(num_layers=2, hidden=96, intermediate=160, vocab=300, n_q_heads=8, n_kv_heads=2,
               head_dim=16, rms_eps=1e-6, rope_theta=1e6, max_pos=64)
    case = dict(cfg=cfg, prompt=4, steps=6)
    w = synth_weights(synth, cfg, seed=99, std=0.15)
    tokens = ((np.arange(2 * 10).reshape(2, 10) * 53 + 11) % cfg["vocab"]).astype(np.int32)
    want = ref.qwen3_forward(w, cfg, tokens, case["prompt"])
    got = _decode_teacher_forced(oracle, case, w, tokens)
    assert np.abs(got - want).max() <= 1e-4
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-5


def test_mistake_swapped_gate_up_is_caught(oracle):
    """silu(up) * gate instead of silu(gate) * up fails the decoder golden."""
    case = gi.MODEL_CASES[0]
    _, g = gi.load("qwen3_forward")
    w, tokens = gi.model_inputs(case)
    I = case["cfg"]["intermediate"]
    for L in w["layers"]:
        L["gate_up"] = np.concatenate([L["gate_up"][I:], L["gate_up"][:I]])
    got = _decode_teacher_forced(oracle, case, w, tokens)
    assert np.abs(got - g["logits0"]).max() > 1e-3


def test_mistake_rope_position_off_by_one_is_caught(oracle):
    """Rotating q at position len + 1 while k sits at len fails the golden.
    (Shifting every position alike would not: RoPE scores depend only on
    position differences.)"""
    case = gi.MODEL_CASES[0]
    _, g = gi.load("qwen3_forward")
    w, tokens = gi.model_inputs(case)
    Hq = case["cfg"]["n_q_heads"]

    class ShiftQ:
        def __init__(self, inner):
            self.inner = inner

        def __getattr__(self, name):
            return getattr(self.inner, name)

        def apply_rope(self, x, pos, cos, sin):
            return self.inner.apply_rope(x, pos + 1 if x.shape[1] == Hq else pos, cos, sin)

    def shift_q(dec):
        dec.or_ = ShiftQ(dec.or_)

    got = _decode_teacher_forced(oracle, case, w, tokens, mutate=shift_q)
    assert np.abs(got - g["logits0"]).max() > 1e-3
