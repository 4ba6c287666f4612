"""GPU parity: paged KV cache, fused QK-norm + RoPE + append, paged GQA decode,
and the one-layer Qwen3-0.6B-shape decode loop (128-token prompt + 100 steps).

fp32 KV: max-abs <= 1e-4 and relative L2 <= 1e-5 against the oracle.
bf16 KV: relative L2 <= 2e-2 against the fp32 oracle, and the oracle run on
the same bf16-rounded K/V agrees to fp32 rounding.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import golden_inputs as gi

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128
SCALE = np.float32(1.0 / np.sqrt(D))


def dev(a, dtype=np.float32):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=dtype)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def assert_f32(out, want, max_abs=1e-4, rl2=1e-5):
    assert np.abs(out - want).max() <= max_abs, np.abs(out - want).max()
    assert rel_l2(out, want) <= rl2, rel_l2(out, want)


def make_cache(sa, kv_dtype, max_seqs=4, max_pages=80, num_pages=300, layers=2):
    return sa.KVCache(layers, HKV, D, max_seqs, max_pages, num_pages, kv_dtype)


@pytest.mark.parametrize("bf16", [False, True])
def test_append_gather_roundtrip_shuffled_pages(sa, synth, bf16):
    cache = make_cache(sa, sa.SA_DTYPE_BF16 if bf16 else sa.SA_DTYPE_F32)
    perm = synth.permutation(21, 1, 300)
    lens = [1, 64, 65, 1000]
    off = 0
    for s, L in enumerate(lens):
        n = (L + 63) // 64
        cache.set_pages(s, perm[off:off + n])
        off += n
    for s, L in enumerate(lens):
        k = synth.normal(22, s, (1, L, HKV, D))
        v = synth.normal(23, s, (1, L, HKV, D))
        ids = [s]
        cache.append(1, None, dev(k), dev(v), seq_ids=ids)
        cache.commit(L, seqs=[s])
        gk, gv = cache.gather(1, s, L)
        want_k = k[0].transpose(1, 0, 2)
        want_v = v[0].transpose(1, 0, 2)
        if bf16:
            want_k, want_v = synth.bf16_round(want_k), synth.bf16_round(want_v)
        np.testing.assert_array_equal(host(gk), want_k)
        np.testing.assert_array_equal(host(gv), want_v)
        assert cache.length(s) == L
    cache.close()


def test_fused_append_matches_oracle(sa, oracle, synth):
    """q/k RMSNorm (eps in the sqrt) + rotate-half RoPE at pos = len + s."""
    cache = make_cache(sa, sa.SA_DTYPE_F32)
    cos, sin = sa.rope_tables(4096, D, 1e6)
    ocos, osin = oracle.rope_tables(4096, D, 1e6)
    np.testing.assert_array_equal(host(cos), ocos)
    np.testing.assert_array_equal(host(sin), osin)
    wq = 1 + synth.normal(24, 1, D, 0.02)
    wk = 1 + synth.normal(24, 2, D, 0.02)
    start = [0, 5, 70]
    S = 3
    for s, L0 in enumerate(start):
        cache.reserve(s, L0 + S)
        cache.set_len(s, L0)
    q = synth.normal(25, 1, (3, S, HQ, D))
    k = synth.normal(25, 2, (3, S, HKV, D))
    v = synth.normal(25, 3, (3, S, HKV, D))
    q_out = cache.append(0, dev(q), dev(k), dev(v), dev(wq), dev(wk), 1e-6, rope=(cos, sin))
    q_out = host(q_out)
    for s, L0 in enumerate(start):
        pos_q = np.repeat(L0 + np.arange(S), HQ)
        want_q = oracle.apply_rope(oracle.rms_norm_rows(q[s], wq, 1e-6), pos_q, ocos, osin)
        assert_f32(q_out[s], want_q, 1e-5, 1e-6)
    cache.commit(S, n_seqs=3)
    for s, L0 in enumerate(start):
        gk, gv = cache.gather(0, s, L0 + S)
        pos_k = np.repeat(L0 + np.arange(S), HKV)
        want_k = oracle.apply_rope(oracle.rms_norm_rows(k[s], wk, 1e-6), pos_k, ocos, osin)
        assert_f32(host(gk)[:, L0:].transpose(1, 0, 2), want_k, 1e-5, 1e-6)
        np.testing.assert_array_equal(host(gv)[:, L0:].transpose(1, 0, 2), v[s])
    cache.close()


@pytest.mark.parametrize("bf16", [False, True])
def test_paged_decode_matches_oracle(sa, oracle, synth, bf16):
    lens = [1, 63, 64, 65, 1000, 5000]
    cache = sa.KVCache(1, HKV, D, len(lens), 80, 400, sa.SA_DTYPE_BF16 if bf16 else sa.SA_DTYPE_F32)
    perm = synth.permutation(26, 1, 400)
    off = 0
    ks, vs = [], []
    for s, L in enumerate(lens):
        n = (L + 63) // 64
        cache.set_pages(s, perm[off:off + n])
        off += n
        k = synth.normal(27, s, (1, L, HKV, D))
        v = synth.normal(28, s, (1, L, HKV, D))
        cache.append(0, None, dev(k), dev(v), seq_ids=[s])
        cache.commit(L, seqs=[s])
        ks.append(k[0].transpose(1, 0, 2))
        vs.append(v[0].transpose(1, 0, 2))
    q = synth.normal(29, 1, (len(lens), HQ, D))
    out = host(cache.decode(0, dev(q), float(SCALE)))
    for s in range(len(lens)):
        k, v = ks[s][None], vs[s][None]
        exact = oracle.decode_gqa(q[s][None], k, v, SCALE)[0]
        if bf16:
            same_in = oracle.decode_gqa(q[s][None], synth.bf16_round(k), synth.bf16_round(v), SCALE)[0]
            assert_f32(out[s], same_in)
            assert rel_l2(out[s], exact) <= 2e-2
        else:
            assert_f32(out[s], exact)
    cache.close()


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("d,hq,hkv", [(8, 4, 2), (16, 4, 2), (32, 4, 4), (32, 16, 2), (64, 16, 8), (256, 8, 8)])
def test_head_dims_append_gather_decode(sa, oracle, synth, bf16, d, hq, hkv):
    """Head sizes other than 128 through the cache, in fp32 and bf16: the
    fused q/k norm + RoPE append (against the oracle), the gather (bit-exact
    round trip of what the append stored) and the paged decode (against the
    oracle's STANDARD decode on the stored K/V), on shuffled pages, lengths
    1 .. 700.  A K/V row then spans 1 to 64 lanes of a wave."""
    lens = [1, 63, 64, 65, 700]
    dt = sa.SA_DTYPE_BF16 if bf16 else sa.SA_DTYPE_F32
    cache = sa.KVCache(1, hkv, d, len(lens), 16, 64, dt)
    perm = synth.permutation(90 + d, 1, 64)
    off = 0
    cos, sin = sa.rope_tables(1024, d, 1e6)
    ocos, osin = oracle.rope_tables(1024, d, 1e6)
    wk = (1 + synth.normal(91, d, d, 0.1)).astype(np.float32)
    for s, L in enumerate(lens):
        n = (L + 63) // 64
        cache.set_pages(s, perm[off:off + n])
        off += n
        k = synth.normal(92 + d, s, (1, L, hkv, d))
        v = synth.normal(93 + d, s, (1, L, hkv, d))
        cache.append(0, None, dev(k), dev(v), None, dev(wk), 1e-6, rope=(cos, sin), seq_ids=[s])
        cache.commit(L, seqs=[s])
        gk, gv = cache.gather(0, s, L)
        want_k = oracle.apply_rope(oracle.rms_norm_rows(k[0].reshape(-1, d), wk, 1e-6),
                                   np.repeat(np.arange(L), hkv), ocos, osin).reshape(L, hkv, d).transpose(1, 0, 2)
        want_v = v[0].transpose(1, 0, 2)
        if bf16:
            np.testing.assert_array_equal(host(gv), synth.bf16_round(want_v))
            assert rel_l2(host(gk), want_k) <= 4e-3
        else:
            np.testing.assert_array_equal(host(gv), want_v)
            assert_f32(host(gk), want_k, 1e-5, 1e-6)
    q = synth.normal(94 + d, 1, (len(lens), hq, d))
    sc = float(1 / np.sqrt(d))
    out = host(cache.decode(0, dev(q), sc))
    for s, L in enumerate(lens):
        gk, gv = cache.gather(0, s, L)
        want = oracle.decode_gqa(q[s][None], host(gk)[None], host(gv)[None], np.float32(sc))[0]
        assert_f32(out[s], want)
    cache.close()


def test_paged_decode_seq_ids_subset(sa, oracle, synth):
    """Decode a permuted subset of cache rows through host seq_ids."""
    cache = sa.KVCache(1, HKV, D, 4, 20, 64, sa.SA_DTYPE_F32)
    data = {}
    for s, L in enumerate([100, 300, 7, 900]):
        cache.reserve(s, L)
        k = synth.normal(30, s, (1, L, HKV, D))
        v = synth.normal(31, s, (1, L, HKV, D))
        cache.append(0, None, dev(k), dev(v), seq_ids=[s])
        cache.commit(L, seqs=[s])
        data[s] = (k[0].transpose(1, 0, 2)[None], v[0].transpose(1, 0, 2)[None])
    ids = [3, 0, 2]
    q = synth.normal(32, 1, (3, HQ, D))
    out = host(cache.decode(0, dev(q), float(SCALE), seq_ids=ids))
    for i, s in enumerate(ids):
        assert_f32(out[i], oracle.decode_gqa(q[i][None], *data[s], SCALE)[0])
    cache.close()


def run_layer_decode_loop(sa, synth, bf16, steps=100, prompt=128, seed=40, fused=False):
    """One layer, B=1, 16q/8kv, D=128: prompt append, then `steps` decode steps
    (append, decode, commit as three calls, or fused: one sa_append_decode
    call that commits).  Returns (GPU outputs [steps, 16, 128], the dense fp32
    K/V the oracle needs, the roped q of each step)."""
    cache = sa.KVCache(1, HKV, D, 1, (prompt + steps + 63) // 64, (prompt + steps + 63) // 64,
                       sa.SA_DTYPE_BF16 if bf16 else sa.SA_DTYPE_F32)
    cos, sin = sa.rope_tables(prompt + steps, D, 1e6)
    wq = dev(1 + synth.normal(seed, 1, D, 0.02))
    wk = dev(1 + synth.normal(seed, 2, D, 0.02))
    cache.reserve(0, prompt + steps)
    kp = synth.normal(seed, 3, (1, prompt, HKV, D))
    vp = synth.normal(seed, 4, (1, prompt, HKV, D))
    cache.append(0, None, dev(kp), dev(vp), None, wk, 1e-6, rope=(cos, sin))
    cache.commit(prompt, n_seqs=1)
    outs, qs = [], []
    q_all = synth.normal(seed, 5, (steps, 1, 1, HQ, D))
    k_all = synth.normal(seed, 6, (steps, 1, 1, HKV, D))
    v_all = synth.normal(seed, 7, (steps, 1, 1, HKV, D))
    ws = torch.zeros(max(cache.decode_ws_bytes(1, HQ), 1), dtype=torch.uint8, device="cuda")
    out = torch.empty(1, HQ, D, device="cuda")
    q_r = torch.empty(1, HQ, D, device="cuda")
    for t in range(steps):
        if fused:
            cache.append_decode(0, dev(q_all[t]).view(1, HQ, D), dev(k_all[t]).view(1, HKV, D),
                                dev(v_all[t]).view(1, HKV, D), float(SCALE), wq, wk, 1e-6, rope=(cos, sin), out=out,
                                q_out=q_r, ws=ws, commit=True)
        else:
            q_r = cache.append(0, dev(q_all[t]), dev(k_all[t]), dev(v_all[t]), wq, wk, 1e-6, rope=(cos, sin))
            cache.decode(0, q_r.view(1, HQ, D), float(SCALE), n_pending=1, out=out, ws=ws)
            cache.commit(1, n_seqs=1)
        assert cache.length(0) == prompt + t + 1
        outs.append(host(out).copy())
        qs.append(host(q_r).reshape(HQ, D))
    gk, gv = cache.gather(0, 0, prompt + steps)
    cache.close()
    return (np.stack(outs)[:, 0], host(gk), host(gv), np.stack(qs),
            (kp, vp, q_all, k_all, v_all, host(wq), host(wk)))


@pytest.mark.parametrize("fused", [False, True])
def test_layer_decode_loop_fp32(sa, oracle, synth, fused):
    prompt, steps = 128, 100
    outs, gk, gv, qs, raw = run_layer_decode_loop(sa, synth, False, steps, prompt, fused=fused)
    kp, vp, q_all, k_all, v_all, wq, wk = raw
    cos, sin = oracle.rope_tables(prompt + steps, D, 1e6)
    # oracle K/V: normed + roped keys at their positions, raw values
    k_tok = np.concatenate([kp[0], k_all[:, 0, 0]], 0)          # [N, HKV, D]
    v_tok = np.concatenate([vp[0], v_all[:, 0, 0]], 0)
    N = prompt + steps
    kk = oracle.apply_rope(oracle.rms_norm_rows(k_tok, wk, 1e-6), np.repeat(np.arange(N), HKV), cos, sin)
    assert_f32(gk.transpose(1, 0, 2), kk, 1e-5, 1e-6)
    np.testing.assert_array_equal(gv.transpose(1, 0, 2), v_tok)
    K = kk.transpose(1, 0, 2)[None]
    V = v_tok.transpose(1, 0, 2)[None]
    for t in range(steps):
        pos = prompt + t
        q_want = oracle.apply_rope(oracle.rms_norm_rows(q_all[t, 0, 0], wq, 1e-6), np.full(HQ, pos), cos, sin)
        assert_f32(qs[t], q_want, 1e-5, 1e-6)
        want = oracle.decode_gqa(q_want[None], K[:, :, : pos + 1], V[:, :, : pos + 1], SCALE)[0]
        assert_f32(outs[t], want)


@pytest.mark.parametrize("fused", [False, True])
def test_layer_decode_loop_bf16(sa, oracle, synth, fused):
    """bf16 KV: relative L2 <= 2e-2 per step, and a greedy readout of the
    attention output (fixed random projection to 512 logits) picks the same
    token as the oracle on the same bf16 K/V for 32 steps."""
    prompt, steps = 128, 32
    outs, gk, gv, qs, raw = run_layer_decode_loop(sa, synth, True, steps, prompt, fused=fused)
    kp, vp, q_all, k_all, v_all, wq, wk = raw
    cos, sin = oracle.rope_tables(prompt + steps, D, 1e6)
    N = prompt + steps
    k_tok = np.concatenate([kp[0], k_all[:, 0, 0]], 0)
    v_tok = np.concatenate([vp[0], v_all[:, 0, 0]], 0)
    kk = oracle.apply_rope(oracle.rms_norm_rows(k_tok, wk, 1e-6), np.repeat(np.arange(N), HKV), cos, sin)
    K = kk.transpose(1, 0, 2)[None]
    V = v_tok.transpose(1, 0, 2)[None]
    # stored K is the fp32 normed+roped key rounded to bf16; the fp32 key may
    # differ from the oracle's by an ulp, so the rounding may land one bf16 ulp
    # away.  V is stored as given, so its rounding is exact.
    assert np.all(np.abs(gk - synth.bf16_round(K)[0]) <= np.abs(K[0]) * 2.0 ** -7)
    np.testing.assert_array_equal(gv, synth.bf16_round(V)[0])
    Kb, Vb = gk[None], gv[None]       # the bf16 K/V the GPU attends over
    head = synth.normal(41, 9, (HQ * D, 512), 0.02)
    for t in range(steps):
        pos = prompt + t
        q_want = oracle.apply_rope(oracle.rms_norm_rows(q_all[t, 0, 0], wq, 1e-6), np.full(HQ, pos), cos, sin)
        exact = oracle.decode_gqa(q_want[None], K[:, :, : pos + 1], V[:, :, : pos + 1], SCALE)[0]
        same = oracle.decode_gqa(q_want[None], Kb[:, :, : pos + 1], Vb[:, :, : pos + 1], SCALE)[0]
        assert rel_l2(outs[t], exact) <= 2e-2
        assert_f32(outs[t], same, 1e-4, 1e-5)
        assert int(np.argmax(outs[t].reshape(-1) @ head)) == int(np.argmax(same.reshape(-1) @ head))


def test_reference_layer_golden(sa):
    """The reference decoder layer (KVCache, prompt of 8 + 4 steps) reproduced by
    append + prefill + paged decode: STANDARD exactly, STREAMING with its
    scale-on-output applied afterwards."""
    meta, g = gi.load("layer")
    _, _, _, wq, wk = gi.layer_inputs()
    Hq, Hkv, P = 4, 2, meta["prompt"]
    eff = g["qkv_eff"]
    N = eff.shape[0]
    q = eff[:, : Hq * D].reshape(N, Hq, D)
    k = eff[:, Hq * D:(Hq + Hkv) * D].reshape(N, Hkv, D)
    v = eff[:, (Hq + Hkv) * D:].reshape(N, Hkv, D)
    cache = sa.KVCache(1, Hkv, D, 1, 1, 1, sa.SA_DTYPE_F32)
    cache.reserve(0, N)
    cos, sin = sa.rope_tables(4096, D, 1e6)
    dwq, dwk = dev(wq), dev(wk)
    # prompt: append all P tokens, prefill attention on the normed+roped q/k
    qr = cache.append(0, dev(q[:P][None]), dev(k[:P][None]), dev(v[:P][None]), dwq, dwk, 1e-6, rope=(cos, sin))
    cache.commit(P, n_seqs=1)
    gk, gv = cache.gather(0, 0, P)
    pre = sa.prefill_causal(qr[0].transpose(0, 1).contiguous()[None], gk[None].contiguous(),
                            gv[None].contiguous(), float(SCALE))
    std = [host(pre)[0].transpose(1, 0, 2)]
    strm = [std[0]]
    for t in range(P, N):
        qr = cache.append(0, dev(q[t][None, None]), dev(k[t][None, None]), dev(v[t][None, None]), dwq, dwk,
                          1e-6, rope=(cos, sin))
        qv = qr.view(1, Hq, D)
        std.append(host(cache.decode(0, qv, float(SCALE), n_pending=1)))
        strm.append(host(cache.decode(0, qv, 1.0, n_pending=1)) * SCALE)
        cache.commit(1, n_seqs=1)
    cache.close()
    assert_f32(np.concatenate(std, 0), g["attn_avx0_str0"])
    assert_f32(np.concatenate(strm, 0), g["attn_avx0_str1"])
    # the AVX2 path puts eps outside the sqrt: inside both bars
    assert_f32(np.concatenate(std, 0), g["attn_avx1_str0"])


def test_cache_errors(sa):
    cache = sa.KVCache(2, HKV, D, 2, 4, 6, sa.SA_DTYPE_F32)
    with pytest.raises(sa.SaError) as e:
        cache.reserve(0, 4 * 64 + 1)               # beyond the table row
    assert e.value.status == sa.SA_EFULL
    cache.reserve(0, 4 * 64)
    assert cache.capacity(0) == 4 * 64 and cache.capacity(1) == 0
    assert cache.capacity(2) == -1                 # no such sequence
    with pytest.raises(sa.SaError) as e:
        cache.reserve(1, 3 * 64)                   # only 2 pages left in the pool
    assert e.value.status == sa.SA_EFULL
    with pytest.raises(sa.SaError) as e:
        cache.commit(1, seqs=[1])                  # nothing reserved for seq 1
    assert e.value.status == sa.SA_EFULL
    with pytest.raises(sa.SaError) as e:
        cache.gather(5, 0, 1)                      # bad layer
    assert e.value.status == sa.SA_ERANGE
    with pytest.raises(sa.SaError) as e:
        cache.gather(0, 0, 1)                      # longer than committed
    assert e.value.status == sa.SA_ERANGE
    with pytest.raises(sa.SaError):
        cache.set_pages(1, [99])                   # page id out of range
    cache.reset()
    assert cache.length(0) == 0 and cache.capacity(0) == 0
    cache.reserve(1, 6 * 64 - 64 * 2)              # pages are back after reset
    cache.close()


@pytest.mark.parametrize("d", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("norm,rope", [(True, True), (True, False), (False, True), (False, False)])
def test_qk_norm_rope_standalone(sa, oracle, synth, d, norm, rope):
    """sa_qk_norm_rope against the oracle's RMSNorm and rotate-half RoPE; rows
    whose position is outside the table stay unrotated; out may alias x."""
    rows, max_pos = 300, 96
    x = synth.normal(95, d, (rows, d))
    w = (1 + synth.normal(95, d + 1, d, 0.1)).astype(np.float32)
    pos = (np.arange(rows) * 7 % (max_pos + 20)).astype(np.int32)   # some beyond the table
    cos, sin = sa.rope_tables(max_pos, d, 1e6)
    ocos, osin = oracle.rope_tables(max_pos, d, 1e6)
    want = oracle.rms_norm_rows(x, w, 1e-6) if norm else x.copy()
    if rope:
        inside = pos < max_pos
        want[inside] = oracle.apply_rope(want[inside], pos[inside], ocos, osin)
    xd = dev(x)
    got = sa.qk_norm_rope(xd, dev(pos, np.int32), dev(w) if norm else None, 1e-6,
                          rope=(cos, sin) if rope else None)
    assert_f32(host(got), want)
    sa.qk_norm_rope(xd, dev(pos, np.int32), dev(w) if norm else None, 1e-6,
                    rope=(cos, sin) if rope else None, out=xd)
    assert np.array_equal(host(xd), host(got))


def test_qk_norm_rope_rejects(sa):
    x = torch.zeros(4, 128, device="cuda")
    with pytest.raises(ValueError):
        sa.qk_norm_rope(x, torch.zeros(3, dtype=torch.int32, device="cuda"))
    with pytest.raises(sa.SaError):
        sa.qk_norm_rope(torch.zeros(4, 96, device="cuda"), torch.zeros(4, dtype=torch.int32, device="cuda"))


def test_set_pages_shrink_then_decode(sa, oracle, synth):
    """A 1000-token sequence cut to 4 pages decodes over its first 256 tokens:
    the device length follows the host's, so the decode sizes its grid and
    workspace for 256 tokens and reads no partial it did not write."""
    cache = sa.KVCache(1, HKV, D, 2, 20, 40, sa.SA_DTYPE_F32)
    pages = [int(p) for p in synth.permutation(33, 1, 40)[:16]]
    cache.set_pages(0, pages)
    k = synth.normal(33, 2, (1, 1000, HKV, D))
    v = synth.normal(33, 3, (1, 1000, HKV, D))
    cache.append(0, None, dev(k), dev(v), seq_ids=[0])
    cache.commit(1000, seqs=[0])
    cache.set_pages(0, pages[:4])
    assert cache.length(0) == 256 and cache.capacity(0) == 256
    q = synth.normal(33, 4, (1, HQ, D))
    out = host(cache.decode(0, dev(q), float(SCALE)))
    K = k[0, :256].transpose(1, 0, 2)[None]
    V = v[0, :256].transpose(1, 0, 2)[None]
    assert_f32(out[0], oracle.decode_gqa(q, K, V, SCALE)[0])
    # the released pages are free again: another sequence can take them
    cache.set_pages(1, pages[4:16])
    cache.close()


@pytest.mark.parametrize("bf16", [False, True])
def test_empty_sequence_decodes_to_zero(sa, oracle, synth, bf16):
    """In a batch, a sequence with no tokens gets a zero output (as the dense
    path writes for T = 0); its neighbours are unaffected."""
    cache = sa.KVCache(1, HKV, D, 3, 40, 60, sa.SA_DTYPE_BF16 if bf16 else sa.SA_DTYPE_F32)
    lens = [700, 0, 2000]
    for s, L in enumerate(lens):
        cache.reserve(s, max(L, 1))
        if L:
            k = synth.normal(34, 2 * s, (1, L, HKV, D))
            v = synth.normal(34, 2 * s + 1, (1, L, HKV, D))
            cache.append(0, None, dev(k), dev(v), seq_ids=[s])
            cache.commit(L, seqs=[s])
    q = synth.normal(34, 9, (3, HQ, D))
    out = torch.full((3, HQ, D), 7.0, device="cuda")          # stale contents
    got = host(cache.decode(0, dev(q), float(SCALE), out=out))
    assert np.all(got[1] == 0.0)
    for s in (0, 2):
        gk, gv = cache.gather(0, s, lens[s])
        assert_f32(got[s], oracle.decode_gqa(q[s][None], host(gk)[None], host(gv)[None], SCALE)[0])
    cache.close()


def test_set_pages_rejects_conflicts(sa):
    cache = sa.KVCache(1, HKV, D, 3, 8, 10, sa.SA_DTYPE_F32)
    cache.set_pages(0, [3, 4])
    with pytest.raises(sa.SaError, match="another sequence") as e:
        cache.set_pages(1, [5, 4])                 # page 4 is sequence 0's
    assert e.value.status == sa.SA_EINVAL
    with pytest.raises(sa.SaError, match="twice") as e:
        cache.set_pages(1, [6, 6])
    assert e.value.status == sa.SA_EINVAL
    cache.set_pages(0, [4, 7])                     # keeps 4, drops 3, takes 7
    cache.set_pages(1, [3])                        # 3 is free again
    cache.reserve(2, 64 * 7)                       # the other 7 pages
    with pytest.raises(sa.SaError) as e:
        cache.reserve(2, 64 * 8)
    assert e.value.status == sa.SA_EFULL
    cache.close()


def test_row_ids_checked_before_launch(sa, synth):
    """With explicit cache rows, an append past a row's pages, a bad row, a
    repeated row and a decode past a row's pages are refused on the host, and
    nothing is written."""
    cache = sa.KVCache(1, HKV, D, 4, 4, 8, sa.SA_DTYPE_F32)
    cache.reserve(0, 64)
    cache.reserve(2, 128)
    k = torch.ones(2, 1, HKV, D, device="cuda")
    cache.append(0, None, k, k, seq_ids=[2, 0])
    cache.commit(1, seqs=[2, 0])
    cache.set_len(0, 64)
    with pytest.raises(sa.SaError) as e:
        cache.append(0, None, k, k, seq_ids=[2, 0])   # row 0 is full
    assert e.value.status == sa.SA_EFULL
    with pytest.raises(sa.SaError) as e:
        cache.append(0, None, k, k, seq_ids=[2, 9])   # no row 9
    assert e.value.status == sa.SA_ERANGE
    with pytest.raises(sa.SaError) as e:
        cache.append(0, None, k, k, seq_ids=[2, 2])   # same row twice
    assert e.value.status == sa.SA_EINVAL
    q = torch.zeros(2, HQ, D, device="cuda")
    with pytest.raises(sa.SaError) as e:
        cache.decode(0, q, 1.0, n_pending=1, seq_ids=[2, 0])   # row 0 has no page for token 64
    assert e.value.status == sa.SA_ERANGE
    # the refused calls wrote nothing: row 2 holds one token of ones, row 1
    # (no pages, no tokens) decodes to zeros
    got = host(cache.decode(0, torch.ones(2, HQ, D, device="cuda"), 1.0, seq_ids=[2, 1]))
    assert cache.length(2) == 1 and cache.length(0) == 64
    np.testing.assert_array_equal(got[0], np.ones((HQ, D), np.float32))
    np.testing.assert_array_equal(got[1], np.zeros((HQ, D), np.float32))
    cache.close()


def test_cache_on_nonblocking_stream(sa, oracle, synth):
    """Reset, reserve, set_pages, append, commit and decode issued on one
    non-blocking stream run in call order (the table and length updates go on
    that stream)."""
    side = torch.cuda.Stream()
    cache = sa.KVCache(1, HKV, D, 2, 16, 32, sa.SA_DTYPE_F32)
    k = synth.normal(35, 1, (1, 900, HKV, D))
    v = synth.normal(35, 2, (1, 900, HKV, D))
    q = synth.normal(35, 3, (1, HQ, D))
    dk, dv, dq = dev(k), dev(v), dev(q)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        for rep in range(3):
            cache.reset(stream=side)
            cache.set_pages(1, [int(p) for p in synth.permutation(35, 4 + rep, 32)[:15]], stream=side)
            cache.append(0, None, dk, dv, seq_ids=[1], stream=side)
            cache.commit(900, seqs=[1], stream=side)
            out = cache.decode(0, dq, float(SCALE), seq_ids=[1], stream=side)
    side.synchronize()
    K = k[0].transpose(1, 0, 2)[None]
    V = v[0].transpose(1, 0, 2)[None]
    assert_f32(host(out)[0], oracle.decode_gqa(q, K, V, SCALE)[0])
    cache.close()
