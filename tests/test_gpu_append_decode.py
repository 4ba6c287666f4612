"""GPU: sa_append_decode, one decode step of a layer in one call (q/k RMSNorm
+ RoPE at the committed length, the K/V append, paged decode over the cache
plus the new token, and optionally the commit), against the three calls it
replaces (sa_qknorm_rope_append, sa_paged_decode with n_pending = 1,
sa_kvcache_commit) on an identical cache.  The arithmetic is the same code,
so outputs, the normed and rotated q, the cache contents and the lengths must
be equal bit for bit; the output is also held to the fp32 bar against the
oracle's STANDARD decode (reference tensor_cpp/src/ops.cpp:514-641) on the
K/V the cache holds.  Sequences of lengths 0, 37, 64, 191 and 700 on
shuffled pages, called in a shuffled row order; single-chunk launches and
forced 128-token chunks (the LSE merge path).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

LENS = [0, 37, 700, 64, 191]
ORDER = [3, 0, 4, 2, 1]


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def make_cache(sa, synth, hkv, d, dt, seed):
    pages_per = [(n + 1 + 63) // 64 for n in LENS]
    n_pages = sum(pages_per) + 2
    cache = sa.KVCache(1, hkv, d, len(LENS), max(pages_per), n_pages, dt)
    perm = synth.permutation(seed, 1, n_pages)
    off = 0
    for s, n in enumerate(LENS):
        cache.set_pages(s, perm[off:off + pages_per[s]])
        off += pages_per[s]
        if n:
            k = synth.normal(seed, 10 + s, (1, n, hkv, d))
            v = synth.normal(seed, 20 + s, (1, n, hkv, d))
            cache.append(0, None, dev(k), dev(v), seq_ids=[s])
            cache.commit(n, seqs=[s])
    return cache


@pytest.fixture
def chunk_env(request):
    old = os.environ.pop("SA_DECODE_CHUNK", None)
    if request.param is not None:
        os.environ["SA_DECODE_CHUNK"] = str(request.param)
    yield request.param
    os.environ.pop("SA_DECODE_CHUNK", None)
    if old is not None:
        os.environ["SA_DECODE_CHUNK"] = old


@pytest.mark.parametrize("chunk_env", [None, 128], indirect=True)
@pytest.mark.parametrize("commit", [False, True])
@pytest.mark.parametrize("hq,hkv,d,kv", [(16, 8, 128, "f32"), (16, 8, 128, "bf16"), (8, 8, 64, "f32"),
                                         (32, 8, 128, "bf16"), (16, 4, 256, "f32")])
def test_append_decode_equals_three_calls(sa, oracle, synth, chunk_env, commit, hq, hkv, d, kv):
    dt = sa.SA_DTYPE_F32 if kv == "f32" else sa.SA_DTYPE_BF16
    seed = 50 + d + hq
    a = make_cache(sa, synth, hkv, d, dt, seed)
    b = make_cache(sa, synth, hkv, d, dt, seed)
    n = len(ORDER)
    cos, sin = sa.rope_tables(max(LENS) + 2, d, 1e6)
    wq = dev(1 + synth.normal(seed, 1, d, 0.05))
    wk = dev(1 + synth.normal(seed, 2, d, 0.05))
    q = dev(synth.normal(seed, 3, (n, hq, d)))
    k = dev(synth.normal(seed, 4, (n, hkv, d)))
    v = dev(synth.normal(seed, 5, (n, hkv, d)))
    sc = float(1 / np.sqrt(d))

    qa = torch.empty_like(q)
    out_a = a.append_decode(0, q, k, v, sc, wq, wk, 1e-6, rope=(cos, sin), q_out=qa, commit=commit, seq_ids=ORDER)
    qb = b.append(0, q.view(n, 1, hq, d), k.view(n, 1, hkv, d), v.view(n, 1, hkv, d), wq, wk, 1e-6,
                  rope=(cos, sin), seq_ids=ORDER)
    out_b = b.decode(0, qb.view(n, hq, d), sc, n_pending=1, seq_ids=ORDER)
    if commit:
        b.commit(1, seqs=ORDER)
    torch.cuda.synchronize()
    dq = (qa - qb.view(n, hq, d)).abs()
    assert torch.equal(qa, qb.view(n, hq, d)), (float(dq.max()), dq.amax(dim=2).nonzero().tolist()[:8])
    do = (out_a - out_b).abs()
    assert torch.equal(out_a, out_b), (float(do.max()), do.amax(dim=2).nonzero().tolist()[:8])
    for s, L in enumerate(LENS):
        assert a.length(s) == b.length(s) == L + int(commit)
    if not commit:                  # the appended token is there, uncommitted
        a.commit(1, seqs=ORDER)
        b.commit(1, seqs=ORDER)
    for s, L in enumerate(LENS):
        ka, va = a.gather(0, s, L + 1)
        kb, vb = b.gather(0, s, L + 1)
        assert torch.equal(ka, kb) and torch.equal(va, vb)
    # the oracle on the K/V the cache holds (its bf16 values, for a bf16 cache)
    got = out_a.cpu().numpy()
    qh = qa.cpu().numpy()
    for i, s in enumerate(ORDER):
        gk, gv = a.gather(0, s, LENS[s] + 1)
        want = oracle.decode_gqa(qh[i][None], gk.cpu().numpy()[None], gv.cpu().numpy()[None], np.float32(sc))[0]
        err = float(np.abs(got[i] - want).max())
        rel = float(np.linalg.norm(got[i] - want) / np.linalg.norm(want))
        assert err <= 1e-4 and rel <= 1e-5, (s, LENS[s], err, rel)
    a.close()
    b.close()


def test_append_decode_refusals_enqueue_nothing(sa, synth):
    hq, hkv, d = 16, 8, 128
    cache = sa.KVCache(1, hkv, d, 2, 1, 2, sa.SA_DTYPE_F32)
    cache.reserve(0, 64)
    cache.reserve(1, 64)
    k = dev(synth.normal(60, 1, (1, 64, hkv, d)))
    cache.append(0, None, k, k, seq_ids=[0])
    cache.commit(64, seqs=[0])                       # row 0 full: no room for a new token
    q = dev(synth.normal(60, 2, (2, hq, d)))
    kv = dev(synth.normal(60, 3, (2, hkv, d)))
    out = torch.full((2, hq, d), 7.0, device="cuda")
    with pytest.raises(sa.SaError) as e:
        cache.append_decode(0, q, kv, kv, 0.1, out=out, commit=True, seq_ids=[1, 0])
    assert e.value.status == sa.SA_EFULL
    with pytest.raises(sa.SaError) as e:
        cache.append_decode(0, q, kv, kv, 0.1, out=out, commit=True, seq_ids=[1, 1])
    assert e.value.status == sa.SA_EINVAL
    with pytest.raises(sa.SaError) as e:
        cache.append_decode(1, q, kv, kv, 0.1, out=out, seq_ids=[1, 0])
    assert e.value.status == sa.SA_ERANGE
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())                  # nothing ran
    assert cache.length(0) == 64 and cache.length(1) == 0
    out1 = cache.append_decode(0, q[:1], kv[:1], kv[:1], 0.1, commit=True, seq_ids=[1])
    torch.cuda.synchronize()
    assert cache.length(1) == 1
    # one token attends to itself: the output is its V in every query head of the group
    np.testing.assert_array_equal(out1.cpu().numpy()[0].reshape(hkv, 2, d),
                                  np.repeat(kv[:1].cpu().numpy()[0][:, None], 2, 1))
    cache.close()
