"""GPU: the fused decode step on grids of more than one workgroup per CU.

sa_append_decode and sa_append_decode_partials run one workgroup per (KV
head, chunk, sequence).  When that grid has more workgroups than the device
has CUs, the launch takes the 4-wave workgroup instantiation (the one the
64-sequence, 28-layer decode step runs); smaller grids take the 8-wave one.
Every launch here has at least 8 KV heads x 40 sequences = 320 workgroups,
so every call below runs the 4-wave kernel; 72 sequences also take two
launches (64 rows per launch) and, with commit, the deferred length update.

Each call is compared with the three calls it replaces
(sa_qknorm_rope_append, sa_paged_decode with n_pending = 1,
sa_kvcache_commit) on an identical cache, bit for bit: the output, the normed
and rotated q, the cache contents and the lengths.  The partials form is
compared with the same three calls on q/k/v summed from the partials in the
kernel's order.  Outputs of the longest, an empty, a one-token and five
seeded sequences are also held to the fp32 bar (max-abs 1e-4, relative L2
1e-5) against the oracle's STANDARD decode (reference
tensor_cpp/src/ops.cpp:514-641) on the K/V the cache holds.

Lengths span 0 .. 4,095 cached tokens (1 to 16 chunks of the default 256
tokens; up to 32 forced chunks of 128 and 64 of 64, where bf16 workgroups
have waves without a tile), on shuffled pages, called in a shuffled row
order.  The fused launch's grid covers only the chunks that hold tokens;
SA_DECODE_COMPACT=0 runs the full (KV head, chunk, sequence) grid, and both
are held to the same bit-equality.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D = 16, 8, 128


def lengths(synth, n_seq, seed):
    fixed = [0, 1, 63, 64, 255, 256, 257, 4095]
    u = synth.uniform(seed, 7, n_seq - len(fixed))
    return fixed + [int(x * 4095) for x in u]


def make_pair(sa, synth, lens, dt, seed):
    """Two caches with identical pages and contents: every pool element
    N(0,1) (device generator), committed lengths lens, room for one token."""
    pages_per = [(n + 1 + 63) // 64 for n in lens]
    n_pages = sum(pages_per) + 3
    caches = [sa.KVCache(1, HKV, D, len(lens), max(pages_per), n_pages, dt) for _ in range(2)]
    perm = synth.permutation(seed, 1, n_pages)
    off = 0
    for s, n in enumerate(lens):
        for c in caches:
            c.set_pages(s, perm[off:off + pages_per[s]])
            c.set_len(s, n)
        off += pages_per[s]
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    for pa, pb in zip(sa.kv_pool_views(caches[0], 0), sa.kv_pool_views(caches[1], 0)):
        pa.normal_(generator=gen)
        pb.copy_(pa)
    torch.cuda.synchronize()
    return caches


@pytest.fixture
def chunk_env(request):
    old = os.environ.pop("SA_DECODE_CHUNK", None)
    if request.param is not None:
        os.environ["SA_DECODE_CHUNK"] = str(request.param)
    yield request.param
    os.environ.pop("SA_DECODE_CHUNK", None)
    if old is not None:
        os.environ["SA_DECODE_CHUNK"] = old


def three_calls(cache, q, k, v, sc, wq, wk, rope, order, commit):
    n = len(order)
    qb = cache.append(0, q.view(n, 1, HQ, D), k.view(n, 1, HKV, D), v.view(n, 1, HKV, D), wq, wk, 1e-6,
                      rope=rope, seq_ids=order)
    out = cache.decode(0, qb.view(n, HQ, D), sc, n_pending=1, seq_ids=order)
    if commit:
        cache.commit(1, seqs=order)
    return out, qb.view(n, HQ, D)


def compare(sa, oracle, synth, a, b, lens, order, out_a, qa, out_b, qb, commit, seed):
    torch.cuda.synchronize()
    dq = (qa - qb).abs()
    assert torch.equal(qa, qb), (float(dq.max()), dq.amax(dim=2).nonzero().tolist()[:8])
    do = (out_a - out_b).abs()
    assert torch.equal(out_a, out_b), (float(do.max()), do.amax(dim=2).nonzero().tolist()[:8])
    for s, L in enumerate(lens):
        assert a.length(s) == b.length(s) == L + int(commit), s
    if not commit:
        a.commit(1, seqs=order)
        b.commit(1, seqs=order)
    for pa, pb in zip(sa.kv_pool_views(a, 0), sa.kv_pool_views(b, 0)):
        assert torch.equal(pa, pb)
    got, qh = out_a.cpu().numpy(), qa.cpu().numpy()
    row_of = {s: i for i, s in enumerate(order)}
    longest = int(np.argmax(lens))
    check = [longest, lens.index(0), lens.index(1)]
    check += [int(s) for s in synth.permutation(seed, 9, len(lens)) if int(s) not in check][:5]
    sc = np.float32(1 / np.sqrt(D))
    for s in check:
        i = row_of[s]
        gk, gv = a.gather(0, s, lens[s] + 1)
        want = oracle.decode_gqa(qh[i][None], gk.cpu().numpy()[None], gv.cpu().numpy()[None], sc)[0]
        err = float(np.abs(got[i] - want).max())
        rel = float(np.linalg.norm((got[i] - want).astype(np.float64)) / np.linalg.norm(want.astype(np.float64)))
        assert err <= 1e-4 and rel <= 1e-5, (s, lens[s], err, rel)


@pytest.fixture(params=["compact", "full"])
def grid_env(request, monkeypatch):
    if request.param == "full":
        monkeypatch.setenv("SA_DECODE_COMPACT", "0")
    else:
        monkeypatch.delenv("SA_DECODE_COMPACT", raising=False)
    return request.param


@pytest.mark.parametrize("chunk_env", [None, 128, 64], indirect=True)
@pytest.mark.parametrize("n_seq,commit", [(40, True), (72, True), (72, False)])
@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_fused_wide_grid_equals_three_calls(sa, oracle, synth, chunk_env, n_seq, commit, kv, grid_env):
    assert HKV * min(n_seq, 64) > torch.cuda.get_device_properties(0).multi_processor_count
    dt = sa.SA_DTYPE_F32 if kv == "f32" else sa.SA_DTYPE_BF16
    seed = 300 + n_seq + (chunk_env or 0)
    lens = lengths(synth, n_seq, seed)
    a, b = make_pair(sa, synth, lens, dt, seed)
    order = [int(x) for x in synth.permutation(seed, 2, n_seq)]
    cos, sin = sa.rope_tables(max(lens) + 2, D, 1e6)
    wq = torch.from_numpy(1 + synth.normal(seed, 3, D, 0.05)).cuda()
    wk = torch.from_numpy(1 + synth.normal(seed, 4, D, 0.05)).cuda()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 1)
    q = torch.randn(n_seq, HQ, D, device="cuda", generator=gen)
    k = torch.randn(n_seq, HKV, D, device="cuda", generator=gen)
    v = torch.randn(n_seq, HKV, D, device="cuda", generator=gen)
    sc = float(1 / np.sqrt(D))
    qa = torch.empty_like(q)
    out_a = a.append_decode(0, q, k, v, sc, wq, wk, 1e-6, rope=(cos, sin), q_out=qa, commit=commit, seq_ids=order)
    out_b, qb = three_calls(b, q, k, v, sc, wq, wk, (cos, sin), order, commit)
    compare(sa, oracle, synth, a, b, lens, order, out_a, qa, out_b, qb, commit, seed)
    a.close()
    b.close()


@pytest.mark.parametrize("chunk_env", [None, 128, 64], indirect=True)
@pytest.mark.parametrize("n_seq,n_part", [(40, 8), (72, 3)])
@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_fused_partials_wide_grid_equals_three_calls(sa, oracle, synth, chunk_env, n_seq, n_part, kv):
    """The decoder step's form: q, k and v of the new token as the sum of the
    qkv projection's split-K partials [n_part][n_seq][(Hq + 2 Hkv) D]."""
    dt = sa.SA_DTYPE_F32 if kv == "f32" else sa.SA_DTYPE_BF16
    seed = 400 + n_seq + n_part + (chunk_env or 0)
    lens = lengths(synth, n_seq, seed)
    a, b = make_pair(sa, synth, lens, dt, seed)
    order = [int(x) for x in synth.permutation(seed, 2, n_seq)]
    cos, sin = sa.rope_tables(max(lens) + 2, D, 1e6)
    wq = torch.from_numpy(1 + synth.normal(seed, 3, D, 0.05)).cuda()
    wk = torch.from_numpy(1 + synth.normal(seed, 4, D, 0.05)).cuda()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 1)
    part = torch.randn(n_part, n_seq, (HQ + 2 * HKV) * D, device="cuda", generator=gen) * 0.5
    # the kernel's sum: fp32 adds in partial order, starting from zero
    acc = torch.zeros(n_seq, (HQ + 2 * HKV) * D, device="cuda")
    for t in range(n_part):
        acc = acc + part[t]
    q = acc[:, :HQ * D].reshape(n_seq, HQ, D).contiguous()
    k = acc[:, HQ * D:(HQ + HKV) * D].reshape(n_seq, HKV, D).contiguous()
    v = acc[:, (HQ + HKV) * D:].reshape(n_seq, HKV, D).contiguous()
    sc = float(1 / np.sqrt(D))
    qa = torch.empty(n_seq, HQ, D, device="cuda")
    out_a = a.append_decode_partials(0, part, HQ, sc, wq, wk, 1e-6, rope=(cos, sin), q_out=qa, commit=True,
                                     seq_ids=order)
    out_b, qb = three_calls(b, q, k, v, sc, wq, wk, (cos, sin), order, True)
    compare(sa, oracle, synth, a, b, lens, order, out_a, qa, out_b, qb, True, seed)
    a.close()
    b.close()
