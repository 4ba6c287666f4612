"""GPU parity of batched paged GQA decode at the shape the 64-sequence
benchmark measures: B = 64 sequences of U[512, 32768] tokens (seeded: 979 to
31,078), 16 query / 8 KV heads, D = 128, bf16 KV in 64-token pages assigned
from a seeded shuffle of the pool.  At this size the default launch picks
2,048-token chunks (32 pages each), so chunks span many pages and page
switches fall inside a wave's tiles.

Each checked sequence is compared with the oracle's STANDARD decode
(reference tensor_cpp/src/ops.cpp:514-641) on the K/V the cache holds (the
bf16 values, gathered as fp32) at the fp32 bar: max-abs <= 1e-4, relative L2
<= 1e-5.  Checked: the shortest, the longest and 8 seeded random sequences,
at the default chunk and at forced chunks of 256, 1088, 4096 and 16384
tokens (SA_DECODE_CHUNK).
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D, B = 16, 8, 128, 64
SCALE = np.float32(1.0 / np.sqrt(D))


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def batch(sa, synth):
    """The filled cache, the queries, and the sequences to check."""
    lens = synth.batch_lengths(B)
    pages_per = [(L + 63) // 64 for L in lens]
    n_pages = sum(pages_per)
    cache = sa.KVCache(1, HKV, D, B, max(pages_per), n_pages, sa.SA_DTYPE_BF16)
    perm = synth.permutation(70, 2, n_pages)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(72)
    off = 0
    for s, L in enumerate(lens):
        cache.set_pages(s, perm[off:off + pages_per[s]])
        off += pages_per[s]
        for t0 in range(0, L, 4096):
            n = min(4096, L - t0)
            k = torch.randn(1, n, HKV, D, device="cuda", generator=gen)
            v = torch.randn(1, n, HKV, D, device="cuda", generator=gen)
            cache.append(0, None, k, v, seq_ids=[s])
            cache.commit(n, seqs=[s])
    q = torch.from_numpy(synth.normal(73, 1, (B, HQ, D))).cuda()
    order = np.argsort(lens)
    rnd = [int(x) for x in synth.permutation(73, 2, B) if x not in (order[0], order[-1])][:8]
    check = [int(order[0]), int(order[-1])] + rnd
    want = {}
    qh = q.cpu().numpy()
    for s in check:
        gk, gv = cache.gather(0, s, lens[s])
        torch.cuda.synchronize()
        want[s] = (gk.cpu().numpy()[None], gv.cpu().numpy()[None])
    yield cache, q, qh, lens, check, want
    cache.close()


@pytest.mark.parametrize("chunk", [None, 256, 1088, 4096, 16384])
def test_batched_paged_decode_bench_shape(sa, oracle, batch, chunk):
    cache, q, qh, lens, check, kv = batch
    assert min(lens) == 979 and max(lens) == 31078
    old = os.environ.pop("SA_DECODE_CHUNK", None)
    if chunk is not None:
        os.environ["SA_DECODE_CHUNK"] = str(chunk)
    try:
        out = cache.decode(0, q, float(SCALE))
        torch.cuda.synchronize()
    finally:
        os.environ.pop("SA_DECODE_CHUNK", None)
        if old is not None:
            os.environ["SA_DECODE_CHUNK"] = old
    got = out.cpu().numpy()
    for s in check:
        want = oracle.decode_gqa(qh[s][None], kv[s][0], kv[s][1], SCALE)[0]
        err = float(np.abs(got[s] - want).max())
        assert err <= 1e-4, (s, lens[s], chunk, err)
        assert rel_l2(got[s], want) <= 1e-5, (s, lens[s], chunk, rel_l2(got[s], want))
