"""Decode steps captured into a HIP graph and replayed.

Each step (fused q/k norm + RoPE + append, paged decode, commit; or the same
as one sa_append_decode launch) is a fixed set of launches whose parameters
the host derives from the committed lengths, so a capture of n steps replays
them exactly from the same starting length.  A replay advances the lengths on the device only; the caller sets
the host's view (sa_kvcache_set_len) before and after.  The replays run several times with eager work and synchronisations
in between, and every replay's per-step outputs must equal the eager run's
bit for bit (the same kernels with the same arguments).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_graph_replay_equals_eager(sa, synth, kv, fused):
    HQ, HKV, D, P, N = 8, 4, 128, 70, 24
    dt = sa.SA_DTYPE_F32 if kv == "f32" else sa.SA_DTYPE_BF16
    cache = sa.KVCache(1, HKV, D, 1, 2, 2, dt)
    cos, sin = sa.rope_tables(P + N, D, 1e6)
    wq = torch.from_numpy(1 + synth.normal(90, 1, D, 0.02)).cuda()
    wk = torch.from_numpy(1 + synth.normal(90, 2, D, 0.02)).cuda()
    q = torch.from_numpy(synth.normal(90, 3, (N, 1, 1, HQ, D))).cuda()
    k = torch.from_numpy(synth.normal(90, 4, (N, 1, 1, HKV, D))).cuda()
    v = torch.from_numpy(synth.normal(90, 5, (N, 1, 1, HKV, D))).cuda()
    kp = torch.from_numpy(synth.normal(90, 6, (1, P, HKV, D))).cuda()
    vp = torch.from_numpy(synth.normal(90, 7, (1, P, HKV, D))).cuda()
    ws = torch.zeros(max(cache.decode_ws_bytes(1, HQ), 1), dtype=torch.uint8, device="cuda")
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
                cache.append_decode(0, q[t].view(1, HQ, D), k[t].view(1, HKV, D), v[t].view(1, HKV, D), sc, wq, wk,
                                    1e-6, rope=(cos, sin), out=outs[t], ws=ws, commit=True)
            else:
                cache.append(0, q[t], k[t], v[t], wq, wk, 1e-6, rope=(cos, sin), q_out=qo)
                cache.decode(0, qo.view(1, HQ, D), sc, n_pending=1, out=outs[t], ws=ws)
                cache.commit(1, n_seqs=1)

    eager = torch.empty(N, 1, HQ, D, device="cuda")
    prompt()
    steps(eager)
    torch.cuda.synchronize()

    prompt()
    torch.cuda.synchronize()
    replayed = torch.empty(N, 1, HQ, D, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        steps(replayed)
    for rep in range(3):
        replayed.fill_(float("nan"))
        scratch = torch.randn(1 << 20, device="cuda")     # eager work between the replays
        (scratch * 2).sum().item()
        cache.set_len(0, P)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay {rep}"
        # the replay advanced the device lengths; the host mirror follows
        cache.set_len(0, P + N)
        assert cache.gather(0, 0, P + N)[0].isfinite().all()
    del graph
    cache.close()
