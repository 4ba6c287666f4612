"""Greedy-step parity of the device decoder (include/sa_qwen3.h) against the
CPU decoder oracle (oracle/qwen3_model.py), for a chosen subset of a batch.

Used by the GPU tests and, outside its timed region, by bench.py's 28-layer
decode workload.  The oracle runs on the model's own weights (read back from
the device, bf16 widened exactly) and on the cache's own contents (gathered
per sequence), so a comparison isolates one decode step.  Rows of a batched
step are independent (per-row GEMMs, per-sequence attention), so the chosen
rows of the device's B-row step are compared with an oracle step over those
rows alone.
"""
from __future__ import annotations

import numpy as np


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def host_weights(sa, model, cfg):
    """The model's weights as the oracle's fp32 dict (exact: bf16 widens exactly)."""
    from oracle.qwen3_model import TENSORS
    H, I, V = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    Hq, Hkv, D = cfg["n_q_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    shapes = {sa.QW_EMBED: (V, H), sa.QW_LM_HEAD: (V, H), sa.QW_FINAL_NORM: (H,), sa.QW_IN_NORM: (H,),
              sa.QW_QKV: ((Hq + 2 * Hkv) * D, H), sa.QW_Q_NORM: (D,), sa.QW_K_NORM: (D,),
              sa.QW_O: (H, Hq * D), sa.QW_POST_NORM: (H,), sa.QW_GATE_UP: (2 * I, H), sa.QW_DOWN: (H, I)}

    def get(which, layer=0):
        return model.tensor(which, layer).float().cpu().numpy().reshape(shapes[which])

    ids = dict(zip(TENSORS, (sa.QW_IN_NORM, sa.QW_QKV, sa.QW_Q_NORM, sa.QW_K_NORM, sa.QW_O, sa.QW_POST_NORM,
                             sa.QW_GATE_UP, sa.QW_DOWN)))
    return {"embed": get(sa.QW_EMBED), "final_norm": get(sa.QW_FINAL_NORM), "lm_head": get(sa.QW_LM_HEAD),
            "layers": [{t: get(ids[t], l) for t in TENSORS} for l in range(cfg["num_layers"])]}


def subset_store(cache, cfg, seqs, room: int, kv_bf16: bool):
    """An oracle KvStore holding cache rows `seqs` at their committed lengths,
    each with room for `room` more tokens (per-sequence capacities, so one long
    sequence does not size the others)."""
    from oracle.qwen3_model import KvStore
    st = KvStore(cfg["num_layers"], len(seqs), cfg["n_kv_heads"], cfg["head_dim"], 1, kv_bf16)
    lens = [cache.length(s) for s in seqs]
    for l in range(cfg["num_layers"]):
        for b, (s, L) in enumerate(zip(seqs, lens)):
            K = np.zeros((cfg["n_kv_heads"], L + room, cfg["head_dim"]), np.float32)
            V = np.zeros_like(K)
            if L:
                k, v = cache.gather(l, s, L)
                K[:, :L] = k.cpu().numpy()
                V[:, :L] = v.cpu().numpy()
            st.K[l][b], st.V[l][b] = K, V
    st.lens[:] = lens
    return st


class SubsetChecker:
    """Oracle steps for rows `seqs` of a device batch, started from the cache
    as it stands at construction; step(tokens_all, logits_all) compares the
    device's logits rows of the step just taken and returns the worst-row
    relative L2, the max-abs error and whether the greedy tokens agree."""

    def __init__(self, sa, oracle, model, cache, cfg, seqs, max_steps: int, kv_bf16: bool):
        from oracle.qwen3_model import Qwen3Decoder
        self.seqs = list(seqs)
        self.store = subset_store(cache, cfg, self.seqs, max_steps, kv_bf16)
        max_pos = int(self.store.lens.max()) + max_steps + 1
        self.dec = Qwen3Decoder(host_weights(sa, model, cfg), dict(cfg, max_pos=max_pos), oracle)

    def want(self, tokens_all):
        """The oracle's logits [len(seqs)][vocab] for this step's input tokens."""
        tok = np.asarray(tokens_all)[self.seqs]
        return self.dec.step(tok, self.store)

    def compare(self, want, got_logits_all, got_tokens_all):
        got = np.asarray(got_logits_all)[self.seqs]
        rows = [rel_l2(g, w) for g, w in zip(got, want)]
        same = bool(np.array_equal(np.asarray(got_tokens_all)[self.seqs], want.argmax(-1)))
        return {"worst_row_rel_l2": max(rows), "max_abs_err": float(np.abs(got - want).max()),
                "tokens_identical": same, "row_rel_l2": rows}
