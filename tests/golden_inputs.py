"""Inputs of the golden fixtures, rebuilt from (seed, stream) pairs.

Shared by tests/golden/make_golden.py (which runs the reference on them) and
the tests (which run the oracle and the GPU path on them).
"""
from __future__ import annotations

import numpy as np

from util import load_synth

synth = load_synth()

UNIT_GRID = [(512, 64), (1024, 128), (2048, 256), (4096, 128)]
ROPE_MAX_POS = 33024
ROPE_ROWS = [0, 1, 2, 3, 63, 64, 127, 128, 227, 1000, 4095, 8191, 16384, 32767, 32895, 33023]
PREFILL_ROWS = [0, 1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 150, 191, 199]
LAYER_PROMPT = 8


def t1024_inputs():
    """Single head, T=1024, d=128, i.i.d. N(0,1)."""
    return synth.stream_inputs(1024, 128, seed=1)


def long_inputs(T: int):
    """d=128, 0.5 N(0,1), 1% of K rows x8 (the long-context outlier workload)."""
    return synth.stream_inputs(T, 128, seed=2, scale=0.5, outlier_frac=0.01)


def unit_inputs(T: int, d: int):
    """U(-1, 1) like the reference unit test, from the package generator."""
    u = [synth.uniform(42, s, n) for s, n in ((11, d), (12, T * d), (13, T * d))]
    Q, K, V = [(2.0 * x - 1.0).astype(np.float32) for x in u]
    return Q, K.reshape(T, d), V.reshape(T, d)


def rope_inputs():
    return synth.normal(5, 1, (1, 4, 6, 128)), synth.normal(5, 2, (1, 2, 6, 128))


def decode_inputs():
    """q [2, 4, 128], k/v [2, 2, 300, 128]."""
    return (synth.normal(6, 1, (2, 4, 128)), synth.normal(6, 2, (2, 2, 300, 128)),
            synth.normal(6, 3, (2, 2, 300, 128)))


def prefill_inputs():
    """q [1, 4, 200, 128], k/v [1, 2, 200, 128]."""
    return (synth.normal(7, 1, (1, 4, 200, 128)), synth.normal(7, 2, (1, 2, 200, 128)),
            synth.normal(7, 3, (1, 2, 200, 128)))


def layer_inputs():
    """12 tokens (8-token prompt + 4 steps) of q [Hq=4], k/v [Hkv=2], D=128; norm weights."""
    n = LAYER_PROMPT + 4
    return (synth.normal(8, 1, (n, 4, 128)), synth.normal(8, 2, (n, 2, 128)),
            synth.normal(8, 3, (n, 2, 128)), 1 + synth.normal(8, 4, 128, 0.02),
            1 + synth.normal(8, 5, 128, 0.02))


# Small whole-model configurations for the decoder oracle (reference
# qwen3_forward_with_cache): shape, weight seed / std, batch, prompt, steps.
MODEL_CASES = [
    dict(cfg=dict(num_layers=2, hidden=64, intermediate=128, vocab=256, n_q_heads=4, n_kv_heads=2,
                  head_dim=16, rms_eps=1e-6, rope_theta=1e6, max_pos=64),
         seed=7, std=0.2, batch=2, prompt=5, steps=4),
    dict(cfg=dict(num_layers=3, hidden=128, intermediate=256, vocab=512, n_q_heads=4, n_kv_heads=4,
                  head_dim=32, rms_eps=1e-6, rope_theta=1e6, max_pos=64),
         seed=8, std=0.1, batch=3, prompt=3, steps=5),
    # head_dim 64 and 128: also the head sizes of the bf16 device model
    dict(cfg=dict(num_layers=2, hidden=128, intermediate=192, vocab=320, n_q_heads=4, n_kv_heads=2,
                  head_dim=64, rms_eps=1e-6, rope_theta=1e6, max_pos=64),
         seed=9, std=0.1, batch=2, prompt=6, steps=4),
    dict(cfg=dict(num_layers=2, hidden=256, intermediate=384, vocab=384, n_q_heads=4, n_kv_heads=2,
                  head_dim=128, rms_eps=1e-6, rope_theta=1e6, max_pos=64),
         seed=10, std=0.08, batch=2, prompt=5, steps=3),
]


def model_inputs(case: dict):
    """(weights, tokens [B][prompt + steps]) of one MODEL_CASES entry."""
    from oracle.qwen3_model import synth_weights
    c = case["cfg"]
    w = synth_weights(synth, c, case["seed"], case["std"])
    n = case["prompt"] + case["steps"]
    tokens = ((np.arange(case["batch"] * n).reshape(case["batch"], n) * 37 + case["seed"]) % c["vocab"])
    return w, tokens.astype(np.int32)


def load(name: str):
    import json
    from pathlib import Path
    path = Path(__file__).resolve().parent / "golden" / f"{name}.npz"
    z = np.load(path, allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    return meta, {k: z[k] for k in z.files if k != "meta"}
