"""GPU parity of the whole-model prefill (sa_qwen3_prefill): a prompt run as
one causal forward, then single-token decode steps, against the reference's
qwen3_forward_with_cache on the same weights (prompt as one forward, then
single tokens; compiled from the reference's sources into oracle/_ref).

fp32 KV cache: logits max-abs <= 1e-4 and relative L2 <= 1e-5 at the last
prompt position and after every later token, argmax identical.  Prompts of
one to several hundred tokens cover several 64-row GEMM tiles and query
tiles of the prefill kernel; the cache contents after prefill equal what
token-by-token decode steps append.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from test_gpu_model import SHAPE_KEYS, host_weights, rel_l2

pytestmark = pytest.mark.gpu

CFG = dict(num_layers=2, hidden=128, intermediate=192, vocab=256, n_q_heads=4, n_kv_heads=2, head_dim=64,
           rms_eps=1e-6, rope_theta=1e6)


def empty_cache(sa, cfg, B, cap, kv_dtype):
    per = (cap + 63) // 64
    cache = sa.KVCache(cfg["num_layers"], cfg["n_kv_heads"], cfg["head_dim"], B, per, B * per, kv_dtype)
    for s in range(B):
        cache.set_pages(s, list(range(s * per, (s + 1) * per)))
        cache.set_len(s, 0)
    return cache


def run(sa, cfg, model, tokens, prompt, kv_dtype):
    """Prefill tokens[:, :prompt], then decode the rest one at a time; logits
    at the last prompt position and after each later token."""
    B, N = tokens.shape
    cache = empty_cache(sa, cfg, B, N + 1, kv_dtype)
    logits = torch.empty(B, cfg["vocab"], dtype=torch.float32, device="cuda")
    dev = torch.from_numpy(np.ascontiguousarray(tokens)).to("cuda")
    nxt = model.prefill(cache, dev[:, :prompt], logits=logits)
    out, toks = [logits.cpu().numpy()], [nxt.cpu().numpy()]
    assert [cache.length(s) for s in range(B)] == [prompt] * B
    for t in range(prompt, N):
        nxt = model.decode_step(cache, dev[:, t].contiguous(), logits=logits)
        out.append(logits.cpu().numpy())
        toks.append(nxt.cpu().numpy())
    return np.stack(out), np.stack(toks), cache


# head_dim 128: the prompt's attention runs on the three-term kernel, and
# prompts of 8 or more 32-query tiles take its paired key ranges (the model
# passes the workspace).
CFG128 = dict(CFG, hidden=256, head_dim=128)


@pytest.mark.parametrize("B,prompt,steps,cfg", [(1, 1, 3, CFG), (2, 7, 4, CFG), (3, 130, 3, CFG), (1, 300, 2, CFG),
                                                (2, 300, 2, CFG128), (1, 77, 2, CFG128)])
def test_prefill_then_decode_matches_reference(sa, ref, B, prompt, steps, cfg):
    max_pos = prompt + steps + 1
    model = sa.Qwen3(B, max_pos, **{k: cfg[k] for k in SHAPE_KEYS})
    model.init_random(11 + prompt, 0.1)
    w = host_weights(sa, model, cfg)
    if cfg is CFG128 and prompt >= 256:
        assert sa.prefill_ws_bytes(sa.SA_DTYPE_F32, B, cfg["n_q_heads"], cfg["n_kv_heads"], prompt, 128) > 0
    tokens = ((np.arange(B * (prompt + steps)).reshape(B, -1) * 41 + 5 * prompt) % cfg["vocab"]).astype(np.int32)
    want = ref.qwen3_forward(w, dict(cfg, max_pos=max_pos), tokens, prompt)
    got, toks, cache = run(sa, cfg, model, tokens, prompt, sa.SA_DTYPE_F32)
    cache.close()
    model.close()
    assert np.abs(got - want).max() <= 1e-4
    for t in range(got.shape[0]):
        assert rel_l2(got[t], want[t]) <= 1e-5, t
    assert (toks == want.argmax(-1)).all()


def test_prefill_cache_equals_decode_appends(sa):
    """The K/V a prefill appends (normed, rotated K; V as projected) equal what
    the same tokens appended one decode step at a time leave in the cache."""
    B, P = 2, 70
    model = sa.Qwen3(B, P + 1, **{k: CFG[k] for k in SHAPE_KEYS})
    model.init_random(3, 0.1)
    tokens = torch.from_numpy(((np.arange(B * P).reshape(B, P) * 13 + 1) % CFG["vocab"]).astype(np.int32)).cuda()
    a = empty_cache(sa, CFG, B, P, sa.SA_DTYPE_F32)
    model.prefill(a, tokens)
    b = empty_cache(sa, CFG, B, P, sa.SA_DTYPE_F32)
    for t in range(P):
        model.decode_step(b, tokens[:, t].contiguous())
    torch.cuda.synchronize()
    for layer in range(CFG["num_layers"]):
        for s in range(B):
            ka, va = a.gather(layer, s, P)
            kb, vb = b.gather(layer, s, P)
            assert (ka - kb).abs().max().item() <= 1e-4
            assert (va - vb).abs().max().item() <= 1e-4
    a.close()
    b.close()
    model.close()


def test_prefill_rejects_bad_calls(sa):
    model = sa.Qwen3(2, 16, **{k: CFG[k] for k in SHAPE_KEYS})
    model.init_random(1, 0.1)
    cache = empty_cache(sa, CFG, 2, 16, sa.SA_DTYPE_F32)
    toks = torch.zeros(2, 17, dtype=torch.int32, device="cuda")
    with pytest.raises(sa.SaError):          # longer than the RoPE table
        model.prefill(cache, toks)
    model.prefill(cache, toks[:, :4].contiguous())
    with pytest.raises(sa.SaError, match="empty"):
        model.prefill(cache, toks[:, :4].contiguous())
    bare = sa.KVCache(CFG["num_layers"], CFG["n_kv_heads"], CFG["head_dim"], 2, 1, 2, sa.SA_DTYPE_F32)
    with pytest.raises(sa.SaError, match="full") as e:   # no pages reserved
        model.prefill(bare, toks[:, :4].contiguous())
    assert e.value.status == sa.SA_EFULL and bare.length(0) == 0
    bare.close()
    cache.close()
    model.close()
