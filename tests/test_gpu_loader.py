"""GPU parity of checkpoint loading: sa_qwen3_load_safetensors fills the
device model so that its greedy decode reproduces the reference's forward
on the weights the reference's own loader reads from the same file.

fp32 KV cache, tokens fed one at a time (the reference runs the prompt as
one prefill, then single tokens): logits max-abs <= 1e-4 at the last prompt
position and after every later token, argmax identical.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import checkpoint as ck
from test_loader import REF_CFG, tokens_for

pytestmark = pytest.mark.gpu

SHAPE_KEYS = ("num_layers", "hidden", "intermediate", "vocab", "n_q_heads", "n_kv_heads", "head_dim",
              "rms_eps", "rope_theta")


def gpu_decode(sa, model, cfg, tokens, prompt):
    """Feed tokens [B][N] one at a time through decode steps over an fp32
    paged cache; logits at the positions decode_teacher_forced reports."""
    B, N = tokens.shape
    cache = sa.KVCache(cfg["num_layers"], cfg["n_kv_heads"], cfg["head_dim"], B, 1, B, sa.SA_DTYPE_F32)
    for s in range(B):
        cache.set_pages(s, [s])
        cache.set_len(s, 0)
    logits = torch.empty(B, cfg["vocab"], dtype=torch.float32, device="cuda")
    out = []
    for t in range(N):
        tok = torch.from_numpy(np.ascontiguousarray(tokens[:, t])).to("cuda")
        model.decode_step(cache, tok, logits=logits)
        if t >= prompt - 1:
            out.append(logits.cpu().numpy())
    cache.close()
    return np.stack(out)


@pytest.fixture(scope="module")
def ref_file(tmp_path_factory, synth):
    from oracle.qwen3_model import synth_weights
    w = ck.bf16_exact(synth_weights(synth, REF_CFG, seed=31, std=0.1))
    path = tmp_path_factory.mktemp("gpu_ckpt") / "model.safetensors"
    ck.write(path, w, REF_CFG)
    return path, w


def test_loaded_model_matches_reference_loader(sa, ref, ref_file):
    path, _ = ref_file
    assert sa.Qwen3.checkpoint_shape(path)["num_layers"] == 28
    tokens = tokens_for(REF_CFG)
    model = sa.Qwen3.from_safetensors(path, max_batch=tokens.shape[0], max_pos=64)
    got = gpu_decode(sa, model, REF_CFG, tokens, prompt=3)
    model.close()
    want = ref.qwen3_forward_file(path, REF_CFG["vocab"], tokens, prompt_len=3)
    assert np.abs(got - want).max() <= 1e-4
    assert (got.argmax(-1) == want.argmax(-1)).all()


def test_tied_f32_checkpoint_matches_oracle(sa, oracle, synth, tmp_path):
    """An F32 checkpoint without lm_head.weight (tied word embeddings), GQA 4:1
    and head_dim 64: the lm_head is the embedding, matrices round to bf16
    (exact here), norm weights stay fp32."""
    from oracle.qwen3_model import synth_weights
    cfg = dict(num_layers=2, hidden=128, intermediate=96, vocab=192, n_q_heads=8, n_kv_heads=2, head_dim=64,
               rms_eps=1e-6, rope_theta=1e6, max_pos=64)
    w = synth_weights(synth, cfg, seed=4, std=0.1)
    path = tmp_path / "tied.safetensors"
    ck.write(path, w, cfg, dtype="F32", tie=True)
    model = sa.Qwen3.from_safetensors(path, max_batch=2, max_pos=64)
    tokens = tokens_for(cfg, N=7)
    got = gpu_decode(sa, model, cfg, tokens, prompt=4)
    model.close()
    want = ck.decode_teacher_forced(oracle, cfg, dict(w, lm_head=w["embed"]), tokens, prompt=4)
    assert np.abs(got - want).max() <= 1e-4
    assert (got.argmax(-1) == want.argmax(-1)).all()


def test_checkpoint_of_another_shape_is_rejected(sa, ref_file):
    path, _ = ref_file
    model = sa.Qwen3(1, 32, **dict({k: REF_CFG[k] for k in SHAPE_KEYS}, hidden=128))
    with pytest.raises(sa.SaError, match="does not match"):
        model.load_safetensors(path)
    model.close()
