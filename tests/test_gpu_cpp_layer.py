"""GPU: the C++ mirror's decoder layer and forward against the reference's own
golden vectors.

tests/cpp/libdrive_compat.cpp drives qwen3_decoder_layer[_avx]_with_cache and
qwen3_forward[_avx]_with_cache of include/tensor_cpp exactly as
oracle/ref_shim.cpp drives the reference when it writes tests/golden: the
identity-projection layer (its attention output appears verbatim in its
output) over an 8-token prompt and 4 single-token steps -> layer.npz, and
teacher-forced forwards of the small models (head_dim 16, 32, 64 and 128) ->
qwen3_forward.npz.  Bar (fp32 weights and activations on both sides):
max-abs <= 1e-4 and relative L2 <= 1e-5, and the same argmax for logits.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import golden_inputs as gi

pytestmark = pytest.mark.gpu

DRIVER = Path(__file__).resolve().parent / "cpp" / "bin" / "libdrive_compat.so"
_I, _F, _P = C.c_int, C.c_float, C.c_void_p


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.fixture(scope="module")
def drv(sa):
    assert DRIVER.exists(), "driver missing: python streaming-attention_amd/build.py --tests"
    lib = C.CDLL(str(DRIVER))
    lib.drv_last_error.restype = C.c_char_p
    lib.drv_layer_attention.argtypes = [_I] * 5 + [_P] * 5 + [_F, _I, _I, _I, _P, _P]
    weights = [_P] * 12 + [_I, _P]
    lib.drv_qwen3_forward.argtypes = [_I] * 7 + [_F, _I, _I, _I] + weights
    lib.drv_qwen3_forward_nocache.argtypes = [_I] * 7 + [_F, _I, _I] + weights
    for f in (lib.drv_layer_attention, lib.drv_qwen3_forward, lib.drv_qwen3_forward_nocache):
        f.restype = _I
    return lib


def close(got, want, what):
    err = float(np.abs(got - want).max())
    rel = float(np.linalg.norm((got - want).ravel()) / np.linalg.norm(want.ravel()))
    assert err <= 1e-4 and rel <= 1e-5, (what, err, rel)


@pytest.mark.parametrize("streaming", [0, 1])
@pytest.mark.parametrize("avx2", [0, 1])
def test_layer_with_cache_matches_reference_golden(drv, avx2, streaming):
    meta, g = gi.load("layer")
    q, k, v, wq, wk = (np.ascontiguousarray(a, np.float32) for a in gi.layer_inputs())
    N, Hq, D = q.shape
    Hkv = k.shape[1]
    attn = np.empty((N, Hq, D), np.float32)
    eff = np.empty((N, (Hq + 2 * Hkv) * D), np.float32)
    rc = drv.drv_layer_attention(Hq, Hkv, D, meta["prompt"], N - meta["prompt"], _p(q), _p(k), _p(v), _p(wq),
                                 _p(wk), 1e-6, 4096, avx2, streaming, _p(attn), _p(eff))
    assert rc == 0, drv.drv_last_error()
    close(eff, g["qkv_eff"], "input RMSNorm")
    close(attn, g[f"attn_avx{avx2}_str{streaming}"], f"attention avx2={avx2} streaming={streaming}")


def _forward(drv, cached, case, avx2):
    """Logits of a MODEL_CASES entry through the driver: cached, the
    teacher-forced forwards [steps + 1][B][V]; otherwise one forward over all
    tokens [B][N][V].  Returns (status, logits)."""
    c = case["cfg"]
    w, tokens = gi.model_inputs(case)
    L = w["layers"]
    stack = {t: np.ascontiguousarray(np.stack([layer[t] for layer in L]), np.float32) for t in L[0]}
    glob = {t: np.ascontiguousarray(w[t], np.float32) for t in ("embed", "final_norm", "lm_head")}
    tokens = np.ascontiguousarray(tokens, np.int32)
    B, N = tokens.shape
    P = case["prompt"]
    shape = [c[k] for k in ("num_layers", "hidden", "intermediate", "vocab", "n_q_heads", "n_kv_heads",
                            "head_dim")] + [c["rms_eps"], B]
    weights = [_p(tokens), _p(glob["embed"]), _p(stack["in_norm"]), _p(stack["qkv"]), _p(stack["q_norm"]),
               _p(stack["k_norm"]), _p(stack["o"]), _p(stack["post_norm"]), _p(stack["gate_up"]),
               _p(stack["down"]), _p(glob["final_norm"]), _p(glob["lm_head"]), avx2]
    if cached:
        out = np.empty((N - P + 1, B, c["vocab"]), np.float32)
        rc = drv.drv_qwen3_forward(*shape, P, N - P, *weights, _p(out))
    else:
        out = np.empty((B, N, c["vocab"]), np.float32)
        rc = drv.drv_qwen3_forward_nocache(*shape, N, *weights, _p(out))
    return rc, out


def _check_logits(got, want, what):
    close(got, want, what)
    assert (got.argmax(-1) == want.argmax(-1)).all(), what


@pytest.mark.parametrize("avx2", [0, 1])
@pytest.mark.parametrize("i", range(len(gi.MODEL_CASES)))
def test_forward_with_cache_matches_reference_golden(drv, i, avx2):
    case = gi.MODEL_CASES[i]
    _, g = gi.load("qwen3_forward")
    rc, got = _forward(drv, True, case, avx2)
    assert rc == 0, drv.drv_last_error()
    _check_logits(got, g[f"logits_avx{i}" if avx2 else f"logits{i}"], f"case {i} avx2={avx2}")


@pytest.mark.parametrize("avx2", [0, 1])
@pytest.mark.parametrize("i", range(len(gi.MODEL_CASES)))
def test_forward_without_cache_matches_reference_golden(drv, i, avx2):
    """qwen3_forward over the whole sequence at once (causal prefill of
    prompt + steps tokens): the logits at the prompt's last position and at
    every later one equal the reference's teacher-forced cached forwards."""
    case = gi.MODEL_CASES[i]
    _, g = gi.load("qwen3_forward")
    rc, got = _forward(drv, False, case, avx2)
    assert rc == 0, drv.drv_last_error()
    P = case["prompt"]
    _check_logits(got[:, P - 1:].transpose(1, 0, 2), g[f"logits_avx{i}" if avx2 else f"logits{i}"],
                  f"case {i} avx2={avx2}")
