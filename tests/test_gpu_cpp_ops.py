"""GPU: the C++ mirror's ops::RotaryEmbedding, ops::cross_attention,
ops::avx2::self_attention_avx2 / linear_avx2 and qwen3::test_qwen3_forward
(include/tensor_cpp/ops.h, attention_avx.h, qwen3_loader.h).

- RotaryEmbedding against the mathematics it states (element i paired with
  i + dim/2, rotated by t * theta^(-i/dim) at sequence index t, zeros past
  seq_len) in float64, and against the reference's own class
  (tensor_cpp/src/ops.cpp:424-487, compiled into oracle/_ref) where built.
  A 2i/dim frequency, a swapped sign or a rotation by head index instead of
  sequence index misses the 1e-5 bar by orders of magnitude.
- cross_attention against the oracle's decode (every query row sees every
  key) and the reference's function; a mask changes nothing, as there.
- self_attention_avx2 against the oracle (decode rows with no -inf in the
  mask, causal prefill with the causal -inf pattern; finite mask values are
  ignored, as in the reference) and the reference's function; linear_avx2
  against float64.
- test_qwen3_forward on a checkpoint file: the final-norm hidden states equal
  the oracle decoder's with an identity lm_head.
Bars: max-abs <= 1e-4 and relative L2 <= 1e-5 (fp32 on both sides) unless
stated.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

import checkpoint as ck

pytestmark = pytest.mark.gpu

DRIVER = Path(__file__).resolve().parent / "cpp" / "bin" / "libdrive_compat.so"
_I, _F, _P = C.c_int, C.c_float, C.c_void_p


@pytest.fixture(scope="module")
def drv(sa):
    assert DRIVER.exists(), "driver missing: python streaming-attention_amd/build.py --tests"
    lib = C.CDLL(str(DRIVER))
    lib.drv_last_error.restype = C.c_char_p
    lib.drv_rotary.argtypes = [_P, _I, _I, _I, _I, _I, _F, _I, _P]
    lib.drv_cross_attention.argtypes = [_P, _P, _P] + [_I] * 6 + [_F, _P, _P]
    lib.drv_test_forward.argtypes = [C.c_char_p, _P, _I, _I, _P, C.c_int64]
    lib.drv_self_attention_avx2.argtypes = [_P, _P, _P] + [_I] * 6 + [_F, _P, _I, _P]
    lib.drv_linear_avx2.argtypes = [_P, _P, _P, _I, _I, _I, _P]
    for f in (lib.drv_rotary, lib.drv_cross_attention, lib.drv_test_forward, lib.drv_self_attention_avx2,
              lib.drv_linear_avx2):
        f.restype = _I
    return lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def close(got, want, what, abs_bar=1e-4, rel_bar=1e-5):
    err = float(np.abs(got - want).max())
    rel = float(np.linalg.norm((got - want).ravel()) / max(np.linalg.norm(want.ravel()), 1e-30))
    assert err <= abs_bar and rel <= rel_bar, (what, err, rel)


def rotary_f64(x, theta, seq_len):
    B, S, H, D = x.shape
    half = D // 2
    freq = np.float64(theta) ** (-np.arange(half, dtype=np.float64) / D)
    ang = np.arange(S, dtype=np.float64)[:, None] * freq[None, :]          # [S][half]
    c, s = np.cos(ang)[None, :, None, :], np.sin(ang)[None, :, None, :]
    x0, x1 = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    out = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)
    out[:, seq_len:] = 0.0
    return out


def run_rotary(drv, x, max_seq, theta, seq_len):
    x = np.ascontiguousarray(x, np.float32)
    out = np.full_like(x, np.nan)
    rc = drv.drv_rotary(_p(x), *x.shape, max_seq, theta, seq_len, _p(out))
    return rc, out


@pytest.mark.parametrize("B,S,H,D,seq_len,theta", [(2, 10, 3, 64, 7, 10000.0), (1, 40, 2, 128, 40, 1e6),
                                                   (3, 5, 4, 256, 1, 10000.0), (2, 9, 8, 16, 9, 10000.0)])
def test_rotary_embedding(drv, ref_opt, synth, B, S, H, D, seq_len, theta):
    x = synth.normal(71, D + S, (B, S, H, D))
    rc, got = run_rotary(drv, x, 64, theta, seq_len)
    assert rc == 0, drv.drv_last_error()
    assert not got[:, seq_len:].any()                            # zeros past seq_len
    # float tables (the angle t * freq rounded to fp32) against float64: 1e-5
    close(got, rotary_f64(x, theta, seq_len), (B, S, H, D), abs_bar=1e-5, rel_bar=1e-5)
    if ref_opt is not None:
        close(got, ref_opt.rotary(x, 64, theta, seq_len), "reference", abs_bar=2e-6, rel_bar=1e-6)


def test_rotary_embedding_refusals(drv, synth):
    x = synth.normal(72, 1, (1, 4, 1, 64))
    assert run_rotary(drv, x, 64, 1e4, 5)[0] == -1                # seq_len past the input
    assert drv.drv_last_error().startswith(b"I:")
    assert run_rotary(drv, x, 3, 1e4, 4)[0] == -1                 # past max_seq_len
    assert run_rotary(drv, synth.normal(72, 2, (1, 4, 1, 7)), 64, 1e4, 4)[0] == -1   # odd dim: constructor
    assert drv.drv_last_error() == b"I:Rotary embedding dimension must be even"
    assert run_rotary(drv, synth.normal(72, 3, (1, 4, 1, 96)), 64, 1e4, 4)[0] == -1  # not a kernel head size
    assert drv.drv_last_error().startswith(b"I:")


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D", [(2, 4, 4, 3, 77, 128), (1, 16, 8, 5, 300, 64), (2, 8, 2, 1, 1, 128)])
def test_cross_attention(drv, oracle, ref_opt, synth, B, Hq, Hkv, Sq, Sk, D):
    q = synth.normal(73, Sq, (B, Hq, Sq, D))
    k = synth.normal(74, Sk, (B, Hkv, Sk, D))
    v = synth.normal(75, Sk, (B, Hkv, Sk, D))
    scale = float(1 / np.sqrt(D))
    out = np.empty_like(q)
    assert drv.drv_cross_attention(_p(q), _p(k), _p(v), B, Hq, Hkv, Sq, Sk, D, scale, None, _p(out)) == 0, \
        drv.drv_last_error()
    want = np.stack([oracle.decode_gqa(np.ascontiguousarray(q[:, :, i]), k, v, np.float32(scale))
                     for i in range(Sq)], axis=2)
    close(out, want, "oracle")
    mask = np.triu(np.full((Sq, Sk), -np.inf, np.float32), 1)     # read by nobody, as in the reference
    out_m = np.empty_like(q)
    assert drv.drv_cross_attention(_p(q), _p(k), _p(v), B, Hq, Hkv, Sq, Sk, D, scale, _p(mask), _p(out_m)) == 0
    assert np.array_equal(out, out_m)
    if ref_opt is not None and Hq == Hkv:
        close(out, ref_opt.cross_attention(q, k, v, scale), "reference")


def run_sa_avx2(drv, q, k, v, scale, mask=None):
    """mask [mrows][Sk], passed as [1][1][mrows][Sk], or None."""
    B, Hq, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    out = np.full_like(q, np.nan)
    m = None if mask is None else np.ascontiguousarray(mask, np.float32)
    rc = drv.drv_self_attention_avx2(_p(q), _p(k), _p(v), B, Hq, Hkv, Sq, Sk, D, scale,
                                     None if m is None else _p(m), 0 if m is None else m.shape[0], _p(out))
    return rc, out


@pytest.mark.parametrize("B,Hq,Hkv,Sq,Sk,D", [(2, 4, 4, 1, 300, 128), (1, 16, 8, 3, 77, 64), (2, 4, 4, 5, 5, 128)])
def test_self_attention_avx2_rows(drv, oracle, ref_opt, synth, B, Hq, Hkv, Sq, Sk, D):
    """No -inf in the mask: every query row attends to every key."""
    q = synth.normal(76, Sq, (B, Hq, Sq, D))
    k = synth.normal(77, Sk, (B, Hkv, Sk, D))
    v = synth.normal(78, Sk, (B, Hkv, Sk, D))
    scale = float(1 / np.sqrt(D))
    rc, out = run_sa_avx2(drv, q, k, v, scale)
    assert rc == 0, drv.drv_last_error()
    want = np.stack([oracle.decode_gqa(np.ascontiguousarray(q[:, :, i]), k, v, np.float32(scale))
                     for i in range(Sq)], axis=2)
    close(out, want, "oracle")
    # finite mask entries are ignored, row mask [1][1][1][Sk] or full [Sq][Sk]
    for mask in (np.zeros((1, Sk)), synth.normal(79, 1, (1, Sk)), synth.normal(79, 2, (Sq, Sk))):
        rc, out_m = run_sa_avx2(drv, q, k, v, scale, mask)
        assert rc == 0, drv.drv_last_error()
        assert np.array_equal(out, out_m)
    if ref_opt is not None and Hq == Hkv:
        close(out, ref_opt.self_attention_avx2(q, k, v, scale), "reference")
        close(out, ref_opt.self_attention_avx2(q, k, v, scale, synth.normal(79, 2, (Sq, Sk))), "reference, mask")


@pytest.mark.parametrize("B,Hq,Hkv,L,D", [(1, 4, 4, 70, 128), (2, 8, 2, 33, 64), (1, 2, 2, 1, 128)])
def test_self_attention_avx2_causal(drv, oracle, ref_opt, synth, B, Hq, Hkv, L, D):
    """The causal -inf pattern (finite values elsewhere) runs the causal prefill."""
    q = synth.normal(80, L, (B, Hq, L, D))
    k = synth.normal(81, L, (B, Hkv, L, D))
    v = synth.normal(82, L, (B, Hkv, L, D))
    scale = float(1 / np.sqrt(D))
    mask = synth.normal(83, L, (L, L))
    mask[np.triu_indices(L, 1)] = -np.inf
    rc, out = run_sa_avx2(drv, q, k, v, scale, mask)
    assert rc == 0, drv.drv_last_error()
    close(out, oracle.prefill_blockwise(q, k, v, np.float32(scale), 64), "oracle")
    if ref_opt is not None and Hq == Hkv:
        close(out, ref_opt.self_attention_avx2(q, k, v, scale, mask), "reference")


def test_self_attention_avx2_refusals(drv, synth):
    q = synth.normal(84, 1, (1, 2, 4, 64))
    k = synth.normal(84, 2, (1, 2, 6, 64))
    mask = np.zeros((4, 6), np.float32)
    mask[1, 3] = -np.inf                                          # not the causal pattern
    assert run_sa_avx2(drv, q, k, k, 0.125, mask)[0] == -1
    assert drv.drv_last_error().startswith(b"I:")
    row = np.zeros((1, 6), np.float32)
    row[0, 2] = -np.inf                                           # a key masked for every row
    assert run_sa_avx2(drv, q, k, k, 0.125, row)[0] == -1
    assert run_sa_avx2(drv, q, synth.normal(84, 3, (1, 3, 6, 64)), synth.normal(84, 3, (1, 3, 6, 64)),
                       0.125)[0] == -1                            # 2 query heads over 3 key heads


@pytest.mark.parametrize("M,K,N,bias", [(5, 33, 70, True), (64, 256, 64, False)])
def test_linear_avx2(drv, synth, M, K, N, bias):
    x = synth.normal(85, M * 7 + K, (M, K))
    w = synth.normal(86, N * 3 + K, (N, K), 0.05)
    b = synth.normal(87, N, (N,)) if bias else None
    out = np.empty((M, N), np.float32)
    assert drv.drv_linear_avx2(_p(x), _p(w), None if b is None else _p(b), M, K, N, _p(out)) == 0, \
        drv.drv_last_error()
    want = x.astype(np.float64) @ w.astype(np.float64).T + (b if bias else 0.0)
    scale = max(1.0, float(np.abs(want).max()))
    assert float(np.abs(out - want).max()) <= 1e-5 * scale


def test_test_qwen3_forward_hidden_states(drv, oracle, synth, tmp_path):
    from oracle.qwen3_model import synth_weights
    cfg = dict(num_layers=2, hidden=128, intermediate=96, vocab=160, n_q_heads=4, n_kv_heads=2, head_dim=128,
               rms_eps=1e-6, rope_theta=1e6, max_pos=16)
    w = synth_weights(synth, cfg, seed=8, std=0.1)
    path = tmp_path / "m.safetensors"
    ck.write(path, w, cfg, dtype="F32")
    B, N = 2, 6
    tokens = ((np.arange(B * N).reshape(B, N) * 37 + 5) % cfg["vocab"]).astype(np.int32)
    got = np.empty((B, N, cfg["hidden"]), np.float32)
    rc = drv.drv_test_forward(str(path).encode(), _p(tokens), B, N, _p(got), got.size)
    assert rc == 0, drv.drv_last_error()
    eye = dict(w, lm_head=np.eye(cfg["hidden"], dtype=np.float32))
    want = ck.decode_teacher_forced(oracle, dict(cfg, vocab=cfg["hidden"]), eye, tokens, prompt=1)   # [N][B][H]
    close(got, want.transpose(1, 0, 2), "hidden states")
