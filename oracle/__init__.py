"""ctypes bindings of the CPU oracle (liboracle.so) and of the reference built
from its own sources (_ref/libsa_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  All
arrays are numpy float32, C-contiguous.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
ORACLE_LIB = ORACLE_DIR / "liboracle.so"
REF_LIB = ORACLE_DIR / "_ref" / "libsa_ref.so"

_P = C.c_void_p
_I = C.c_int
_F = C.c_float
_D = C.c_double

_ORACLE_SIGS = {
    "or_streaming_serial": (None, [_P, _P, _P, _I, _I, _I, _P]),
    "or_naive_serial": (None, [_P, _P, _P, _I, _I, _P]),
    "or_streaming_omp": (None, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "or_l2_error": (_F, [_P, _P, _I]),
    "or_max_error": (_F, [_P, _P, _I]),
    "or_rms_norm_rows": (None, [_P, _P, _I, _I, _F, _I, _P]),
    "or_rope_tables": (None, [_I, _I, _F, _P, _P]),
    "or_apply_rope": (None, [_P, _I, _I, _P, _P, _P, _P]),
    "or_decode_gqa": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _F, _P]),
    "or_decode_streaming_compat": (None, [_P, _P, _P, _I, _I, _I, _I, _F, _I, _P]),
    "or_prefill_blockwise": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _P, _I, _P]),
    "or_sdpa_f64": (None, [_P, _P, _P, _I, _I, _I, _D, _I, _I, _P]),
    "or_sequence_np1": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _F, _I, _I, _P]),
}

_REF_SIGS = {
    "ref_streaming_serial": (None, [_P, _P, _P, _I, _I, _I, _P]),
    "ref_naive_serial": (None, [_P, _P, _P, _I, _I, _P]),
    "ref_streaming_omp": (None, [_P, _P, _P, _I, _I, _I, _I, _P]),
    "ref_naive_omp": (None, [_P, _P, _P, _I, _I, _I, _P]),
    "ref_l2_error": (_F, [_P, _P, _I]),
    "ref_max_error": (_F, [_P, _P, _I]),
    "ref_rope_freqs": (None, [_I, _I, _F, _P, _P]),
    "ref_apply_rope": (None, [_P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    "ref_repeat_kv": (None, [_P, _I, _I, _I, _I, _I, _P]),
    "ref_self_attention": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P]),
    "ref_self_attention_streaming": (None, [_P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _P]),
    "ref_blockwise": (None, [_P, _P, _P, _I, _I, _I, _I, _F, _I, _I, _I, _P]),
    "ref_layer_attention": (_I, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _F, _I, _I, _I, _P, _P]),
    "ref_qwen3_forward": (_I, [_I, _I, _I, _I, _I, _I, _I, _F, _I, _I, _I] + [_P] * 12 + [_I, _P]),
    "ref_set_threads": (None, [_I]),
    "ref_qwen3_forward_file": (_I, [C.c_char_p, _F, _I, _I, _I, _P, _P]),
    "ref_load_weights": (_I, [C.c_char_p, _P, _P, C.c_int64]),
    "ref_rotary": (_I, [_P, _I, _I, _I, _I, _I, _F, _I, _P]),
    "ref_argmax": (C.c_long, [_P, _P, _I, _I, _I, _P, C.c_long, _P, _P]),
    "ref_cross_attention": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _F, _P]),
    "ref_self_attention_avx2": (None, [_P, _P, _P, _I, _I, _I, _I, _I, _F, _P, _I, _P]),
    "ref_time_decode_layer": (_I, [_I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
}


def _bind(path: Path, sigs: dict) -> C.CDLL:
    lib = C.CDLL(str(path))
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def _p(a: np.ndarray) -> int:
    assert a.flags.c_contiguous, "arrays must be C-contiguous"
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class Oracle:
    """The C restatement of the reference (oracle.c)."""

    def __init__(self, path: Path = ORACLE_LIB):
        if not path.exists():
            raise RuntimeError(f"{path} missing: run `make -C oracle oracle`")
        self.lib = _bind(path, _ORACLE_SIGS)

    def streaming_serial(self, Q, K, V, block):
        Q, K, V = _f32(Q), _f32(K), _f32(V)
        T, d = (K.shape[0], K.shape[1]) if K.ndim == 2 else (0, Q.size)
        O = np.empty(d, np.float32)
        self.lib.or_streaming_serial(_p(Q), _p(K), _p(V), T, d, block, _p(O))
        return O

    def naive_serial(self, Q, K, V):
        Q, K, V = _f32(Q), _f32(K), _f32(V)
        T, d = K.shape
        O = np.empty(d, np.float32)
        self.lib.or_naive_serial(_p(Q), _p(K), _p(V), T, d, _p(O))
        return O

    def streaming_omp(self, Q, K, V, block, nthreads=0):
        Q, K, V = _f32(Q), _f32(K), _f32(V)
        T, d = K.shape
        O = np.empty(d, np.float32)
        self.lib.or_streaming_omp(_p(Q), _p(K), _p(V), T, d, block, nthreads, _p(O))
        return O

    def l2_error(self, a, b):
        a, b = _f32(a).ravel(), _f32(b).ravel()
        return float(self.lib.or_l2_error(_p(a), _p(b), a.size))

    def max_error(self, a, b):
        a, b = _f32(a).ravel(), _f32(b).ravel()
        return float(self.lib.or_max_error(_p(a), _p(b), a.size))

    def rms_norm_rows(self, x, w, eps=1e-6, eps_outside=False):
        x, w = _f32(x), _f32(w)
        D = x.shape[-1]
        y = np.empty_like(x)
        self.lib.or_rms_norm_rows(_p(x), _p(w), x.size // D, D, eps, int(eps_outside), _p(y))
        return y

    def rope_tables(self, max_pos, D, theta=1e6):
        c = np.empty((max_pos, D // 2), np.float32)
        s = np.empty_like(c)
        self.lib.or_rope_tables(max_pos, D, theta, _p(c), _p(s))
        return c, s

    def apply_rope(self, x, pos, cos, sin):
        """x [..., D] rows; pos int array with one entry per row."""
        x = _f32(x)
        D = x.shape[-1]
        rows = x.size // D
        pos = np.ascontiguousarray(np.broadcast_to(pos, (rows,)), dtype=np.int32)
        y = np.empty_like(x)
        self.lib.or_apply_rope(_p(x), rows, D, _p(pos), _p(_f32(cos)), _p(_f32(sin)), _p(y))
        return y

    def decode_gqa(self, q, k, v, scale):
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, Hq, D = q.shape
        Hkv, L = k.shape[1], k.shape[2]
        out = np.empty_like(q)
        self.lib.or_decode_gqa(_p(q), _p(k), _p(v), B, Hq, Hkv, L, D, scale, _p(out))
        return out

    def decode_streaming_compat(self, q, k, v, scale, block=64):
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, H, D = q.shape
        L = k.shape[2]
        out = np.empty_like(q)
        self.lib.or_decode_streaming_compat(_p(q), _p(k), _p(v), B, H, L, D, scale, block, _p(out))
        return out

    def prefill_blockwise(self, q, k, v, scale, kv_block=64, rows=None):
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, Hq, L, D = q.shape
        Hkv = k.shape[1]
        out = np.zeros_like(q)
        r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
        self.lib.or_prefill_blockwise(_p(q), _p(k), _p(v), B, Hq, Hkv, L, D, scale, kv_block,
                                      None if r is None else _p(r), 0 if r is None else r.size, _p(out))
        return out

    def sdpa_f64(self, q, k, v, scale, causal=False, pos0=0):
        """q [nq, D], k/v [L, D] -> fp64 [nq, D]."""
        q, k, v = _f32(q), _f32(k), _f32(v)
        nq, D = q.shape
        L = k.shape[0]
        out = np.empty((nq, D), np.float64)
        self.lib.or_sdpa_f64(_p(q), _p(k), _p(v), nq, L, D, float(scale), int(causal), pos0, _p(out))
        return out


    def sequence_np1(self, q, k, v, scale, heads=None):
        """TIMING ONLY: the np = 1 loop of the reference's MPI sequence-parallel
        prefill (numerically wrong there and here).  q [B, Hq, L, D], k/v
        [B, Hkv, L, D]; heads (first, count) limits the work to a head range
        (the other heads' rows stay zero)."""
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, Hq, L, D = q.shape
        Hkv = k.shape[1]
        h0, nh = (0, Hq) if heads is None else heads
        if not (0 <= h0 and nh >= 0 and h0 + nh <= Hq):
            raise ValueError("head range outside [0, Hq)")
        out = np.zeros_like(q)
        self.lib.or_sequence_np1(_p(q), _p(k), _p(v), B, Hq, Hkv, L, D, scale, h0, nh, _p(out))
        return out


class Reference:
    """The reference compiled from its own sources (oracle/_ref/libsa_ref.so)."""

    def __init__(self, path: Path = REF_LIB):
        if not path.exists():
            raise RuntimeError(f"{path} missing: run `make -C oracle ref` where the reference is mounted")
        self.lib = _bind(path, _REF_SIGS)

    @staticmethod
    def available(path: Path = REF_LIB) -> bool:
        return path.exists()

    def streaming_serial(self, Q, K, V, block):
        Q, K, V = _f32(Q), _f32(K), _f32(V)
        T, d = K.shape
        O = np.empty(d, np.float32)
        self.lib.ref_streaming_serial(_p(Q), _p(K), _p(V), T, d, block, _p(O))
        return O

    def naive_serial(self, Q, K, V):
        Q, K, V = _f32(Q), _f32(K), _f32(V)
        T, d = K.shape
        O = np.empty(d, np.float32)
        self.lib.ref_naive_serial(_p(Q), _p(K), _p(V), T, d, _p(O))
        return O

    def streaming_omp(self, Q, K, V, block, nthreads=0):
        Q, K, V = _f32(Q), _f32(K), _f32(V)
        T, d = K.shape
        O = np.empty(d, np.float32)
        self.lib.ref_streaming_omp(_p(Q), _p(K), _p(V), T, d, block, nthreads, _p(O))
        return O

    def naive_omp(self, Q, K, V, nthreads=0):
        Q, K, V = _f32(Q), _f32(K), _f32(V)
        T, d = K.shape
        O = np.empty(d, np.float32)
        self.lib.ref_naive_omp(_p(Q), _p(K), _p(V), T, d, nthreads, _p(O))
        return O

    def l2_error(self, a, b):
        a, b = _f32(a).ravel(), _f32(b).ravel()
        return float(self.lib.ref_l2_error(_p(a), _p(b), a.size))

    def max_error(self, a, b):
        a, b = _f32(a).ravel(), _f32(b).ravel()
        return float(self.lib.ref_max_error(_p(a), _p(b), a.size))

    def rope_freqs(self, seq_len, D, theta):
        c = np.empty((seq_len, D // 2), np.float32)
        s = np.empty_like(c)
        self.lib.ref_rope_freqs(seq_len, D, theta, _p(c), _p(s))
        return c, s

    def apply_rope(self, q, k, cos, sin):
        q, k = _f32(q), _f32(k)
        B, Hq, S, D = q.shape
        Hkv = k.shape[1]
        qo, ko = np.empty_like(q), np.empty_like(k)
        self.lib.ref_apply_rope(_p(q), _p(k), B, Hq, Hkv, S, D, _p(_f32(cos)), _p(_f32(sin)), _p(qo),
                                _p(ko))
        return qo, ko

    def repeat_kv(self, x, n_rep):
        x = _f32(x)
        B, H, S, D = x.shape
        out = np.empty((B, H * n_rep, S, D), np.float32)
        self.lib.ref_repeat_kv(_p(x), B, H, S, D, n_rep, _p(out))
        return out

    def self_attention(self, q, k, v, scale, causal):
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, H, Sq, D = q.shape
        Sk = k.shape[2]
        out = np.empty_like(q)
        self.lib.ref_self_attention(_p(q), _p(k), _p(v), B, H, Sq, Sk, D, int(causal), scale, _p(out))
        return out

    def self_attention_streaming(self, q, k, v, scale, block=64, nthreads=0):
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, H, D = q.shape[0], q.shape[1], q.shape[-1]
        L = k.shape[2]
        out = np.empty((B, H, 1, D), np.float32)
        self.lib.ref_self_attention_streaming(_p(q), _p(k), _p(v), B, H, L, D, scale, block, nthreads,
                                              _p(out))
        return out

    def blockwise(self, q, k, v, scale, q_block=32, kv_block=64, variant=0):
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, H, L, D = q.shape
        out = np.empty_like(q)
        self.lib.ref_blockwise(_p(q), _p(k), _p(v), B, H, L, D, scale, q_block, kv_block, variant,
                               _p(out))
        return out

    def layer_attention(self, q, k, v, wq, wk, prompt_len, eps=1e-6, max_seq=4096, avx2=False,
                        streaming=False):
        """q [N, Hq, D], k/v [N, Hkv, D] token rows -> (attn [N, Hq, D], qkv_eff [N, (Hq+2Hkv)*D])."""
        q, k, v, wq, wk = _f32(q), _f32(k), _f32(v), _f32(wq), _f32(wk)
        N, Hq, D = q.shape
        Hkv = k.shape[1]
        attn = np.empty((N, Hq, D), np.float32)
        eff = np.empty((N, (Hq + 2 * Hkv) * D), np.float32)
        rc = self.lib.ref_layer_attention(Hq, Hkv, D, prompt_len, N - prompt_len, _p(q), _p(k), _p(v),
                                          _p(wq), _p(wk), eps, max_seq, int(avx2), int(streaming),
                                          _p(attn), _p(eff))
        if rc != 0:
            raise RuntimeError("reference layer raised")
        return attn, eff

    def qwen3_forward_file(self, path, vocab, tokens, prompt_len, eps=1e-6):
        """qwen3_forward_with_cache (teacher forcing, as qwen3_forward) on the
        weights the reference's load_qwen3_weights reads from a safetensors
        file.  Returns logits [n + 1][B][vocab]."""
        import os
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        B, N = tokens.shape
        logits = np.empty((N - prompt_len + 1, B, vocab), np.float32)
        rc = self.lib.ref_qwen3_forward_file(os.fsencode(str(path)), eps, B, prompt_len, N - prompt_len,
                                             _p(tokens), _p(logits))
        if rc != 0:
            raise RuntimeError("reference loader or forward raised")
        return logits

    def load_weights(self, path):
        """(meta [7], flat fp32 weights) as the reference's load_qwen3_weights
        reads them (layout: ref_load_weights in oracle/ref_shim.cpp)."""
        import os
        meta = np.zeros(7, np.int64)
        if self.lib.ref_load_weights(os.fsencode(str(path)), _p(meta), None, 0) != 0:
            raise RuntimeError("reference loader raised")
        out = np.empty(int(meta[6]), np.float32)
        if self.lib.ref_load_weights(os.fsencode(str(path)), _p(meta), _p(out), out.size) != 0:
            raise RuntimeError("reference loader raised")
        return meta, out

    def rotary(self, x, max_seq, theta, seq_len):
        """ops::RotaryEmbedding(D, max_seq, theta).apply(x [B][S][H][D], seq_len)."""
        x = _f32(x)
        B, S, H, D = x.shape
        out = np.empty_like(x)
        if self.lib.ref_rotary(_p(x), B, S, H, D, max_seq, float(theta), seq_len, _p(out)) != 0:
            raise RuntimeError("reference RotaryEmbedding raised")
        return out

    def argmax(self, x, dim=-1, keepdim=False):
        """ops::argmax -> (indices, shape), or None where the reference raises."""
        x = _f32(x)
        dims = np.asarray(x.shape, np.int64)
        idx = np.zeros(max(1, x.size), np.int64)
        shape = np.zeros(8, np.int64)
        nd = C.c_int(0)
        n = self.lib.ref_argmax(_p(x), _p(dims), x.ndim, dim, int(keepdim), _p(idx), idx.size, _p(shape),
                                C.byref(nd))
        return None if n < 0 else (idx[:n].copy(), tuple(int(s) for s in shape[:nd.value]))

    def cross_attention(self, q, k, v, scale):
        """ops::cross_attention(q [B][H][Sq][D], k/v [B][H][Sk][D], nullptr, scale)."""
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, H, Sq, D = q.shape
        out = np.empty_like(q)
        self.lib.ref_cross_attention(_p(q), _p(k), _p(v), B, H, Sq, k.shape[2], D, float(scale), _p(out))
        return out

    def self_attention_avx2(self, q, k, v, scale, mask=None):
        """ops::avx2::self_attention_avx2(q [B][H][Sq][D], k/v [B][H][Sk][D],
        mask [mrows][Sk] (given as [1][1][mrows][Sk]) or nullptr, scale)."""
        q, k, v = _f32(q), _f32(k), _f32(v)
        B, H, Sq, D = q.shape
        out = np.empty_like(q)
        m = None if mask is None else _f32(mask)
        mrows = 0 if m is None else m.shape[0]
        self.lib.ref_self_attention_avx2(_p(q), _p(k), _p(v), B, H, Sq, k.shape[2], D, float(scale),
                                         None if m is None else _p(m), mrows, _p(out))
        return out

    def set_threads(self, n):
        """omp_set_num_threads(n) for the reference's later OpenMP regions."""
        self.lib.ref_set_threads(int(n))

    def time_decode_layer(self, hidden, intermediate, Hq, Hkv, D, batch, L0, n_steps, nthreads):
        """Wall seconds of n_steps one-token calls of the reference's
        qwen3_decoder_layer_avx_with_cache (STREAMING) over a cache holding L0
        tokens per sequence (timing only: LCG-filled weights and inputs)."""
        secs = np.empty(n_steps, np.float64)
        rc = self.lib.ref_time_decode_layer(hidden, intermediate, Hq, Hkv, D, batch, L0, n_steps, nthreads,
                                            secs.ctypes.data)
        if rc != 0:
            raise RuntimeError("reference layer raised")
        return secs

    def qwen3_forward(self, weights, cfg, tokens, prompt_len, avx2=False):
        """qwen3_forward_with_cache (avx2: qwen3_forward_avx_with_cache) over
        tokens [B][P + n] (teacher forcing): a P-token prompt, then n one-token
        forwards.  weights as in oracle.qwen3_model.  Returns logits
        [n + 1][B][V] at the last position of each forward."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        B, N = tokens.shape
        n_steps = N - prompt_len
        c = cfg
        L = weights["layers"]
        stack = {t: _f32(np.stack([layer[t] for layer in L])) for t in L[0]}
        glob = {t: _f32(weights[t]) for t in ("embed", "final_norm", "lm_head")}
        logits = np.empty((n_steps + 1, B, c["vocab"]), np.float32)
        rc = self.lib.ref_qwen3_forward(
            c["num_layers"], c["hidden"], c["intermediate"], c["vocab"], c["n_q_heads"], c["n_kv_heads"],
            c["head_dim"], c["rms_eps"], B, prompt_len, n_steps, _p(tokens), _p(glob["embed"]),
            _p(stack["in_norm"]), _p(stack["qkv"]), _p(stack["q_norm"]), _p(stack["k_norm"]), _p(stack["o"]),
            _p(stack["post_norm"]), _p(stack["gate_up"]), _p(stack["down"]), _p(glob["final_norm"]),
            _p(glob["lm_head"]), int(avx2), _p(logits))
        if rc != 0:
            raise RuntimeError("reference forward raised")
        return logits
