"""CPU restatement of the Qwen3 decoder's greedy decode step.

TEST INFRASTRUCTURE ONLY: the checker of the GPU model step (tests/) and
nothing else.

Follows qwen3_forward_with_cache (reference tensor_cpp/src/qwen3_ops.cpp:936-1014)
one token per sequence at a time:
    x = embedding(token)                                  ops.cpp:278-313
    per layer (qwen3_decoder_layer_with_cache, qwen3_ops.cpp:620-934):
        h = rms_norm(x, input_layernorm)                  ops.cpp:375-417
        q | k | v = h @ qkv_projs^T                       qwen3_ops.cpp:652-688
        per-head rms_norm(q, q_norm), rms_norm(k, k_norm) qwen3_ops.cpp:697-753
        RoPE at position = cached length                  qwen3_ops.cpp:757-788
        append k, v; attention over the cache (STANDARD)  qwen3_ops.cpp:790-909
        x = x + attn @ o_proj^T                           qwen3_ops.cpp:911-925
        h = rms_norm(x, post_attention_layernorm)
        x = x + down(silu(gate(h)) * up(h))               qwen3_ops.cpp:265-296
    logits = rms_norm(x, norm) @ lm_head^T                qwen3_ops.cpp:994-1012
and the cache length grows by one after the last layer (:988-992).

Weights are numpy float32 in the reference's row-major layouts:
embed [V][H]; per layer in_norm [H], qkv [(Hq+2Hkv)D][H], q_norm [D],
k_norm [D], o [H][Hq D], post_norm [H], gate_up [2I][H] (gate rows, then up
rows), down [H][I]; final_norm [H]; lm_head [V][H].  The QK-norm and RoPE
pieces are the C oracle's (or_rms_norm_rows, or_apply_rope), pinned by their
own tests; matmuls and the attention are numpy fp32 (BLAS), so only the
summation order differs from the reference's loops.
"""
from __future__ import annotations

import numpy as np

TENSORS = ("in_norm", "qkv", "q_norm", "k_norm", "o", "post_norm", "gate_up", "down")


def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """ops::rms_norm: x / sqrt(mean(x^2) + eps) * w over the last axis (fp32)."""
    x = x.astype(np.float32)
    ms = (x * x).mean(axis=-1, keepdims=True, dtype=np.float32)
    return ((x / np.sqrt(ms + np.float32(eps))) * w).astype(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as fp32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


class KvStore:
    """Per-layer, per-sequence K/V with spare capacity, fp32:
    K[l][b], V[l][b] [Hkv][cap][D]; lens[b] committed tokens of sequence b.
    kv_bf16: appended K/V are stored rounded to bf16, as a bf16 cache holds them."""

    def __init__(self, num_layers: int, batch: int, n_kv_heads: int, head_dim: int, cap: int,
                 kv_bf16: bool = False):
        self.kv_bf16 = kv_bf16
        shape = (n_kv_heads, cap, head_dim)
        self.K = [[np.zeros(shape, np.float32) for _ in range(batch)] for _ in range(num_layers)]
        self.V = [[np.zeros(shape, np.float32) for _ in range(batch)] for _ in range(num_layers)]
        self.lens = np.zeros(batch, np.int64)


class Qwen3Decoder:
    """Greedy decode over per-sequence caches of any lengths.

    cfg: num_layers, hidden, intermediate, vocab, n_q_heads, n_kv_heads,
    head_dim, rms_eps, rope_theta, max_pos.  weights: dict with "embed",
    "final_norm", "lm_head" and "layers" (a list of dicts keyed by TENSORS).
    step() appends one token per sequence to a KvStore and returns the logits.
    """

    def __init__(self, weights: dict, cfg: dict, oracle, qk_eps_outside: bool = False):
        self.w = weights
        self.cfg = cfg
        self.or_ = oracle
        # q/k RMSNorm as the AVX2 layer: x / (sqrt(mean(x^2)) + eps)
        # (reference tensor_cpp/src/qwen3_ops_avx.cpp:537, :566)
        self.qk_eps_outside = qk_eps_outside
        self.cos, self.sin = oracle.rope_tables(cfg["max_pos"], cfg["head_dim"], cfg["rope_theta"])

    def step(self, tokens, kv: KvStore):
        c, w, o = self.cfg, self.w, self.or_
        B = len(tokens)
        Hq, Hkv, D, eps = c["n_q_heads"], c["n_kv_heads"], c["head_dim"], c["rms_eps"]
        nq, nk, rep = Hq * D, Hkv * D, Hq // Hkv
        scale = np.float32(1.0 / np.sqrt(np.float32(D)))
        pos = kv.lens[:B].astype(np.int32)       # position = cached length
        x = w["embed"][np.asarray(tokens, np.int64)].astype(np.float32)
        for l, L in enumerate(w["layers"]):
            h = rms_norm(x, L["in_norm"], eps)
            qkv = h @ L["qkv"].T
            # the q/k RMSNorm's eps is 1e-6 whatever rms_eps is (qwen3_ops.cpp:716)
            q = o.rms_norm_rows(qkv[:, :nq].reshape(B, Hq, D), L["q_norm"], 1e-6, self.qk_eps_outside)
            k = o.rms_norm_rows(qkv[:, nq:nq + nk].reshape(B, Hkv, D), L["k_norm"], 1e-6, self.qk_eps_outside)
            v = qkv[:, nq + nk:].reshape(B, Hkv, D)
            q = o.apply_rope(q, np.repeat(pos, Hq), self.cos, self.sin)
            k = o.apply_rope(k, np.repeat(pos, Hkv), self.cos, self.sin)
            attn = np.empty((B, Hkv, rep, D), np.float32)
            for b in range(B):
                n = pos[b] + 1
                K, V = kv.K[l][b], kv.V[l][b]
                K[:, pos[b]] = bf16_round(k[b]) if kv.kv_bf16 else k[b]
                V[:, pos[b]] = bf16_round(v[b]) if kv.kv_bf16 else v[b]
                # query head h reads KV head h // rep (repeat_kv, qwen3_ops.cpp:194-234);
                # softmax(q k^T scale) v over the n cached tokens (ops.cpp:514-641)
                s = np.matmul(q[b].reshape(Hkv, rep, D), K[:, :n].transpose(0, 2, 1)) * scale
                s = np.exp(s - s.max(axis=-1, keepdims=True))
                s /= s.sum(axis=-1, keepdims=True)
                attn[b] = np.matmul(s, V[:, :n])
            x = (x + attn.reshape(B, nq) @ L["o"].T).astype(np.float32)
            h = rms_norm(x, L["post_norm"], eps)
            gu = h @ L["gate_up"].T
            I = c["intermediate"]
            g, u = gu[:, :I], gu[:, I:]
            act = (g * (np.float32(1.0) / (np.float32(1.0) + np.exp(-g))) * u).astype(np.float32)
            x = (x + act @ L["down"].T).astype(np.float32)
        kv.lens[:B] += 1                          # increment_seq_len after the last layer
        h = rms_norm(x, w["final_norm"], eps)
        return (h @ w["lm_head"].T).astype(np.float32)


def synth_weights(synth, cfg: dict, seed: int, std: float = 0.02) -> dict:
    """Weights drawn as the GPU model's sa_qwen3_init_random draws them:
    tensor `which` of layer l is stream 1000 + 16 l + which of `seed`;
    matrices std * N(0,1) rounded to bf16, norm weights 1 + std * N(0,1).
    The device takes std as an fp32 value, so the draws scale by float32(std)."""
    std = float(np.float32(std))
    H, I, V = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    Hq, Hkv, D = cfg["n_q_heads"], cfg["n_kv_heads"], cfg["head_dim"]
    shapes = {"embed": (0, (V, H)), "in_norm": (1, (H,)), "qkv": (2, ((Hq + 2 * Hkv) * D, H)),
              "q_norm": (3, (D,)), "k_norm": (4, (D,)), "o": (5, (H, Hq * D)), "post_norm": (6, (H,)),
              "gate_up": (7, (2 * I, H)), "down": (8, (H, I)), "final_norm": (9, (H,)),
              "lm_head": (10, (V, H))}

    def draw(name, layer):
        which, shape = shapes[name]
        z = synth.normal(seed, 1000 + 16 * layer + which, shape, std)
        if len(shape) == 1:
            return (np.float32(1.0) + z).astype(np.float32)
        return synth.bf16_round(z)

    return {"embed": draw("embed", 0), "final_norm": draw("final_norm", 0), "lm_head": draw("lm_head", 0),
            "layers": [{t: draw(t, l) for t in TENSORS} for l in range(cfg["num_layers"])]}
