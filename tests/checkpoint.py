"""Qwen3 checkpoints in safetensors format for the loader tests.

The weights come as the oracle's dict (oracle/qwen3_model.py: fused qkv rows
q | k | v, gate_up rows gate | up, fp32 values) and are written under the
Hugging Face tensor names the reference's load_qwen3_weights reads
(reference tensor_cpp/src/qwen3_loader.cpp:188-296), with the `safetensors`
package.
"""
from __future__ import annotations

import numpy as np


def bf16_exact(w: dict) -> dict:
    """w with every tensor rounded to bf16 (RNE), as a BF16 checkpoint holds it."""
    import torch

    def r(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()

    return {"embed": r(w["embed"]), "final_norm": r(w["final_norm"]), "lm_head": r(w["lm_head"]),
            "layers": [{k: r(v) for k, v in L.items()} for L in w["layers"]]}


def hf_tensors(w: dict, cfg: dict, tie: bool = False) -> dict:
    """{Hugging Face name: fp32 array}; tie=True leaves lm_head out (tied word embeddings)."""
    Hq, Hkv, D, I = cfg["n_q_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["intermediate"]
    out = {"model.embed_tokens.weight": w["embed"], "model.norm.weight": w["final_norm"]}
    if not tie:
        out["lm_head.weight"] = w["lm_head"]
    for i, L in enumerate(w["layers"]):
        p = f"model.layers.{i}."
        q, k, v = np.split(L["qkv"], [Hq * D, (Hq + Hkv) * D])
        out[p + "input_layernorm.weight"] = L["in_norm"]
        out[p + "post_attention_layernorm.weight"] = L["post_norm"]
        out[p + "self_attn.q_proj.weight"] = q
        out[p + "self_attn.k_proj.weight"] = k
        out[p + "self_attn.v_proj.weight"] = v
        out[p + "self_attn.q_norm.weight"] = L["q_norm"]
        out[p + "self_attn.k_norm.weight"] = L["k_norm"]
        out[p + "self_attn.o_proj.weight"] = L["o"]
        out[p + "mlp.gate_proj.weight"] = L["gate_up"][:I]
        out[p + "mlp.up_proj.weight"] = L["gate_up"][I:]
        out[p + "mlp.down_proj.weight"] = L["down"]
    return out


def write(path, w: dict, cfg: dict, dtype: str = "BF16", tie: bool = False, drop=()) -> None:
    """Write w as a safetensors checkpoint (dtype "BF16" or "F32"); names in
    `drop` are left out."""
    import torch
    from safetensors.torch import save_file
    tdt = torch.bfloat16 if dtype == "BF16" else torch.float32
    tensors = {k: torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(tdt)
               for k, v in hf_tensors(w, cfg, tie).items() if k not in drop}
    save_file(tensors, str(path), metadata={"format": "pt"})


def decode_teacher_forced(oracle, cfg: dict, w: dict, tokens: np.ndarray, prompt: int) -> np.ndarray:
    """The oracle decoder fed tokens [B][N] one at a time; logits [N - prompt + 1][B][V]
    at the last prompt position and after each later token."""
    from oracle.qwen3_model import KvStore, Qwen3Decoder
    dec = Qwen3Decoder(w, cfg, oracle)
    B, N = tokens.shape
    kv = KvStore(cfg["num_layers"], B, cfg["n_kv_heads"], cfg["head_dim"], N)
    out = []
    for t in range(N):
        lg = dec.step(tokens[:, t], kv)
        if t >= prompt - 1:
            out.append(lg)
    return np.stack(out)
