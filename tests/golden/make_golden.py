"""Write the golden vectors in tests/golden/*.npz from the reference itself.

The reference is compiled from its own sources by oracle/Makefile into
oracle/_ref/libsa_ref.so (only possible where the reference is mounted).
Inputs are rebuilt from (seed, stream) with the package's generator, so only
the reference outputs and a SHA-256 of the inputs are stored.

    make -C oracle ref && python tests/golden/make_golden.py [name ...]

With names (e.g. qwen3_forward), only those files are rewritten.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

from oracle import Reference  # noqa: E402
from util import load_synth  # noqa: E402
import golden_inputs as gi  # noqa: E402

synth = load_synth()
ONLY = set(sys.argv[1:])


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def save(name: str, meta: dict, **arrays) -> None:
    if ONLY and name not in ONLY:
        return
    path = HERE / f"{name}.npz"
    np.savez(path, meta=np.array(json.dumps(meta)), **arrays)
    print(f"wrote {path.name}: {sorted(arrays)} ({path.stat().st_size} B)")


def main() -> None:
    ref = Reference()

    # Single-query streaming attention (T = 1024, d = 128) and the reference's
    # unit-test grid (tensor_cpp/tests/unit/test_streaming_attention.cpp:65-108).
    Q, K, V = gi.t1024_inputs()
    scale = np.float32(1.0 / np.sqrt(128.0))
    out = {}
    for blk in (64, 128):
        out[f"serial_b{blk}"] = ref.streaming_serial(Q, K, V, blk)
        out[f"serial_scaled_b{blk}"] = ref.streaming_serial(Q * scale, K, V, blk)
    out["naive"] = ref.naive_serial(Q, K, V)
    out["omp_b64_t4"] = ref.streaming_omp(Q, K, V, 64, 4)
    save("stream_t1024", {"inputs_sha256": digest(Q, K, V), "T": 1024, "d": 128}, **out)

    out = {}
    for T, d in gi.UNIT_GRID:
        Qu, Ku, Vu = gi.unit_inputs(T, d)
        out[f"serial_T{T}_d{d}"] = ref.streaming_serial(Qu, Ku, Vu, 64)
    save("stream_unit", {"grid": gi.UNIT_GRID}, **out)

    out, sha = {}, {}
    for T in (8192, 65536):
        Q2, K2, V2 = gi.long_inputs(T)
        sha[str(T)] = digest(Q2, K2, V2)
        for blk in (64, 128):
            out[f"serial_T{T}_b{blk}"] = ref.streaming_serial(Q2, K2, V2, blk)
    save("stream_long", {"inputs_sha256": sha}, **out)

    # RoPE tables at theta 1e6 (tensor_cpp/src/qwen3_ops.cpp:70-104), sampled rows.
    cos, sin = ref.rope_freqs(gi.ROPE_MAX_POS, 128, 1e6)
    rows = np.array(gi.ROPE_ROWS)
    q, k = gi.rope_inputs()
    qo, ko = ref.apply_rope(q, k, cos[: q.shape[2]], sin[: q.shape[2]])
    save("rope", {"rows": gi.ROPE_ROWS, "max_pos": gi.ROPE_MAX_POS}, cos=cos[rows], sin=sin[rows],
         q_rope=qo, k_rope=ko)

    # Decode attention over a dense cache: STANDARD (self_attention, zero mask)
    # and the STREAMING wrapper with its scale-on-output, both on repeat_kv heads.
    qd, kd, vd = gi.decode_inputs()
    rep = qd.shape[1] // kd.shape[1]
    kr, vr = ref.repeat_kv(kd, rep), ref.repeat_kv(vd, rep)
    sc = np.float32(1.0 / np.sqrt(qd.shape[-1]))
    std = ref.self_attention(qd[:, :, None, :], kr, vr, sc, causal=False)[:, :, 0, :]
    # One thread: the reference's nested OpenMP region then covers every chunk.
    strm = ref.self_attention_streaming(qd[:, :, None, :], kr, vr, sc, 64, nthreads=1)[:, :, 0, :]
    # Eight threads: the nested streaming_attention_omp runs on one thread but
    # still splits T into min(8, ceil(T/128)) chunks, so only chunk 0 is used.
    strm8 = ref.self_attention_streaming(qd[:, :, None, :], kr, vr, sc, 64, nthreads=8)[:, :, 0, :]
    save("decode", {"inputs_sha256": digest(qd, kd, vd)}, standard=std, streaming=strm,
         streaming_nested_t8=strm8)

    # Causal prefill: blockwise (q 32 / kv 64, the reference decoder's choice)
    # and its AVX2 twin at 128/128 (benchmark_qwen3's setting); sampled rows.
    qp, kp, vp = gi.prefill_inputs()
    rep = qp.shape[1] // kp.shape[1]
    kr, vr = ref.repeat_kv(kp, rep), ref.repeat_kv(vp, rep)
    sc = np.float32(1.0 / np.sqrt(qp.shape[-1]))
    rows = np.array(gi.PREFILL_ROWS)
    bw = ref.blockwise(qp, kr, vr, sc, 32, 64, 0)[:, :, rows, :]
    bw2 = ref.blockwise(qp, kr, vr, sc, 128, 128, 1)[:, :, rows, :]
    save("prefill", {"rows": gi.PREFILL_ROWS, "inputs_sha256": digest(qp, kp, vp)}, blockwise=bw,
         blockwise_avx2=bw2)

    # One reference decoder layer with a KVCache: prompt, then single-token steps.
    ql, kl, vl, wq, wk = gi.layer_inputs()
    out = {}
    for avx2 in (False, True):
        for streaming in (False, True):
            attn, eff = ref.layer_attention(ql, kl, vl, wq, wk, gi.LAYER_PROMPT, avx2=avx2,
                                            streaming=streaming)
            out[f"attn_avx{int(avx2)}_str{int(streaming)}"] = attn
            out["qkv_eff"] = eff
    save("layer", {"prompt": gi.LAYER_PROMPT, "inputs_sha256": digest(ql, kl, vl, wq, wk)}, **out)

    # Whole-model forwards (STANDARD attention): qwen3_forward_with_cache and
    # qwen3_forward_avx_with_cache.
    out, shas = {}, []
    for i, case in enumerate(gi.MODEL_CASES):
        w, tokens = gi.model_inputs(case)
        out[f"logits{i}"] = ref.qwen3_forward(w, case["cfg"], tokens, case["prompt"])
        out[f"logits_avx{i}"] = ref.qwen3_forward(w, case["cfg"], tokens, case["prompt"], avx2=True)
        shas.append(digest(tokens, w["embed"], w["lm_head"], *[v for L in w["layers"] for v in L.values()]))
    save("qwen3_forward", {"inputs_sha256": shas}, **out)


if __name__ == "__main__":
    main()
