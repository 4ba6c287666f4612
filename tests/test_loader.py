"""The safetensors checkpoint path on the CPU.

- The reference's own loader (load_qwen3_weights, compiled into oracle/_ref)
  and forward read a checkpoint written here exactly as the oracle decoder
  reads the weights dict it came from: this pins the tensor names and the
  q | k | v and gate | up fusion the GPU loader uses.
- sa_qwen3_desc_from_safetensors (host-only part of the C ABI) reads the
  model shape, and rejects truncated, malformed or incomplete files with the
  documented status codes.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np
import pytest

import checkpoint as ck

# The reference loader assumes 28 layers, 16/8 heads and head_dim 128
# (reference tensor_cpp/src/qwen3_loader.cpp:217-221); hidden, intermediate and
# vocab are small so the CPU forward stays quick.
REF_CFG = dict(num_layers=28, hidden=64, intermediate=64, vocab=128, n_q_heads=16, n_kv_heads=8,
               head_dim=128, rms_eps=1e-6, rope_theta=1e6, max_pos=32)


@pytest.fixture(scope="module")
def ref_ckpt(tmp_path_factory, synth):
    from oracle.qwen3_model import synth_weights
    w = ck.bf16_exact(synth_weights(synth, REF_CFG, seed=31, std=0.1))
    path = tmp_path_factory.mktemp("ckpt") / "model.safetensors"
    ck.write(path, w, REF_CFG)
    return path, w


def tokens_for(cfg, B=2, N=6, seed=3):
    return ((np.arange(B * N).reshape(B, N) * 29 + seed) % cfg["vocab"]).astype(np.int32)


def test_reference_loader_reads_what_the_oracle_reads(oracle, ref, ref_ckpt):
    """load_qwen3_weights + qwen3_forward_with_cache on the file equal the oracle
    decoder on the weights dict the file was written from."""
    path, w = ref_ckpt
    tokens = tokens_for(REF_CFG)
    want = ref.qwen3_forward_file(path, REF_CFG["vocab"], tokens, prompt_len=3)
    got = ck.decode_teacher_forced(oracle, REF_CFG, w, tokens, prompt=3)
    assert np.abs(got - want).max() <= 1e-4
    assert (got.argmax(-1) == want.argmax(-1)).all()


def test_reference_loader_catches_swapped_gate_up(oracle, ref, tmp_path, synth):
    """Writing up_proj under gate_proj's name (and back) changes the reference's
    logits: the file test above would catch a loader that swapped them."""
    from oracle.qwen3_model import synth_weights
    w = ck.bf16_exact(synth_weights(synth, REF_CFG, seed=31, std=0.1))
    I = REF_CFG["intermediate"]
    swapped = {**w, "layers": [dict(L, gate_up=np.concatenate([L["gate_up"][I:], L["gate_up"][:I]]))
                               for L in w["layers"]]}
    path = tmp_path / "swapped.safetensors"
    ck.write(path, swapped, REF_CFG)
    tokens = tokens_for(REF_CFG)
    got = ref.qwen3_forward_file(path, REF_CFG["vocab"], tokens, prompt_len=3)
    want = ck.decode_teacher_forced(oracle, REF_CFG, w, tokens, prompt=3)
    assert np.abs(got - want).max() > 1e-3


def _desc(sa_lib, path):
    from util import load_pkg
    pkg = load_pkg()
    d = pkg.Qwen3Desc()
    st = pkg.lib().sa_qwen3_desc_from_safetensors(str(path).encode(), C.byref(d))
    return st, d, pkg


def test_desc_from_checkpoint(ref_ckpt):
    path, _ = ref_ckpt
    st, d, pkg = _desc(None, path)
    assert st == pkg.SA_OK, pkg.lib().sa_last_error()
    for k in ("num_layers", "hidden", "intermediate", "vocab", "n_q_heads", "n_kv_heads", "head_dim"):
        assert getattr(d, k) == REF_CFG[k], k
    assert d.max_pos == 0
    assert d.rms_eps == np.float32(1e-6) and d.rope_theta == np.float32(1e6)


def test_desc_gqa_and_head_dim_64(tmp_path, synth):
    """Shapes come from the tensors, not from Qwen3-0.6B constants."""
    from oracle.qwen3_model import synth_weights
    cfg = dict(num_layers=3, hidden=128, intermediate=96, vocab=192, n_q_heads=8, n_kv_heads=2, head_dim=64,
               rms_eps=1e-6, rope_theta=1e6)
    path = tmp_path / "m.safetensors"
    ck.write(path, synth_weights(synth, cfg, seed=2, std=0.1), cfg, dtype="F32", tie=True)
    st, d, pkg = _desc(None, path)
    assert st == pkg.SA_OK, pkg.lib().sa_last_error()
    assert (d.num_layers, d.hidden, d.intermediate, d.vocab, d.n_q_heads, d.n_kv_heads, d.head_dim) == \
        (3, 128, 96, 192, 8, 2, 64)


def test_desc_errors(tmp_path, ref_ckpt):
    path, _ = ref_ckpt
    raw = path.read_bytes()
    from util import load_pkg
    pkg = load_pkg()

    def status(data, name):
        p = tmp_path / name
        p.write_bytes(data)
        return _desc(None, p)[0]

    assert status(raw[:5], "short") == pkg.SA_EIO                       # no header length
    (n,) = struct.unpack("<Q", raw[:8])
    assert status(raw[:8 + n // 2], "cut_header") == pkg.SA_EIO          # header past the end
    assert status(raw[:8 + n + 100], "cut_data") == pkg.SA_EIO           # data ranges past the end
    bad = bytearray(raw)
    bad[8] = ord("[")                                                    # header not an object
    assert status(bytes(bad), "not_object") == pkg.SA_EIO
    missing = _desc(None, tmp_path / "does_not_exist.safetensors")[0]
    assert missing == pkg.SA_EIO


def test_desc_missing_tensor(tmp_path, synth):
    from oracle.qwen3_model import synth_weights
    cfg = dict(REF_CFG, num_layers=2)
    path = tmp_path / "m.safetensors"
    ck.write(path, synth_weights(synth, cfg, seed=2, std=0.1), cfg, drop=("model.layers.0.self_attn.q_norm.weight",))
    st, _, pkg = _desc(None, path)
    assert st == pkg.SA_EINVAL
    assert b"q_norm" in pkg.lib().sa_last_error()


# --- load_qwen3_weights of include/tensor_cpp/qwen3_loader.h (host tensors) ---

DRIVER = __import__("pathlib").Path(__file__).resolve().parent / "cpp" / "bin" / "libdrive_compat.so"


@pytest.fixture(scope="module")
def drv():
    if not DRIVER.exists():
        pytest.fail("driver missing: python streaming-attention_amd/build.py --tests")
    lib = C.CDLL(str(DRIVER))
    lib.drv_last_error.restype = C.c_char_p
    lib.drv_load_weights.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p, C.c_int64]
    lib.drv_load_weights.restype = C.c_int
    return lib


def load_mirror(drv, path):
    """(meta [7], flat fp32 weights) from the mirror's load_qwen3_weights, or
    raises RuntimeError with the exception's kind and text."""
    meta = np.zeros(7, np.int64)
    if drv.drv_load_weights(str(path).encode(), meta.ctypes.data, None, 0) != 0:
        raise RuntimeError(drv.drv_last_error().decode())
    out = np.empty(int(meta[6]), np.float32)
    assert drv.drv_load_weights(str(path).encode(), meta.ctypes.data, out.ctypes.data, out.size) == 0
    return meta, out


def flat_expected(w, cfg, tie):
    """The flat layout of drv_load_weights / ref_load_weights from the weights dict."""
    Hq, Hkv, D, I = cfg["n_q_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["intermediate"]
    parts = [w["embed"], w["final_norm"], w["embed"] if tie else w["lm_head"]]
    for L in w["layers"]:
        q, k, v = np.split(L["qkv"], [Hq * D, (Hq + Hkv) * D])
        parts += [L["in_norm"], L["post_norm"], L["qkv"], q, k, v, L["q_norm"], L["k_norm"], L["o"],
                  L["gate_up"][:I], L["gate_up"][I:], L["down"]]
    return np.concatenate([np.asarray(p, np.float32).ravel() for p in parts])


def test_mirror_loader_equals_reference_loader(drv, ref, ref_ckpt):
    """On the reference's model shape (28 layers, 16/8 heads of 128, BF16) the
    mirror's load_qwen3_weights returns, bit for bit, the tensors and config
    the reference's own loader returns."""
    path, w = ref_ckpt
    meta_ref, flat_ref = ref.load_weights(path)
    meta, flat = load_mirror(drv, path)
    assert meta.tolist() == meta_ref.tolist()
    assert np.array_equal(flat.view(np.uint32), flat_ref.view(np.uint32))
    assert np.array_equal(flat, flat_expected(w, REF_CFG, tie=False))


@pytest.mark.parametrize("dtype,tie", [("BF16", False), ("F32", True), ("F32", False)])
def test_mirror_loader_reads_any_shape(drv, tmp_path, synth, dtype, tie):
    """GQA 8/2, head_dim 64, three layers, F32 or BF16, tied or separate lm_head:
    the shape comes from the file, F32 values arrive unrounded, a tied
    checkpoint gets the embedding as lm_head."""
    from oracle.qwen3_model import synth_weights
    cfg = dict(num_layers=3, hidden=128, intermediate=96, vocab=192, n_q_heads=8, n_kv_heads=2, head_dim=64,
               rms_eps=1e-6, rope_theta=1e6)
    w = synth_weights(synth, cfg, seed=5, std=0.1)
    if dtype == "BF16":
        w = ck.bf16_exact(w)
    path = tmp_path / "m.safetensors"
    ck.write(path, w, cfg, dtype=dtype, tie=tie)
    meta, flat = load_mirror(drv, path)
    assert meta[:6].tolist() == [3, 8, 2, 64, 128, 192]
    assert np.array_equal(flat, flat_expected(w, cfg, tie))


def test_mirror_loader_errors(drv, tmp_path, synth):
    """The reference's messages for a file it cannot open and a missing tensor
    (std::runtime_error both); a wrong shape names the tensor."""
    from oracle.qwen3_model import synth_weights
    cfg = dict(num_layers=2, hidden=64, intermediate=64, vocab=96, n_q_heads=4, n_kv_heads=2, head_dim=64,
               rms_eps=1e-6, rope_theta=1e6)
    w = synth_weights(synth, cfg, seed=6, std=0.1)
    with pytest.raises(RuntimeError, match=r"^R:Failed to open safetensors file: .*nope\.safetensors"):
        load_mirror(drv, tmp_path / "nope.safetensors")
    ck.write(tmp_path / "a.safetensors", w, cfg, drop=("model.layers.1.mlp.up_proj.weight",))
    with pytest.raises(RuntimeError, match=r"^R:Tensor not found: model\.layers\.1\.mlp\.up_proj\.weight$"):
        load_mirror(drv, tmp_path / "a.safetensors")
    ck.write(tmp_path / "b.safetensors", w, cfg, drop=("model.norm.weight",))
    with pytest.raises(RuntimeError, match=r"^R:Tensor not found: model\.norm\.weight$"):
        load_mirror(drv, tmp_path / "b.safetensors")
    bad = dict(w, layers=[dict(L) for L in w["layers"]])
    bad["layers"][1]["down"] = bad["layers"][1]["down"][:, :32]
    ck.write(tmp_path / "c.safetensors", bad, cfg)
    with pytest.raises(RuntimeError, match=r"^R:model\.layers\.1\.mlp\.down_proj\.weight: shape"):
        load_mirror(drv, tmp_path / "c.safetensors")
