"""CPU checks of the C ABI: the library loads without a GPU and exports every
function include/sa_*.h declares, with the argument counts the Python
binding assumes."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from util import load_pkg

HEADERS = sorted((Path(__file__).resolve().parents[1] / "include").glob("sa_*.h"))


def declared_functions():
    text = "\n".join(re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S) for h in HEADERS)
    decls = {}
    for m in re.finditer(r"^\s*[\w\s\*]+?\b(sa_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S):
        args = m.group(2).strip()
        n = 0 if args in ("", "void") else args.count(",") + 1
        decls[m.group(1)] = n
    return decls


def test_header_declares_entry_points():
    decls = declared_functions()
    for name in ("sa_stream_attn_f32", "sa_decode_dense_f32", "sa_kvcache_create", "sa_qknorm_rope_append",
                 "sa_paged_decode", "sa_prefill_causal", "sa_last_error", "sa_qwen3_decode_step"):
        assert name in decls


def test_library_exports_every_declared_symbol():
    sa = load_pkg()
    lib = sa.lib()
    decls = declared_functions()
    missing = [n for n in decls if not hasattr(lib, n)]
    assert not missing, missing
    # the ctypes binding covers the header exactly, with matching arity
    assert set(sa.SIGNATURES) == set(decls)
    for name, n_args in decls.items():
        assert len(sa.SIGNATURES[name][1]) == n_args, name


def test_last_error_starts_empty():
    lib = load_pkg().lib()
    assert lib.sa_last_error() == b""


def test_library_does_not_interpose_on_the_reference(ref):
    """libsa_amd exports the reference API's names (streaming_attention_serial,
    ...); loading it first must not redirect the reference build's own calls."""
    import numpy as np
    load_pkg().lib()
    Q = np.ones(64, np.float32)
    K = np.ones((3, 64), np.float32)
    V = np.arange(192, dtype=np.float32).reshape(3, 64)
    np.testing.assert_allclose(ref.streaming_serial(Q, K, V, 64), V.mean(0), rtol=1e-6)


def test_no_gpu_compute_without_device():
    """Argument validation runs on the host: a bad call fails before any launch."""
    sa = load_pkg()
    lib = sa.lib()
    st = lib.sa_stream_attn_f32(None, None, None, 10, 128, 64, 1.0, None, None, 0, None)
    assert st == sa.SA_EINVAL
    assert b"null" in lib.sa_last_error()
    st = lib.sa_stream_attn_f32(None, None, None, 10, 128, 0, 1.0, None, None, 0, None)
    assert st == sa.SA_EINVAL and b"block_size" in lib.sa_last_error()
    assert lib.sa_stream_attn_ws_bytes(0, 128) == 0
    assert lib.sa_kvcache_len(None, 0) == -1
    with pytest.raises(Exception):
        ctypes.CDLL(str(sa.LIB_PATH)).sa_not_a_symbol  # noqa: B018
