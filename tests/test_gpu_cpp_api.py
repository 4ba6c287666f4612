"""GPU: the C++ mirror of the reference API (attention.h, KVCache, ops,
qwen3 attention path), exercised by tests/cpp/test_compat.cpp against the
oracle (one PASS/FAIL line per check), and four of the reference's own unit
tests (tensor_cpp/tests/unit/test_streaming_attention.cpp, test_attention.cpp,
test_ops.cpp, test_avx_ops.cpp), compiled unchanged against include/ and
linked to the library by oracle/Makefile (ref-on-lib), run on the GPU
kernels."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cpp" / "bin" / "test_compat"
REF_BIN = Path(__file__).resolve().parents[1] / "oracle" / "_ref"
REF_TEST = REF_BIN / "test_streaming_attention_on_sa_amd"


def test_cpp_api_mirror():
    assert EXE.exists(), "C++ driver missing: python streaming-attention_amd/build.py --tests"
    r = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    failed = [line for line in r.stdout.splitlines() if line.startswith("FAIL")]
    assert r.returncode == 0 and not failed, "\n".join(failed) + r.stderr
    assert r.stdout.count("PASS") >= 40


def test_reference_unit_test_on_the_gpu():
    """The reference's correctness grid (T 512..4096 x d 64/128/256 at a 1e-5
    max-abs bar against naive attention), its OpenMP-vs-serial check (1e-4)
    and its block-size sweep, all through the library."""
    if not REF_TEST.exists():
        pytest.skip("built only where the reference sources are mounted (make -C oracle ref-on-lib)")
    r = subprocess.run([str(REF_TEST)], capture_output=True, text=True, timeout=600)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert r.stdout.count("Status: OK") == 4


def _run_reference_program(name, tmp_path):
    exe = REF_BIN / f"{name}_on_sa_amd"
    if not exe.exists():
        pytest.skip("built only where the reference sources are mounted (make -C oracle ref-on-lib)")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, cwd=tmp_path)
    print(r.stdout[-4000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    return r.stdout


def test_reference_attention_unit_test_on_the_gpu(tmp_path):
    """The reference's self/cross attention suite (head_dim 8 .. 128, query
    lengths 4 .. 64, key lengths up to 20 beyond the queries), which throws
    on any failure."""
    out = _run_reference_program("test_attention", tmp_path)
    assert "All Attention Tests PASSED" in out
    assert out.count("Status: OK") >= 6


def test_reference_ops_unit_test_on_the_gpu(tmp_path):
    """The reference's operator suite (add, argmax, embedding, linear, rms_norm,
    RotaryEmbedding, swiglu, self_attention, Tensor matmul): every case must
    report PASSED and none ERROR."""
    out = _run_reference_program("test_ops", tmp_path)
    assert "All tests PASSED" in out and "ERROR" not in out
    assert "Failed: 0" in out


def test_reference_avx_ops_unit_test_on_the_gpu(tmp_path):
    """The reference's checks of matmul_avx (relative 1e-3 against a scalar
    product), dot_avx (1e-4), add_avx (1e-6) and rms_norm_avx (1e-5 against
    ops::rms_norm), all four through the library."""
    out = _run_reference_program("test_avx_ops", tmp_path)
    assert out.count("Status: PASSED") == 4 and "FAILED" not in out
