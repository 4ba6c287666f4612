"""GPU: the C++ mirror of the reference API (attention.h, KVCache, ops,
qwen3 attention path), exercised by tests/cpp/test_compat.cpp against the
oracle.  The driver prints one PASS/FAIL line per check."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cpp" / "bin" / "test_compat"


def test_cpp_api_mirror():
    assert EXE.exists(), "C++ driver missing: python streaming-attention_amd/build.py --tests"
    r = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=600)
    print(r.stdout)
    failed = [line for line in r.stdout.splitlines() if line.startswith("FAIL")]
    assert r.returncode == 0 and not failed, "\n".join(failed) + r.stderr
    assert r.stdout.count("PASS") >= 40
