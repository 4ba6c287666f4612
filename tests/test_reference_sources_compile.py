"""CPU: the reference's own programs over the attention API compile and link
unchanged against include/ and libsa_amd.so: its attention benchmark
(tensor_cpp/tests/benchmark/benchmark_attention.cpp, which reaches OpenMP
through tensor_cpp/ops.h) and its attention unit test
(tensor_cpp/tests/unit/test_streaming_attention.cpp).  Needs the reference
sources; skipped where they are not mounted."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
REF = Path(os.environ.get("SA_REFERENCE", "/root/reference"))
LIB_DIR = ROOT / "streaming-attention_amd" / "lib"

PROGRAMS = ["tensor_cpp/tests/benchmark/benchmark_attention.cpp",
            "tensor_cpp/tests/unit/test_streaming_attention.cpp"]


@pytest.mark.parametrize("src", PROGRAMS)
def test_reference_program_builds_against_include(src, tmp_path):
    path = REF / src
    if not path.exists():
        pytest.skip("reference sources not mounted")
    if not (LIB_DIR / "libsa_amd.so").exists():
        pytest.skip("libsa_amd.so not built")
    exe = tmp_path / Path(src).stem
    cmd = ["g++", "-std=c++17", "-O0", "-fopenmp", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}",
           "-I/opt/rocm/include", str(path), "-o", str(exe), f"-L{LIB_DIR}", "-lsa_amd"]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    assert exe.exists()
