"""CPU test of the paged cache's host bookkeeping (csrc/page_table.cpp): the
C++ unit test in tests/cpp_host is compiled with g++ (no HIP) and run.  It
covers every refusal the cache makes before enqueuing device work: pages
beyond a sequence's table row or the pool, pages owned by another sequence or
listed twice, a length cut when a sequence shrinks, appends and decodes past
a row's pages or the RoPE table, bad or repeated rows, all-or-nothing commits
(reference tensor_cpp/include/tensor_cpp/kv_cache.h:94-130 throws on
overflow; the C ABI returns SA_EFULL / SA_ERANGE / SA_EINVAL instead)."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_page_table_host_checks(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path / "test_page_table"
    cmd = [gxx, "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{ROOT / 'include'}",
           f"-I{ROOT / 'streaming-attention_amd' / 'csrc'}",
           str(ROOT / "tests" / "cpp_host" / "test_page_table.cpp"),
           str(ROOT / "streaming-attention_amd" / "csrc" / "page_table.cpp"), "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all checks passed" in res.stdout
