"""benchmark_qwen3, the reference-compatible command line (built by build()).

CPU: options are parsed as the reference parses them (help, unknown options,
bad values) without touching a GPU.  GPU: each phase runs and prints the
result lines the reference's experiment scripts read (总时间, 平均时间/token,
吞吐量, second field numeric), and --verify agrees between one prefill and
token-by-token decode.
"""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

BIN = Path(__file__).resolve().parents[1] / "streaming-attention_amd" / "bin" / "benchmark_qwen3"


def run(*args, timeout=240):
    if not BIN.exists():
        pytest.fail(f"{BIN} not built (run __graft_entry__.build())")
    return subprocess.run([str(BIN), *args], capture_output=True, text=True, timeout=timeout)


def field(out: str, label: str) -> float:
    """The second whitespace-separated field of the line starting with label,
    as the reference's scripts read it (grep label | awk '{print $2}')."""
    for line in out.splitlines():
        if line.startswith(label):
            return float(line.split()[1])
    raise AssertionError(f"no line '{label}' in:\n{out}")


def test_help_and_bad_options():
    r = run("--help")
    assert r.returncode == 0 and "--prompt-len" in r.stdout
    r = run("--no-such-option")
    assert r.returncode == 1 and "unknown option" in r.stderr
    r = run("--prompt-len", "abc")
    assert r.returncode == 1
    r = run("--batch-size", "65")
    assert r.returncode == 1
    r = run("--phase", "prefill")          # neither --model nor --synthetic
    assert r.returncode == 1


@pytest.mark.gpu
def test_prefill_phase_result_lines():
    r = run("--synthetic", "--phase", "prefill", "--prompt-len", "64", "--iters", "2", "--warmup", "1")
    assert r.returncode == 0, r.stderr
    total = field(r.stdout, "总时间:")
    assert field(r.stdout, "处理token数:") == 128
    assert abs(field(r.stdout, "平均时间/token:") - total / 128) < 1e-3
    assert field(r.stdout, "吞吐量:") > 0


@pytest.mark.gpu
@pytest.mark.parametrize("cache_flag", ["--use-kv-cache", "--no-kv-cache"])
def test_decode_phase_result_lines(cache_flag):
    r = run("--synthetic", "--phase", "decode", "--gen-len", "4", "--batch-size", "2", cache_flag)
    assert r.returncode == 0, r.stderr
    assert field(r.stdout, "处理token数:") == 8
    assert field(r.stdout, "吞吐量:") > 0


@pytest.mark.gpu
def test_verify_matches():
    r = run("--synthetic", "--verify", "151644,872,198,35127,752")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "MATCH" in r.stdout
    toks = re.findall(r"next token (\d+)", r.stdout)
    assert len(toks) == 2 and toks[0] == toks[1]
