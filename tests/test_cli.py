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
    r = run("--batch-size", "1025")
    assert r.returncode == 1
    r = run("--phase", "prefill")          # neither --model nor --synthetic
    assert r.returncode == 1
    for opt, bad in (("--q-block-size", "48"), ("--q-block-size", "256"), ("--kv-block-size", "100"),
                     ("--kv-block-size", "32768")):
        r = run("--synthetic", opt, bad)
        assert r.returncode == 1 and "error:" in r.stderr and "block" in r.stderr, (opt, bad, r.stderr)


# q_block:kv_block pairs of the reference's block-size sweep
# (tensor_cpp/scripts/exp6_block_size_tuning.sh:28-34), at its prompt lengths.
EXP6_BLOCKS = ["32:64", "64:128", "64:64", "128:128", "128:256"]


@pytest.mark.gpu
@pytest.mark.parametrize("seq_len", [128, 1024])
def test_block_size_sweep_prefill(seq_len):
    """The sweep's prefill runs: every setting prints the result lines and
    the query tile it asked for."""
    for cfg in EXP6_BLOCKS:
        q, kv = cfg.split(":")
        r = run("--synthetic", "--phase", "prefill", "--prompt-len", str(seq_len), "--q-block-size", q,
                "--kv-block-size", kv, "--iters", "2", "--warmup", "1")
        assert r.returncode == 0, (cfg, r.stderr)
        assert field(r.stdout, "处理token数:") == 2 * seq_len
        assert field(r.stdout, "吞吐量:") > 0
        assert re.search(rf"attention tiles: prefill {q} queries per workgroup and head", r.stdout), r.stdout
        assert f"decode split-KV chunk {kv} tokens" in r.stdout


@pytest.mark.gpu
def test_block_sizes_change_only_rounding(tmp_path):
    """--verify (a 300-token prefill, and a one-token prefill followed by 299
    decode steps) under each block setting of the sweep and the automatic
    one: the last-position logits of both paths agree with the automatic
    setting's to fp32 rounding (max-abs <= 1e-4 relative to the largest
    logit, same greedy token), and each run's two paths MATCH."""
    import numpy as np
    toks = ",".join(str((7 * i * i + 3 * i + 11) % 151936) for i in range(300))
    res = {}
    for cfg in ["0:0"] + EXP6_BLOCKS:
        q, kv = cfg.split(":")
        out = tmp_path / f"logits_{q}_{kv}.bin"
        r = run("--synthetic", "--synthetic-shape", "2,1024,3072,151936,16,8,128", "--q-block-size", q,
                "--kv-block-size", kv, "--verify", toks, "--logits-out", str(out))
        assert r.returncode == 0 and "MATCH" in r.stdout, (cfg, r.stdout, r.stderr)
        res[cfg] = np.fromfile(out, np.float32).reshape(2, 1, -1)
    base = res["0:0"]
    scale = float(np.abs(base).max())
    for cfg, got in res.items():
        err = float(np.abs(got - base).max())
        assert err <= 1e-4 * scale, (cfg, err, scale)
        assert (got.argmax(-1) == base.argmax(-1)).all(), cfg


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


VERIFY_CFG = dict(num_layers=2, hidden=128, intermediate=192, vocab=320, n_q_heads=4, n_kv_heads=2, head_dim=64,
                  rms_eps=1e-6, rope_theta=1e6, max_pos=64)


@pytest.mark.gpu
@pytest.mark.parametrize("batch", [1, 3])
def test_verify_against_host_forward(tmp_path, oracle, synth, batch):
    """--verify on a small synthetic model (seed 9, std 0.1): the next token and
    the last-position logits of both GPU paths (one prefill; a one-token
    prefill then decode steps) against the oracle decoder on the same weights
    (oracle.qwen3_model.synth_weights draws what sa_qwen3_init_random draws)
    and, where it is built, the reference's qwen3_forward_with_cache.  fp32
    bar: max-abs <= 1e-4, relative L2 <= 1e-5, same argmax."""
    import numpy as np
    from oracle import Reference
    from oracle.qwen3_model import KvStore, Qwen3Decoder, synth_weights

    c = VERIFY_CFG
    tokens = [3, 17, 99, 250, 7, 120, 64]
    out = tmp_path / "logits.bin"
    shape = ",".join(str(c[k]) for k in ("num_layers", "hidden", "intermediate", "vocab", "n_q_heads",
                                         "n_kv_heads", "head_dim"))
    r = run("--synthetic", "--synthetic-shape", shape, "--seed", "9", "--std", "0.1", "--batch-size", str(batch),
            "--verify", ",".join(map(str, tokens)), "--logits-out", str(out))
    assert r.returncode == 0, r.stdout + r.stderr
    got = np.fromfile(out, np.float32).reshape(2, batch, c["vocab"])
    next_tok = [int(t) for t in re.findall(r"next token (\d+)", r.stdout)]

    w = synth_weights(synth, c, 9, 0.1)
    dec = Qwen3Decoder(w, c, oracle)
    kv = KvStore(c["num_layers"], batch, c["n_kv_heads"], c["head_dim"], len(tokens))
    for t in tokens:
        want = dec.step([t] * batch, kv)
    wants = [("oracle", want)]
    if Reference.available():
        seq = np.array([tokens] * batch, np.int32)
        wants.append(("reference", Reference().qwen3_forward(w, c, seq, len(tokens))[0]))
    for name, wt in wants:
        for path in range(2):
            g = got[path]
            err = float(np.abs(g - wt).max())
            rel = float(np.linalg.norm(g - wt) / np.linalg.norm(wt))
            assert err <= 1e-4 and rel <= 1e-5, (name, path, err, rel)
            assert (g.argmax(-1) == wt.argmax(-1)).all(), (name, path)
        assert next_tok == [int(wt[0].argmax())] * 2, (name, next_tok)
