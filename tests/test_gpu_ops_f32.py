"""GPU numerics of the dense fp32 operators (sa_linear_f32, sa_rms_norm_f32,
sa_swiglu_f32, sa_axpby_f32) and of the eps placement of sa_qk_norm_rope_ex,
each against a float64 host restatement of the reference formula
(tensor_cpp/src/ops.cpp linear :315-369, rms_norm :375-418, swiglu :493-509,
add :194-207) or the oracle (or_rms_norm_rows).

Bars: relative L2 <= 2e-6 and max-abs <= 1e-5 x the output's scale, which an
fp32 computation in any summation order meets; a dropped bias, a transposed
weight or a wrong row stride misses them by orders of magnitude.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def near(got, want, what):
    got = np.asarray(got, np.float64)
    scale = max(float(np.abs(want).max()), 1e-30)
    assert rel_l2(got, want) <= 2e-6, (what, rel_l2(got, want))
    assert float(np.abs(got - want).max()) <= 1e-5 * scale, (what, float(np.abs(got - want).max()), scale)


@pytest.mark.parametrize("M,K,N,bias", [(1, 1024, 3072, False), (5, 33, 70, True), (64, 256, 64, False),
                                        (130, 128, 200, True), (3, 1, 7, False), (17, 4096, 96, False)])
def test_linear_matches_float64(sa, synth, M, K, N, bias):
    x = synth.normal(40, M * 7 + K, (M, K))
    w = synth.normal(41, N * 3 + K, (N, K), 0.05)
    b = synth.normal(42, N, (N,)) if bias else None
    got = sa.linear(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(),
                    torch.from_numpy(b).cuda() if bias else None).cpu().numpy()
    want = x.astype(np.float64) @ w.astype(np.float64).T + (b if bias else 0.0)
    near(got, want, (M, K, N, bias))


def test_linear_unaligned_rows_and_zero_k(sa, synth):
    """x starting 4 bytes past an allocation (no float4 loads), and K = 0
    (y = bias)."""
    M, K, N = 9, 64, 40
    buf = torch.from_numpy(synth.normal(43, 1, (M * K + 1,))).cuda()
    x = buf[1:].view(M, K)
    w = torch.from_numpy(synth.normal(43, 2, (N, K))).cuda()
    got = sa.linear(x, w).cpu().numpy()
    near(got, x.cpu().double().numpy() @ w.cpu().double().numpy().T, "unaligned x")
    b = torch.from_numpy(synth.normal(43, 3, (N,))).cuda()
    y = sa.linear(torch.empty(M, 0, device="cuda"), torch.empty(N, 0, device="cuda"), b).cpu().numpy()
    assert np.array_equal(y, np.broadcast_to(b.cpu().numpy(), (M, N)))


@pytest.mark.parametrize("rows,n,weighted", [(7, 1000, True), (1, 1024, True), (33, 64, False), (4, 5120, True)])
def test_rms_norm_matches_float64(sa, synth, rows, n, weighted):
    x = synth.normal(44, rows, (rows, n), 3.0)
    w = (1 + synth.normal(45, n, (n,), 0.1)) if weighted else None
    xd = torch.from_numpy(x).cuda()
    got = sa.rms_norm(xd, torch.from_numpy(w).cuda() if weighted else None, 1e-6).cpu().numpy()
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + 1e-6) * (w if weighted else 1.0)
    near(got, want, (rows, n))
    sa.rms_norm(xd, None, 1e-6, out=xd)        # in place
    near(xd.cpu().numpy(), x64 / np.sqrt((x64 * x64).mean(-1, keepdims=True) + 1e-6), "in place")


def test_swiglu_and_axpby_match_float64(sa, synth):
    n = 10001
    g = synth.normal(46, 1, (n,), 4.0)
    g[:4] = [-100.0, -80.0, 80.0, 0.0]          # exp overflow / underflow ends
    u = synth.normal(46, 2, (n,))
    gd, ud = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    got = sa.swiglu(gd, ud).cpu().numpy()
    g64 = g.astype(np.float64)
    want = u * (g64 / (1.0 + np.exp(-g64)))
    assert np.isfinite(got).all()
    near(got, want, "swiglu")
    near(sa.axpby(gd, 1.0, ud, -0.5).cpu().numpy(), g64 - 0.5 * u, "x + alpha y")
    near(sa.axpby(gd, 0.25).cpu().numpy(), 0.25 * g64, "a x")
    sa.axpby(gd, 1.0, ud, 1.0, out=ud)          # out aliases y
    near(ud.cpu().numpy(), g64 + u, "aliased residual add")


@pytest.mark.parametrize("eps_outside", [False, True])
def test_qk_norm_eps_placement(sa, oracle, synth, eps_outside):
    """Rows of magnitude 1e-4 (mean square 1e-8, far below eps = 1e-6) tell
    x / sqrt(ms + eps) from x / (sqrt(ms) + eps) by a factor of ten."""
    D = 128
    x = synth.normal(47, 1, (6, D))
    x[3:] *= 1e-4
    w = 1 + synth.normal(47, 2, (D,), 0.1)
    pos = torch.zeros(6, dtype=torch.int32, device="cuda")
    got = sa.qk_norm_rope(torch.from_numpy(x).cuda(), pos, torch.from_numpy(w).cuda(), 1e-6,
                          eps_outside=eps_outside).cpu().numpy()
    want = oracle.rms_norm_rows(x, w, 1e-6, eps_outside)
    other = oracle.rms_norm_rows(x, w, 1e-6, not eps_outside)
    near(got, want, eps_outside)
    assert rel_l2(got[3:], other[3:]) > 0.5
