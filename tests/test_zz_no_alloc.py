"""GPU test of sa_stream_attn_f32_noalloc, the allocation-free variant of
sa_stream_attn_f32 (its split-KV partials live in the library's 1 MiB device
scratch array instead of a caller workspace).  Called through the C ABI, it
must equal the workspace entry point bit for bit on two calls in a row, the
second with a smaller input, and both must match the oracle at the fp32 bar
(max-abs <= 1e-4, relative L2 <= 1e-5)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _call_both(sa, Q, K, V, T, d):
    lib = sa.lib()
    dq, dk, dv = (torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (Q, K, V))
    out_ws = torch.full((d,), float("nan"), device="cuda")
    out_na = torch.full((d,), float("nan"), device="cuda")
    need = lib.sa_stream_attn_ws_bytes(T, d)
    ws = torch.zeros(max(need, 1), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    sa.check(lib.sa_stream_attn_f32(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), T, d, 64, 1.0,
                                    out_ws.data_ptr(), ws.data_ptr(), ws.numel(), stream))
    sa.check(lib.sa_stream_attn_f32_noalloc(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), T, d, 64, 1.0,
                                            out_na.data_ptr(), stream))
    torch.cuda.synchronize()
    return out_ws.cpu().numpy(), out_na.cpu().numpy()


def test_noalloc_matches_workspace_entry(sa, synth, oracle):
    # first a long context (256 chunks of partials), then a shorter one that
    # uses fewer chunks of the same scratch
    for T, d, seed in ((262144, 128, 80), (5000, 64, 81)):
        Q, K, V = synth.stream_inputs(T, d, seed=seed, scale=0.5, outlier_frac=0.01)
        got_ws, got_na = _call_both(sa, Q, K, V, T, d)
        np.testing.assert_array_equal(got_na, got_ws)
        want = oracle.streaming_serial(Q, K, V, 64)
        assert np.abs(got_na - want).max() <= 1e-4
        assert np.linalg.norm(got_na - want) / np.linalg.norm(want) <= 1e-5


def test_noalloc_argument_errors(sa):
    lib = sa.lib()
    assert lib.sa_stream_attn_f32_noalloc(None, None, None, 10, 128, 0, 1.0, None, None) == sa.SA_EINVAL
    assert b"block_size" in lib.sa_last_error()
    assert lib.sa_stream_attn_f32_noalloc(None, None, None, 10, 128, 64, 1.0, None, None) == sa.SA_EINVAL
    x = torch.zeros(100, 96, device="cuda")
    o = torch.zeros(96, device="cuda")
    st = lib.sa_stream_attn_f32_noalloc(x.data_ptr(), x.data_ptr(), x.data_ptr(), 100, 96, 64, 1.0,
                                        o.data_ptr(), None)
    assert st == sa.SA_EINVAL and b"head_dim" in lib.sa_last_error()
