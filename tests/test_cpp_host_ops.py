"""CPU: ops::argmax of the C++ mirror (include/tensor_cpp/ops.h), a host scan,
against numpy's argmax (the first of equal maxima) and against the
reference's own ops::argmax (tensor_cpp/src/ops.cpp:213-272, compiled into
oracle/_ref) on the same inputs: indices, result shape, and the cases where
the reference's TensorL refuses the shape it builds (std::invalid_argument).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

DRIVER = Path(__file__).resolve().parent / "cpp" / "bin" / "libdrive_compat.so"

CASES = [((7,), -1, False), ((3, 50), -1, False), ((1, 50), 1, False), ((3, 50), 1, True), ((3, 50), 1, False),
         ((2, 1, 9), 2, False), ((2, 3, 9), 2, False), ((2, 3, 9), 2, True), ((4, 6), 0, False),
         ((5,), 0, False), ((2, 2, 1, 5), 3, True)]


@pytest.fixture(scope="module")
def drv():
    if not DRIVER.exists():
        pytest.fail("driver missing: python streaming-attention_amd/build.py --tests")
    lib = C.CDLL(str(DRIVER))
    lib.drv_last_error.restype = C.c_char_p
    lib.drv_argmax.restype = C.c_long
    lib.drv_argmax.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_long, C.c_void_p,
                               C.c_void_p]
    return lib


def mirror_argmax(drv, x, dim, keepdim):
    """(indices, shape), or the exception's kind and text."""
    x = np.ascontiguousarray(x, np.float32)
    dims = np.asarray(x.shape, np.int64)
    idx = np.zeros(max(1, x.size), np.int64)
    shape = np.zeros(8, np.int64)
    nd = C.c_int(0)
    n = drv.drv_argmax(x.ctypes.data, dims.ctypes.data, x.ndim, dim, int(keepdim), idx.ctypes.data, idx.size,
                       shape.ctypes.data, C.byref(nd))
    if n < 0:
        return drv.drv_last_error().decode()
    return idx[:n].copy(), tuple(int(s) for s in shape[:nd.value])


def inputs(shape, seed):
    x = np.random.default_rng(seed).integers(-4, 5, size=shape).astype(np.float32)   # many ties
    return x


@pytest.mark.parametrize("shape,dim,keepdim", CASES)
def test_argmax_matches_numpy(drv, shape, dim, keepdim):
    x = inputs(shape, len(shape) * 10 + dim)
    got = mirror_argmax(drv, x, dim, keepdim)
    if dim == -1:
        assert got[0].tolist() == [int(np.argmax(x))] and got[1] == (1,)
        return
    if dim != x.ndim - 1:
        assert isinstance(got, str) and got.startswith("R:"), got
        return
    if x.ndim < 2:
        assert got == "I:Argmax along last dim requires at least 2D input", got
        return
    rows = np.argmax(x.reshape(-1, x.shape[-1]), axis=-1)
    lead = list(x.shape[:-1]) if keepdim else list(x.shape[:-2])
    shape_want = tuple(lead) if lead else (1,)
    if int(np.prod(shape_want)) != rows.size:      # the reference's TensorL refuses it
        assert isinstance(got, str) and got.startswith("I:Data size does not match shape"), got
        return
    assert got[1] == shape_want
    assert got[0].tolist() == rows.tolist()


@pytest.mark.parametrize("shape,dim,keepdim", CASES)
def test_argmax_matches_reference(drv, ref, shape, dim, keepdim):
    x = inputs(shape, len(shape) * 10 + dim + 1)
    want = ref.argmax(x, dim, keepdim)
    got = mirror_argmax(drv, x, dim, keepdim)
    if want is None:
        assert isinstance(got, str), got
    else:
        assert not isinstance(got, str), got
        assert got[1] == want[1] and got[0].tolist() == want[0].tolist()
