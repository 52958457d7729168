"""GPU test of wm_reduce_noalloc, the allocation-free variant of wm_reduce
(no counterpart in the reference; for callers that cannot allocate device
memory).  It runs the same kernels as wm_reduce with its chunk partials in a
fixed device array, so its outputs must equal wm_reduce's bit for bit on
every op and shape (the partitions, and so every summation order, are the
same), and the library's pool must hand out no block during the call.  Two
calls in a row, the second on a smaller input, check that nothing of the
first call's contents leaks into the second.
"""
import ctypes as C
import functools

import numpy as np
import pytest

from gpu_helpers import rng_normal
from whitematter_amd import _lib as W

pytestmark = pytest.mark.gpu

OPS = [W.R_SUM, W.R_MEAN, W.R_MAX, W.R_MIN, W.R_ARGMAX, W.R_ARGMIN]

# (outer, n, inner): split columns (config 3's dim 0, chunk partials), rows
# one wave each (dim 1), one long row split in chunks (a full reduction),
# ragged shapes on the scalar paths
SHAPES = [(1, 16384, 4096), (16384, 4096, 1), (1, 1 << 22, 1), (3, 1000, 37), (5, 4093, 1), (2, 777, 64)]


def handouts():
    n = C.c_int64()
    W.call("wm_pool_handouts", C.byref(n))
    return n.value


def run(name, op, x, outer, n, inner):
    val = W.DeviceArray((outer * inner,))
    idx = W.DeviceArray((outer * inner,), np.int64) if op >= W.R_MAX else None
    before = handouts()
    W.call(name, op, x.vp, outer, n, inner, val.vp, W.ptr(idx))
    after = handouts()
    W.sync()
    return val.to_host(), (idx.to_host() if idx is not None else None), after - before


@functools.lru_cache(maxsize=4)
def quantised(size, seed):
    # ties are frequent (values on a 1/64 grid), as in config 3
    return (np.rint(rng_normal((size,), seed) * 64) / 64).astype(np.float32)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("op", OPS)
def test_noalloc_matches_wm_reduce(wm, shape, op):
    outer, n, inner = shape
    x = W.DeviceArray.from_host(quantised(outer * n * inner, 40 + len(shape)))
    rv, ri, _ = run("wm_reduce", op, x, outer, n, inner)
    gv, gi, allocs = run("wm_reduce_noalloc", op, x, outer, n, inner)
    assert allocs == 0, "wm_reduce_noalloc took blocks from the pool"
    assert np.array_equal(gv.view(np.uint32), rv.view(np.uint32))
    if ri is not None:
        assert np.array_equal(gi, ri)


@pytest.mark.parametrize("op", OPS)
def test_noalloc_two_calls_second_smaller(wm, op):
    """The array keeps the last call's contents: a second, smaller call must
    not see the first call's partials."""
    first, second = (1, 16384, 4096), (1, 3000, 1000)
    outs = []
    for k, (outer, n, inner) in enumerate((first, second)):
        x = W.DeviceArray.from_host(quantised(outer * n * inner, 90 + k))
        gv, gi, allocs = run("wm_reduce_noalloc", op, x, outer, n, inner)
        rv, ri, _ = run("wm_reduce", op, x, outer, n, inner)
        assert allocs == 0
        assert np.array_equal(gv.view(np.uint32), rv.view(np.uint32))
        if ri is not None:
            assert np.array_equal(gi, ri)
        outs.append(gv)
    assert outs[1].shape == (second[0] * second[2],)


def test_noalloc_argument_errors(wm):
    x = W.DeviceArray.from_host(np.ones(16, np.float32))
    out = W.DeviceArray((1,))
    L = W.lib()
    assert L.wm_reduce_noalloc(W.R_SUM, x.vp, 1, -1, 1, out.vp, None) == 1
    assert L.wm_reduce_noalloc(99, x.vp, 1, 16, 1, out.vp, None) == 1
    assert L.wm_reduce_noalloc(W.R_SUM, None, 1, 16, 1, out.vp, None) == 1
    assert L.wm_reduce_noalloc(W.R_MAX, x.vp, 1, 16, 1, None, None) == 1
    assert b"wm_reduce_noalloc" in L.wm_last_error()
