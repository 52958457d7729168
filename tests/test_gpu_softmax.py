"""GPU parity: row softmax / log_softmax forward and backward through the C ABI.

Reference: softmax core/tensor.cpp:1548-1591 (three passes; backward is the
explicit O(C^2) Jacobian), log_softmax :1593-1635.  The fp64 oracle follows
those loops literally (the Jacobian included); the GPU uses the closed form.
Contract: within 1e-5 of the fp64 oracle, relative to max(|exact|, sum of
|terms|) for the quantities that cancel.
"""
import numpy as np
import pytest

import oracle
from gpu_helpers import rng_normal, softmax_bwd, softmax_fwd
from whitematter_amd import synth

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (4, 3), (33, 100), (16, 1000), (8, 2048), (4, 2049), (4, 4096), (3, 10001),
          (2, 32000), (2, 32768), (1, 40000)]


def logits(shape, seed):
    x = rng_normal(shape, seed, 3.0)
    return synth.spikes(x, seed, 0.01, 20.0)


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("shape", SHAPES)
def test_softmax_forward(wm, shape, log):
    x = logits(shape, shape[1])
    got = softmax_fwd(x, log)
    ref = oracle.get("f64").softmax(x, log)
    scale = oracle.get("abs").softmax(x, log)
    ok, worst = oracle.close_scaled(got, ref, scale, 1e-5)
    assert ok, f"{worst:.3g}x tolerance"
    if not log:
        assert np.allclose(got.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("shape", [(4, 3), (33, 100), (8, 2048), (4, 4096), (2, 5003), (1, 32000), (1, 40000)])
def test_softmax_backward(wm, shape, log, accumulate):
    x = logits(shape, 5)
    out = softmax_fwd(x, log)
    g = rng_normal(shape, 6)
    gx0 = rng_normal(shape, 7) if accumulate else None
    got = softmax_bwd(g, out, gx0, log)
    ref = oracle.get("f64").softmax_bwd(g, out, log)
    scale = oracle.get("abs").softmax_bwd(g, out, log)
    if accumulate:
        ref = ref + gx0
        scale = scale + np.abs(gx0)
    ok, worst = oracle.close_scaled(got, ref, scale, 1e-5, atol=1e-30)
    assert ok, f"{worst:.3g}x tolerance"
    if not log and not accumulate:
        # softmax backward is orthogonal to the ones vector per row
        s = got.astype(np.float64).sum(axis=1)
        assert np.all(np.abs(s) <= 1e-5 * np.abs(g).sum(axis=1))


def test_softmax_all_neg_inf_row(wm):
    """A row of -inf gives NaN (exp(-inf - -inf)), as in the reference."""
    x = np.full((2, 64), -np.inf, np.float32)
    x[1] = 0.0
    got = softmax_fwd(x)
    assert np.isnan(got[0]).all() and np.allclose(got[1], 1 / 64)
