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


@pytest.mark.parametrize("log", [False, True])
@pytest.mark.parametrize("cols", [64, 100, 4096, 32000])
def test_softmax_special_rows(wm, log, cols):
    """NaN / inf / -inf inputs and wide spreads, row by row (both tile sizes).

    Reference semantics (core/tensor.cpp:1553-1575): any NaN or +inf in a row
    makes the whole row NaN (NaN propagates through the sum; +inf - +inf is
    NaN); -inf elements give exactly 0 (softmax) / -inf (log_softmax) while
    the rest of the row is normal.  Spreads of 100 reach subnormal outputs,
    which fp32 stores with absolute spacing 2^-149 (hence the atol)."""
    rows = []
    r = rng_normal((cols,), 31, 3.0); r[0] = np.nan; rows.append(r)               # NaN first
    r = rng_normal((cols,), 32, 3.0); r[cols // 2] = np.nan; rows.append(r)       # NaN inside
    r = rng_normal((cols,), 33, 3.0); r[-1] = np.inf; rows.append(r)              # +inf
    r = rng_normal((cols,), 34, 3.0); r[::3] = -np.inf; rows.append(r)            # many -inf
    r = np.full((cols,), -np.inf, np.float32); r[-1] = 1.5; rows.append(r)        # one finite, last
    r = np.full((cols,), -np.inf, np.float32); r[0] = -3.0; rows.append(r)        # one finite, first
    r = np.linspace(0.0, -110.0, cols).astype(np.float32); rows.append(r)        # subnormal tail
    r = rng_normal((cols,), 35, 40.0); rows.append(r)                              # huge spread
    r = np.full((cols,), 88.0, np.float32); rows.append(r)                         # large equal values
    x = np.ascontiguousarray(np.stack(rows).astype(np.float32))
    got = softmax_fwd(x, log)
    ref = oracle.get("f64").softmax(x, log)
    scale = oracle.get("abs").softmax(x, log)
    ok, worst = oracle.close_scaled(got, ref, scale, 1e-5, atol=0.0 if log else 3e-45)
    assert ok, f"{worst:.3g}x tolerance"
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
