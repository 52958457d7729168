"""GPU parity: sum/mean/max/min/argmax/argmin over the middle axis of an
[outer, n, inner] view, and their backward passes, through the C ABI.

Contract: max/min values and all indices bit-exact against the strict fp32
oracle (the reference's strict-compare scans: first index wins ties, a NaN
wins only as the first element); sum/mean within 1e-5 of the fp64 oracle
relative to max(|sum|, sum of |terms|).  With inputs quantised to 1/64 (the
config-3 recipe) every partial sum is exact in fp32, so sums must be
bit-identical to fp64 there.
"""
import numpy as np
import pytest

import oracle
from gpu_helpers import reduce, reduce_bwd, rng_normal
from whitematter_amd import synth

pytestmark = pytest.mark.gpu

VIEWS = [
    (1, 1, 1),
    (1, 1000, 1),          # full reduction, small
    (1, 1 << 20, 1),       # full reduction, split into chunks + second pass
    (1, 1000003, 1),       # odd length, scalar path
    (300, 257, 1),         # rows, n % 4 != 0
    (4096, 1024, 1),       # many rows (one wave per row)
    (3, 200000, 1),        # few long rows (split rows)
    (1, 2048, 64),         # dim 0 of [2048, 64]
    (1, 5000, 1000),       # dim 0, inner % 4 == 0 -> float4 columns
    (1, 333, 77),          # dim 0, scalar columns
    (7, 50, 9),            # 3-D middle axis
    (16, 3, 4096),
]

OPS = ["sum", "mean", "max", "min", "argmax", "argmin"]


def quantised(shape, seed):
    return synth.quantize(rng_normal(shape, seed))


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("view", VIEWS)
def test_reduce_forward(wm, op, view):
    outer, n, inner = view
    x = quantised((outer * n * inner,), outer * 7 + n * 3 + inner)
    val, idx = reduce(op, x, outer, n, inner, want_idx=op not in ("sum", "mean"))
    if op in ("sum", "mean"):
        ref, _ = oracle.get("f64").reduce(op, x, outer, n, inner)
        scale, _ = oracle.get("abs").reduce(op, x, outer, n, inner)
        ok, worst = oracle.close_scaled(val, ref, scale, 1e-5)
        assert ok, f"{worst:.3g}x tolerance"
        if op == "sum":
            # quantised inputs: exact partial sums
            assert np.array_equal(val.astype(np.float64), ref), "quantised sums must be exact"
    else:
        ref, ridx = oracle.get("f32").reduce(op, x, outer, n, inner)
        assert oracle.bit_equal(val, ref)
        assert np.array_equal(idx, ridx)


@pytest.mark.parametrize("op", ["max", "min", "argmax", "argmin"])
def test_reduce_nan_and_ties(wm, op):
    """NaN first element wins; later NaNs never win; +0/-0 tie -> first."""
    n = 4096
    rows = []
    base = rng_normal((n,), 3)
    r0 = base.copy(); r0[0] = np.nan                       # NaN first
    r1 = base.copy(); r1[5] = np.nan; r1[999] = np.nan      # NaN later
    r2 = np.zeros(n, np.float32); r2[::2] = -0.0            # signed zero ties
    r3 = np.full(n, -np.inf, np.float32)                    # all -inf
    r4 = np.full(n, np.nan, np.float32)                     # all NaN
    r5 = np.full(n, 7.0, np.float32)                        # all equal
    for r in (r0, r1, r2, r3, r4, r5):
        rows.append(r)
    x = np.stack(rows).astype(np.float32)
    R = x.shape[0]
    # rows (inner == 1) and columns (transpose: inner == R)
    for arr, view in ((x.reshape(-1), (R, n, 1)), (np.ascontiguousarray(x.T).reshape(-1), (1, n, R))):
        val, idx = reduce(op, arr, *view, want_idx=True)
        ref, ridx = oracle.get("f32").reduce(op, arr, *view)
        assert oracle.bit_equal(val, ref), view
        assert np.array_equal(idx, ridx), view
    # split rows (few long rows) take the chunked path with a second pass
    long = np.concatenate([r0, r1, r5] * 64).astype(np.float32)
    val, idx = reduce(op, long, 1, long.size, 1, want_idx=True)
    ref, ridx = oracle.get("f32").reduce(op, long, 1, long.size, 1)
    assert oracle.bit_equal(val, ref) and np.array_equal(idx, ridx)


def special_slices(outer, n, inner, seed):
    """[outer, n, inner] quantised normals where each (outer, inner) slice is
    one of: plain, NaN first, NaNs later, signed zeros only, all -inf, all
    +inf, all NaN, all equal (ties)."""
    x = quantised((outer, n, inner), seed).reshape(outer, n, inner)
    rng = np.random.default_rng(seed)
    kind = rng.integers(0, 8, size=(outer, inner))
    for o, c in zip(*np.nonzero(kind)):
        k = kind[o, c]
        if k == 1:
            x[o, 0, c] = np.nan
        elif k == 2 and n > 1:
            x[o, rng.choice(np.arange(1, n), size=min(3, n - 1), replace=False), c] = np.nan
        elif k == 3:
            x[o, :, c] = np.where(rng.integers(0, 2, size=n) == 1, np.float32(-0.0), np.float32(0.0))
        elif k == 4:
            x[o, :, c] = -np.inf
        elif k == 5:
            x[o, :, c] = np.inf
        elif k == 6:
            x[o, :, c] = np.nan
        elif k == 7:
            x[o, :, c] = 7.0
    return x.reshape(-1)


@pytest.mark.parametrize("op", ["max", "min", "argmax", "argmin"])
@pytest.mark.parametrize("view", [
    (1, 4096, 8),       # float4 columns, split into chunks + second pass
    (1024, 16, 8),      # float4 columns, one workgroup per column tile
    (1, 3000, 1024),    # several column tiles, split
    (2, 100, 520),      # partial last tile (dead lanes), split
    (64, 50, 7),        # scalar columns, one workgroup per column tile
    (1, 3000, 7),       # scalar columns, split
    (512, 300, 1),      # rows, one wave per row
    (2, 300000, 1),     # long rows, split + second pass
    (9000, 5, 256),     # float4 columns: 9000 items on an 8192-workgroup grid (some workgroups take two)
    (9000, 3, 63),      # scalar columns, the same with a partial tile
])
def test_reduce_special_values(wm, op, view):
    """Bit-exact values and first-occurrence indices with NaNs, signed zeros,
    infinities and ties mixed per slice, on every launch shape of the max
    family: the cross-wave and cross-chunk folds see every kind of state."""
    outer, n, inner = view
    x = special_slices(outer, n, inner, outer * 31 + n + inner)
    val, idx = reduce(op, x, outer, n, inner, want_idx=True)
    ref, ridx = oracle.get("f32").reduce(op, x, outer, n, inner)
    assert oracle.bit_equal(val, ref)
    assert np.array_equal(idx, ridx)


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("op", ["sum", "mean", "max", "min"])
@pytest.mark.parametrize("view", [(1, 1000, 1), (300, 257, 1), (1, 500, 64), (7, 50, 9), (64, 1024, 1)])
def test_reduce_backward(wm, op, view, accumulate):
    outer, n, inner = view
    x = quantised((outer * n * inner,), 11)
    g = rng_normal((outer, inner), 12)
    gx0 = rng_normal((outer, n, inner), 13) if accumulate else None
    idx = None
    if op in ("max", "min"):
        _, idx = reduce(op, x, outer, n, inner, want_idx=True)
    got = reduce_bwd(op, g, idx, outer, n, inner, gx0)
    ref = oracle.get("f64").reduce_bwd(op, g, idx, outer, n, inner)
    if accumulate:
        ref = ref + gx0
    scale = np.abs(ref) + (np.abs(gx0) if accumulate else 0)
    ok, worst = oracle.close_scaled(got, ref, scale, 1e-6 if accumulate else 0.0)
    assert ok, f"{worst:.3g}x tolerance"
