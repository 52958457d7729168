"""GPU parity: broadcast binary ops, forward and backward, through the C ABI.

Contract (forward): add/sub/mul/div/max/min bit-exact against the strict fp32
oracle (the reference's broadcast loops, core/tensor.cpp:926-947 and twins);
pow within 2 ulp of the fp64 oracle, NaN positions identical.
Contract (backward): within 1e-5 of the fp64 oracle, relative to
max(|exact|, sum of |terms|) -- the broadcast-gradient sums of N(0,1) terms
cancel, so a plain relative bound would not hold for the reference either.
"""
import zlib

import numpy as np
import pytest

import oracle
from gpu_helpers import binary_bwd, binary_fwd, rng_normal, rng_uniform

pytestmark = pytest.mark.gpu

RTOL = 1e-5

SHAPES = [
    ((257, 129), (257, 129)),        # same shape, n % 4 != 0 (scalar path)
    ((64, 1024), (64, 1024)),        # same shape, float4 path
    ((64, 1024), (1024,)),           # row vector, missing leading dim (bias add)
    ((64, 1024), (1, 1024)),         # row vector
    ((96, 1000), (96, 1)),           # column vector
    ((1, 1000), (96, 1000)),         # broadcast on the left operand
    ((3, 1, 5), (1, 4, 1)),          # both broadcast: generic path
    ((2, 3, 4, 5), (3, 1, 5)),       # 4-D vs 3-D
    ((4096,), (1,)),                 # scalar operand
    ((1,), (37,)),                   # scalar on the left
    ((5, 7, 64), (7, 1)),            # middle-dim broadcast
    ((8, 2048), (8, 2048)),
    ((5, 70000), (5, 1)),            # column vector, few long rows: split into chunks
    ((40, 1024), (40, 1)),           # column vector, one workgroup per row (256 threads)
    ((24, 2052), (24, 1)),           # ... 512 threads, the last float4s idle
    ((16, 4096), (16, 1)),
    ((8, 6000), (8, 1)),             # ... 1024 threads
    ((40, 1), (40, 2048)),           # column vector on the left
    ((8, 8196), (8, 1)),             # beyond one workgroup's row: the wave kernel
    ((6, 8192), (1, 8192)),          # row vector, rows of >= 8192 floats: two rows per item
    ((4, 8196), (8196,)),            # ... with a partial last tile
    ((1, 8192), (6, 8192)),          # ... row vector on the left
    ((6, 1), (6, 8192)),             # ... column vector on the left
    ((7, 8192), (1, 8192)),          # odd row count: single rows
    ((3, 16384), (16384,)),          # row vector's gradient: 64-column slots in the second pass
    ((4, 16388), (16388,)),          # ... with a partial last slot
    ((6, 8192), (6, 1)),             # column vector, rows of >= 8192 floats: two rows per item (pow too)
    ((4, 8196), (4, 1)),             # ... with a partial last tile
    ((7, 8192), (7, 1)),             # ... odd row count: single rows
    ((0, 16), (16,)),                # empty
]

OPS = ["add", "sub", "mul", "div", "pow", "max", "min"]


def make_inputs(op, sa, sb, seed):
    a = rng_normal(sa, seed)
    b = rng_normal(sb, seed + 1)
    if op == "div":
        b = rng_uniform(sb, seed + 1, 0.5, 2.0) * np.where(rng_normal(sb, seed + 2) > 0, 1, -1).astype(np.float32)
    if op == "pow":
        a = np.abs(a) + np.float32(0.25)
        b = rng_uniform(sb, seed + 1, -1.5, 2.5)
    if op in ("max", "min"):
        # force ties so the ">=" / "<=" routing is exercised
        a = synth_quant(a)
        b = synth_quant(b)
    return a.astype(np.float32), b.astype(np.float32)


def stable_seed(*key):
    return zlib.crc32(repr(key).encode()) & 0xFFFF


def synth_quant(x):
    return (np.rint(x * 4) / 4).astype(np.float32)


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("sa,sb", SHAPES)
def test_binary_forward(wm, op, sa, sb):
    a, b = make_inputs(op, sa, sb, stable_seed(op, sa, sb))
    got = binary_fwd(op, a, b)
    if op == "pow":
        ref = oracle.get("f64").binary("pow", a, b)
        assert got.shape == ref.shape
        u = oracle.ulp_vs_f64(got, ref)
        assert u.size == 0 or u.max() <= 2.0, f"pow max ulp {u.max()}"
    else:
        ref = oracle.get("f32").binary(op, a, b)
        assert oracle.bit_equal(got, ref), f"{op} {sa} {sb} not bit-exact"


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("sa,sb", SHAPES)
@pytest.mark.parametrize("accumulate", [False, True])
def test_binary_backward(wm, op, sa, sb, accumulate):
    seed = stable_seed(op, sa, sb, "bwd")
    a, b = make_inputs(op, sa, sb, seed)
    out = binary_fwd(op, a, b)
    g = rng_normal(out.shape, seed + 7)
    ga0 = rng_normal(sa, seed + 8) if accumulate else None
    gb0 = rng_normal(sb, seed + 9) if accumulate else None
    ga, gb = binary_bwd(op, g, a, b, out, ga0, gb0)
    ra, rb = oracle.get("f64").binary_bwd(op, g, a, b, out)
    sa_, sb_ = oracle.get("abs").binary_bwd(op, g, a, b, out)
    if accumulate:
        ra, rb = ra + ga0, rb + gb0
        sa_, sb_ = sa_ + np.abs(ga0), sb_ + np.abs(gb0)
    ok_a, wa = oracle.close_scaled(ga, ra, sa_, RTOL)
    ok_b, wb = oracle.close_scaled(gb, rb, sb_, RTOL)
    assert ok_a, f"grad a off by {wa:.3g}x tolerance"
    assert ok_b, f"grad b off by {wb:.3g}x tolerance"


@pytest.mark.parametrize("op", ["add", "mul"])
def test_binary_backward_one_side(wm, op):
    """Only one input requires grad (the other pointer is NULL)."""
    a, b = make_inputs(op, (64, 1024), (1024,), 5)
    out = binary_fwd(op, a, b)
    g = rng_normal(out.shape, 6)
    ra, rb = oracle.get("f64").binary_bwd(op, g, a, b, out)
    sa_, sb_ = oracle.get("abs").binary_bwd(op, g, a, b, out)
    ga, gb = binary_bwd(op, g, a, b, out, need_b=False)
    assert gb is None and oracle.close_scaled(ga, ra, sa_, RTOL)[0]
    ga, gb = binary_bwd(op, g, a, b, out, need_a=False)
    assert ga is None and oracle.close_scaled(gb, rb, sb_, RTOL)[0]


def test_c2_shapes_forward_bitexact(wm):
    """Config-2 layouts (row and column broadcast) on a row slice of A."""
    from whitematter_amd import synth
    A, c, r, G = synth.config2(rows=512, cols=8192)
    o32 = oracle.get("f32")
    for op, other in (("add", r), ("mul", c), ("div", r)):
        got = binary_fwd(op, A, other)
        assert oracle.bit_equal(got, o32.binary(op, A, other)), op
    # pow with negative bases: NaN positions must match, the rest within 2 ulp
    got = binary_fwd("pow", A, c)
    ref = oracle.get("f64").binary("pow", A, c)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert oracle.ulp_vs_f64(got, ref).max() <= 2.0


def test_pow_nan_grad_positions(wm):
    """c.grad of A->pow(c) with negative A is NaN where the reference's is."""
    from whitematter_amd import synth
    A, c, r, G = synth.config2(rows=64, cols=512)
    out = binary_fwd("pow", A, c)
    ga, gc = binary_bwd("pow", G, A, c, out)
    ra, rc = oracle.get("f64").binary_bwd("pow", G, A, c, out)
    assert np.array_equal(np.isnan(ga), np.isnan(ra))
    assert np.array_equal(np.isnan(gc), np.isnan(rc))


def test_div_row_vector_special_divisors(wm):
    """a / b with b a row vector: columns whose divisor is zero, infinite,
    NaN, subnormal or outside [2^-62, 2^62] take the divisions, the others
    one reciprocal per column; both match the reference's fp32 expressions
    (g / b, -(g a / (b b))) to the gradient tolerance, with the same NaN and
    infinity positions."""
    cols = 1024
    a = rng_normal((96, cols), 41)
    b = rng_uniform((1, cols), 42, 0.5, 2.0)
    special = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 1e-30, -1e30, 2.0 ** -62, 2.0 ** -63,
               2.0 ** 62, 2.0 ** 63, -(2.0 ** -62) * 1.5, 3.0e18]
    for i, v in enumerate(special):
        col = 7 + 61 * i
        b[0, col] = np.float32(v)
        if 0 < abs(v) < 1e-18:
            # keep g a / b^2 far below the float range, so that no column sum
            # of finite terms overflows (where that happens depends on the
            # summation order, which differs from the reference's)
            a[:, col] *= np.float32(1e-25)
    out = binary_fwd("div", a, b)
    g = rng_normal(out.shape, 43)
    ga, gb = binary_bwd("div", g, a, b, out)
    ra, rb = oracle.get("f32").binary_bwd("div", g, a, b, out)
    sa_, sb_ = oracle.get("abs").binary_bwd("div", g, a, b, out)
    ok_a, wa = oracle.close_scaled(ga, ra, np.abs(sa_), RTOL)
    ok_b, wb = oracle.close_scaled(gb, rb, np.abs(sb_), RTOL)
    assert ok_a, f"grad a off by {wa:.3g}x tolerance"
    assert ok_b, f"grad b off by {wb:.3g}x tolerance"


@pytest.mark.parametrize("sa,sb", [((96, 1000), (96, 1)), ((40, 1), (40, 2048)), ((5, 70000), (5, 1)),
                                   ((33, 1001), (33, 1)), ((64, 1024), (1024,))])
@pytest.mark.parametrize("need", [(True, True), (True, False), (False, True)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_pow_backward_recomputes_output(wm, sa, sb, need, accumulate):
    """pow's backward without the forward output (as config 2's bench step
    calls it): the power is recomputed in the kernel; every layout and
    gradient subset against the fp64 oracle."""
    seed = stable_seed("pow-noout", sa, sb)
    a, b = make_inputs("pow", sa, sb, seed)
    out = binary_fwd("pow", a, b)
    g = rng_normal(out.shape, seed + 7)
    ga0 = rng_normal(sa, seed + 8) if accumulate else None
    gb0 = rng_normal(sb, seed + 9) if accumulate else None
    ga, gb = binary_bwd("pow", g, a, b, None, ga0, gb0, need_a=need[0], need_b=need[1])
    ra, rb = oracle.get("f64").binary_bwd("pow", g, a, b, out)
    sa_, sb_ = oracle.get("abs").binary_bwd("pow", g, a, b, out)
    if accumulate:
        ra, rb = ra + ga0, rb + gb0
        sa_, sb_ = sa_ + np.abs(ga0), sb_ + np.abs(gb0)
    if need[0]:
        ok, w = oracle.close_scaled(ga, ra, sa_, RTOL)
        assert ok, f"grad a off by {w:.3g}x tolerance"
    else:
        assert ga is None
    if need[1]:
        ok, w = oracle.close_scaled(gb, rb, sb_, RTOL)
        assert ok, f"grad b off by {w:.3g}x tolerance"
    else:
        assert gb is None
