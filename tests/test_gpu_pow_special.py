"""GPU parity: pow on special operands, through every forward and backward
kernel layout.

The pow kernels evaluate a branch-free table path for every element and
repair the operands it does not cover (zero, subnormal, infinite and NaN
bases, |x| == 1, infinite, NaN and zero exponents) in a second step; a
negative base takes C pow's sign rule inside the table path.  These tests
put every such operand pair through each kernel: the flat and row-broadcast
vector kernels, their scalar twins (rows not a multiple of 4) and the
generic kernel, forward and backward, and pow(Tensor, float).

Contract: forward within 2 ulp of the fp64 oracle (C pow, core/tensor.cpp:1394
std::pow), with identical NaN and infinity positions and the sign of zero
results preserved; gradients within 1e-5 (scale-aware) of the strict fp32
oracle, NaN / infinity positions identical.
"""
import numpy as np
import pytest

import oracle
from gpu_helpers import binary_bwd, binary_fwd, rng_normal, unary_bwd, unary_fwd

pytestmark = pytest.mark.gpu

F = np.float32
SPECIAL = np.array([
    0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan,
    2.0, 0.5, -2.0, -0.5, 3.0, -3.0, 0.25, 7.5, -7.5, 0.3, -0.3,
    1e-45, -1e-45, 1.1754942e-38, 1.17549435e-38, -1.17549435e-38, 3.4028235e38, -3.4028235e38,
    16777216.0, -16777216.0, 2.0 ** 31, -(2.0 ** 31), 2.0 ** 40,
    1.0000001, 0.99999994, -1.0000001, 1e10, -1e10, 1e-10,
    127.5, 128.0, -149.0, -150.0, 150.0, -126.0, 1e6, -1e6,
], dtype=F)


def check_fwd(got, a, b):
    ref = oracle.get("f64").binary("pow", a, b)
    assert got.shape == ref.shape
    u = oracle.ulp_vs_f64(got, ref)
    bad = np.argwhere(u > 2.0)
    assert bad.size == 0, "pow(%r, %r) = %r, exact %r" % (
        np.broadcast_to(a, ref.shape)[tuple(bad[0])], np.broadcast_to(b, ref.shape)[tuple(bad[0])],
        got[tuple(bad[0])], ref[tuple(bad[0])])
    zero = ref == 0
    assert np.array_equal(np.signbit(got[zero]), np.signbit(ref[zero])), "sign of a zero result"


def grid(n_rows_pad=0):
    """a[i, j] = SPECIAL[j], b[i, j] = SPECIAL[i]: every (base, exponent)
    pair once; optional extra columns of ordinary values keep the row length
    off a multiple of 4 or 4096."""
    m = len(SPECIAL)
    a = np.broadcast_to(SPECIAL[None, :], (m, m))
    b = np.broadcast_to(SPECIAL[:, None], (m, m))
    if n_rows_pad:
        pad = rng_normal((m, n_rows_pad), 91)
        a = np.concatenate([a, pad], axis=1)
        b = np.concatenate([b, np.broadcast_to(b[:, :1], (m, n_rows_pad))], axis=1)
    return np.ascontiguousarray(a, F), np.ascontiguousarray(b, F)


@pytest.mark.parametrize("pad", [0, 3, 4052])
def test_pow_special_flat(wm, pad):
    a, b = grid(pad)
    check_fwd(binary_fwd("pow", a, b), a, b)


@pytest.mark.parametrize("pad", [0, 1, 4052, 8148, 8152])
def test_pow_special_column_exponent(wm, pad):
    """b is a column vector [m, 1]: the row-broadcast kernel (cached b);
    rows of 8192 and 8196 floats (an even row count) take its two-row
    items."""
    a, b = grid(pad)
    bc = np.ascontiguousarray(b[:, :1])
    check_fwd(binary_fwd("pow", a, bc), a, bc)


@pytest.mark.parametrize("pad", [0, 1])
def test_pow_special_row_base(wm, pad):
    """a is a row vector [1, n] and b a column [m, 1]: both broadcast."""
    a, b = grid(pad)
    ar = np.ascontiguousarray(a[:1])
    bc = np.ascontiguousarray(b[:, :1])
    check_fwd(binary_fwd("pow", ar, bc), ar, bc)


def test_pow_special_generic(wm):
    """3-D broadcast on both sides: the generic per-element kernel."""
    m = len(SPECIAL)
    a = SPECIAL.reshape(1, m, 1)
    b = SPECIAL.reshape(m, 1, 1)
    b2 = np.ascontiguousarray(np.concatenate([b, b], axis=2))
    check_fwd(binary_fwd("pow", a, b2), a, b2)


def test_pow_special_scalar_exponent(wm):
    """pow(Tensor, float): the unary kernel, every special exponent."""
    x = np.ascontiguousarray(np.concatenate([SPECIAL, rng_normal((4096 - len(SPECIAL),), 92)]), F)
    for p in SPECIAL:
        got = unary_fwd("pows", x, float(p))
        check_fwd(got, x, np.full_like(x, p))


# Gradients of extreme operands overflow, underflow or turn NaN inside the
# reference's float arithmetic (g * b * pow(a, b - 1) with pow(a, b - 1)
# beyond float range, g * out overflowing, 0 * inf), which the fp64 oracle
# would carry through in double; so these tests compare with the strict fp32
# oracle, the reference's own arithmetic in IEEE mode.  ATOL covers results
# in the subnormal range, where a 2e-7 relative difference in a factor can
# move the rounded product by one subnormal step.
ATOL = 3e-45


def close_grads(ga, gb, a, b, g, out):
    ra, rb = oracle.get("f32").binary_bwd("pow", g, a, b, out)
    sa, sb = oracle.get("abs").binary_bwd("pow", g, a, b, out)
    ok_a, wa = oracle.close_scaled(ga, ra, sa, 1e-5, ATOL)
    ok_b, wb = oracle.close_scaled(gb, rb, sb, 1e-5, ATOL)
    assert ok_a, "grad a off by %.3g x tolerance" % wa
    assert ok_b, "grad b off by %.3g x tolerance" % wb


@pytest.mark.parametrize("layout", ["flat", "column", "generic"])
@pytest.mark.parametrize("recompute", [False, True])
def test_pow_special_backward(wm, layout, recompute):
    """Gradients on every special pair, with the forward output passed in or
    recomputed on the device (out = NULL, what Tensor::pow's closure does)."""
    a, b = grid(5)
    if layout == "column":
        b = np.ascontiguousarray(b[:, :1])
    elif layout == "generic":
        m = len(SPECIAL)
        a = np.ascontiguousarray(SPECIAL.reshape(1, m, 1))
        b = np.ascontiguousarray(np.concatenate([SPECIAL.reshape(m, 1, 1)] * 2, axis=2))
    out = binary_fwd("pow", a, b)
    g = rng_normal(out.shape, 93)
    if recompute:
        from whitematter_amd import _lib as W
        from gpu_helpers import dev
        dg, da, db = dev(g), dev(a), dev(b)
        dga, dgb = W.DeviceArray(a.shape), W.DeviceArray(b.shape)
        dga.fill(np.nan)
        dgb.fill(np.nan)
        W.binary_bwd(W.BINARY_OPS["pow"], dg, da, db, None, dga, False, dgb, False)
        ga, gb = dga.to_host(), dgb.to_host()
    else:
        ga, gb = binary_bwd("pow", g, a, b, out)
    close_grads(ga, gb, a, b, g, out)


def test_pow_special_scalar_exponent_backward(wm):
    x = np.ascontiguousarray(np.concatenate([SPECIAL, rng_normal((1024 - len(SPECIAL),), 94)]), F)
    g = rng_normal(x.shape, 95)
    for p in SPECIAL:
        out = unary_fwd("pows", x, float(p))
        got = unary_bwd("pows", g, x, out, p0=float(p))
        ref = oracle.get("f32").unary_bwd("pows", g, x, out, float(p))
        scale = oracle.get("abs").unary_bwd("pows", g, x, out, float(p))
        ok, w = oracle.close_scaled(got, ref, scale, 1e-5, ATOL)
        assert ok, "pow(x, %r) backward off by %.3g x tolerance" % (p, w)
