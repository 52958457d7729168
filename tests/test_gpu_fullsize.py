"""GPU parity at the benchmark configurations' full sizes (c2 A[8192, 8192],
c3 X[16384, 4096], c4 logits[8192, 32000], c5 h, res[32 x 1024, 4096]),
through properties that hold at any size, so no oracle run is needed at
these sizes:

- element-wise forwards of add / sub / mul / div equal IEEE fp32 arithmetic
  bit for bit (the reference's broadcast loops, core/tensor.cpp:926-947 and
  twins, are single IEEE operations; numpy's float32 operators are the same
  operations);
- pow is within 2 ulp of float64 pow, with the same NaN positions;
- gradients agree with the derivative formulas evaluated in float64 within
  the sums contract (1e-5 of the sum of |terms|), broadcast gradients being
  the row or column sums of the element terms;
- sums of values quantised to 1/64 are exact in fp32 whatever the order
  while every partial sum stays below 2^24 / 64, so dim-0 / dim-1 sums and
  means are bit-exact, and max / min / argmax / argmin with their
  first-index ties equal numpy's;
- softmax rows sum to 1 and match the float64 closed form; log_softmax
  likewise, and their closures match their closed forms;
- the fused fp16 epilogue stores the truncating fp16 of the fp32 tanh the
  unary kernel computes (pinned in test_gpu_unary.py), bit for bit.

The inputs come from numpy's seeded generator; test_gpu_recipe.py runs the
same configurations on the bench recipe's own bytes (whitematter_amd/synth.py).
"""
import numpy as np
import pytest

import oracle
from gpu_helpers import binary_bwd, binary_fwd, reduce, softmax_bwd, softmax_fwd
from whitematter_amd import _lib as W

pytestmark = pytest.mark.gpu


def normal(shape, seed, std=1.0):
    x = np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)
    return x * np.float32(std) if std != 1.0 else x


def uniform(shape, seed, lo, hi):
    return np.random.default_rng(seed).uniform(lo, hi, shape).astype(np.float32)


def close(got, ref, scale, rtol=1e-5, atol=1e-30):
    ok, worst = oracle.close_scaled(got, ref, scale, rtol, atol)
    assert ok, f"{worst:.3g}x tolerance"


# ---- config 2: A[8192, 8192] with r[1, 8192], c[8192, 1] ---------------------

@pytest.fixture(scope="module")
def c2():
    R = C = 8192
    return normal((R, C), 201), uniform((R, 1), 202, 0.5, 2.0), uniform((1, C), 203, 0.5, 2.0), normal((R, C), 204)


@pytest.mark.parametrize("op,vec", [("add", "r"), ("sub", "c"), ("mul", "c"), ("div", "r")])
def test_c2_forward_is_ieee_fp32(wm, c2, op, vec):
    A, c, r, _ = c2
    b = r if vec == "r" else c
    ref = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide}[op](A, b)
    assert oracle.bit_equal(binary_fwd(op, A, b), ref)


def test_c2_pow_within_2_ulp(wm, c2):
    A, c, _, _ = c2
    got = binary_fwd("pow", A, c)
    with np.errstate(invalid="ignore"):
        ref = np.power(A.astype(np.float64), c.astype(np.float64))
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    u = oracle.ulp_vs_f64(got, ref)
    assert u.max() <= 2.0, f"pow max ulp {u.max()}"


def grad_terms(op, G, A, b):
    """Element terms of dA and db in float64, and their magnitudes."""
    g, a, v = G.astype(np.float64), A.astype(np.float64), b.astype(np.float64)
    with np.errstate(invalid="ignore", divide="ignore"):
        if op == "add":
            return g, g
        if op == "sub":
            return g, -g
        if op == "mul":
            return g * v, g * a
        if op == "div":
            return g / v, -g * a / (v * v)
        p = np.power(a, v)
        return g * v * np.power(a, v - 1.0), g * p * np.log(a)


@pytest.mark.parametrize("op,vec,give_out", [("add", "r", True), ("sub", "c", True), ("mul", "c", True),
                                             ("div", "r", True), ("pow", "c", True), ("pow", "c", False)])
def test_c2_backward_accumulates(wm, c2, op, vec, give_out):
    """give_out=False: no forward output passed, as the bench step calls pow's
    backward (the kernel recomputes the power)."""
    A, c, r, G = c2
    if op == "pow":
        A = np.abs(A)  # finite log(a), so c's row sums are finite (negative bases: test_gpu_binary.py)
    b = r if vec == "r" else c
    out = binary_fwd(op, A, b)
    ga0, gb0 = normal(A.shape, 205), normal(b.shape, 206)
    ga, gb = binary_bwd(op, G, A, b, out if give_out else None, ga0, gb0)
    da, db = grad_terms(op, G, A, b)
    axis = 0 if vec == "r" else 1
    close(ga, ga0 + da, np.abs(ga0) + np.abs(da))
    ref_b = gb0.astype(np.float64) + db.sum(axis=axis, keepdims=True)
    scale_b = np.abs(gb0) + np.abs(db).sum(axis=axis, keepdims=True)
    close(gb, ref_b, scale_b)


# ---- config 3: X[16384, 4096] quantised to 1/64 -------------------------------

@pytest.fixture(scope="module")
def c3():
    return np.round(normal((16384, 4096), 301) * np.float32(64)) / np.float32(64)


@pytest.mark.parametrize("dim", [0, 1])
def test_c3_sums_and_means_are_exact(wm, c3, dim):
    R, C = c3.shape
    outer, n, inner = (1, R, C) if dim == 0 else (R, C, 1)
    exact = c3.astype(np.float64).sum(axis=dim)
    assert np.abs(c3).sum(axis=dim).max() < 2 ** 24 / 64   # every partial sum is representable
    s, _ = reduce("sum", c3, outer, n, inner)
    assert np.array_equal(s.ravel(), exact.astype(np.float32))
    m, _ = reduce("mean", c3, outer, n, inner)
    assert np.array_equal(m.ravel(), exact.astype(np.float32) / np.float32(n))


@pytest.mark.parametrize("dim", [0, 1])
@pytest.mark.parametrize("op", ["max", "min", "argmax", "argmin"])
def test_c3_extrema_with_first_index_ties(wm, c3, op, dim):
    R, C = c3.shape
    outer, n, inner = (1, R, C) if dim == 0 else (R, C, 1)
    v, i = reduce(op, c3, outer, n, inner, want_idx=True)
    pick = np.argmax if op in ("max", "argmax") else np.argmin
    ref_i = pick(c3, axis=dim)
    assert np.array_equal(i.ravel(), ref_i)
    if op in ("max", "min"):
        assert np.array_equal(v.ravel(), np.take_along_axis(c3, np.expand_dims(ref_i, dim), dim).ravel())
    else:
        assert np.array_equal(v.ravel(), ref_i.astype(np.float32))


def test_c3_full_sum(wm, c3):
    s, _ = reduce("sum", c3, 1, c3.size, 1)
    x = c3.astype(np.float64)
    close(s.ravel(), [x.sum()], [np.abs(x).sum()])


# ---- config 4: logits[8192, 32000] --------------------------------------------

@pytest.fixture(scope="module")
def c4():
    x = normal((8192, 32000), 401, 3.0)
    spike = np.random.default_rng(402).random(x.shape) < 0.01
    x[spike] = np.float32(20.0)       # the config's spikes: 1% of the logits set to +20
    return x


def test_c4_softmax_forward_backward(wm, c4):
    x = c4.astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    s = e / e.sum(axis=1, keepdims=True)
    del e
    got = softmax_fwd(c4)
    close(got, s, s)
    assert np.abs(got.astype(np.float64).sum(axis=1) - 1.0).max() <= 1e-5
    g = normal(c4.shape, 403)
    g64 = g.astype(np.float64)
    gs = g64 * s
    dot = gs.sum(axis=1, keepdims=True)
    ref = gs - s * dot
    scale = np.abs(gs) + s * np.abs(gs).sum(axis=1, keepdims=True)
    del gs, s
    dx = softmax_bwd(g, got)
    close(dx, ref, scale)
    # orthogonal to the ones vector per row
    assert np.all(np.abs(dx.astype(np.float64).sum(axis=1)) <= 1e-5 * np.abs(g64).sum(axis=1))


def test_c4_log_softmax_forward_backward(wm, c4):
    x = c4.astype(np.float64)
    m = x.max(axis=1, keepdims=True)
    lse = np.log(np.exp(x - m).sum(axis=1, keepdims=True))
    ref = x - m - lse
    got = softmax_fwd(c4, log=True)
    close(got, ref, np.abs(x) + np.abs(m + lse))  # the operands of x - (max + lse), as the abs oracle
    assert np.abs(np.exp(got.astype(np.float64)).sum(axis=1) - 1.0).max() <= 1e-4
    del x
    g = normal(c4.shape, 404)
    g64 = g.astype(np.float64)
    p = np.exp(got.astype(np.float64))
    gsum = g64.sum(axis=1, keepdims=True)
    close(softmax_bwd(g, got, log=True), g64 - p * gsum, np.abs(g64) + p * np.abs(g64).sum(axis=1, keepdims=True))


# ---- config 5: fp16 epilogue on [32 x 1024, 4096] -----------------------------

def test_c5_epilogue(wm):
    rows, cols, lo, hi = 32 * 1024, 4096, -4.0, 4.0
    o32 = oracle.get("f32")
    h16 = o32.f32_to_f16(normal((rows, cols), 501))
    r16 = o32.f32_to_f16(normal((rows, cols), 502))
    g = uniform((cols,), 503, 0.8, 1.2)
    dm = normal((rows,), 504)
    dh, dr, dg_, ddm = (W.DeviceArray.from_host(a) for a in (h16, r16, g, dm))
    out = W.DeviceArray((rows, cols), np.uint16)
    mean = W.DeviceArray((rows,))
    W.call("wm_epilogue_f16_fwd", out.vp, mean.vp, dh.vp, dr.vp, dg_.vp, rows, cols, W.C.c_float(lo),
           W.C.c_float(hi))
    gh, gr, gg = W.DeviceArray((rows, cols)), W.DeviceArray((rows, cols)), W.DeviceArray((cols,))
    W.call("wm_epilogue_f16_bwd", ddm.vp, dh.vp, dr.vp, dg_.vp, gh.vp, 0, gr.vp, 0, gg.vp, 0, rows, cols,
           W.C.c_float(lo), W.C.c_float(hi))
    # forward chain in fp32 (single IEEE operations), tanh from the unary kernel
    t = o32.f16_to_f32(h16) + o32.f16_to_f32(r16)
    u = t * g
    v = np.minimum(np.maximum(u, np.float32(lo)), np.float32(hi))
    w = W.unary(W.TANH, W.DeviceArray.from_host(v)).to_host()
    del v
    assert np.array_equal(out.to_host(), o32.f32_to_f16(w))
    w64 = w.astype(np.float64)
    close(mean.to_host(), w64.sum(axis=1) / cols, np.abs(w64).sum(axis=1) / cols)
    du = np.where((u > lo) & (u < hi), dm.astype(np.float64)[:, None] * (1.0 - w64 * w64), 0.0)
    del w64
    dt = du * g.astype(np.float64)[None, :]
    close(gh.to_host(), dt, np.abs(dt))
    close(gr.to_host(), dt, np.abs(dt))
    dgt = du * t.astype(np.float64)
    close(gg.to_host(), dgt.sum(axis=0), np.abs(dgt).sum(axis=0))


def _f16_bounds_check(out16, w64, ulps=2):
    """out16 (fp16 bits) is the truncating fp16 of some fp32 value within
    `ulps` fp32 ulps of w64 (the fp32 contract of tanh, then the reference's
    float_to_half).  Truncation toward zero is monotone, so that holds iff
    out16 lies between the truncations of the interval's two ends."""
    o32 = oracle.get("f32")
    w32 = w64.astype(np.float32)
    lo, hi = w32.copy(), w32.copy()
    for _ in range(ulps):
        lo = np.nextafter(lo, np.float32(-np.inf))
        hi = np.nextafter(hi, np.float32(np.inf))
    f = o32.f16_to_f32
    got = f(out16)
    assert np.all((got >= f(o32.f32_to_f16(lo))) & (got <= f(o32.f32_to_f16(hi))))


def test_c5_epilogue_forward_against_fp64(wm):
    """The fused forward's fp16 output against fp64 tanh directly (not the
    GPU's own unary tanh): within the 2-ulp contract before truncation."""
    rows, cols, lo, hi = 32 * 1024, 4096, -4.0, 4.0
    o32 = oracle.get("f32")
    h16 = o32.f32_to_f16(normal((rows, cols), 511))
    r16 = o32.f32_to_f16(normal((rows, cols), 512))
    g = uniform((cols,), 513, 0.8, 1.2)
    dh, dr, dg_ = (W.DeviceArray.from_host(a) for a in (h16, r16, g))
    out = W.DeviceArray((rows, cols), np.uint16)
    mean = W.DeviceArray((rows,))
    W.call("wm_epilogue_f16_fwd", out.vp, mean.vp, dh.vp, dr.vp, dg_.vp, rows, cols, W.C.c_float(lo),
           W.C.c_float(hi))
    v = np.clip((o32.f16_to_f32(h16) + o32.f16_to_f32(r16)) * g, np.float32(lo), np.float32(hi))
    _f16_bounds_check(out.to_host(), np.tanh(v.astype(np.float64)))


def test_c5_tensor_api_chain(wm):
    """Config 5 as a caller of the drop-in Tensor API writes it (core/amp.h
    HalfTensor :256-286, then core/tensor.cpp add :897, mul :1063 (row
    broadcast of g), clamp :1524, tanh_ :1302, reshape :2250, mean :1709,
    reshape), at full size, forward and every closure of the backward with
    the upstream gradient injected at the root (y->grad = dm; y->grad_fn()).
    Forward: fp16 storage bit-exact, add / mul / clamp bit-exact IEEE fp32,
    tanh within 2 ulp of fp64, the mean within the sums contract; backward:
    every gradient within 1e-5 of the fp64 closed form (the mean's gradient
    unscaled, S6; clamp passes only strictly inside, S11)."""
    from whitematter_amd import _tensor as T
    B, S, C, lo, hi = 32, 1024, 4096, -4.0, 4.0
    rows = B * S
    o32 = oracle.get("f32")
    h = normal((B, S, C), 521)
    res = normal((B, S, C), 522)
    g = uniform((C,), 523, 0.8, 1.2)
    dm = normal((B, S, 1), 524)
    hh, rr = T.HalfTensor(T.Tensor.from_array(h)), T.HalfTensor(T.Tensor.from_array(res))
    h16, r16 = o32.f32_to_f16(h), o32.f32_to_f16(res)
    del h, res
    assert np.array_equal(np.asarray(hh.data).reshape(B, S, C), h16)
    assert np.array_equal(np.asarray(rr.data).reshape(B, S, C), r16)
    gt = T.Tensor.from_array(g, requires_grad=True)
    hf, rf = hh.to_float(True), rr.to_float(True)
    t1 = hf.add(rf)
    t2 = t1.mul(gt)
    t3 = t2.clamp(lo, hi)
    t4 = t3.tanh_()
    t5 = t4.reshape([rows, C])
    m = t5.mean(1, True)
    m3 = m.reshape([B, S, 1])
    assert list(m3.shape) == [B, S, 1]
    # forward
    a = o32.f16_to_f32(h16) + o32.f16_to_f32(r16)
    assert np.array_equal(np.asarray(t1.data), a)
    b = a * g
    assert np.array_equal(np.asarray(t2.data), b)
    c = np.minimum(np.maximum(b, np.float32(lo)), np.float32(hi))
    assert np.array_equal(np.asarray(t3.data), c)
    w = np.asarray(t4.data)
    u = oracle.ulp_vs_f64(w, np.tanh(c.astype(np.float64)))
    assert float(np.nanmax(u)) <= 2.0
    w64 = w.astype(np.float64).reshape(rows, C)
    close(np.asarray(m3.data).reshape(rows), w64.sum(axis=1) / C, np.abs(w64).sum(axis=1) / C)
    # backward: dm injected at the root, then every closure in order
    m3.run_grad_fn(dm)
    for node in (m, t5, t4, t3, t2, t1):
        node.call_grad_fn()
    dw = np.broadcast_to(dm.astype(np.float64).reshape(rows, 1), (rows, C)).reshape(B, S, C)
    du = np.where((b > lo) & (b < hi), dw * (1.0 - w.astype(np.float64) ** 2), 0.0)
    del w64, dw
    dt = du * g.astype(np.float64)
    close(np.asarray(hf.grad), dt, np.abs(dt))
    close(np.asarray(rf.grad), dt, np.abs(dt))
    dgt = (du * a.astype(np.float64)).reshape(rows, C)
    close(np.asarray(gt.grad), dgt.sum(axis=0), np.abs(dgt).sum(axis=0))
