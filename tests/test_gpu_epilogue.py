"""GPU parity: fp16 storage conversions and the fused config-5 epilogue
out = tanh_(clamp((h + res) * g, -4, 4)), m = mean(out, last dim, keepdim).

fp16 conversions are bit-exact against the oracle (the reference's
float_to_half / half_to_float, core/amp.h:15-72): every one of the 65536
half values, and fp32 inputs covering every rounding / overflow branch.

The fused kernels are checked against the chain of reference ops they
replace: t = h + res and u = t * g are bit-exact fp32 ops, the clamp mask is
exact, and the fp64 oracle evaluates the backward chain (the reference
closures of mean, tanh_, clamp, mul, add) on the fp32 tanh values the forward
produced -- the values the reference closure reads from result->data.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from gpu_helpers import dev
from whitematter_amd import _lib as W
from whitematter_amd import synth

pytestmark = pytest.mark.gpu

LO, HI = -4.0, 4.0


def f16_to_f32_gpu(h16):
    d = dev(h16)
    out = W.DeviceArray(h16.shape)
    W.call("wm_f16_to_f32", out.vp, d.vp, h16.size)
    return out.to_host()


def f32_to_f16_gpu(x):
    d = dev(x)
    out = W.DeviceArray(x.shape, np.uint16)
    W.call("wm_f32_to_f16_rtz", out.vp, d.vp, x.size)
    return out.to_host()


def test_f16_to_f32_exhaustive(wm):
    allh = np.arange(65536, dtype=np.uint16)
    assert oracle.bit_equal(f16_to_f32_gpu(allh), oracle.get("f32").f16_to_f32(allh))


def test_f32_to_f16_branches(wm):
    special = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e5, -1e5, 6.1e-5, 6.0e-5, 5.96e-8,
                        2.98e-8, 1e-40, -1e-40, np.inf, -np.inf, np.nan, 3.14159, -2.71828], np.float32)
    bits = np.random.default_rng(5).integers(0, 2 ** 32, 200003, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([special, bits.view(np.float32), synth.normal((100001,), 3)]).astype(np.float32)
    assert np.array_equal(f32_to_f16_gpu(x), oracle.get("f32").f32_to_f16(x))


def run_fused(h16, r16, g, dm, acc=None, lo=None, hi=None):
    lo = LO if lo is None else lo
    hi = HI if hi is None else hi
    rows, cols = h16.shape
    dh, dr, dg_, ddm = dev(h16), dev(r16), dev(g), dev(dm)
    out = W.DeviceArray((rows, cols), np.uint16)
    m = W.DeviceArray((rows,))
    W.call("wm_epilogue_f16_fwd", out.vp, m.vp, dh.vp, dr.vp, dg_.vp, rows, cols, C.c_float(lo), C.c_float(hi))
    if acc is None:
        gh, gr, gg = W.DeviceArray((rows, cols)), W.DeviceArray((rows, cols)), W.DeviceArray((cols,))
        for d in (gh, gr, gg):
            d.fill(np.nan)      # overwrite mode must not read them
        flags = (0, 0, 0)
    else:
        gh, gr, gg = dev(acc[0]), dev(acc[1]), dev(acc[2])
        flags = (1, 1, 1)
    W.call("wm_epilogue_f16_bwd", ddm.vp, dh.vp, dr.vp, dg_.vp, gh.vp, flags[0], gr.vp, flags[1], gg.vp, flags[2],
           rows, cols, C.c_float(lo), C.c_float(hi))
    return out.to_host(), m.to_host(), gh.to_host(), gr.to_host(), gg.to_host()


def tanh_gpu(v):
    return W.unary(W.TANH, dev(v)).to_host()


def reference_chain(h16, r16, g, dm, lo=None, hi=None):
    """fp32 forward intermediates (exact ops), the GPU's fp32 tanh, and the
    fp64 backward chain of the reference closures."""
    lo = LO if lo is None else lo
    hi = HI if hi is None else hi
    o32 = oracle.get("f32")
    h = o32.f16_to_f32(h16)
    r = o32.f16_to_f32(r16)
    t = o32.binary("add", h, r)
    u = o32.binary("mul", t, g)
    v = o32.unary("clamp", u, lo, hi)
    w = tanh_gpu(v)                                  # pinned by test_gpu_unary
    w64 = w.astype(np.float64)
    dv = dm.astype(np.float64)[:, None] * (1.0 - w64 * w64)
    du = np.where((u > lo) & (u < hi), dv, 0.0)
    dt = du * g.astype(np.float64)[None, :]
    dg = (du * t.astype(np.float64)).sum(axis=0)
    dg_scale = np.abs(du * t.astype(np.float64)).sum(axis=0)
    mean = w64.sum(axis=1) / h16.shape[1]
    mean_scale = np.abs(w64).sum(axis=1) / h16.shape[1]
    return w, mean, mean_scale, dt, dg, dg_scale


# (-4, 4): the bounds for which the kernels clamp with the hardware min /
# max; a zero bound takes the compare-and-select path
@pytest.mark.parametrize("bounds", [(-4.0, 4.0), (0.0, 4.0), (-1.5, -0.0)], ids=str)
@pytest.mark.parametrize("shape", [(64, 4096), (37, 1000), (5, 13), (1, 8), (300, 256), (40, 1024), (24, 2056), (9, 6144), (6, 8200)])
@pytest.mark.parametrize("accumulate", [False, True])
def test_fused_epilogue(wm, shape, accumulate, bounds):
    lo, hi = bounds
    rows, cols = shape
    h = synth.normal(shape, synth.seed_for(5, 0))
    r = synth.normal(shape, synth.seed_for(5, 1))
    g = synth.uniform((cols,), synth.seed_for(5, 2), 0.8, 1.2)
    dm = synth.normal((rows,), synth.seed_for(5, 3))
    o32 = oracle.get("f32")
    h16, r16 = o32.f32_to_f16(h), o32.f32_to_f16(r)
    acc = None
    if accumulate:
        acc = (synth.normal(shape, 91), synth.normal(shape, 92), synth.normal((cols,), 93))
    out16, m, gh, gr, gg = run_fused(h16, r16, g, dm, acc, lo, hi)
    w, mean, mean_scale, dt, dg, dg_scale = reference_chain(h16, r16, g, dm, lo, hi)
    # forward: out is the truncating fp16 of the fp32 tanh value, bit for bit
    assert np.array_equal(out16, o32.f32_to_f16(w))
    assert oracle.close_scaled(m, mean, mean_scale, 1e-5)[0]
    # backward
    if accumulate:
        dt_h, dt_r, dg = dt + acc[0], dt + acc[1], dg + acc[2]
        s_h, s_r, dg_scale = np.abs(dt) + np.abs(acc[0]), np.abs(dt) + np.abs(acc[1]), dg_scale + np.abs(acc[2])
    else:
        dt_h = dt_r = dt
        s_h = s_r = np.abs(dt)
    assert oracle.close_scaled(gh, dt_h, s_h, 1e-5, atol=1e-30)[0], "h.grad"
    assert oracle.close_scaled(gr, dt_r, s_r, 1e-5, atol=1e-30)[0], "res.grad"
    ok, worst = oracle.close_scaled(gg, dg, dg_scale, 1e-5, atol=1e-30)
    assert ok, f"g.grad off by {worst:.3g}x tolerance"


def test_fused_matches_composed_tensor_ops(wm):
    """The fused kernels equal the chain of drop-in Tensor ops on fp32 copies
    of the fp16 inputs (reshape to 2-D, mean(1, keepdim), backward)."""
    from whitematter_amd import _tensor
    T = _tensor.Tensor
    b, t_, c = 2, 16, 256
    h = synth.normal((b, t_, c), 7)
    r = synth.normal((b, t_, c), 8)
    g = synth.uniform((c,), 9, 0.8, 1.2)
    dm = synth.normal((b, t_, 1), 10)
    o32 = oracle.get("f32")
    h16, r16 = o32.f32_to_f16(h), o32.f32_to_f16(r)
    th = T.from_array(o32.f16_to_f32(h16), [b, t_, c], True)
    tr = T.from_array(o32.f16_to_f32(r16), [b, t_, c], True)
    tg = T.from_array(g, [c], True)
    out = th.add(tr).mul(tg).clamp(LO, HI).tanh_()
    m = out.reshape([b * t_, c]).mean(1, True).reshape([b, t_, 1])
    # backward() needs a scalar root: (m * dm).sum() injects dm as dL/dm
    m.mul(T.from_array(dm, [b, t_, 1], False)).sum().backward()
    out16, mf, gh, gr, gg = run_fused(h16.reshape(b * t_, c), r16.reshape(b * t_, c), g, dm.reshape(-1))
    assert np.array_equal(out16.reshape(b, t_, c), o32.f32_to_f16(out.data))
    assert np.allclose(mf.reshape(b, t_, 1), m.data, rtol=1e-6, atol=1e-7)
    assert np.allclose(gh.reshape(b, t_, c), th.grad, rtol=1e-5, atol=1e-7)
    assert np.allclose(gr.reshape(b, t_, c), tr.grad, rtol=1e-5, atol=1e-7)
    assert np.allclose(gg, tg.grad, rtol=1e-4, atol=1e-5)
