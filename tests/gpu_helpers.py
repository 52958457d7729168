"""Helpers shared by the GPU parity tests: run one op through the C ABI and
return host arrays."""
import numpy as np

from whitematter_amd import _lib as W
from whitematter_amd import synth


def dev(a):
    return W.DeviceArray.from_host(np.ascontiguousarray(a))


def rng_normal(shape, seed, std=1.0):
    return synth.normal(shape, 0xC0FFEE00 + seed, 0.0, std)


def rng_uniform(shape, seed, lo, hi):
    return synth.uniform(shape, 0xC0FFEE00 + seed, lo, hi)


def binary_fwd(op, a, b):
    da, db = dev(a), dev(b)
    out = W.binary(W.BINARY_OPS[op], da, db)
    return out.to_host()


def binary_bwd(op, g, a, b, out, ga0=None, gb0=None, need_a=True, need_b=True):
    """Backward through wm_binary_bwd.  ga0/gb0: initial gradient buffers for
    the accumulate mode (None = known-zero, overwrite mode)."""
    dg, da, db, dout = dev(g), dev(a), dev(b), dev(out)
    dga = (dev(ga0) if ga0 is not None else W.DeviceArray(a.shape)) if need_a else None
    dgb = (dev(gb0) if gb0 is not None else W.DeviceArray(b.shape)) if need_b else None
    if dga is not None and ga0 is None:
        dga.fill(np.nan)  # overwrite mode must not read it
    if dgb is not None and gb0 is None:
        dgb.fill(np.nan)
    W.binary_bwd(W.BINARY_OPS[op], dg, da, db, dout, dga, ga0 is not None, dgb, gb0 is not None)
    return (dga.to_host() if dga is not None else None, dgb.to_host() if dgb is not None else None)


def unary_fwd(op, x, p0=0.0, p1=0.0):
    return W.unary(W.UNARY_OPS[op], dev(x), p0, p1).to_host()


def unary_bwd(op, g, x, out, gx0=None, p0=0.0, p1=0.0):
    dgx = dev(gx0) if gx0 is not None else W.DeviceArray(g.shape)
    if gx0 is None:
        dgx.fill(np.nan)
    W.unary_bwd(W.UNARY_OPS[op], dev(g), dev(x), dev(out), dgx, gx0 is not None, p0, p1)
    return dgx.to_host()


def reduce(op, x, outer, n, inner, want_idx=False):
    v, i = W.reduce(W.REDUCE_OPS[op], dev(x), outer, n, inner, want_val=True, want_idx=want_idx)
    return v.to_host(), (i.to_host() if i is not None else None)


def reduce_bwd(op, g, idx, outer, n, inner, gx0=None):
    dgx = dev(gx0) if gx0 is not None else W.DeviceArray((outer, n, inner))
    if gx0 is None:
        dgx.fill(np.nan)
    W.reduce_bwd(W.REDUCE_OPS[op], dev(g), dev(idx) if idx is not None else None, outer, n, inner, dgx,
                 gx0 is not None)
    return dgx.to_host()


def softmax_fwd(x, log=False):
    dx = dev(x)
    out = W.DeviceArray(x.shape)
    W.call("wm_log_softmax_fwd" if log else "wm_softmax_fwd", out.vp, dx.vp, x.shape[0], x.shape[1])
    return out.to_host()


def softmax_bwd(g, out, gx0=None, log=False):
    dgx = dev(gx0) if gx0 is not None else W.DeviceArray(g.shape)
    if gx0 is None:
        dgx.fill(np.nan)
    # Keep the device copies referenced until the call returns: a temporary
    # freed mid-expression goes back to the pool and the next allocation of
    # the same size would alias it.
    dg, dout = dev(g), dev(out)
    W.call("wm_log_softmax_bwd" if log else "wm_softmax_bwd", dg.vp, dout.vp, dgx.vp,
           int(gx0 is not None), g.shape[0], g.shape[1])
    return dgx.to_host()
