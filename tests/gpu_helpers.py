"""Helpers shared by the GPU parity tests: run one op through the C ABI and
return host arrays."""
import ctypes as C

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
    the accumulate mode (None = known-zero, overwrite mode).  out=None passes
    no forward output (pow then recomputes it)."""
    dg, da, db = dev(g), dev(a), dev(b)
    dout = dev(out) if out is not None else None
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


# ---- loss heads (include/wm_loss.h) -------------------------------------------

def _scalar_dev(v):
    return dev(np.float32([v]))


def _grad_buffer(shape, g0):
    """Gradient buffer: g0 for the accumulate mode, else NaN-filled (a
    known-zero buffer that the kernel must overwrite without reading)."""
    if g0 is not None:
        return dev(g0), 1
    d = W.DeviceArray(shape)
    d.fill(np.nan)
    return d, 0


def ce_fwd(x, lab):
    """-> (loss, stats [rows, 2]) through wm_cross_entropy_fwd."""
    rows, cols = x.shape
    dx, dl = dev(x), dev(lab)
    stats, loss = W.DeviceArray((max(rows, 1), W.CE_STATS)), W.DeviceArray((1,))
    W.call("wm_cross_entropy_fwd", dx.vp, dl.vp, rows, cols, stats.vp, loss.vp)
    return loss.to_host()[0], stats.to_host()[:rows]


def ce_bwd(x, lab, loss_grad=1.0, g0=None):
    rows, cols = x.shape
    dx, dl = dev(x), dev(lab)
    stats, loss = W.DeviceArray((max(rows, 1), W.CE_STATS)), W.DeviceArray((1,))
    W.call("wm_cross_entropy_fwd", dx.vp, dl.vp, rows, cols, stats.vp, loss.vp)
    gx, acc = _grad_buffer(x.shape, g0)
    lg = _scalar_dev(loss_grad)  # referenced until the call returns
    W.call("wm_cross_entropy_bwd", dx.vp, dl.vp, stats.vp, lg.vp, gx.vp, acc, rows, cols)
    return gx.to_host()


def nll_fwd(x, lab):
    rows, cols = x.shape
    dx, dl, loss = dev(x), dev(lab), W.DeviceArray((1,))
    W.call("wm_nll_fwd", dx.vp, dl.vp, rows, cols, loss.vp)
    return loss.to_host()[0]


def nll_bwd(shape, lab, loss_grad=1.0, g0=None):
    dl = dev(lab)
    gx, acc = _grad_buffer(shape, g0)
    lg = _scalar_dev(loss_grad)
    W.call("wm_nll_bwd", dl.vp, lg.vp, gx.vp, acc, shape[0], shape[1])
    return gx.to_host()


def focal_fwd(x, lab, gamma, alpha):
    rows, cols = x.shape
    dx, dl = dev(x), dev(lab)
    stats, loss = W.DeviceArray((max(rows, 1), W.FOCAL_STATS)), W.DeviceArray((1,))
    W.call("wm_focal_fwd", dx.vp, dl.vp, rows, cols, C.c_float(gamma), C.c_float(alpha), stats.vp, loss.vp)
    return loss.to_host()[0], stats.to_host()[:rows]


def focal_bwd(x, lab, gamma, alpha, loss_grad=1.0, g0=None):
    rows, cols = x.shape
    dx, dl = dev(x), dev(lab)
    stats, loss = W.DeviceArray((max(rows, 1), W.FOCAL_STATS)), W.DeviceArray((1,))
    W.call("wm_focal_fwd", dx.vp, dl.vp, rows, cols, C.c_float(gamma), C.c_float(alpha), stats.vp, loss.vp)
    gx, acc = _grad_buffer(x.shape, g0)
    lg = _scalar_dev(loss_grad)
    W.call("wm_focal_bwd", dx.vp, dl.vp, stats.vp, lg.vp, gx.vp, acc, rows, cols,
           C.c_float(gamma), C.c_float(alpha))
    return gx.to_host()


POINTWISE_KIND = {"smooth_l1": 0, "bce": 1, "bce_logits": 2, "kldiv": 3, "kldiv_log": 4, "binary_focal": 5}


def _offset_dev(a, offset):
    """a on the device starting `offset` floats into its allocation (offset 1
    gives a pointer that is not 16-byte aligned, the kernels' scalar path)."""
    buf = np.zeros(a.size + offset, np.float32)
    buf[offset:] = a.ravel()
    d = dev(buf)
    return d, C.c_void_p(d.ptr + 4 * offset)


def pw_fwd(kind, x, y, p0=0.0, p1=0.0, denom=None, offset=0):
    dxa, dx = _offset_dev(x, offset)
    dya, dy = _offset_dev(y, offset)
    loss = W.DeviceArray((1,))
    d = float(x.size if denom is None else denom)
    W.call("wm_pointwise_loss_fwd", POINTWISE_KIND[kind], dx, dy, x.size, C.c_float(p0), C.c_float(p1),
           C.c_float(d), loss.vp)
    return loss.to_host()[0]


def pw_bwd(kind, x, y, p0=0.0, p1=0.0, denom=None, loss_grad=1.0, g0=None, offset=0):
    dxa, dx = _offset_dev(x, offset)
    dya, dy = _offset_dev(y, offset)
    if g0 is not None:
        dga, dg = _offset_dev(g0, offset)
        acc = 1
    else:
        dga, dg = _offset_dev(np.full(x.size, np.nan, np.float32), offset)
        acc = 0
    d = float(x.size if denom is None else denom)
    lg = _scalar_dev(loss_grad)
    W.call("wm_pointwise_loss_bwd", POINTWISE_KIND[kind], dx, dy, x.size, C.c_float(p0), C.c_float(p1),
           C.c_float(d), lg.vp, dg, acc)
    return dga.to_host()[offset:].reshape(x.shape)


# ---- LayerNorm / BatchNorm2d / attention softmax (include/wm_layers.h) ---------

def _opt_grad(shape, g0, want):
    """(device buffer or None, accumulate flag) for an optional gradient."""
    if not want:
        return None, 0
    return _grad_buffer(shape, g0)


def layernorm_fwd(x, gamma, beta, eps=1e-5):
    n = gamma.size
    rows = x.size // n
    dx, dgm, dbt = dev(x), dev(gamma), dev(beta)
    y, mean, inv = W.DeviceArray(x.shape), W.DeviceArray((max(rows, 1),)), W.DeviceArray((max(rows, 1),))
    W.call("wm_layernorm_fwd", dx.vp, dgm.vp, dbt.vp, rows, n, C.c_float(eps), y.vp, mean.vp, inv.vp)
    return y.to_host(), mean.to_host()[:rows], inv.to_host()[:rows]


def layernorm_bwd(g, x, gamma, mean, inv, gx0=None, dg0=None, db0=None, want=(True, True, True)):
    n = gamma.size
    rows = x.size // n
    dg_, dx, dgm, dm, di = dev(g), dev(x), dev(gamma), dev(mean), dev(inv)
    gx, ax = _opt_grad(x.shape, gx0, want[0])
    gg, ag = _opt_grad((n,), dg0, want[1])
    gb, ab = _opt_grad((n,), db0, want[2])
    W.call("wm_layernorm_bwd", dg_.vp, dx.vp, dgm.vp, dm.vp, di.vp, rows, n, gx.vp if gx else None, ax,
           gg.vp if gg else None, ag, gb.vp if gb else None, ab)
    return tuple(b.to_host() if b is not None else None for b in (gx, gg, gb))


def batchnorm_fwd(x, gamma, beta, rm, rv, training=True, eps=1e-5, momentum=0.1):
    B, Cc = x.shape[0], x.shape[1]
    S = x.size // (B * Cc) if B * Cc else 0
    dx, dgm, dbt, drm, drv = dev(x), dev(gamma), dev(beta), dev(rm), dev(rv)
    y, mean, inv = W.DeviceArray(x.shape), W.DeviceArray((max(Cc, 1),)), W.DeviceArray((max(Cc, 1),))
    W.call("wm_batchnorm2d_fwd", dx.vp, dgm.vp, dbt.vp, drm.vp, drv.vp, B, Cc, S, C.c_float(eps),
           C.c_float(momentum), int(training), y.vp, mean.vp, inv.vp)
    return y.to_host(), mean.to_host()[:Cc], inv.to_host()[:Cc], drm.to_host(), drv.to_host()


def batchnorm_bwd(g, x, gamma, mean, inv, gx0=None, dg0=None, db0=None, want=(True, True, True)):
    B, Cc = x.shape[0], x.shape[1]
    S = x.size // (B * Cc) if B * Cc else 0
    dg_, dx, dgm, dm, di = dev(g), dev(x), dev(gamma), dev(mean), dev(inv)
    gx, ax = _opt_grad(x.shape, gx0, want[0])
    gg, ag = _opt_grad((Cc,), dg0, want[1])
    gb, ab = _opt_grad((Cc,), db0, want[2])
    W.call("wm_batchnorm2d_bwd", dg_.vp, dx.vp, dgm.vp, dm.vp, di.vp, B, Cc, S, gx.vp if gx else None, ax,
           gg.vp if gg else None, ag, gb.vp if gb else None, ab)
    return tuple(b.to_host() if b is not None else None for b in (gx, gg, gb))


def attn_softmax_fwd(scores, mask=None):
    B, H, tq, tk = scores.shape
    ds_ = dev(scores)
    dm = dev(mask) if mask is not None else None
    out = W.DeviceArray(scores.shape)
    W.call("wm_attention_softmax_fwd", ds_.vp, dm.vp if dm else None, mask.shape[0] if mask is not None else 0,
           B, H, tq, tk, out.vp)
    return out.to_host()


def attn_softmax_bwd(attn, d_attn):
    tk = attn.shape[-1]
    da, dd = dev(attn), dev(d_attn)
    out = W.DeviceArray(attn.shape)
    out.fill(np.nan)
    W.call("wm_attention_softmax_bwd", da.vp, dd.vp, attn.size // tk, tk, out.vp)
    return out.to_host()


# ---- matrix products (include/wm_gemm.h) ------------------------------------------

def matmul(a, b):
    """a [m, k] @ b [k, n] (2-D) or bmm for 3-D operands."""
    da, db = dev(a), dev(b)
    if a.ndim == 2:
        m, k = a.shape
        n = b.shape[1]
        out = W.DeviceArray((m, n))
        out.fill(np.nan)
        W.call("wm_matmul", da.vp, db.vp, m, k, n, out.vp)
    else:
        P, m, k = a.shape
        n = b.shape[2]
        out = W.DeviceArray((P, m, n))
        out.fill(np.nan)
        W.call("wm_bmm", da.vp, db.vp, P, m, k, n, out.vp)
    return out.to_host()


def matmul_bwd(g, a, b, ga0=None, gb0=None, need_a=True, need_b=True):
    """(ga0 + g @ b^T, gb0 + a^T @ g) per problem through wm_matmul_bwd /
    wm_bmm_bwd; a gradient without a start value is written (accumulate 0)
    into a NaN-filled buffer."""
    dg, da, db = dev(g), dev(a), dev(b)
    keep = []

    def grad_buf(shape, start, need):
        if not need:
            return None, 0
        if start is not None:
            d = dev(np.asarray(start, np.float32))
            keep.append(d)
            return d, 1
        d = W.DeviceArray(shape)
        d.fill(np.nan)
        keep.append(d)
        return d, 0

    ga, acc_a = grad_buf(a.shape, ga0, need_a)
    gb, acc_b = grad_buf(b.shape, gb0, need_b)
    if a.ndim == 2:
        m, k = a.shape
        n = b.shape[1]
        W.call("wm_matmul_bwd", dg.vp, da.vp, db.vp, m, k, n, W.ptr(ga), acc_a, W.ptr(gb), acc_b)
    else:
        P, m, k = a.shape
        n = b.shape[2]
        W.call("wm_bmm_bwd", dg.vp, da.vp, db.vp, P, m, k, n, W.ptr(ga), acc_a, W.ptr(gb), acc_b)
    return (ga.to_host() if ga else None), (gb.to_host() if gb else None)


def gemm(ta, tb, m, n, k, alpha, a, lda, b, ldb, c0, ldc, accumulate, bias=None, batch=1, batch_inner=1,
         strides=None):
    """wm_gemm on host arrays holding the operands' storage (flat); returns
    the C storage after the call (c0 is its initial content)."""
    da, db, dc = dev(np.asarray(a, np.float32)), dev(np.asarray(b, np.float32)), dev(np.asarray(c0, np.float32))
    dbias = dev(np.asarray(bias, np.float32)) if bias is not None else None
    st = (C.c_int64 * 6)(*strides) if strides is not None else None
    W.call("wm_gemm", int(ta), int(tb), m, n, k, C.c_float(alpha), da.vp, lda, db.vp, ldb, dc.vp, ldc,
           int(accumulate), W.ptr(dbias), batch, batch_inner, st)
    return dc.to_host()


def mha_fwd(q, k, v, params, heads, mask=None):
    """wm_mha_fwd; returns dict(out, attn, Q, K, V, ctx) as host arrays."""
    B, Sq, E = q.shape
    Sk = k.shape[1]
    d_in = [dev(x) for x in (q, k, v)]
    dm = dev(mask) if mask is not None else None
    dp = [dev(np.asarray(p, np.float32)) for p in params]
    outs = {"out": (B, Sq, E), "attn": (B, heads, Sq, Sk), "Q": (B, Sq, E), "K": (B, Sk, E), "V": (B, Sk, E),
            "ctx": (B, Sq, E)}
    dev_out = {n: W.DeviceArray(s) for n, s in outs.items()}
    for d in dev_out.values():
        d.fill(np.nan)
    W.call("wm_mha_fwd", *[x.vp for x in d_in], W.ptr(dm), mask.shape[0] if mask is not None else 0,
           *[p.vp for p in dp], B, Sq, Sk, E, heads, *[dev_out[n].vp for n in outs])
    return {n: d.to_host() for n, d in dev_out.items()}


def mha_bwd(dout, q, k, v, params, heads, saved, need=(True, True, True), alias=False, start=None):
    """wm_mha_bwd adding into gradient buffers that start at `start[name]`
    (default zeros); returns dict of host gradients (gq only, with alias)."""
    B, Sq, E = q.shape
    Sk = k.shape[1]
    start = start or {}
    shapes = {"gWq": (E, E), "gWk": (E, E), "gWv": (E, E), "gWo": (E, E), "gbq": (E,), "gbk": (E,), "gbv": (E,),
              "gbo": (E,), "gq": q.shape, "gk": k.shape, "gv": v.shape}
    bufs = {}
    for n, s in shapes.items():
        if n in ("gq", "gk", "gv"):
            i = ("gq", "gk", "gv").index(n)
            if not need[i] or (alias and n != "gq"):
                continue
        bufs[n] = dev(np.asarray(start.get(n, np.zeros(s, np.float32)), np.float32))
    if alias:
        for i, n in ((1, "gk"), (2, "gv")):
            if need[i]:
                bufs[n] = bufs["gq"]
    ins = [dev(x) for x in (dout, q, k, v)] + [dev(np.asarray(p, np.float32)) for p in params[:4]]
    sv = [dev(saved[n]) for n in ("Q", "K", "V", "attn", "ctx")]
    W.call("wm_mha_bwd", *[x.vp for x in ins], *[x.vp for x in sv], B, Sq, Sk, E, heads,
           *[W.ptr(bufs.get(n)) for n in shapes])
    return {n: d.to_host() for n, d in bufs.items() if not (alias and n in ("gk", "gv"))}


def mha_forward_scales(q, k, v, params, H, f):
    """First-order error scales of Q, K, V, attn, ctx, out from the fp64
    forward f: |x| |W|^T + |b| for projections; for a weight a_ij of a row
    with score scales s_ij, a_ij * (s_ij + sum_j a_ij s_ij); the context and
    output carry both their own sums of |terms| and their inputs' scales."""
    Wq, Wk, Wv, Wo, bq, bk, bv, bo = [np.abs(np.asarray(p, np.float64)) for p in params]
    B, Sq, E = q.shape
    Sk = k.shape[1]
    hd = E // H

    def proj(x, Wa, ba):
        return np.abs(x.astype(np.float64)) @ Wa.T + ba

    sQ, sK, sV = proj(q, Wq, bq), proj(k, Wk, bk), proj(v, Wv, bv)
    scale = 1.0 / np.sqrt(hd)
    heads = lambda X, S: X.reshape(B, S, H, hd).transpose(0, 2, 1, 3)  # noqa: E731
    s_sc = scale * (heads(sQ, Sq) @ heads(sK, Sk).transpose(0, 1, 3, 2))
    a = f["attn"]
    s_at = a * (s_sc + (a * s_sc).sum(-1, keepdims=True))
    Vh, sVh = np.abs(heads(f["V"], Sk)), heads(sV, Sk)
    s_ctx = (s_at @ Vh + a @ sVh + a @ Vh).transpose(0, 2, 1, 3).reshape(B, Sq, E)
    s_out = s_ctx @ Wo.T + bo
    return {"Q": sQ, "K": sK, "V": sV, "attn": s_at + 1e-30, "ctx": s_ctx, "out": s_out}
