"""GPU parity on the benchmark configurations' own seeded inputs (the recipe
of whitematter_amd/synth.py, byte for byte what bench.py times), at full
size.

Row-local outputs (element-wise forwards and gradients, dim-1 reductions,
softmax rows, the epilogue's rows) are checked on three blocks of rows --
the first, a middle and the last -- against the CPU oracle (oracle/) run on
those rows; outputs that combine every row (dim-0 and full reductions, the
broadcast vectors' gradients, the epilogue's g.grad) are checked in full
against the fp64 oracle or fp64 numpy on the whole input.  The bars are the
contract's: bit-exact for the IEEE element-wise ops and the max family
(values and first-index positions), <= 2 ulp of fp64 for pow and tanh,
1e-5 of the sum of |terms| for sums, means, softmax and gradients.

References: core/tensor.cpp add/mul/div/pow :897-1475, sum/mean/max/min
:1637-1899, argmax/argmin :2075-2221, softmax/log_softmax :1548-1635,
clamp/tanh_ :1302-1321, :1524-1546; core/amp.h float_to_half :15-72.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from whitematter_amd import _lib as W
from whitematter_amd import synth

pytestmark = pytest.mark.gpu

BLOCK = 32


def blocks(rows):
    """Row indices of the first, a middle and the last block."""
    mid = rows // 2 - BLOCK // 2
    return np.concatenate([np.arange(BLOCK), np.arange(mid, mid + BLOCK), np.arange(rows - BLOCK, rows)])


def close(got, ref, scale, rtol=1e-5):
    ok, worst = oracle.close_scaled(got, ref, scale, rtol, atol=1e-30)
    assert ok, f"{worst:.3g}x tolerance"


def host(d):
    return d.to_host()


# ---- config 2: A[8192, 8192], c[8192, 1], r[1, 8192] ---------------------------

@pytest.fixture(scope="module")
def c2(wm):
    A, c, r, G = synth.config2()
    return {"A": A, "c": c, "r": r, "G": G, "dA": W.DeviceArray.from_host(A), "dc": W.DeviceArray.from_host(c),
            "dr": W.DeviceArray.from_host(r), "dG": W.DeviceArray.from_host(G)}


@pytest.mark.parametrize("name,op,vec", [("A+r", "add", "r"), ("A*c", "mul", "c"), ("A/r", "div", "r"),
                                         ("A^c", "pow", "c")])
def test_c2_recipe(wm, c2, name, op, vec):
    A, G = c2["A"], c2["G"]
    other = c2[vec]
    dother = c2["d" + vec]
    R, Cc = A.shape
    idx = blocks(R)
    o32, o64, oab = oracle.get("f32"), oracle.get("f64"), oracle.get("abs")
    out = W.binary(W.BINARY_OPS[op], c2["dA"], dother)
    o = host(out)[idx]
    sub_other = other[idx] if vec == "c" else other
    if op == "pow":
        d = oracle.ulp_vs_f64(o, o64.binary("pow", A[idx], sub_other))
        assert d.max() <= 2.0, f"pow forward {d.max():.3g} ulp"
    else:
        assert oracle.bit_equal(o, o32.binary(op, A[idx], sub_other)), name + " forward"
    gA, gv = W.DeviceArray(A.shape), W.DeviceArray(other.shape)
    gA.fill(0.0)
    gv.fill(0.0)
    W.binary_bwd(W.BINARY_OPS[op], c2["dG"], c2["dA"], dother, None, gA, True, gv, True)
    fwd = o if op == "pow" else None
    ga64, gb64 = o64.binary_bwd(op, G[idx], A[idx], sub_other, out=fwd)
    gaab, gbab = oab.binary_bwd(op, G[idx], A[idx], sub_other, out=fwd)
    close(host(gA)[idx], ga64, gaab)
    gvh = host(gv)
    if vec == "c":          # row sums: row-local
        close(gvh[idx], gb64, gbab)
    else:                   # column sums over every row: fp64 over the whole tensor
        A64, G64, r64 = A.astype(np.float64), G.astype(np.float64), other.astype(np.float64)
        if op == "add":
            terms = G64
        else:               # div: gb -= g a / (b b)
            terms = -(G64 * A64) / (r64 * r64)
        close(gvh, terms.sum(axis=0, keepdims=True), np.abs(terms).sum(axis=0, keepdims=True))


# ---- config 3: X[16384, 4096] quantised to 1/64 -----------------------------------

@pytest.fixture(scope="module")
def c3(wm):
    X = synth.config3()
    return X, W.DeviceArray.from_host(X)


@pytest.mark.parametrize("dim", [0, 1])
def test_c3_recipe(wm, c3, dim):
    X, dX = c3
    R, Cc = X.shape
    outer, n, inner = (1, R, Cc) if dim == 0 else (R, Cc, 1)
    o32, o64, oab = oracle.get("f32"), oracle.get("f64"), oracle.get("abs")
    for name in ("sum", "mean", "max", "min", "argmax", "argmin"):
        want_idx = name in ("max", "min", "argmax", "argmin")
        v, i = W.reduce(W.REDUCE_OPS[name], dX, outer, n, inner, want_val=True, want_idx=want_idx)
        v, i = host(v).reshape(-1), (host(i).reshape(-1) if i is not None else None)
        if dim == 1:   # row-local: the three row blocks through the oracle
            idx = blocks(R)
            xs, so, sn, si = X[idx], len(idx), Cc, 1
            v, i = v[idx], (i[idx] if i is not None else None)
        else:
            xs, so, sn, si = X, outer, n, inner
        if name in ("sum", "mean"):
            close(v, o64.reduce(name, xs, so, sn, si)[0].reshape(-1), oab.reduce(name, xs, so, sn, si)[0].reshape(-1))
            # quantised values: every partial sum is exact in fp32
            assert oracle.bit_equal(v, o32.reduce(name, xs, so, sn, si)[0].reshape(-1)), name + " not exact"
        else:
            rv, ri = o32.reduce(name, xs, so, sn, si)
            assert oracle.bit_equal(v, rv.reshape(-1)), f"{name} dim{dim} values"
            assert np.array_equal(i, ri.reshape(-1)), f"{name} dim{dim} positions (first index wins)"


def test_c3_recipe_full_sum_and_max_backward(wm, c3):
    X, dX = c3
    R, Cc = X.shape
    o32, o64, oab = oracle.get("f32"), oracle.get("f64"), oracle.get("abs")
    v, _ = W.reduce(W.R_SUM, dX, 1, X.size, 1)
    close(host(v).reshape(-1), o64.reduce("sum", X, 1, X.size, 1)[0].reshape(-1),
          oab.reduce("sum", X, 1, X.size, 1)[0].reshape(-1))
    for dim, (outer, n, inner) in ((0, (1, R, Cc)), (1, (R, Cc, 1))):
        g = synth.normal((outer * inner,), synth.seed_for(3, 5 + dim))
        _, i = W.reduce(W.R_MAX, dX, outer, n, inner, want_val=False, want_idx=True)
        gx = W.DeviceArray(X.shape)
        gx.fill(0.0)
        W.reduce_bwd(W.R_MAX, W.DeviceArray.from_host(g), i, outer, n, inner, gx, True)
        ref = o32.reduce_bwd("max", g, o32.reduce("max", X, outer, n, inner)[1], outer, n, inner)
        assert oracle.bit_equal(host(gx).reshape(-1), ref.reshape(-1)), f"max dim{dim} backward"


# ---- config 4: logits[8192, 32000] ~N(0,3), 1% set to +20 ---------------------------

@pytest.fixture(scope="module")
def c4(wm):
    L, G = synth.config4()
    return L, G, W.DeviceArray.from_host(L), W.DeviceArray.from_host(G)


@pytest.mark.parametrize("log", [False, True], ids=["softmax", "log_softmax"])
def test_c4_recipe(wm, c4, log):
    L, G, dL, dG = c4
    R, Cc = L.shape
    assert np.count_nonzero(L == np.float32(20.0)) > 0.009 * L.size   # the spikes are set to +20
    idx = blocks(R)
    o64, oab = oracle.get("f64"), oracle.get("abs")
    y = W.DeviceArray(L.shape)
    W.call("wm_log_softmax_fwd" if log else "wm_softmax_fwd", y.vp, dL.vp, R, Cc)
    gx = W.DeviceArray(L.shape)
    gx.fill(0.0)
    W.call("wm_log_softmax_bwd" if log else "wm_softmax_bwd", dG.vp, y.vp, gx.vp, 1, R, Cc)
    ys, gxs = host(y)[idx], host(gx)[idx]
    Ls, Gs = L[idx], G[idx]
    ref = o64.softmax(Ls, log=log)
    close(ys, ref, oab.softmax(Ls, log=log) if log else ref)
    if log:
        close(gxs, o64.softmax_bwd(Gs, ys, log=True), oab.softmax_bwd(Gs, ys, log=True))
    else:
        # the closure's value in closed form, fp64: s_j (g_j - sum_k g_k s_k)
        g64, s = Gs.astype(np.float64), ys.astype(np.float64)
        gs = g64 * s
        close(gxs, gs - s * gs.sum(axis=1, keepdims=True),
              np.abs(gs) + s * np.abs(gs).sum(axis=1, keepdims=True))
        # and the reference's explicit Jacobian (O(C^2)) on two of those rows
        for r in (0, 2 * BLOCK):
            jac = o64.softmax_bwd(Gs[r:r + 1], ys[r:r + 1])
            close(gxs[r:r + 1], jac, np.abs(gs[r:r + 1]) + s[r:r + 1] * np.abs(gs[r:r + 1]).sum())


# ---- config 5: h, res[32, 1024, 4096] -> fp16 (truncating), g[4096] -------------------

def test_c5_recipe(wm):
    h, res, g, dm = synth.config5()
    B, S, Cc = h.shape
    R = B * S
    lo, hi = -4.0, 4.0
    o32 = oracle.get("f32")
    dh32 = W.DeviceArray.from_host(h)
    h16 = W.DeviceArray((R, Cc), np.uint16)
    W.call("wm_f32_to_f16_rtz", h16.vp, dh32.vp, R * Cc)
    dh32.free()
    dr32 = W.DeviceArray.from_host(res)
    r16 = W.DeviceArray((R, Cc), np.uint16)
    W.call("wm_f32_to_f16_rtz", r16.vp, dr32.vp, R * Cc)
    dr32.free()
    h16h, r16h = host(h16), host(r16)
    idx = blocks(R)
    hb, rb = h.reshape(R, Cc)[idx], res.reshape(R, Cc)[idx]
    del h, res
    assert np.array_equal(h16h[idx], o32.f32_to_f16(hb)) and np.array_equal(r16h[idx], o32.f32_to_f16(rb))
    dg_, ddm = W.DeviceArray.from_host(g), W.DeviceArray.from_host(dm.reshape(-1))
    out, m = W.DeviceArray((R, Cc), np.uint16), W.DeviceArray((R,))
    W.call("wm_epilogue_f16_fwd", out.vp, m.vp, h16.vp, r16.vp, dg_.vp, R, Cc, C.c_float(lo), C.c_float(hi))
    gh, gr, gg = W.DeviceArray((R, Cc)), W.DeviceArray((R, Cc)), W.DeviceArray((Cc,))
    W.call("wm_epilogue_f16_bwd", ddm.vp, h16.vp, r16.vp, dg_.vp, gh.vp, 0, gr.vp, 0, gg.vp, 0, R, Cc,
           C.c_float(lo), C.c_float(hi))
    out_h, m_h, gh_h, gr_h, gg_h = host(out), host(m), host(gh), host(gr), host(gg)
    dm = dm.reshape(-1)
    g64 = g.astype(np.float64)
    dg64 = np.zeros(Cc)
    dg_scale = np.zeros(Cc)
    step = 2048
    for r0 in range(0, R, step):
        rows = np.arange(r0, r0 + step)
        t = o32.f16_to_f32(h16h[rows]) + o32.f16_to_f32(r16h[rows])    # IEEE fp32, as the reference's add
        u = t * g                                                        # and mul
        v = np.minimum(np.maximum(u, np.float32(lo)), np.float32(hi))
        w = W.unary(W.TANH, W.DeviceArray.from_host(v)).to_host()        # the fp32 tanh (pinned to 2 ulp)
        w64 = w.astype(np.float64)
        du = np.where((u > lo) & (u < hi), dm[rows, None].astype(np.float64) * (1.0 - w64 * w64), 0.0)
        dgt = du * t.astype(np.float64)
        dg64 += dgt.sum(axis=0)
        dg_scale += np.abs(dgt).sum(axis=0)
        sel = np.isin(rows, idx)
        if sel.any():
            rs = rows[sel]
            # forward: out is the truncating fp16 of the fp32 tanh, bit for bit; fp64 tanh within 2 ulp
            assert np.array_equal(out_h[rs], o32.f32_to_f16(w[sel]))
            assert oracle.ulp_vs_f64(w[sel], np.tanh(v[sel].astype(np.float64))).max() <= 2.0
            close(m_h[rs], w64[sel].sum(axis=1) / Cc, np.abs(w64[sel]).sum(axis=1) / Cc)
            dt = du[sel] * g64[None, :]
            close(gh_h[rs], dt, np.abs(dt))
            close(gr_h[rs], dt, np.abs(dt))
    close(gg_h, dg64, dg_scale)
