"""Benchmark of the MI355X Tensor elementwise / broadcast / reduction path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c2]

Metric: achieved HBM GB/s (% of MI355X peak) per op, and the
speedup over the host-CPU reference path.  A "step" is one pass of the
configuration's ops, forward and backward, over inputs already resident in
HBM.  Each op is timed with HIP events recorded on the library stream (the
stream every kernel is launched on); a 512 MiB fill runs between ops (outside
the timed region) so no op starts with its inputs in L2 / Infinity Cache.

Bytes are ALGORITHMIC: every distinct input read once (broadcast operands at
their real size), every output written once, read + write for every gradient
accumulated with "+=".  pow's backward recomputes pow(a, b) instead of
reading the saved output, so its bytes are the recompute figure.

The default workload is config 2: A[8192,8192]
with r[1,8192] and c[8192,1]; A+r, A*c, A/r, A->pow(c), forward and backward.
``value`` is the step's total algorithmic bytes over its total kernel time.
Other configs (--config c1/c3/c4/c5) print the same line for that workload.

The CPU baseline is the reference's own core/tensor.cpp (oracle/_ref, built
with the reference's flags) -- or, where that is not built, the oracle's
restatement compiled with the same flags -- timed single-threaded on one host
core over a row slice of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from whitematter_amd import _lib as W  # noqa: E402
from whitematter_amd import synth  # noqa: E402

PEAK_GBPS = 8000.0  # MI355X HBM3E
PEAK_F32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix
METRIC = "achieved HBM GB/s (% of MI355X peak) per op; speedup vs host-CPU ref"
METRIC_MFMA = "achieved fp32 matrix-core TFLOP/s (% of MI355X dense fp32 peak) per op"
F32 = 4


class Op:
    def __init__(self, name, launch, nbytes, kernel, elems, flops=None):
        self.name, self.launch, self.bytes, self.kernel, self.elems = name, launch, nbytes, kernel, elems
        self.flops = flops  # set for matrix-core ops: their roofline is TFLOP/s, not HBM
        self.ms = []   # event basis: markers before and after the op on the library stream
        self.kms = []  # kernel basis: first kernel's start to last kernel's end (wm_span_*)


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------

def shape_arg(s):
    return W.shape_arg(s)


def c2_ops(rows=8192, cols=8192):
    A, c, r, G = synth.config2(rows, cols)
    dA, dc, dr, dG = (W.DeviceArray.from_host(x) for x in (A, c, r, G))
    out = W.DeviceArray((rows, cols))
    gA = W.DeviceArray((rows, cols)); gA.fill(0.0)
    gc = W.DeviceArray((rows, 1)); gc.fill(0.0)
    gr = W.DeviceArray((1, cols)); gr.fill(0.0)
    N = rows * cols
    big = N * F32
    ops = []
    for name, code, other, gother, vec in (("A+r", W.ADD, dr, gr, cols), ("A*c", W.MUL, dc, gc, rows),
                                           ("A/r", W.DIV, dr, gr, cols), ("A^c", W.POW, dc, gc, rows)):
        sa, na = shape_arg(dA.shape)
        sb, nb = shape_arg(other.shape)

        def fwd(code=code, other=other, sa=sa, na=na, sb=sb, nb=nb):
            W.call("wm_binary", code, out.vp, dA.vp, sa, na, other.vp, sb, nb)

        def bwd(code=code, other=other, gother=gother, sa=sa, na=na, sb=sb, nb=nb):
            W.call("wm_binary_bwd", code, dG.vp, dA.vp, sa, na, other.vp, sb, nb, W.nullp(),
                   gA.vp, 1, gother.vp, 1)

        vb = vec * F32
        fwd_bytes = big + vb + big                     # A, vector, out
        if code == W.ADD:
            bwd_bytes = big + 2 * big + 2 * vb         # G; A.grad RMW; r.grad RMW
        else:
            bwd_bytes = big + big + vb + 2 * big + 2 * vb  # G, A, vector; grads RMW
        # rocprof kernel-name prefixes (template arguments: op code, operand inner strides)
        kf = "binary_rows_kernel<%d, 1, %d," % (code, 1 if other is dr else 0)
        kb = ("bwd_colsum_kernel<%d," % code) if other is dr else ("bwd_rowsum_kernel<%d," % code)
        ops.append(Op(name + " fwd", fwd, fwd_bytes, kf, N))
        ops.append(Op(name + " bwd", bwd, bwd_bytes, kb, N))
    keep = [dA, dc, dr, dG, out, gA, gc, gr]
    workload = {"workload": "c2: A[%d,%d] fp32 with r[1,%d], c[%d,1]; A+r, A*c, A/r, A->pow(c), fwd+bwd "
                            "(grads accumulated, all inputs require grad)" % (rows, cols, cols, rows),
                "elements": N}
    return ops, keep, workload


def c1_ops():
    a, b = synth.config1()
    rows, cols = a.shape
    da, db = W.DeviceArray.from_host(a), W.DeviceArray.from_host(b)
    t = W.DeviceArray((rows, cols)); rl = W.DeviceArray((rows, cols))
    s1 = W.DeviceArray((rows, 1)); y = W.DeviceArray((1, 1))
    dy = W.DeviceArray.from_host(np.ones((1, 1), np.float32))
    ds1 = W.DeviceArray((rows, 1)); dr = W.DeviceArray((rows, cols)); dt = W.DeviceArray((rows, cols))
    ga = W.DeviceArray((rows, cols)); ga.fill(0.0)
    gb = W.DeviceArray((cols,)); gb.fill(0.0)
    sa, na = shape_arg((rows, cols))
    sb, nb = shape_arg((cols,))
    N = rows * cols
    big = N * F32
    ops = [
        Op("add fwd", lambda: W.call("wm_binary", W.ADD, t.vp, da.vp, sa, na, db.vp, sb, nb),
           2 * big + cols * F32, "binary_rows_kernel", N),
        Op("relu fwd", lambda: W.call("wm_unary", W.RELU, rl.vp, t.vp, N, 0.0, 0.0), 2 * big,
           "unary_fwd_kernel", N),
        Op("sum(1) fwd", lambda: W.call("wm_reduce", W.R_SUM, rl.vp, rows, cols, 1, s1.vp, W.nullp()),
           big + rows * F32, "reduce_rows_kernel", N),
        Op("sum() fwd", lambda: W.call("wm_reduce", W.R_SUM, s1.vp, 1, rows, 1, y.vp, W.nullp()),
           rows * F32 + F32, "reduce_rows_kernel", rows),
        Op("sum() bwd", lambda: W.call("wm_reduce_bwd", W.R_SUM, dy.vp, W.nullp(), 1, rows, 1, ds1.vp, 0),
           F32 + rows * F32, "reduce_bwd_sum", rows),
        Op("sum(1) bwd", lambda: W.call("wm_reduce_bwd", W.R_SUM, ds1.vp, W.nullp(), rows, cols, 1, dr.vp, 0),
           rows * F32 + big, "reduce_bwd_sum_vec_kernel", N),
        Op("relu bwd", lambda: W.call("wm_unary_bwd", W.RELU, dr.vp, t.vp, W.nullp(), dt.vp, 0, N, 0.0, 0.0),
           3 * big, "unary_bwd_kernel", N),
        Op("add bwd", lambda: W.call("wm_binary_bwd", W.ADD, dt.vp, da.vp, sa, na, db.vp, sb, nb, W.nullp(),
                                     ga.vp, 1, gb.vp, 1),
           big + 2 * big + 2 * cols * F32, "bwd_colsum_kernel", N),
    ]
    keep = [da, db, t, rl, s1, y, dy, ds1, dr, dt, ga, gb]
    return ops, keep, {"workload": "c1: y = relu(a[1024,1024] + b[1024]).sum(1).sum(), fwd+bwd "
                                   "(L2-resident, launch-bound; not a roofline case)", "elements": N}


def c3_ops(rows=16384, cols=4096):
    X = synth.config3(rows, cols)
    dX = W.DeviceArray.from_host(X)
    N = rows * cols
    big = N * F32
    ops, keep = [], [dX]
    for dim, (outer, n, inner) in ((0, (1, rows, cols)), (1, (rows, cols, 1))):
        nout = outer * inner
        for name, code in (("sum", W.R_SUM), ("mean", W.R_MEAN), ("max", W.R_MAX), ("min", W.R_MIN),
                           ("argmax", W.R_ARGMAX), ("argmin", W.R_ARGMIN)):
            val = W.DeviceArray((nout,))
            idx = W.DeviceArray((nout,), np.int64) if code in (W.R_MAX, W.R_MIN) else None
            keep += [val] + ([idx] if idx is not None else [])
            nbytes = big + nout * F32 + (nout * 8 if idx is not None else 0)
            kern = "reduce_cols_kernel" if inner > 1 else "reduce_rows_kernel"
            ops.append(Op(f"{name} dim{dim}",
                          (lambda code=code, val=val, idx=idx, o=outer, n=n, i=inner:
                           W.call("wm_reduce", code, dX.vp, o, n, i, val.vp, W.ptr(idx))),
                          nbytes, kern, N))
    full = W.DeviceArray((1,))
    keep.append(full)
    ops.append(Op("sum full", lambda: W.call("wm_reduce", W.R_SUM, dX.vp, 1, N, 1, full.vp, W.nullp()),
                  big + F32, "reduce_rows_kernel", N))
    # max backward (scatter to the first winner), dim 0 and dim 1
    gX = W.DeviceArray((rows, cols)); gX.fill(0.0)
    keep.append(gX)
    for dim, (outer, n, inner) in ((0, (1, rows, cols)), (1, (rows, cols, 1))):
        nout = outer * inner
        idx = W.DeviceArray((nout,), np.int64)
        W.call("wm_reduce", W.R_MAX, dX.vp, outer, n, inner, W.nullp(), idx.vp)
        g = W.DeviceArray.from_host(synth.normal((nout,), synth.seed_for(3, 5 + dim)))
        keep += [idx, g]
        ops.append(Op(f"max dim{dim} bwd",
                      (lambda g=g, idx=idx, o=outer, n=n, i=inner:
                       W.call("wm_reduce_bwd", W.R_MAX, g.vp, idx.vp, o, n, i, gX.vp, 1)),
                      nout * (F32 + 8 + 2 * F32), "reduce_bwd_scatter_kernel", nout))
    return ops, keep, {"workload": "c3: X[%d,%d] fp32 quantised to 1/64; sum/mean/max/min/argmax/argmin "
                                   "over dim 0 and dim 1 (+ full sum), max backward" % (rows, cols),
                       "elements": N}


def c4_ops(rows=8192, cols=32000):
    L, G = synth.config4(rows, cols)
    dL, dG = W.DeviceArray.from_host(L), W.DeviceArray.from_host(G)
    y = W.DeviceArray((rows, cols)); ly = W.DeviceArray((rows, cols))
    gx = W.DeviceArray((rows, cols)); gx.fill(0.0)
    N = rows * cols
    big = N * F32
    ops = [
        Op("softmax fwd", lambda: W.call("wm_softmax_fwd", y.vp, dL.vp, rows, cols), 2 * big,
           "softmax_fwd_kernel", N),
        Op("log_softmax fwd", lambda: W.call("wm_log_softmax_fwd", ly.vp, dL.vp, rows, cols), 2 * big,
           "softmax_fwd_kernel", N),
        Op("softmax bwd", lambda: W.call("wm_softmax_bwd", dG.vp, y.vp, gx.vp, 1, rows, cols), 4 * big,
           "softmax_bwd_kernel", N),
        Op("log_softmax bwd", lambda: W.call("wm_log_softmax_bwd", dG.vp, ly.vp, gx.vp, 1, rows, cols), 4 * big,
           "softmax_bwd_kernel", N),
    ]
    return ops, [dL, dG, y, ly, gx], {"workload": "c4: logits[%d,%d] fp32 ~N(0,3) with 1%% +20 spikes; "
                                                 "softmax and log_softmax fwd+bwd (dx accumulated)" % (rows, cols),
                                      "elements": N}


def c5_ops(b=32, t=1024, c=4096):
    h, res, g, dm = synth.config5(b, t, c)
    rows = b * t
    N = rows * c
    # fp16 storage made on the device with the reference's truncating conversion
    h32, r32 = W.DeviceArray.from_host(h), W.DeviceArray.from_host(res)
    h16, r16 = W.DeviceArray((rows, c), np.uint16), W.DeviceArray((rows, c), np.uint16)
    W.call("wm_f32_to_f16_rtz", h16.vp, h32.vp, N)
    W.call("wm_f32_to_f16_rtz", r16.vp, r32.vp, N)
    h32.free(); r32.free()
    dg_, ddm = W.DeviceArray.from_host(g), W.DeviceArray.from_host(dm.reshape(-1))
    out = W.DeviceArray((rows, c), np.uint16)
    m = W.DeviceArray((rows,))
    gh = W.DeviceArray((rows, c)); gh.fill(0.0)
    gr = W.DeviceArray((rows, c)); gr.fill(0.0)
    gg = W.DeviceArray((c,)); gg.fill(0.0)
    lo, hi = W.C.c_float(-4.0), W.C.c_float(4.0)
    ops = [
        Op("epilogue fwd", lambda: W.call("wm_epilogue_f16_fwd", out.vp, m.vp, h16.vp, r16.vp, dg_.vp, rows, c, lo,
                                          hi),
           N * (2 + 2 + 2) + c * F32 + rows * F32, "epilogue_fwd_kernel", N),
        Op("epilogue bwd", lambda: W.call("wm_epilogue_f16_bwd", ddm.vp, h16.vp, r16.vp, dg_.vp, gh.vp, 1, gr.vp, 1,
                                          gg.vp, 1, rows, c, lo, hi),
           N * (2 + 2 + 8 + 8) + c * F32 + rows * F32 + 2 * c * F32, "epilogue_bwd_kernel", N),
    ]
    return ops, [h16, r16, dg_, ddm, out, m, gh, gr, gg], {
        "workload": "c5: h, res[%d,%d,%d] fp16 storage (truncating conversion), g[%d] fp32; "
                    "out = tanh_(clamp((h+res)*g, -4, 4)) stored fp16, mean over the last dim; fused fwd + bwd "
                    "(grads fp32, accumulated)" % (b, t, c, c), "elements": N}


def gpt2_small_shapes():
    """Parameter shapes of a GPT-2-small-sized model (124M parameters): the
    tensor list an optimizer step walks (many small bias / norm vectors next
    to a few large matrices)."""
    d, v, ctx, layers = 768, 50257, 1024, 12
    shapes = [(v, d), (ctx, d)]
    for _ in range(layers):
        shapes += [(d,), (d,), (d, 3 * d), (3 * d,), (d, d), (d,), (d,), (d,), (d, 4 * d), (4 * d,), (4 * d, d), (d,)]
    shapes += [(d,), (d,)]
    return shapes


def opt_ops():
    """Parameter updates: one optimizer step / clipping / unscaling pass over a
    GPT-2-small-sized parameter list, one multi-tensor launch per pass as the
    drop-in optimizers issue them."""
    shapes = gpt2_small_shapes()
    rng = np.random.default_rng(0)
    P, G, S1, S2 = [], [], [], []
    for i, s in enumerate(shapes):
        n = int(np.prod(s))
        P.append(W.DeviceArray.from_host((rng.standard_normal(n) * 0.02).astype(np.float32)))
        G.append(W.DeviceArray.from_host((rng.standard_normal(n) * 1e-3).astype(np.float32)))
        S1.append(W.DeviceArray((n,))); S1[-1].fill(0.0)
        S2.append(W.DeviceArray((n,))); S2[-1].fill(0.0)
    N = sum(int(np.prod(s)) for s in shapes)
    sizes = [int(np.prod(s)) for s in shapes]
    total = W.DeviceArray((1,))
    gptrs = (W.C.c_void_p * len(G))(*[g.ptr for g in G])
    gsizes = (W.C.c_int64 * len(G))(*sizes)
    found = W.C.c_int()
    L = W.lib()
    t = [0]

    pP, _a = W.ptr_array([p.ptr for p in P])
    pG, _b = W.ptr_array([g.ptr for g in G])
    pS1, _c = W.ptr_array([x.ptr for x in S1])
    pS2, _d = W.ptr_array([x.ptr for x in S2])
    pN, _e = W.i64_array(sizes)
    cnt = len(sizes)

    # the drop-in optimizers' step(): one multi-tensor launch over the list
    def adam():
        t[0] += 1
        bc1 = np.float32(1.0 - 0.9 ** t[0]); bc2 = np.float32(1.0 - 0.999 ** t[0])
        W.check(L.wm_adamw_step_multi(cnt, pP, pG, pS1, pS2, pN, 1e-4, 0.9, 0.999, 1e-8, bc1, bc2, 0.01))

    def sgd():
        W.check(L.wm_sgd_step_multi(cnt, pP, pG, pS1, pN, 1e-4, 0.9))

    def rms():
        W.check(L.wm_rmsprop_step_multi(cnt, pP, pG, pS2, None, pN, 1e-4, 0.99, 1e-8, 0.0, 0.0))

    def clip():
        W.check(L.wm_grad_sumsq_multi(cnt, pG, pN, total.vp))
        # max_norm 0 clips on every call (coefficient 0 < 1), so the timed pass
        # always reads and writes every gradient
        W.check(L.wm_clip_grad_norm_scale_multi(cnt, pG, pN, total.vp, 0.0))

    def unscale():
        W.check(L.wm_grad_unscale(len(G), W.C.cast(gptrs, W.C.c_void_p), W.C.cast(gsizes, W.C.c_void_p), 1.0,
                                  W.C.byref(found)))

    ops = [
        Op("AdamW step", adam, N * 28, "multi_update_kernel<wm::Upd<1, true", N),
        Op("SGD momentum step", sgd, N * 20, "multi_update_kernel<wm::Upd<0, true", N),
        Op("RMSprop step", rms, N * 20, "multi_update_kernel<wm::Upd<2, false, false", N),
        # algorithmic bytes: every gradient read once and written once (8 per
        # element); both ops read the gradients twice (the norm, or the first
        # non-finite position, must be known before any write), so they move 12
        Op("clip_grad_norm_", clip, N * 8, "multi_sumsq_kernel", N),
        Op("GradScaler unscale", unscale, N * 8, "multi_first_bad_kernel", N),
    ]
    return ops, P + G + S1 + S2 + [total], {
        "workload": "opt: %d parameter tensors, %d parameters (GPT-2-small shapes), fp32 params / grads / "
                    "state; one AdamW, SGD-momentum and RMSprop step, clip_grad_norm_ and GradScaler unscale, "
                    "each one multi-tensor launch (pair) over the list" % (len(shapes), N), "elements": N}




# ---------------------------------------------------------------------------
# CPU baseline (reference core/tensor.cpp through oracle/_ref, 1 core)
# ---------------------------------------------------------------------------

def cpu_baseline_c2(sample_rows=1024, cols=8192, reps=3):
    sys.path.insert(0, ROOT)
    import oracle
    A, c, r, G = synth.config2(8192, cols)
    A, c, G = A[:sample_rows], c[:sample_rows], G[:sample_rows]
    ref = oracle.reference()
    kind = "reference" if ref is not None else "port"
    N = sample_rows * cols
    big = N * F32
    total_bytes = 0
    times = {}
    cpu0 = os.sched_getaffinity(0)
    core = min(cpu0)
    os.sched_setaffinity(0, {core})
    try:
        for name, op, other in (("A+r", "add", r), ("A*c", "mul", c), ("A/r", "div", r), ("A^c", "pow", c)):
            vb = other.size * F32
            fb = 2 * big + vb
            bb = 3 * big + 2 * vb if op == "add" else 4 * big + 3 * vb
            tf, tb = [], []
            for rep in range(reps + 1):
                if kind == "reference":
                    ta, to = ref.tensor(A, True), ref.tensor(other, True)
                    t0 = time.perf_counter()
                    y = ref.binary(op, ta, to)
                    t1 = time.perf_counter()
                    y.set_grad(G)
                    t2 = time.perf_counter()
                    y.call_grad_fn()
                    t3 = time.perf_counter()
                    del y, ta, to
                else:
                    o = oracle.get("port")
                    t0 = time.perf_counter()
                    out = o.binary(op, A, other)
                    t1 = time.perf_counter()
                    t2 = time.perf_counter()
                    o.binary_bwd(op, G, A, other, out)
                    t3 = time.perf_counter()
                if rep > 0:
                    tf.append(t1 - t0)
                    tb.append(t3 - t2)
            times[name + " fwd"] = (statistics.median(tf), fb)
            times[name + " bwd"] = (statistics.median(tb), bb)
            total_bytes += fb + bb
    finally:
        os.sched_setaffinity(0, cpu0)
    total_t = sum(t for t, _ in times.values())
    value = total_bytes / total_t / 1e9
    return {"value": round(value, 4), "unit": "GB/s", "cores": 1, "kind": kind,
            "sample": f"A[{sample_rows},{cols}] row slice of config 2 (1/{8192 // sample_rows} of A), same ops "
                      f"fwd+bwd, median of {reps} after 1 warm-up, single-threaded on 1 of "
                      f"{len(cpu0)} host cores",
            "per_op_ms": {k: round(t * 1e3, 3) for k, (t, _) in times.items()},
            "per_op_GBps": {k: round(b / t / 1e9, 4) for k, (t, b) in times.items()}}


# ---------------------------------------------------------------------------

def loss_ops(rows=8192, cols=32000):
    """Loss heads on the softmax config's logits: the fused CrossEntropy and
    Focal heads and NLL, forward and backward (prediction gradient known-zero,
    as in a training step), and BCEWithLogits over the same elements."""
    L, _ = synth.config4(rows, cols)
    lab = np.floor(synth.uniform((rows,), synth.seed_for(6, 0), 0, cols)).clip(0, cols - 1).astype(np.float32)
    tgt = synth.uniform((rows, cols), synth.seed_for(6, 1), 0, 1)
    dL, dlab, dt = W.DeviceArray.from_host(L), W.DeviceArray.from_host(lab), W.DeviceArray.from_host(tgt)
    del L, tgt
    ce_st, fo_st = W.DeviceArray((rows, W.CE_STATS)), W.DeviceArray((rows, W.FOCAL_STATS))
    loss = W.DeviceArray((1,))
    one = W.DeviceArray.from_host(np.float32([1.0]))
    gx = W.DeviceArray((rows, cols))
    N = rows * cols
    big = N * F32
    g2, am1 = W.C.c_float(2.0), W.C.c_float(-1.0)
    zero = W.C.c_float(0.0)
    nf = W.C.c_float(float(N))
    ops = [
        Op("CrossEntropy fwd", lambda: W.call("wm_cross_entropy_fwd", dL.vp, dlab.vp, rows, cols, ce_st.vp, loss.vp),
           big + rows * (F32 + 2 * F32), "head_fwd_kernel", N),
        Op("CrossEntropy bwd", lambda: W.call("wm_cross_entropy_bwd", dL.vp, dlab.vp, ce_st.vp, one.vp, gx.vp, 0,
                                              rows, cols),
           2 * big + rows * (F32 + 2 * F32), "head_bwd_kernel<0", N),
        Op("Focal fwd", lambda: W.call("wm_focal_fwd", dL.vp, dlab.vp, rows, cols, g2, am1, fo_st.vp, loss.vp),
           big + rows * (F32 + 8 * F32), "head_fwd_kernel", N),
        Op("Focal bwd", lambda: W.call("wm_focal_bwd", dL.vp, dlab.vp, fo_st.vp, one.vp, gx.vp, 0, rows, cols, g2,
                                       am1),
           2 * big + rows * (F32 + 8 * F32), "head_bwd_kernel<1", N),
        Op("NLL bwd", lambda: W.call("wm_nll_bwd", dlab.vp, one.vp, gx.vp, 0, rows, cols), big + rows * F32,
           "head_bwd_kernel<2", N),
        Op("BCEWithLogits fwd", lambda: W.call("wm_pointwise_loss_fwd", 2, dL.vp, dt.vp, N, zero, zero, nf, loss.vp),
           2 * big, "pw_fwd_kernel", N),
        Op("BCEWithLogits bwd", lambda: W.call("wm_pointwise_loss_bwd", 2, dL.vp, dt.vp, N, zero, zero, nf, one.vp,
                                               gx.vp, 0),
           3 * big, "pw_bwd_kernel", N),
    ]
    return ops, [dL, dlab, dt, ce_st, fo_st, loss, one, gx], {
        "workload": "loss: logits[%d,%d] fp32 (the c4 recipe) with uniform class labels; fused CrossEntropy and "
                    "Focal(gamma 2) heads and NLL fwd+bwd (gradient buffer known-zero), BCEWithLogits over the "
                    "same elements with U[0,1] targets" % (rows, cols), "elements": N}


def norm_ops():
    """Row-3 kernels at transformer / CNN sizes: LayerNorm over [32768, 4096]
    (the c5 block's activations), BatchNorm2d over [64, 256, 56, 56] in
    training mode, and the attention softmax over [8, 16, 1024, 1024] scores
    with a causal mask; each forward and backward (gradients known-zero)."""
    rows, n = 32768, 4096
    x = synth.normal((rows, n), synth.seed_for(7, 0), 1.0, 2.0)
    g = synth.normal((rows, n), synth.seed_for(7, 1))
    dx, dg = W.DeviceArray.from_host(x), W.DeviceArray.from_host(g)
    del x, g
    gam = W.DeviceArray.from_host(synth.uniform((n,), synth.seed_for(7, 2), 0.5, 1.5))
    bet = W.DeviceArray.from_host(synth.normal((n,), synth.seed_for(7, 3)))
    y, gx = W.DeviceArray((rows, n)), W.DeviceArray((rows, n))
    mean, inv = W.DeviceArray((rows,)), W.DeviceArray((rows,))
    dgam, dbet = W.DeviceArray((n,)), W.DeviceArray((n,))
    eps = W.C.c_float(1e-5)

    B, C, H = 64, 256, 56
    S = H * H
    bx = synth.normal((B, C, S), synth.seed_for(8, 0), 0.5, 2.0)
    bg = synth.normal((B, C, S), synth.seed_for(8, 1))
    dbx, dbg = W.DeviceArray.from_host(bx), W.DeviceArray.from_host(bg)
    del bx, bg
    bgam = W.DeviceArray.from_host(synth.uniform((C,), synth.seed_for(8, 2), 0.5, 1.5))
    bbet = W.DeviceArray.from_host(synth.normal((C,), synth.seed_for(8, 3)))
    rm, rv = W.DeviceArray((C,)), W.DeviceArray((C,))
    rm.fill(0.0)
    rv.fill(1.0)
    by, bgx = W.DeviceArray((B, C, S)), W.DeviceArray((B, C, S))
    bmean, binv, bdg, bdb = (W.DeviceArray((C,)) for _ in range(4))
    mom = W.C.c_float(0.1)

    AB, AH, T = 8, 16, 1024
    sc = synth.normal((AB, AH, T, T), synth.seed_for(9, 0), 0.0, 3.0)
    da = synth.normal((AB, AH, T, T), synth.seed_for(9, 1))
    dsc, dda = W.DeviceArray.from_host(sc), W.DeviceArray.from_host(da)
    del sc, da
    mask = W.DeviceArray.from_host(np.where(np.triu(np.ones((T, T)), 1) > 0, -1e9, 0).astype(np.float32))
    att, dsc_out = W.DeviceArray((AB, AH, T, T)), W.DeviceArray((AB, AH, T, T))

    NL, NB, NA = rows * n, B * C * S, AB * AH * T * T
    ops = [
        Op("LayerNorm fwd", lambda: W.call("wm_layernorm_fwd", dx.vp, gam.vp, bet.vp, rows, n, eps, y.vp, mean.vp,
                                           inv.vp),
           2 * NL * F32 + 2 * n * F32 + 2 * rows * F32, "ln_fwd_kernel", NL),
        Op("LayerNorm bwd", lambda: W.call("wm_layernorm_bwd", dg.vp, dx.vp, gam.vp, mean.vp, inv.vp, rows, n, gx.vp,
                                           0, dgam.vp, 0, dbet.vp, 0),
           3 * NL * F32 + 3 * n * F32 + 2 * rows * F32, "ln_bwd_kernel", NL),
        Op("BatchNorm2d fwd (train)", lambda: W.call("wm_batchnorm2d_fwd", dbx.vp, bgam.vp, bbet.vp, rm.vp, rv.vp, B,
                                                     C, S, eps, mom, 1, by.vp, bmean.vp, binv.vp),
           2 * NB * F32, "bn_apply_kernel", NB),
        Op("BatchNorm2d bwd", lambda: W.call("wm_batchnorm2d_bwd", dbg.vp, dbx.vp, bgam.vp, bmean.vp, binv.vp, B, C, S,
                                             bgx.vp, 0, bdg.vp, 0, bdb.vp, 0),
           3 * NB * F32, "bn_bwd_apply_kernel", NB),
        Op("attention softmax fwd", lambda: W.call("wm_attention_softmax_fwd", dsc.vp, mask.vp, 1, AB, AH, T, T,
                                                   att.vp),
           2 * NA * F32 + T * T * F32, "attn_softmax_fwd_kernel", NA),
        Op("attention softmax bwd", lambda: W.call("wm_attention_softmax_bwd", att.vp, dda.vp, AB * AH * T, T,
                                                   dsc_out.vp),
           3 * NA * F32, "attn_softmax_bwd_kernel", NA),
    ]
    keep = [dx, dg, gam, bet, y, gx, mean, inv, dgam, dbet, dbx, dbg, bgam, bbet, rm, rv, by, bgx, bmean, binv, bdg,
            bdb, dsc, dda, mask, att, dsc_out]
    return ops, keep, {
        "workload": "norm: LayerNorm x[%d,%d] fp32 (eps 1e-5); BatchNorm2d x[%d,%d,%d,%d] training mode; "
                    "attention softmax scores[%d,%d,%d,%d] + causal mask [1,1,%d,%d]; fwd+bwd each, gradients "
                    "known-zero; algorithmic bytes = one read of each input and one write of each output"
                    % (rows, n, B, C, H, H, AB, AH, T, T, T, T), "elements": NL + NB + NA}


def gemm_ops(n=8192, batch=64, t=1024, hd=128):
    """Matrix-product kernels (include/wm_gemm.h) on the matrix cores, fp32:
    Tensor::matmul [n, n] @ [n, n] forward and backward (two products), and
    Tensor::bmm at attention shape [batch, t, hd] @ [batch, hd, t] forward and
    backward.  flops = 2 m n k per product."""
    a = W.DeviceArray.from_host(synth.normal((n, n), synth.seed_for(10, 0)))
    b = W.DeviceArray.from_host(synth.normal((n, n), synth.seed_for(10, 1)))
    g = W.DeviceArray.from_host(synth.normal((n, n), synth.seed_for(10, 2)))
    c, ga, gb = W.DeviceArray((n, n)), W.DeviceArray((n, n)), W.DeviceArray((n, n))
    qa = W.DeviceArray.from_host(synth.normal((batch, t, hd), synth.seed_for(11, 0)))
    kb = W.DeviceArray.from_host(synth.normal((batch, hd, t), synth.seed_for(11, 1)))
    sg = W.DeviceArray.from_host(synth.normal((batch, t, t), synth.seed_for(11, 2)))
    sc, gq, gk = W.DeviceArray((batch, t, t)), W.DeviceArray((batch, t, hd)), W.DeviceArray((batch, hd, t))
    mm = 2 * n * n * n
    bm = 2 * batch * t * t * hd
    ops = [
        Op("matmul fwd", lambda: W.call("wm_matmul", a.vp, b.vp, n, n, n, c.vp), 3 * n * n * F32, "gemm_kernel", n * n,
           mm),
        Op("matmul bwd", lambda: W.call("wm_matmul_bwd", g.vp, a.vp, b.vp, n, n, n, ga.vp, 0, gb.vp, 0),
           6 * n * n * F32, "gemm_kernel", 2 * n * n, 2 * mm),
        Op("bmm fwd", lambda: W.call("wm_bmm", qa.vp, kb.vp, batch, t, hd, t, sc.vp),
           (2 * batch * t * hd + batch * t * t) * F32, "gemm_kernel", batch * t * t, bm),
        Op("bmm bwd", lambda: W.call("wm_bmm_bwd", sg.vp, qa.vp, kb.vp, batch, t, hd, t, gq.vp, 0, gk.vp, 0),
           (batch * t * t * 2 + 4 * batch * t * hd) * F32, "gemm_kernel", 2 * batch * t * hd, 2 * bm),
    ]
    keep = [a, b, g, c, ga, gb, qa, kb, sg, sc, gq, gk]
    return ops, keep, {"workload": "gemm: Tensor::matmul [%d,%d]@[%d,%d] and Tensor::bmm [%d,%d,%d]@[%d,%d,%d], fp32 "
                                   "on v_mfma_f32_32x32x2_f32, forward and backward (gradients overwritten)"
                                   % (n, n, n, n, batch, t, hd, batch, hd, t),
                       "elements": n * n + batch * t * t}


def mha_ops(B=8, S=1024, E=1024, H=16):
    """MultiHeadAttention forward and closure (wm_mha_fwd / wm_mha_bwd) at a
    transformer shape: self attention over [B, S, E] with H heads and a
    causal mask.  flops = the products (projections 4 * 2 B S E^2, scores and
    attn V 2 * 2 B H S^2 hd; the closure twice that); the attention softmax
    and the bias column sums ride along in the same time."""
    hd = E // H
    x = W.DeviceArray.from_host(synth.normal((B, S, E), synth.seed_for(13, 0)))
    params = [W.DeviceArray.from_host(synth.normal((E, E), synth.seed_for(13, 1 + i), 0.0, E ** -0.5))
              for i in range(4)]
    params += [W.DeviceArray.from_host(synth.normal((E,), synth.seed_for(13, 5 + i), 0.0, 0.1)) for i in range(4)]
    mask = W.DeviceArray.from_host(np.where(np.triu(np.ones((S, S)), 1) > 0, -1e9, 0).astype(np.float32))
    out, ctx = W.DeviceArray((B, S, E)), W.DeviceArray((B, S, E))
    Q, K, V = (W.DeviceArray((B, S, E)) for _ in range(3))
    attn = W.DeviceArray((B, H, S, S))
    dout = W.DeviceArray.from_host(synth.normal((B, S, E), synth.seed_for(13, 9)))
    grads = [W.DeviceArray((E, E)) for _ in range(4)] + [W.DeviceArray((E,)) for _ in range(4)]
    gx = W.DeviceArray((B, S, E))
    for gbuf in grads + [gx]:
        gbuf.fill(0.0)
    pv = [p.vp for p in params]

    def fwd():
        W.call("wm_mha_fwd", x.vp, x.vp, x.vp, mask.vp, 1, *pv, B, S, S, E, H, out.vp, attn.vp, Q.vp, K.vp, V.vp,
               ctx.vp)

    def bwd():
        W.call("wm_mha_bwd", dout.vp, x.vp, x.vp, x.vp, *pv[:4], Q.vp, K.vp, V.vp, attn.vp, ctx.vp, B, S, S, E, H,
               *[gb.vp for gb in grads], gx.vp, gx.vp, gx.vp)

    fwd()
    f_fl = 4 * 2 * B * S * E * E + 2 * 2 * B * H * S * S * hd
    att = B * H * S * S * F32
    ops = [Op("mha fwd", fwd, 4 * B * S * E * F32 + 3 * att, "gemm_kernel", B * S * E, f_fl),
           Op("mha bwd", bwd, 6 * B * S * E * F32 + 4 * att, "gemm_kernel", B * S * E, 2 * f_fl)]
    keep = [x, mask, out, ctx, Q, K, V, attn, dout, gx] + params + grads
    return ops, keep, {"workload": "mha: MultiHeadAttention self attention x[%d,%d,%d], %d heads (hd %d), causal "
                                   "mask; forward and closure (parameter gradients accumulated, one input gradient "
                                   "for q = k = v)" % (B, S, E, H, hd),
                       "elements": B * S * E}


def io_ops(n_floats=1 << 28):
    """WMT tensor files (core/serialize.cpp:36-108) through the drop-in:
    load_tensor of a 1 GiB file straight into HBM, save_tensor of the same
    tensor from HBM, on a RAM-backed path (/dev/shm when present) so the
    figure is the staging pipeline's (file-cache read, pinned copy, PCIe),
    not a disk's.  Timed with events on the library stream around the whole
    host-driven call; 'bytes' = the payload."""
    from whitematter_amd import _tensor as T
    d = "/dev/shm" if os.path.isdir("/dev/shm") and os.access("/dev/shm", os.W_OK) else "/tmp"
    path = os.path.join(d, "wm_bench_io_%d.wmt" % os.getpid())
    x = T.Tensor.from_array(synth.normal((n_floats,), synth.seed_for(12, 0)), requires_grad=True)
    assert T.save_tensor(x, path)
    holder = {}

    def load():
        holder["t"] = T.load_tensor(path)

    def save():
        assert T.save_tensor(x, path)

    nb = n_floats * F32
    ops = [Op("load_tensor", load, nb, "(host-driven copies)", n_floats),
           Op("save_tensor", save, nb, "(host-driven copies)", n_floats)]
    for op in ops:
        op.host_io = True

    class Cleanup:
        def __del__(self):
            try:
                os.remove(path)
            except OSError:
                pass

    return ops, [x, holder, Cleanup()], {
        "workload": "io: WMT tensor file of %d fp32 (%d MiB) loaded into / saved from HBM through pinned "
                    "double-buffered staging (include/wm_io.h), file on %s" % (n_floats, nb >> 20, d),
        "elements": n_floats, "path": path}


def cpu_baseline_io(path, reps=3):
    """The reference's own load_tensor (oracle/_ref: ifstream read into a
    std::vector, then Tensor::create's copy) on the same file, one thread."""
    sys.path.insert(0, ROOT)
    import oracle
    ref = oracle.reference()
    if ref is None:
        return None
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        t = ref.load_tensor(path)
        ts.append(time.perf_counter() - t0)
        n = int(np.prod(t.shape))
        del t
    sec = statistics.median(ts)
    return {"value": round(n * F32 / sec / 1e9, 2), "unit": "GB/s", "cores": 1, "kind": "reference",
            "sample": "the whole %d MiB file, median of %d loads" % (n * F32 >> 20, reps)}


def traffic_for(op_name: str, config: str):
    """HBM bytes per launch of an op's main kernel, from the committed
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE summary (profiles/traffic.json,
    calibrated against the copy kernel)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    try:
        d = json.load(open(path))
        return d.get(config, {}).get(op_name, {}).get("hbm_bytes")
    except Exception:
        return None


CONFIGS = {"gemm": gemm_ops, "mha": mha_ops, "io": io_ops, "c1": c1_ops, "c2": c2_ops, "c3": c3_ops, "c4": c4_ops, "c5": c5_ops, "opt": opt_ops, "loss": loss_ops,
           "norm": norm_ops}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="c2", choices=sorted(CONFIGS))
    ap.add_argument("--flush-mib", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-rows", type=int, default=1024)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU; multi-GPU runs are not part of it "
              "(value is the single-GPU throughput).", file=sys.stderr)
        sys.exit(2)

    W.call("wm_init", 0)
    cus = W.device_cus()
    ops, keep, workload = CONFIGS[args.config]()
    flush = W.DeviceArray((args.flush_mib * (1 << 20) // 4,))

    def run_op(op, timed):
        flush.fill(1.0)
        if timed:
            W.call("wm_span_begin")
            W.call("wm_timer_start")
        op.launch()
        if timed:
            ms, kms, nk = W.C.c_float(), W.C.c_float(), W.C.c_int()
            W.call("wm_timer_stop", W.C.byref(ms))
            if getattr(op, "host_io", False):
                W.lib().wm_span_end(W.C.byref(kms), W.C.byref(nk))  # no kernels: host-driven copies
                op.kms.append(ms.value)
            else:
                W.call("wm_span_end", W.C.byref(kms), W.C.byref(nk))
                op.kms.append(kms.value)
            op.ms.append(ms.value)

    for _ in range(args.warmup):
        for op in ops:
            run_op(op, False)
    W.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        for op in ops:
            run_op(op, True)
    W.sync()
    wall = time.perf_counter() - t0

    per_op = {}
    step_ms = 0.0
    step_bytes = 0
    for op in ops:
        ms = statistics.mean(op.ms)
        step_ms += ms
        step_bytes += op.bytes
        gbps = op.bytes / (ms * 1e-3) / 1e9
        per_op[op.name] = {"ms": round(ms, 4), "ms_median": round(statistics.median(op.ms), 4),
                           "ms_kernel_median": round(statistics.median(op.kms), 4),
                           "GBps": round(gbps, 1), "pct_peak": round(100 * gbps / PEAK_GBPS, 1),
                           "Gelem_per_s": round(op.elems / (ms * 1e-3) / 1e9, 2), "bytes": op.bytes}
        if op.flops:
            tf = op.flops / (ms * 1e-3) / 1e12
            per_op[op.name].update({"TFLOPs": round(tf, 1), "pct_mfma_peak": round(100 * tf / PEAK_F32_MFMA_TFLOPS, 1),
                                    "flops": op.flops})
    mfma = all(op.flops for op in ops)
    host_io = all(getattr(op, "host_io", False) for op in ops)
    dom = max(ops, key=lambda o: statistics.mean(o.ms))
    dom_ms = statistics.mean(dom.ms)
    if host_io:
        # host-driven file transfers: bounded by the file cache and PCIe, not by
        # an HBM or matrix-core roofline
        value = step_bytes / (step_ms * 1e-3) / 1e9
        roofline = None
    elif mfma:
        value = sum(op.flops for op in ops) / (step_ms * 1e-3) / 1e12
        dom_tf = dom.flops / (dom_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(dom_tf, 2), "peak": PEAK_F32_MFMA_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(dom_tf / PEAK_F32_MFMA_TFLOPS, 4), "traffic": traffic_for(dom.name, args.config),
                    "kernel": dom.kernel, "op": dom.name, "algorithmic_flops": dom.flops,
                    "avg_ms": round(dom_ms, 4)}
    else:
        value = step_bytes / (step_ms * 1e-3) / 1e9
        dom_gbps = dom.bytes / (dom_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(dom_gbps, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                    "frac": round(dom_gbps / PEAK_GBPS, 4), "traffic": traffic_for(dom.name, args.config),
                    "kernel": dom.kernel, "op": dom.name, "algorithmic_bytes": dom.bytes,
                    "avg_ms": round(dom_ms, 4)}

    # calibration copy kernel (its own launches, after the timed region)
    n_copy = 1 << 28  # 1 GiB
    src = W.DeviceArray((n_copy,)); dst = W.DeviceArray((n_copy,))
    src.fill(2.0)
    cms = []
    for _ in range(3):
        flush.fill(1.0)
        W.call("wm_timer_start")
        W.call("wm_copy_kernel", dst.vp, src.vp, n_copy)
        ms = W.C.c_float()
        W.call("wm_timer_stop", W.C.byref(ms))
        cms.append(ms.value)
    copy_gbps = 2 * n_copy * F32 / (statistics.median(cms) * 1e-3) / 1e9
    src.free(); dst.free()

    cpu = None
    if not args.no_cpu and args.config == "io":
        try:
            cpu = cpu_baseline_io(workload["path"])
        except Exception as e:  # the baseline is reported, never the target
            cpu = {"value": None, "error": str(e)}
    if not args.no_cpu and args.config == "c2":
        try:
            cpu = cpu_baseline_c2(args.cpu_rows)
        except Exception as e:  # the baseline is reported, never the target
            cpu = {"value": None, "error": str(e)}
    if cpu and cpu.get("value"):
        for name, d in per_op.items():
            t = cpu.get("per_op_ms", {}).get(name)
            if t:
                # CPU ms scaled from the row sample to the full workload
                scale = 8192 / args.cpu_rows
                d["speedup_vs_cpu"] = round(t * scale / d["ms"], 1)

    line = {
        "metric": METRIC_MFMA if mfma else METRIC,
        "value": round(value, 1),
        "unit": "TFLOP/s" if mfma else "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded splitmix64 -> Box-Muller fp64 -> fp32, BASELINE config recipe)",
        "config": dict(workload, pct_of_peak=round(100 * value / (PEAK_F32_MFMA_TFLOPS if mfma else PEAK_GBPS), 1),
                       cus=cus,
                       timing="HIP events on the library stream per op; 512 MiB flush between ops "
                              "(untimed); ms_per_step = sum of op kernel times",
                       wall_s_timed_loop=round(wall, 3)),
        "roofline": roofline,
        "cpu_baseline": cpu,
        "ops": per_op,
        "copy_kernel_GBps": round(copy_gbps, 1),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
