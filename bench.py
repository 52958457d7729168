"""Benchmark of the MI355X Tensor elementwise / broadcast / reduction path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all] [--detail PATH]

Metric: achieved HBM GB/s (% of MI355X peak) per op, and the
speedup over the host-CPU reference path.  A "step" is one pass of a
configuration's ops, forward and backward, over inputs already resident in
HBM; a 512 MiB fill runs before every op (untimed) so no op starts with its
inputs in L2 / Infinity Cache.

Each op is timed twice per step, in separate launches:
  trace basis   the op's own kernel dispatches, start to end timestamp, as
                the command processor stamps them: read in-process through
                rocprofiler-sdk's kernel-dispatch tracing (libwm_ktrace),
                the numbers a rocprofv3 --kernel-trace of the same run
                shows.  Every GB/s and roofline fraction is computed from
                this basis (median of K steps; an op's time is the sum of
                its dispatches).  Where the process already runs under a
                profiler (rocprofv3), the tracer cannot register: the
                kernels are then launched exactly as on the trace basis and
                the profiler's trace is the measurement ("basis":
                "external"; bench's own figures fall back to the event
                basis).  If it cannot register for any other reason, the
                per-launch event pairs of wm_span_* stand in ("basis":
                "span"); they read ~4 us longer per dispatch.
  event basis   events recorded on the library stream before and after the
                op (wm_timer_*): launch gaps and marker latency included;
                reported beside as value_event.

Bytes are ALGORITHMIC: every distinct input read once (broadcast operands at
their real size), every output written once, read + write for every gradient
accumulated with "+=".  pow's backward recomputes pow(a, b) instead of
reading the saved output, so its bytes are the recompute figure.

The default run (--config all) measures the five BASELINE configurations and
the config-5 chain as a Tensor-API caller issues it:
  c4     (headline: the largest single-GPU configuration) logits[8192,32000]
         softmax / log_softmax fwd + bwd;
  c1     y = relu(a + b).sum(1).sum(), fwd + bwd (L2-resident, launch-bound);
  c2     A[8192,8192] with r[1,8192], c[8192,1]; A+r, A*c, A/r, A->pow(c),
         fwd + bwd;
  c3     X[16384,4096] sum/mean/max/min/argmax/argmin over dims 0 and 1, full
         sum, max backward;
  c5     the fused fp16-storage epilogue (C ABI) fwd + bwd;
  c5api  the same computation through the drop-in Tensor API: HalfTensor
         to_float, add, mul, clamp, tanh_, reshape, mean, reshape, and each
         closure of the backward.
stdout gets ONE JSON line (kept under 4 KB): the top-level value / roofline /
cpu_baseline / parity are c4's, and "configs" holds a compact record per
other configuration.  The per-op figures of every configuration go to
stderr as one "bench.py detail:" JSON line (and to --detail PATH).
--config NAME runs one configuration (also opt, loss, norm, gemm, mha, io).

The CPU baseline is the reference's own core/tensor.cpp (oracle/_ref, built
with the reference's flags), timed single-threaded on one host core over a
bounded row sample of the same workload and scaled to the full size (the
sample is stated in each record).  The same leg checks parity on the recipe's
bytes: the GPU outputs of the timed kernels for the sampled rows (and, for
outputs that sum over all rows, the GPU run on the sample itself) against the
reference build's outputs and the fp64 oracle, to the contract's bars --
bit-exact for add/sub/mul/div/relu/clamp/max/min/arg*, <= 2 ulp of fp64 for
the transcendentals, 1e-5 of the sum of |terms| (fp64) for sums, softmax
and gradients.
"""
from __future__ import annotations

import argparse
import ctypes
import gc
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
        self.kms = []  # kernel basis: the op's dispatch durations summed (trace, or span events)
        self.kparts = []  # the same, dispatch by dispatch
        self.knames = None  # the dispatches' kernel names (trace basis)
        self.prepare = None  # untimed work before each launch (e.g. refilling gradients)


class KTrace:
    """libwm_ktrace: the op's own dispatches' start / end timestamps through
    rocprofiler-sdk's kernel-dispatch tracing (whitematter_amd/csrc/wm_ktrace.cpp).
    Must be created before the process's first HIP call."""

    def __init__(self):
        self.ok, self.err = False, ""
        path = os.path.join(ROOT, "whitematter_amd", "libwm_ktrace.so")
        if not os.path.exists(path):
            self.err = "libwm_ktrace.so is not built"
            return
        try:
            L = ctypes.CDLL(path)
        except OSError as e:
            self.err = str(e)
            return
        L.wm_ktrace_error.restype = ctypes.c_char_p
        L.wm_ktrace_end.argtypes = [ctypes.POINTER(ctypes.c_int)]
        L.wm_ktrace_take.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_double), ctypes.c_int]
        L.wm_ktrace_name.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
        self.L = L
        if L.wm_ktrace_init() == 0:
            self.ok = True
        else:
            self.err = L.wm_ktrace_error().decode(errors="replace")

    @property
    def basis(self):
        """trace: this library's dispatch timestamps; external: another tool
        (rocprofv3) already traces the process, so kernels are launched
        plainly, exactly as on the trace basis, and that tool's trace is the
        kernel measurement (bench's own figures fall back to the event basis);
        span: per-launch event pairs, when the tracer cannot register at all."""
        if self.ok:
            return "trace"
        return "external" if "already configured" in self.err else "span"

    def begin(self):
        if self.L.wm_ktrace_begin() != 0:
            raise RuntimeError("wm_ktrace_begin failed")

    def end(self):
        n = ctypes.c_int()
        if self.L.wm_ktrace_end(ctypes.byref(n)) != 0:
            raise RuntimeError("wm_ktrace_end failed")
        return n.value

    def take(self, n, want_names=False):
        buf = (ctypes.c_double * max(1, n))()
        got = self.L.wm_ktrace_take(10000, buf, n)
        if got != n:
            raise RuntimeError("wm_ktrace_take: " + self.L.wm_ktrace_error().decode(errors="replace"))
        names = None
        if want_names:
            names = []
            nb = ctypes.create_string_buffer(512)
            for i in range(n):
                self.L.wm_ktrace_name(i, nb, 512)
                names.append(nb.value.decode(errors="replace"))
        return [buf[i] for i in range(n)], names


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
    keep = {"ops": ops, "dA": dA, "dc": dc, "dr": dr, "dG": dG, "out": out, "gA": gA, "gc": gc, "gr": gr}
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
    keep = {"ops": ops, "da": da, "db": db, "t": t, "rl": rl, "s1": s1, "y": y, "dy": dy, "ds1": ds1, "dr": dr,
            "dt": dt, "ga": ga, "gb": gb}
    return ops, keep, {"workload": "c1: y = relu(a[1024,1024] + b[1024]).sum(1).sum(), fwd+bwd "
                                   "(L2-resident, launch-bound; not a roofline case)", "elements": N}


def c3_ops(rows=16384, cols=4096):
    X = synth.config3(rows, cols)
    dX = W.DeviceArray.from_host(X)
    N = rows * cols
    big = N * F32
    ops, keep, outs = [], [dX], {}
    for dim, (outer, n, inner) in ((0, (1, rows, cols)), (1, (rows, cols, 1))):
        nout = outer * inner
        for name, code in (("sum", W.R_SUM), ("mean", W.R_MEAN), ("max", W.R_MAX), ("min", W.R_MIN),
                           ("argmax", W.R_ARGMAX), ("argmin", W.R_ARGMIN)):
            val = W.DeviceArray((nout,))
            idx = W.DeviceArray((nout,), np.int64) if code in (W.R_MAX, W.R_MIN) else None
            outs[f"{name} dim{dim}"] = (val, idx)
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
    keep = {"ops": ops, "bufs": keep, "outs": outs}
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
    return ops, {"ops": ops, "dL": dL, "dG": dG, "y": y, "ly": ly, "gx": gx}, {"workload": "c4: logits[%d,%d] fp32 ~N(0,3) with 1%% +20 spikes; "
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
    return ops, {"ops": ops, "h16": h16, "r16": r16, "dg": dg_, "ddm": ddm, "out": out, "m": m, "gh": gh,
                 "gr": gr, "gg": gg, "rows": rows, "c": c}, {
        "workload": "c5: h, res[%d,%d,%d] fp16 storage (truncating conversion), g[%d] fp32; "
                    "out = tanh_(clamp((h+res)*g, -4, 4)) stored fp16, mean over the last dim; fused fwd + bwd "
                    "(grads fp32, accumulated)" % (b, t, c, c), "elements": N}


def c5api_ops(b=32, t=1024, c=4096):
    """Config 5 as a caller of the drop-in Tensor API issues it (core/amp.h
    HalfTensor, core/tensor.h ops): every op materialises its fp32 output, as
    the reference's do, and every closure is timed on its own after the
    upstream gradient dm is injected (y->grad = dm; y->grad_fn(), which
    equals backward() from the scalar (y * dm).sum()).  Intermediate gradients start known-zero each step, so
    each closure's first contribution is written without a read."""
    from whitematter_amd import _tensor as T
    h, res, g, dm = synth.config5(b, t, c)
    rows = b * t
    N = rows * c
    hh = T.HalfTensor(T.Tensor.from_array(h))
    rr = T.HalfTensor(T.Tensor.from_array(res))
    del h, res
    gt = T.Tensor.from_array(g, requires_grad=True)
    dmt = T.Tensor.from_array(dm)
    st = {}

    def to_float_h():
        gt.zero_grad()
        st.clear()
        st["hf"] = hh.to_float(True)

    def fwd(name, fn):
        def run():
            st[name] = fn()
        return run

    def bwd(name, inject=False):
        def run():
            x = st[name]
            if inject:
                x.set_grad_from(dmt)
            x.call_grad_fn()
        return run

    f4 = N * F32
    ops = [
        Op("HalfTensor.to_float(h)", to_float_h, N * 2 + f4, "f16_to_f32_kernel", N),
        Op("HalfTensor.to_float(res)", fwd("rf", lambda: rr.to_float(True)), N * 2 + f4, "f16_to_f32_kernel", N),
        Op("add fwd", fwd("t1", lambda: st["hf"].add(st["rf"])), 3 * f4, "binary_flat_kernel", N),
        Op("mul(g) fwd", fwd("t2", lambda: st["t1"].mul(gt)), 2 * f4 + c * F32, "binary_rows_kernel", N),
        Op("clamp fwd", fwd("t3", lambda: st["t2"].clamp(-4.0, 4.0)), 2 * f4, "unary_fwd_kernel", N),
        Op("tanh_ fwd", fwd("t4", lambda: st["t3"].tanh_()), 2 * f4, "unary_fwd_kernel", N),
        Op("reshape fwd", fwd("t5", lambda: st["t4"].reshape([rows, c])), 2 * f4, "copy", N),
        Op("mean(1) fwd", fwd("m", lambda: st["t5"].mean(1, True)), f4 + rows * F32, "reduce_rows_kernel", N),
        Op("reshape(m) fwd", fwd("m3", lambda: st["m"].reshape([b, t, 1])), 2 * rows * F32, "copy", rows),
        # backward: dm injected into m3, then each node's closure in order
        Op("reshape(m) bwd", bwd("m3", inject=True), 3 * rows * F32, "copy", rows),
        Op("mean(1) bwd", bwd("m"), rows * F32 + f4, "reduce_bwd_sum_vec_kernel", N),
        Op("reshape bwd", bwd("t5"), 2 * f4, "copy", N),
        Op("tanh_ bwd", bwd("t4"), 3 * f4, "unary_bwd_kernel", N),
        Op("clamp bwd", bwd("t3"), 3 * f4, "unary_bwd_kernel", N),
        # G, a (t1), the g vector; t1.grad written; g.grad read + written
        Op("mul(g) bwd", bwd("t2"), 3 * f4 + 3 * c * F32, "bwd_colsum_kernel", N),
        Op("add bwd", bwd("t1"), 3 * f4, "bwd_flat_kernel", N),
    ]
    return ops, {"ops": ops, "hh": hh, "rr": rr, "gt": gt, "dmt": dmt, "st": st}, {
        "workload": "c5api: the c5 chain through the drop-in Tensor API: HalfTensor(h), HalfTensor(res) "
                    "[%d,%d,%d] fp16 -> to_float(requires_grad) -> add -> mul(g[%d]) -> clamp(-4,4) -> tanh_ -> "
                    "reshape([%d,%d]) -> mean(1, keepdim) -> reshape([%d,%d,1]); backward closures with dm "
                    "injected; fp32 intermediates as the Tensor API materialises them" % (b, t, c, c, rows, c, b, t),
        "elements": N}


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

    # clip_grad_norm_ / GradScaler::unscale followed by the step, through the
    # drop-in API (core/optimizer.h, core/amp.h) on a second copy of the list:
    # the norm (or the unscale's finiteness search) reads every gradient once,
    # its multiplication is deferred into the step, which reads the gradients
    # once more -- 4 + 28 bytes per element, the eager in-place multiplication's
    # read + write of every gradient gone.  Before each launch (untimed) the
    # gradients are refilled from their source copy, as a backward pass would
    # rewrite them, so no deferred scaling carries over between launches.
    from whitematter_amd import _tensor as T
    tp, tsrc = [], []
    for i, s in enumerate(shapes):
        n = int(np.prod(s))
        tp.append(T.Tensor.from_array((rng.standard_normal(n) * 0.02).astype(np.float32), list(s), True))
        # mul(1.0): an exact device copy, so the refills are device-to-device
        tsrc.append(T.Tensor.from_array((rng.standard_normal(n) * 1e-3).astype(np.float32), list(s)).mul(1.0))
    topt = T.AdamW(tp, 1e-4, 0.9, 0.999, 1e-8, 0.01)
    scaler = T.GradScaler(1024.0, 2.0, 0.5, 2000)

    def refill():
        for p_, s_ in zip(tp, tsrc):
            p_.set_grad_from(s_)

    def clip_step():
        T.clip_grad_norm_(tp, 1.0)  # norm ~11: clips on every call
        topt.step()

    def unscale_step():
        if not scaler.unscale(topt):
            raise RuntimeError("opt: unscale found a non-finite gradient")
        scaler.step(topt, True)

    ops = [
        Op("AdamW step", adam, N * 28, "multi_update_kernel<wm::Upd<1, true", N),
        Op("SGD momentum step", sgd, N * 20, "multi_update_kernel<wm::Upd<0, true", N),
        Op("RMSprop step", rms, N * 20, "multi_update_kernel<wm::Upd<2, false, false", N),
        Op("clip_grad_norm_ + AdamW step", clip_step, N * 32, "multi_update_kernel<wm::Upd<1, true", N),
        Op("GradScaler unscale + AdamW step", unscale_step, N * 32, "multi_update_kernel<wm::Upd<1, true", N),
    ]
    for op in ops[3:]:
        op.prepare = refill
    return ops, P + G + S1 + S2 + [tp, tsrc, topt, scaler], {
        "workload": "opt: %d parameter tensors, %d parameters (GPT-2-small shapes), fp32 params / grads / "
                    "state; one AdamW, SGD-momentum and RMSprop step (one multi-tensor launch each), and "
                    "clip_grad_norm_ + AdamW step, GradScaler unscale + AdamW step through the drop-in "
                    "optimizer / GradScaler (the gradients refilled, untimed, before each launch)"
                    % (len(shapes), N), "elements": N}




# ---------------------------------------------------------------------------
# CPU baselines (the reference's core/tensor.cpp, oracle/_ref, on 1 host core)
# and parity on the recipe's bytes
# ---------------------------------------------------------------------------

class _OneCore:
    """Pin this process to one host core for the duration (the reference's
    hot-path ops are single-threaded: no OpenMP on the path)."""

    def __enter__(self):
        self.cpus = os.sched_getaffinity(0)
        os.sched_setaffinity(0, {min(self.cpus)})
        return self

    def __exit__(self, *exc):
        os.sched_setaffinity(0, self.cpus)


def _reference():
    sys.path.insert(0, ROOT)
    import oracle
    ref = oracle.reference()
    if ref is None:
        raise RuntimeError("oracle/_ref is not built (the reference build needs /root/reference at build time)")
    return ref


def _oracles():
    sys.path.insert(0, ROOT)
    import oracle
    return oracle, oracle.get("f32"), oracle.get("f64"), oracle.get("abs")


def _timed(fn):
    t0 = time.perf_counter()
    out = fn()
    return out, time.perf_counter() - t0


def host_llc_bytes():
    """The last-level cache one host core sees (its L3 instance): sysfs for
    core 0, else the C library's sysconf; 0 if neither says."""
    base = "/sys/devices/system/cpu/cpu0/cache"
    best = 0
    try:
        for d in os.listdir(base):
            with open(os.path.join(base, d, "size")) as f:
                v = f.read().strip()
            mult = {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}.get(v[-1:], 1)
            best = max(best, int(v.rstrip("KMG")) * mult)
    except (OSError, ValueError):
        pass
    if not best:
        # lscpu -B: "L3 cache: <bytes> (<n> instances)" -> one instance
        try:
            import subprocess
            out = subprocess.run(["lscpu", "-B"], capture_output=True, text=True, timeout=10).stdout
            for line in out.splitlines():
                if line.startswith("L3 cache:") or (line.startswith("L2 cache:") and not best):
                    f = line.split(":", 1)[1].split()
                    n = int(f[1].strip("(")) if len(f) > 1 else 1
                    best = max(best, int(f[0]) // max(n, 1))
        except (OSError, ValueError, IndexError, subprocess.SubprocessError):
            pass
    return max(best, 0)


def host_cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _cpu_record(samples, ncpus, sample, reps, sample_bytes=None):
    """samples: op name -> (list of sample seconds, scale to the full workload,
    full-workload algorithmic bytes).  Per-op figures are the median sample
    time scaled to the full workload."""
    per_ms, per_gbps, tot_t, tot_b = {}, {}, 0.0, 0
    for name, (ts, scale, nbytes) in samples.items():
        t = statistics.median(ts) * scale
        per_ms[name] = round(t * 1e3, 3)
        per_gbps[name] = round(nbytes / t / 1e9, 4)
        tot_t += t
        tot_b += nbytes
    rec = {"value": round(tot_b / tot_t / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "reference",
           "sample": f"{sample}; median of {reps} after 1 warm-up unless stated; per-op times scaled to the full "
                     f"workload; single-threaded on 1 of {ncpus} host cores",
           "per_op_ms_full": per_ms, "per_op_GBps": per_gbps}
    llc = host_llc_bytes()
    rec["host_cpu"] = host_cpu_model()
    if sample_bytes is not None:
        rec["sample_MiB"] = round(sample_bytes / 2 ** 20, 1)
        rec["host_llc_MiB"] = round(llc / 2 ** 20, 1) if llc else None
        rec["sample_exceeds_llc"] = bool(llc and sample_bytes > llc)
    return rec


class Parity:
    """Checks of GPU outputs against the reference build and the fp64 oracle,
    to the contract's bars; `notes` holds how far the reference build's own
    outputs sit from the fp64 oracle on the same bytes (for the record)."""

    def __init__(self):
        self.oracle = _oracles()[0]
        self.items, self.notes = {}, {}

    def _add(self, name, ok, worst, kind):
        self.items[name] = {"ok": bool(ok), "kind": kind, "worst": None if worst is None else float(worst)}

    def exact(self, name, got, ref, zero_sign=False):
        got = np.asarray(got).reshape(np.shape(ref))
        if np.asarray(ref).dtype.kind in "iu":
            self._add(name, np.array_equal(got, ref), None, "exact")
            return
        eq = self.oracle.equal_modulo_zero_sign if zero_sign else self.oracle.bit_equal
        self._add(name, eq(got, ref), None, "exact")

    def ulp(self, name, got, ref64, bound=2.0):
        d = self.oracle.ulp_vs_f64(np.asarray(got).reshape(np.shape(ref64)), ref64)
        worst = float(d.max()) if d.size else 0.0
        self._add(name, worst <= bound, worst, "ulp<=%g" % bound)

    def tol(self, name, got, ref64, scale64, rtol=1e-5):
        ok, worst = self.oracle.close_scaled(np.asarray(got).reshape(np.shape(ref64)), ref64, scale64, rtol,
                                             atol=1e-30)
        self._add(name, ok, worst, "tol %g" % rtol)

    def f16_within(self, name, out16, w64, ulps=2):
        """out16 (fp16 bits) is the truncating fp16 (core/amp.h float_to_half)
        of an fp32 value within `ulps` fp32 ulps of w64: truncation toward zero
        is monotone, so that holds iff out16 lies between the truncations of
        the interval's two ends."""
        o32 = self.oracle.get("f32")
        w32 = np.asarray(w64).astype(np.float32)
        lo, hi = w32.copy(), w32.copy()
        for _ in range(ulps):
            lo = np.nextafter(lo, np.float32(-np.inf))
            hi = np.nextafter(hi, np.float32(np.inf))
        f = o32.f16_to_f32
        got = f(np.asarray(out16).reshape(w32.shape))
        ok = np.all((got >= f(o32.f32_to_f16(lo))) & (got <= f(o32.f32_to_f16(hi))))
        self._add(name, ok, None, "fp16 of fp32 within %d ulp" % ulps)

    def note(self, name, value):
        self.notes[name] = value if isinstance(value, (str, bool, type(None))) else round(float(value), 4)

    def summary(self):
        fails = [k for k, v in self.items.items() if not v["ok"]]
        return {"pass": not fails, "checks": len(self.items), "fail": fails}

    def detail(self):
        return {"checks": self.items, "reference_vs_fp64": self.notes}


def d2h_rows(d, rows):
    """The first `rows` rows (leading dimension) of a device array, to host."""
    per_row = d.size // d.shape[0]
    out = np.empty((rows,) + tuple(d.shape[1:]), d.dtype)
    W.call("wm_d2h", out.ctypes.data_as(ctypes.c_void_p), d.vp, rows * per_row * d.dtype.itemsize)
    return out


# ---- config 1 ------------------------------------------------------------------

def cpu_baseline_c1(reps=3):
    """Returns (record, outputs of the last run: the reference's values and
    gradients on the whole of config 1)."""
    ref = _reference()
    a, b = synth.config1()
    rows, cols = a.shape
    N = rows * cols
    big = N * F32
    bytes_ = {"add fwd": 2 * big + cols * F32, "relu fwd": 2 * big, "sum(1) fwd": big + rows * F32,
              "sum() fwd": rows * F32 + F32, "sum() bwd": F32 + rows * F32, "sum(1) bwd": rows * F32 + big,
              "relu bwd": 3 * big, "add bwd": big + 2 * big + 2 * cols * F32}
    ts = {k: [] for k in bytes_}
    with _OneCore() as oc:
        for rep in range(reps + 1):
            ta, tb = ref.tensor(a, True), ref.tensor(b, True)
            t, d0 = _timed(lambda: ref.binary("add", ta, tb))
            r, d1 = _timed(lambda: ref.unary("relu", t))
            s1, d2 = _timed(lambda: ref.reduce("sum", r, 1, False))
            y, d3 = _timed(lambda: ref.reduce("sum", s1, -1, False))
            y.set_grad(np.ones(1, np.float32))
            _, d4 = _timed(y.call_grad_fn)
            _, d5 = _timed(s1.call_grad_fn)
            _, d6 = _timed(r.call_grad_fn)
            _, d7 = _timed(t.call_grad_fn)
            if rep:
                for k, d in zip(bytes_, (d0, d1, d2, d3, d4, d5, d6, d7)):
                    ts[k].append(d)
        ncpu = len(oc.cpus)
    outs = {"a": a, "b": b, "t": t.data(), "r": r.data(), "s1": s1.data(), "y": y.data(), "ga": ta.grad(),
            "gb": tb.grad()}
    rec = _cpu_record({k: (ts[k], 1, bytes_[k]) for k in bytes_}, ncpu, "the whole of config 1", reps,
                      sample_bytes=2 * big)
    return rec, outs


def parity_c1(ctx, outs):
    """The whole chain once more on the GPU (gradients from zero), every
    output against the reference build / fp64 oracle on the same bytes."""
    _, o32, o64, oab = _oracles()
    ctx["ga"].fill(0.0)
    ctx["gb"].fill(0.0)
    for op in ctx["ops"]:
        op.launch()
    W.sync()
    P = Parity()
    a, b = outs["a"], outs["b"]
    rows, cols = a.shape
    t, r, s1, y = (ctx[k].to_host() for k in ("t", "rl", "s1", "y"))
    P.exact("add fwd", t, outs["t"])
    P.exact("relu fwd", r, outs["r"])
    P.tol("sum(1) fwd", s1.reshape(rows), o64.reduce("sum", r, rows, cols, 1)[0].reshape(rows),
          oab.reduce("sum", r, rows, cols, 1)[0].reshape(rows))
    P.tol("sum() fwd", y.reshape(1), o64.reduce("sum", s1, 1, rows, 1)[0].reshape(1),
          oab.reduce("sum", s1, 1, rows, 1)[0].reshape(1))
    dt = o32.unary_bwd("relu", np.ones_like(t), t, r)    # 0 / 1: exact
    ga64, gb64 = o64.binary_bwd("add", dt, a, b)
    gaab, gbab = oab.binary_bwd("add", dt, a, b)
    ga, gb = ctx["ga"].to_host(), ctx["gb"].to_host()
    P.tol("add bwd a.grad", ga, ga64, gaab)
    P.tol("add bwd b.grad", gb, gb64, gbab)
    # the reference's gradients are small integers (exact in fp32): equal bit for bit
    P.exact("a.grad = reference's", ga, outs["ga"])
    P.exact("b.grad = reference's", gb, outs["gb"])
    P.note("sum() reference", oracle_worst(outs["y"].reshape(1), o64.reduce("sum", s1, 1, rows, 1)[0].reshape(1),
                                           oab.reduce("sum", s1, 1, rows, 1)[0].reshape(1)))
    return P


def oracle_worst(got, ref64, scale64):
    return _oracles()[0].close_scaled(np.asarray(got).reshape(np.shape(ref64)), ref64, scale64, 1e-5, 1e-30)[1]


# ---- config 2 ------------------------------------------------------------------

C2_OPS = (("A+r", "add", "r"), ("A*c", "mul", "c"), ("A/r", "div", "r"), ("A^c", "pow", "c"))


def cpu_baseline_c2(sample_rows=2048, cols=8192, reps=3):
    ref = _reference()
    rows_full = 8192
    A, c, r, G = synth.config2(sample_rows, cols)  # the first sample_rows rows of A, c and G
    scale = rows_full / sample_rows
    N = rows_full * cols
    big = N * F32
    samples, outs = {}, {"inputs": (A, c, r, G)}
    with _OneCore() as oc:
        for name, op, vec in C2_OPS:
            other = c if vec == "c" else r
            vb = (rows_full if vec == "c" else cols) * F32
            fb = 2 * big + vb
            bb = 3 * big + 2 * vb if op == "add" else 4 * big + 3 * vb
            tf, tb = [], []
            for rep in range(reps + 1):
                ta, to = ref.tensor(A, True), ref.tensor(other, True)
                y, d0 = _timed(lambda: ref.binary(op, ta, to))
                y.set_grad(G)
                _, d1 = _timed(y.call_grad_fn)
                if rep:
                    tf.append(d0)
                    tb.append(d1)
                if rep == reps:
                    outs[name + " fwd"] = y.data()
                    outs[name + " bwd"] = (ta.grad(), to.grad())
                del y, ta, to
            samples[name + " fwd"] = (tf, scale, fb)
            samples[name + " bwd"] = (tb, scale, bb)
        ncpu = len(oc.cpus)
    rec = _cpu_record(samples, ncpu, f"A[{sample_rows},{cols}] row slice of config 2 (1/{int(scale)} of A), same ops",
                      reps, sample_bytes=3 * A.nbytes)
    return rec, outs


def parity_c2(ctx, outs):
    """Each op's forward and backward once more at full size (gradients from
    zero); the sampled rows of A's gradient and the row-local c.grad against
    the oracle; r.grad, a sum over every row, from the same kernels run on
    the sample's rows."""
    _, o32, o64, oab = _oracles()
    A, c, r, G = outs["inputs"]
    rows_s, cols = A.shape
    byname = {op.name: op for op in ctx["ops"]}
    P = Parity()
    for name, opname, vec in C2_OPS:
        other = c if vec == "c" else r
        byname[name + " fwd"].launch()
        out = d2h_rows(ctx["out"], rows_s)
        if opname == "pow":
            P.ulp(name + " fwd", out, o64.binary("pow", A, other))
            P.note(name + " fwd reference, max ulp",
                   float(_oracles()[0].ulp_vs_f64(outs[name + " fwd"], o64.binary("pow", A, other)).max()))
        else:
            P.exact(name + " fwd", out, outs[name + " fwd"])
        gvec = ctx["gc"] if vec == "c" else ctx["gr"]
        ctx["gA"].fill(0.0)
        gvec.fill(0.0)
        byname[name + " bwd"].launch()
        gA = d2h_rows(ctx["gA"], rows_s)
        fwd_out = out if opname == "pow" else None
        ga64, gb64 = _bwd_pair(o64, opname, G, A, other, fwd_out)
        gaab, gbab = _bwd_pair(oab, opname, G, A, other, fwd_out)
        P.tol(name + " bwd A.grad", gA, ga64, gaab)
        if vec == "c":
            P.tol(name + " bwd c.grad", d2h_rows(ctx["gc"], rows_s), gb64, gbab)
        else:
            dA_s, dG_s = W.DeviceArray.from_host(A), W.DeviceArray.from_host(G)
            gA_s, gr_s = W.DeviceArray(A.shape), W.DeviceArray(r.shape)
            gA_s.fill(0.0)
            gr_s.fill(0.0)
            sa, na = W.shape_arg(A.shape)
            sb, nb = W.shape_arg(r.shape)
            W.call("wm_binary_bwd", W.BINARY_OPS[opname], dG_s.vp, dA_s.vp, sa, na, ctx["dr"].vp, sb, nb,
                   W.nullp(), gA_s.vp, 1, gr_s.vp, 1)
            P.tol(name + " bwd r.grad (kernels on the sample)", gr_s.to_host(), gb64, gbab)
            for d in (dA_s, dG_s, gA_s, gr_s):
                d.free()
        rga, rgb = outs[name + " bwd"]
        P.note(name + " bwd reference A.grad", oracle_worst(rga, ga64, gaab))
        P.note(name + " bwd reference " + vec + ".grad", oracle_worst(rgb, gb64, gbab))
    return P


def _bwd_pair(o, opname, G, A, other, out):
    return o.binary_bwd(opname, G, A, other, out=out)


# ---- config 3 ------------------------------------------------------------------

C3_OPS = ("sum", "mean", "max", "min", "argmax", "argmin")


def cpu_baseline_c3(sample_rows=8192, cols=4096, reps=3):
    ref = _reference()
    rows_full = 16384
    X = synth.quantize(synth.normal((sample_rows, cols), synth.seed_for(3, 0)))  # first rows of config 3's X
    scale = rows_full / sample_rows
    N = rows_full * cols
    big = N * F32
    samples, outs = {}, {"X": X}
    with _OneCore() as oc:
        tx = ref.tensor(X, False)
        for dim in (0, 1):
            nout = cols if dim == 0 else rows_full
            for name in C3_OPS:
                ts = []
                for rep in range(reps + 1):
                    y, d = _timed(lambda: ref.reduce(name, tx, dim, False))
                    if rep:
                        ts.append(d)
                outs[f"{name} dim{dim}"] = y.data()
                samples[f"{name} dim{dim}"] = (ts, scale, big + nout * F32)
        ts = []
        for rep in range(reps + 1):
            y, d = _timed(lambda: ref.reduce("sum", tx, -1, False))
            if rep:
                ts.append(d)
        outs["sum full"] = y.data()
        samples["sum full"] = (ts, scale, big + F32)
        # max backward: the closure routes g to the first winner (O(outputs))
        for dim in (0, 1):
            nout = cols if dim == 0 else sample_rows
            g = synth.normal((nout,), synth.seed_for(3, 5 + dim))
            ts = []
            for rep in range(reps + 1):
                tg = ref.tensor(X, True)
                m = ref.reduce("max", tg, dim, False)
                m.set_grad(g)
                _, d = _timed(m.call_grad_fn)
                if rep:
                    ts.append(d)
            outs[f"max dim{dim} bwd"] = (g, tg.grad())
            del tg, m
            full_out = cols if dim == 0 else rows_full
            samples[f"max dim{dim} bwd"] = (ts, 1 if dim == 0 else scale, full_out * (F32 + 8 + 2 * F32))
        ncpu = len(oc.cpus)
    rec = _cpu_record(samples, ncpu, f"X[{sample_rows},{cols}] row slice of config 3 (1/{int(scale)} of X), same ops",
                      reps, sample_bytes=X.nbytes)
    return rec, outs


def parity_c3(ctx, outs):
    """dim-1 reductions: the timed kernels' outputs for the sampled rows;
    dim-0 / full reductions and the max backward (sums over every row, or
    scatters into the whole input): the same kernels on the sample."""
    oracle, o32, o64, oab = _oracles()
    X = outs["X"]
    rows_s, cols = X.shape
    P = Parity()
    dXs = W.DeviceArray.from_host(X)
    for dim in (0, 1):
        outer, n, inner = (1, rows_s, cols) if dim == 0 else (rows_s, cols, 1)
        nout = outer * inner
        for name in C3_OPS:
            code = W.REDUCE_OPS[name]
            key = f"{name} dim{dim}"
            if dim == 1:   # row-local: the timed run's own outputs
                val_d, idx_d = ctx["outs"][key]
                got = d2h_rows(val_d, rows_s)
                gidx = d2h_rows(idx_d, rows_s) if idx_d is not None else None
            else:
                val_d = W.DeviceArray((nout,))
                idx_d = W.DeviceArray((nout,), np.int64) if name in ("max", "min") else None
                W.call("wm_reduce", code, dXs.vp, outer, n, inner, val_d.vp, W.ptr(idx_d))
                got = val_d.to_host()
                gidx = idx_d.to_host() if idx_d is not None else None
                val_d.free()
                if idx_d is not None:
                    idx_d.free()
            ref = outs[key].reshape(-1)
            if name in ("sum", "mean"):
                v64 = o64.reduce(name, X, outer, n, inner)[0].reshape(-1)
                P.tol(key, got, v64, oab.reduce(name, X, outer, n, inner)[0].reshape(-1))
                P.note(key + " reference", oracle_worst(ref, v64, oab.reduce(name, X, outer, n, inner)[0].reshape(-1)))
            elif name in ("max", "min"):
                P.exact(key, got, ref, zero_sign=True)
                P.exact(key + " index", gidx, o32.reduce(name, X, outer, n, inner)[1].reshape(-1))
            else:
                P.exact(key, got, ref)
    full = W.DeviceArray((1,))
    W.call("wm_reduce", W.R_SUM, dXs.vp, 1, X.size, 1, full.vp, W.nullp())
    P.tol("sum full", full.to_host(), o64.reduce("sum", X, 1, X.size, 1)[0].reshape(-1),
          oab.reduce("sum", X, 1, X.size, 1)[0].reshape(-1))
    full.free()
    for dim in (0, 1):
        outer, n, inner = (1, rows_s, cols) if dim == 0 else (rows_s, cols, 1)
        g, ref_grad = outs[f"max dim{dim} bwd"]
        idx = W.DeviceArray((outer * inner,), np.int64)
        W.call("wm_reduce", W.R_MAX, dXs.vp, outer, n, inner, W.nullp(), idx.vp)
        dg = W.DeviceArray.from_host(g)
        gX = W.DeviceArray(X.shape)
        gX.fill(0.0)
        W.call("wm_reduce_bwd", W.R_MAX, dg.vp, idx.vp, outer, n, inner, gX.vp, 1)
        P.exact(f"max dim{dim} bwd (scatter to the first winner)", gX.to_host(), ref_grad)
        for d in (idx, dg, gX):
            d.free()
    dXs.free()
    return P


# ---- config 4 ------------------------------------------------------------------

def c4_sample(sample_rows):
    L = synth.spikes(synth.normal((sample_rows, 32000), synth.seed_for(4, 0), 0.0, 3.0), synth.seed_for(4, 1))
    G = synth.normal((sample_rows, 32000), synth.seed_for(4, 2))
    return L, G


def cpu_baseline_c4(sample_rows=512, jac_rows=4, cols=32000, reps=3):
    """softmax / log_softmax forward and log_softmax backward on 512 rows; the
    softmax backward (the reference's explicit Jacobian, O(cols^2) per row)
    on jac_rows rows, each timed on its own (the spread shows the rows cost
    the same), extrapolated by rows."""
    ref = _reference()
    rows_full = 8192
    L, G = c4_sample(sample_rows)
    N = rows_full * cols
    big = N * F32
    samples, outs = {}, {"L": L, "G": G}
    with _OneCore() as oc:
        for log in (False, True):
            nm = "log_softmax" if log else "softmax"
            tf, tb = [], []
            for rep in range(reps + 1):
                tx = ref.tensor(L, True)
                y, d = _timed(lambda: ref.softmax(tx, log))
                if rep:
                    tf.append(d)
                if log:
                    y.set_grad(G)
                    _, d = _timed(y.call_grad_fn)
                    if rep:
                        tb.append(d)
            outs[nm + " fwd"] = y.data()
            if log:
                outs[nm + " bwd"] = tx.grad()
            samples[nm + " fwd"] = (tf, rows_full / sample_rows, 2 * big)
            if log:
                samples[nm + " bwd"] = (tb, rows_full / sample_rows, 4 * big)
        per_row, jac = [], []
        for i in range(jac_rows):
            tx = ref.tensor(L[i:i + 1], True)
            y = ref.softmax(tx, False)
            y.set_grad(G[i:i + 1])
            _, d = _timed(y.call_grad_fn)
            per_row.append(d)
            jac.append((y.data(), tx.grad()))
        outs["softmax bwd"] = jac
        samples["softmax bwd"] = ([sum(per_row) / jac_rows], rows_full, 4 * big)
        ncpu = len(oc.cpus)
    rec = _cpu_record(samples, ncpu, f"logits[{sample_rows},{cols}] row slice of config 4 (softmax bwd: {jac_rows} "
                                     f"rows timed one by one, mean x{rows_full})", reps,
                      sample_bytes=L.nbytes + G.nbytes)
    rec["extrapolated"] = ["softmax bwd"]
    rec["softmax_bwd_row_s"] = [round(t, 3) for t in per_row]
    return rec, outs


def _softmax_bwd64(g, y):
    """The softmax closure's value in fp64, closed form: s_j (g_j - sum_k g_k s_k),
    and the magnitude of its terms, s_j (|g_j| + sum_k |g_k| s_k)."""
    g64, s = g.astype(np.float64), y.astype(np.float64)
    gs = g64 * s
    ref = gs - s * gs.sum(axis=1, keepdims=True)
    scale = np.abs(gs) + s * np.abs(gs).sum(axis=1, keepdims=True)
    return ref, scale


def parity_c4(ctx, outs):
    """Row-local throughout: the timed kernels' outputs for the sampled rows
    (the backward once more, gradient from zero)."""
    _, o32, o64, oab = _oracles()
    L, G = outs["L"], outs["G"]
    rows_s = L.shape[0]
    byname = {op.name: op for op in ctx["ops"]}
    P = Parity()
    y = d2h_rows(ctx["y"], rows_s)
    ly = d2h_rows(ctx["ly"], rows_s)
    s64 = o64.softmax(L)
    P.tol("softmax fwd", y, s64, s64)
    P.note("softmax fwd reference", oracle_worst(outs["softmax fwd"], s64, s64))
    l64, lab = o64.softmax(L, log=True), oab.softmax(L, log=True)
    P.tol("log_softmax fwd", ly, l64, lab)
    P.note("log_softmax fwd reference", oracle_worst(outs["log_softmax fwd"], l64, lab))
    for nm, log in (("softmax bwd", False), ("log_softmax bwd", True)):
        ctx["gx"].fill(0.0)
        byname[nm].launch()
        gx = d2h_rows(ctx["gx"], rows_s)
        saved = ly if log else y
        if log:
            ref, scale = o64.softmax_bwd(G, saved, log=True), oab.softmax_bwd(G, saved, log=True)
        else:
            ref, scale = _softmax_bwd64(G, saved)
        P.tol(nm, gx, ref, scale)
    P.note("log_softmax bwd reference",
           oracle_worst(outs["log_softmax bwd"], o64.softmax_bwd(G, outs["log_softmax fwd"], log=True),
                        oab.softmax_bwd(G, outs["log_softmax fwd"], log=True)))
    # the reference's O(C^2) Jacobian on its rows, and the GPU on the same rows
    jw = 0.0
    for i, (ry, rgx) in enumerate(outs["softmax bwd"]):
        ref, scale = _softmax_bwd64(G[i:i + 1], ry.reshape(1, -1))
        jw = max(jw, oracle_worst(rgx.reshape(1, -1), ref, scale))
    P.note("softmax bwd reference (Jacobian rows)", jw)
    return P


# ---- config 5 (fused) and 5api (the Tensor API chain) -----------------------------

_C5_CHAIN = {}


def _c5_chain_baseline(sample_rows=2048, c=4096, reps=3):
    """The config-5 chain through the reference's Tensor API on the first
    sample_rows rows (t = 0 .. sample_rows - 1 of batch 0); timed once per
    process, shared by the c5 and c5api records."""
    key = (sample_rows, c, reps)
    if key in _C5_CHAIN:
        return _C5_CHAIN[key]
    ref = _reference()
    rows_full = 32 * 1024
    h = synth.normal((1, sample_rows, c), synth.seed_for(5, 0))
    res = synth.normal((1, sample_rows, c), synth.seed_for(5, 1))
    g = synth.uniform((c,), synth.seed_for(5, 2), 0.8, 1.2)
    dm = synth.normal((1, sample_rows, 1), synth.seed_for(5, 3))
    h16, r16 = ref.f32_to_f16(h), ref.f32_to_f16(res)
    scale = rows_full / sample_rows
    N = rows_full * c
    f4 = N * F32
    bytes_ = {"HalfTensor.to_float(h)": N * 2 + f4, "HalfTensor.to_float(res)": N * 2 + f4, "add fwd": 3 * f4,
              "mul(g) fwd": 2 * f4 + c * F32, "clamp fwd": 2 * f4, "tanh_ fwd": 2 * f4, "reshape fwd": 2 * f4,
              "mean(1) fwd": f4 + rows_full * F32, "reshape(m) fwd": 2 * rows_full * F32,
              "reshape(m) bwd": 3 * rows_full * F32, "mean(1) bwd": rows_full * F32 + f4, "reshape bwd": 2 * f4,
              "tanh_ bwd": 3 * f4, "clamp bwd": 3 * f4, "mul(g) bwd": 3 * f4 + 3 * c * F32, "add bwd": 3 * f4}
    ts = {k: [] for k in bytes_}
    outs = {"h16": h16.reshape(sample_rows, c), "r16": r16.reshape(sample_rows, c), "g": g,
            "dm": dm.reshape(sample_rows)}
    with _OneCore() as oc:
        for rep in range(reps + 1):
            d = {}
            hf, d["HalfTensor.to_float(h)"] = _timed(lambda: ref.tensor(ref.f16_to_f32(h16), True))
            rf, d["HalfTensor.to_float(res)"] = _timed(lambda: ref.tensor(ref.f16_to_f32(r16), True))
            gt = ref.tensor(g, True)
            t1, d["add fwd"] = _timed(lambda: ref.binary("add", hf, rf))
            t2, d["mul(g) fwd"] = _timed(lambda: ref.binary("mul", t1, gt))
            t3, d["clamp fwd"] = _timed(lambda: ref.unary("clamp", t2, -4.0, 4.0))
            t4, d["tanh_ fwd"] = _timed(lambda: ref.unary("tanh", t3))
            t5, d["reshape fwd"] = _timed(lambda: ref.reshape(t4, (sample_rows, c)))
            m, d["mean(1) fwd"] = _timed(lambda: ref.reduce("mean", t5, 1, True))
            m3, d["reshape(m) fwd"] = _timed(lambda: ref.reshape(m, (1, sample_rows, 1)))
            m3.set_grad(dm)
            for name, node in (("reshape(m) bwd", m3), ("mean(1) bwd", m), ("reshape bwd", t5), ("tanh_ bwd", t4),
                               ("clamp bwd", t3), ("mul(g) bwd", t2), ("add bwd", t1)):
                _, d[name] = _timed(node.call_grad_fn)
            if rep:
                for k in bytes_:
                    ts[k].append(d[k])
            if rep == reps:
                outs.update({"t1": t1.data(), "t2": t2.data(), "t3": t3.data(), "t4": t4.data(), "m": m.data(),
                             "gh": hf.grad(), "gr": rf.grad(), "gg": gt.grad()})
            del hf, rf, gt, t1, t2, t3, t4, t5, m, m3
        ncpu = len(oc.cpus)
    # the (m) reshapes and their closure move rows-sized vectors: scale by rows too
    rec = _cpu_record({k: (ts[k], scale, bytes_[k]) for k in bytes_}, ncpu,
                      f"h, res[1,{sample_rows},{c}] (the first {sample_rows} of 32768 rows of config 5) through "
                      f"the same chain, the (h, res) fp16 bits made by the reference's float_to_half", reps,
                      sample_bytes=2 * sample_rows * c * 2 + 8 * sample_rows * c * F32)
    _C5_CHAIN[key] = (rec, outs)
    return rec, outs


def cpu_baseline_c5api(sample_rows=2048, c=4096, reps=3):
    return _c5_chain_baseline(sample_rows, c, reps)


def cpu_baseline_c5(b=32, t=1024, c=4096):
    """Config 5 has no fused op in the reference: its CPU path is the chain
    cpu_baseline_c5api times (HalfTensor -> add -> mul -> clamp -> tanh_ ->
    reshape -> mean and the closures).  The chain's forward and backward
    times are reported against the fused ops, and value is the fused step's
    algorithmic bytes over the chain's time, so that value / value is the
    time ratio."""
    chain, outs = _c5_chain_baseline(c=c)
    rows, N = b * t, b * t * c
    fwd_b = N * (2 + 2 + 2) + c * F32 + rows * F32           # as c5_ops
    bwd_b = N * (2 + 2 + 8 + 8) + c * F32 + rows * F32 + 2 * c * F32
    per = chain["per_op_ms_full"]
    t_fwd = sum(v for k, v in per.items() if k.endswith("fwd") or k.startswith("HalfTensor"))
    t_bwd = sum(v for k, v in per.items() if k.endswith("bwd"))
    rec = {"value": round((fwd_b + bwd_b) / ((t_fwd + t_bwd) * 1e-3) / 1e9, 4), "unit": "GB/s", "cores": 1,
           "kind": "reference",
           "sample": "the reference's chain for config 5 (no fused op there): " + chain["sample"] +
                     "; its forward and backward times set against the fused ops",
           "per_op_ms_full": {"epilogue fwd": round(t_fwd, 3), "epilogue bwd": round(t_bwd, 3)}}
    return rec, outs


def _c5_expected(outs, tanh32):
    """fp32 forward intermediates of the chain on the sample (exact IEEE ops),
    and the fp64 backward chain of the reference closures on the fp32 tanh
    values the forward produced (the values a closure reads from
    result->data)."""
    _, o32, _, _ = _oracles()
    lo, hi = -4.0, 4.0
    h = o32.f16_to_f32(outs["h16"])
    r = o32.f16_to_f32(outs["r16"])
    g, dm = outs["g"], outs["dm"]
    t = o32.binary("add", h, r)
    u = o32.binary("mul", t, g)
    v = o32.unary("clamp", u, lo, hi)
    w = tanh32(v)
    w64 = w.astype(np.float64)
    du = np.where((u > lo) & (u < hi), dm.astype(np.float64)[:, None] * (1.0 - w64 * w64), 0.0)
    dt = du * g.astype(np.float64)[None, :]
    dgt = du * t.astype(np.float64)
    return {"t": t, "u": u, "v": v, "w": w, "mean": w64.sum(axis=1) / w.shape[1],
            "mean_scale": np.abs(w64).sum(axis=1) / w.shape[1], "dt": dt, "dg": dgt.sum(axis=0),
            "dg_scale": np.abs(dgt).sum(axis=0)}


def _gpu_tanh(v):
    d = W.DeviceArray.from_host(v)
    out = W.unary(W.TANH, d)
    res = out.to_host()
    d.free()
    out.free()
    return res


def parity_c5(ctx, outs):
    """The fused kernels' outputs for the sampled rows (the backward once more,
    overwriting); g.grad, a column sum over every row, from the same kernel
    on the sample."""
    _, o32, _, _ = _oracles()
    S = outs["h16"].shape[0]
    P = Parity()
    P.exact("float_to_half(h), (res) on the device", np.stack([d2h_rows(ctx["h16"], S), d2h_rows(ctx["r16"], S)]),
            np.stack([outs["h16"], outs["r16"]]))
    e = _c5_expected(outs, _gpu_tanh)
    out16 = d2h_rows(ctx["out"], S)
    P.exact("epilogue fwd out = float_to_half(fp32 tanh)", out16, o32.f32_to_f16(e["w"]))
    P.f16_within("epilogue fwd out vs fp64 tanh", out16, np.tanh(e["v"].astype(np.float64)))
    P.tol("epilogue fwd mean", d2h_rows(ctx["m"], S), e["mean"], e["mean_scale"])
    lo, hi = W.C.c_float(-4.0), W.C.c_float(4.0)
    rows, c = ctx["rows"], ctx["c"]
    W.call("wm_epilogue_f16_bwd", ctx["ddm"].vp, ctx["h16"].vp, ctx["r16"].vp, ctx["dg"].vp, ctx["gh"].vp, 0,
           ctx["gr"].vp, 0, ctx["gg"].vp, 0, rows, c, lo, hi)
    P.tol("epilogue bwd h.grad", d2h_rows(ctx["gh"], S), e["dt"], np.abs(e["dt"]))
    P.tol("epilogue bwd res.grad", d2h_rows(ctx["gr"], S), e["dt"], np.abs(e["dt"]))
    dh, dr, ddm = (W.DeviceArray.from_host(outs[k]) for k in ("h16", "r16", "dm"))
    gh, gr, gg = W.DeviceArray((S, c)), W.DeviceArray((S, c)), W.DeviceArray((c,))
    W.call("wm_epilogue_f16_bwd", ddm.vp, dh.vp, dr.vp, ctx["dg"].vp, gh.vp, 0, gr.vp, 0, gg.vp, 0, S, c, lo, hi)
    P.tol("epilogue bwd g.grad (kernel on the sample)", gg.to_host(), e["dg"], e["dg_scale"])
    for d in (dh, dr, ddm, gh, gr, gg):
        d.free()
    _c5_reference_notes(P, outs, e)
    return P


def _c5_reference_notes(P, outs, e):
    oracle, o32, _, _ = _oracles()
    P.note("tanh_ reference, max ulp vs fp64",
           float(oracle.ulp_vs_f64(outs["t4"].reshape(e["v"].shape), np.tanh(e["v"].astype(np.float64))).max()))
    P.note("add / mul / clamp reference bit-exact",
           bool(oracle.bit_equal(outs["t1"].reshape(e["t"].shape), e["t"]) and
                oracle.bit_equal(outs["t2"].reshape(e["u"].shape), e["u"]) and
                oracle.bit_equal(outs["t3"].reshape(e["v"].shape), e["v"])))


def parity_c5api(ctx, outs):
    """The Tensor-API chain's tensors from the last timed step, sampled rows;
    g.grad (a column sum over every row) from the same chain on the sample."""
    from whitematter_amd import _tensor as T
    oracle, o32, o64, _ = _oracles()
    st, gt = ctx["st"], ctx["gt"]
    S, c = outs["h16"].shape
    P = Parity()

    def rows_of(x):
        return np.asarray(x).reshape(-1, c)[:S]

    e = _c5_expected(outs, _gpu_tanh)
    P.exact("HalfTensor(h).to_float", rows_of(st["hf"].data), o32.f16_to_f32(outs["h16"]))
    P.exact("add fwd", rows_of(st["t1"].data), outs["t1"])
    P.exact("mul(g) fwd", rows_of(st["t2"].data), outs["t2"])
    P.exact("clamp fwd", rows_of(st["t3"].data), outs["t3"])
    w = rows_of(st["t4"].data)
    P.ulp("tanh_ fwd", w, np.tanh(e["v"].astype(np.float64)))
    P.exact("tanh_ fwd = the unary kernel's", w, e["w"])
    P.tol("mean(1) fwd", np.asarray(st["m3"].data).reshape(-1)[:S], e["mean"], e["mean_scale"])
    P.tol("add bwd h.grad", rows_of(st["hf"].grad), e["dt"], np.abs(e["dt"]))
    P.tol("add bwd res.grad", rows_of(st["rf"].grad), e["dt"], np.abs(e["dt"]))
    # g.grad sums over all rows: the same chain on the sample
    hs = T.HalfTensor(T.Tensor.from_array(o32.f16_to_f32(outs["h16"]).reshape(1, S, c)))
    rs = T.HalfTensor(T.Tensor.from_array(o32.f16_to_f32(outs["r16"]).reshape(1, S, c)))
    gs = T.Tensor.from_array(outs["g"], requires_grad=True)
    m3 = hs.to_float(True).add(rs.to_float(True)).mul(gs).clamp(-4.0, 4.0).tanh_().reshape([S, c]).mean(
        1, True).reshape([1, S, 1])
    (m3 * T.Tensor.from_array(outs["dm"].reshape(1, S, 1))).sum().backward()
    P.tol("mul(g) bwd g.grad (chain on the sample)", np.asarray(gs.grad).reshape(-1), e["dg"], e["dg_scale"])
    _c5_reference_notes(P, outs, e)
    return P


CPU_BASELINES = {"c1": cpu_baseline_c1, "c2": cpu_baseline_c2, "c3": cpu_baseline_c3, "c4": cpu_baseline_c4,
                 "c5": cpu_baseline_c5, "c5api": cpu_baseline_c5api}
PARITY = {"c1": parity_c1, "c2": parity_c2, "c3": parity_c3, "c4": parity_c4, "c5": parity_c5,
          "c5api": parity_c5api}


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
        Op("matmul fwd", lambda: W.call("wm_matmul", a.vp, b.vp, n, n, n, c.vp), 3 * n * n * F32, "rocBLAS sgemm",
           n * n, mm),
        Op("matmul bwd", lambda: W.call("wm_matmul_bwd", g.vp, a.vp, b.vp, n, n, n, ga.vp, 0, gb.vp, 0),
           6 * n * n * F32, "rocBLAS sgemm", 2 * n * n, 2 * mm),
        Op("bmm fwd", lambda: W.call("wm_bmm", qa.vp, kb.vp, batch, t, hd, t, sc.vp),
           (2 * batch * t * hd + batch * t * t) * F32, "gemm_dma3_kernel", batch * t * t, bm),
        Op("bmm bwd", lambda: W.call("wm_bmm_bwd", sg.vp, qa.vp, kb.vp, batch, t, hd, t, gq.vp, 0, gk.vp, 0),
           (batch * t * t * 2 + 4 * batch * t * hd) * F32, "gemm_dma_kernel", 2 * batch * t * hd, 2 * bm),
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
    and the bias column sums ride along in the same time (the score product, mask
    and softmax run as one kernel)."""
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
    kn = "rocBLAS sgemm + head_rows_kernel + gemm_kernel + gemm_dma32_kernel"
    ops = [Op("mha fwd", fwd, 4 * B * S * E * F32 + 3 * att, kn, B * S * E, f_fl),
           Op("mha bwd", bwd, 6 * B * S * E * F32 + 4 * att, kn, B * S * E, 2 * f_fl)]
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


CONFIGS = {"c1": c1_ops, "c2": c2_ops, "c3": c3_ops, "c4": c4_ops, "c5": c5_ops, "c5api": c5api_ops, "opt": opt_ops,
           "loss": loss_ops, "norm": norm_ops, "gemm": gemm_ops, "mha": mha_ops, "io": io_ops}
# --config all: the headline (the largest single-GPU configuration, c4) first, then the rest
ALL = ["c4", "c1", "c2", "c3", "c5", "c5api"]
# broadcast-elementwise and dim-reduction configurations: the >= 70 % of HBM target applies to their ops
TARGET_CONFIGS = ("c2", "c3", "c4", "c5", "c5api")
TARGET_FRAC = 0.70


def _launch(op, basis, flush, kt):
    """One launch of op after the 512 MiB flush fill (and the op's untimed
    preparation, if it has one), timed in `basis`."""
    if op.prepare is not None:
        op.prepare()
        W.sync()  # its copies dispatched and done before the timed window opens
    flush.fill(1.0)
    if basis in ("trace", "span", "external") and getattr(op, "host_io", False):
        return  # host-driven copies: timed on the event basis only
    if basis is None:
        op.launch()
    elif basis == "external":
        # another tool (rocprofv3) traces this process: launch exactly as the
        # trace basis does (no event markers), counting the dispatches
        c0, c1 = ctypes.c_int64(), ctypes.c_int64()
        W.call("wm_launch_count", ctypes.byref(c0))
        op.launch()
        W.call("wm_launch_count", ctypes.byref(c1))
        op.ndisp = c1.value - c0.value
    elif basis == "trace":
        c0, c1 = ctypes.c_int64(), ctypes.c_int64()
        W.call("wm_launch_count", ctypes.byref(c0))
        kt.begin()
        op.launch()
        n = kt.end()
        W.call("wm_launch_count", ctypes.byref(c1))
        W.sync()
        if n == 0:
            return  # no kernel (host-driven copies): the event basis only
        if n < c1.value - c0.value:
            raise RuntimeError("%s: the tracer saw %d dispatches, the library launched %d"
                               % (op.name, n, c1.value - c0.value))
        ms, names = kt.take(n, want_names=op.knames is None)
        op.kms.append(sum(ms))
        op.kparts.append(ms)
        if names is not None:
            op.knames = names
    elif basis == "span":
        W.call("wm_span_begin")
        op.launch()
        kms, nk = W.C.c_float(), W.C.c_int()
        rc = W.lib().wm_span_end(W.C.byref(kms), None, W.C.byref(nk))
        if rc != 0 and nk.value == 0:
            return
        W.check(rc, "wm_span_end (%s)" % op.name)
        op.kms.append(kms.value)
        per = []
        for i in range(nk.value):
            km = W.C.c_float()
            W.call("wm_span_kernel", i, W.C.byref(km))
            per.append(km.value)
        op.kparts.append(per)
    else:
        W.call("wm_timer_start")
        op.launch()
        ms = W.C.c_float()
        W.call("wm_timer_stop", W.C.byref(ms))
        op.ms.append(ms.value)


def run_config(name, args, flush, want_cpu, kt):
    """Build one configuration, time its ops (kernel basis -- the trace's, or
    span events -- and event basis, one flush before every launch), check
    parity on the recipe's bytes, and return (compact record, detail record)."""
    ops, ctx, workload = CONFIGS[name]()
    basis = kt.basis

    for _ in range(args.warmup):
        for op in ops:
            _launch(op, None, flush, kt)
    W.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        for op in ops:
            _launch(op, basis, flush, kt)
        for op in ops:
            _launch(op, "event", flush, kt)
    W.sync()
    wall = time.perf_counter() - t0

    cpu, parity = None, None
    if want_cpu and (name == "io" or name in CPU_BASELINES):
        try:
            if name == "io":
                cpu = cpu_baseline_io(workload["path"])
            else:
                cpu, outs = CPU_BASELINES[name]()
                P = PARITY[name](ctx, outs)
                parity = (P.summary(), P.detail())
                del outs
        except Exception as e:  # the baseline is reported, never the target
            cpu = {"value": None, "error": "%s: %s" % (type(e).__name__, e)}

    per_op, step_ms, step_bytes, step_flops, step_event_ms = {}, 0.0, 0, 0, 0.0
    host_io = all(getattr(op, "host_io", False) for op in ops)
    mfma = all(op.flops for op in ops)
    for op in ops:
        km = statistics.median(op.kms) if op.kms else statistics.median(op.ms)
        step_ms += km
        step_event_ms += statistics.median(op.ms)
        step_bytes += op.bytes
        step_flops += op.flops or 0
        gbps = op.bytes / (km * 1e-3) / 1e9
        d = {"ms": round(km, 4), "ms_event_median": round(statistics.median(op.ms), 4), "GBps": round(gbps, 1),
             "pct_peak": round(100 * gbps / PEAK_GBPS, 1), "Gelem_per_s": round(op.elems / (km * 1e-3) / 1e9, 2),
             "bytes": op.bytes}
        if op.prepare is not None:
            d["prepared"] = True  # untimed work before each launch (its dispatches precede the flush)
        if getattr(op, "ndisp", None) is not None:
            d["dispatches"] = op.ndisp
        if op.kms:
            nk = len(op.kparts[0])
            d["dispatches"] = nk
            if nk > 1 and all(len(k) == nk for k in op.kparts):
                d["ms_by_dispatch"] = [round(statistics.median(k[i] for k in op.kparts), 4) for i in range(nk)]
            if op.knames:
                d["kernels"] = [kn.split("(")[0][:80] for kn in op.knames]
        if op.flops:
            tf = op.flops / (km * 1e-3) / 1e12
            d.update({"TFLOPs": round(tf, 1), "pct_mfma_peak": round(100 * tf / PEAK_F32_MFMA_TFLOPS, 1),
                      "flops": op.flops})
        if cpu and cpu.get("per_op_ms_full", {}).get(op.name):
            d["speedup_vs_cpu"] = round(cpu["per_op_ms_full"][op.name] / km, 1)
        per_op[op.name] = d

    dom = max(ops, key=lambda o: statistics.median(o.kms) if o.kms else statistics.median(o.ms))
    dom_ms = per_op[dom.name]["ms"]
    if host_io:
        # host-driven file transfers: bounded by the file cache and PCIe, not by
        # an HBM or matrix-core roofline
        value, unit, roofline = step_bytes / (step_ms * 1e-3) / 1e9, "GB/s", None
        value_event = value
    elif mfma:
        value, unit = step_flops / (step_ms * 1e-3) / 1e12, "TFLOP/s"
        value_event = step_flops / (step_event_ms * 1e-3) / 1e12
        dom_tf = dom.flops / (dom_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(dom_tf, 2), "peak": PEAK_F32_MFMA_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(dom_tf / PEAK_F32_MFMA_TFLOPS, 4), "traffic": traffic_for(dom.name, name),
                    "kernel": dom.kernel, "op": dom.name, "algorithmic_flops": dom.flops, "ms": dom_ms}
    else:
        value, unit = step_bytes / (step_ms * 1e-3) / 1e9, "GB/s"
        value_event = step_bytes / (step_event_ms * 1e-3) / 1e9
        dom_gbps = dom.bytes / (dom_ms * 1e-3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(dom_gbps, 1), "peak": PEAK_GBPS, "unit": "GB/s",
                    "frac": round(dom_gbps / PEAK_GBPS, 4), "traffic": traffic_for(dom.name, name),
                    "kernel": dom.kernel, "op": dom.name, "algorithmic_bytes": dom.bytes, "ms": dom_ms}
    peak = PEAK_F32_MFMA_TFLOPS if mfma else PEAK_GBPS
    rec = {"workload": workload["workload"], "elements": workload.get("elements"), "value": round(value, 1),
           "unit": unit, "pct_of_peak": round(100 * value / peak, 1) if not host_io else None,
           "value_event": round(value_event, 1), "basis": basis, "ms_per_step": round(step_ms, 4),
           "roofline": roofline, "cpu_baseline": cpu, "wall_s_timed_loop": round(wall, 3)}
    if cpu and cpu.get("value") and not mfma:
        rec["speedup_vs_cpu_step"] = round(value / cpu["value"], 1)
    if name in TARGET_CONFIGS:
        rec["below_70pct"] = [k for k, v in per_op.items() if v["pct_peak"] < 100 * TARGET_FRAC
                              and not k.startswith(("max dim", "reshape(m)"))]
    if parity is not None:
        rec["parity"] = parity[0]
    detail = dict(rec, ops=per_op, parity_detail=parity[1] if parity else None)
    del ops, ctx
    gc.collect()
    return rec, detail


def compact(rec):
    """A configuration's record for the stdout line: headline figures, the
    dominant kernel's roofline, the CPU baseline's value, parity's verdict."""
    out = {"value": rec["value"], "unit": rec["unit"], "pct": rec["pct_of_peak"], "value_event": rec["value_event"],
           "ms_per_step": rec["ms_per_step"]}
    r = rec.get("roofline")
    if r:
        out["roofline"] = {k: r[k] for k in ("op", "kernel", "frac", "ms", "algorithmic_bytes", "algorithmic_flops",
                                              "traffic") if k in r}
    cpu = rec.get("cpu_baseline")
    if cpu:
        out["cpu_baseline"] = {k: cpu.get(k) for k in ("value", "unit", "cores", "kind")}
        if cpu.get("error"):
            out["cpu_baseline"]["error"] = cpu["error"][:120]
        else:
            out["cpu_baseline"]["sample"] = cpu.get("sample", "").split(";")[0][:110]
    if "speedup_vs_cpu_step" in rec:
        out["speedup_vs_cpu"] = rec["speedup_vs_cpu_step"]
    if "below_70pct" in rec:
        out["below_70pct"] = rec["below_70pct"]
    if "parity" in rec:
        p = rec["parity"]
        out["parity"] = _short_parity(p)
    return out


def _short_parity(p):
    return {"pass": p["pass"], "checks": p["checks"], "fail": [f[:48] for f in p["fail"][:4]],
            "failed": len(p["fail"])}


LINE_LIMIT = 4000  # bytes: the driver keeps the tail of stdout, and must see the whole line


def _fit(line):
    """Drop the least important fields of the compact records until the line
    fits LINE_LIMIT (the top-level contract fields are never dropped)."""
    steps = [("cpu_baseline", "sample"), ("roofline", "kernel"), (None, "below_70pct"), (None, "value_event"),
             ("cpu_baseline", "kind"), ("roofline", "traffic")]
    for parent, key in steps:
        if len(json.dumps(line)) <= LINE_LIMIT:
            break
        for rec in line.get("configs", {}).values():
            tgt = rec.get(parent) if parent else rec
            if isinstance(tgt, dict):
                tgt.pop(key, None)
    for rec in line.get("configs", {}).values():
        if len(json.dumps(line)) > LINE_LIMIT and rec.get("parity"):
            rec["parity"].pop("fail", None)
    if len(json.dumps(line)) > LINE_LIMIT and line.get("cpu_baseline", {}).get("sample"):
        line["cpu_baseline"]["sample"] = line["cpu_baseline"]["sample"][:120]
    return line


def bench_line(head, recs, names, args, cus, basis, copies):
    """The one stdout line: the headline configuration's figures at the top
    level, a compact record per other configuration in "configs"."""
    mfma = head["unit"] == "TFLOP/s"
    cpu = head.get("cpu_baseline")
    cpu_top = None
    if cpu:
        cpu_top = {k: cpu.get(k) for k in ("value", "unit", "cores", "kind", "sample")}
        if cpu.get("error"):
            cpu_top["error"] = cpu["error"][:200]
        if cpu_top.get("sample"):
            cpu_top["sample"] = cpu_top["sample"][:300]
    line = {
        "metric": METRIC_MFMA if mfma else METRIC,
        "value": head["value"],
        "unit": head["unit"],
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded splitmix64 -> Box-Muller fp64 -> fp32, the BASELINE config recipe)",
        "config": {"workload": head["workload"][:400], "pct_of_peak": head["pct_of_peak"], "cus": cus,
                   "basis": basis,
                   "timing": "per op: median over the timed steps of its dispatches' durations (%s basis), one "
                             "512 MiB flush before every launch; ms_per_step = the sum over the step's ops"
                             % basis},
        "roofline": head["roofline"],
        "cpu_baseline": cpu_top,
        "value_event": head["value_event"],
        "copy_kernel_GBps": copies.get("wm_copy_kernel"),
    }
    if "speedup_vs_cpu_step" in head:
        line["speedup_vs_cpu"] = head["speedup_vs_cpu_step"]
    if "below_70pct" in head:
        line["below_70pct"] = [k[:40] for k in head["below_70pct"][:8]]
    if "parity" in head:
        line["parity"] = _short_parity(head["parity"])
    if len(names) > 1:
        line["configs"] = {nm: compact(recs[nm]) for nm in names[1:]}
    return _fit(line)


def copy_calibration(flush, kt):
    """The 1 GiB copy kernels, streaming (the practical read + write ceiling)
    and cached: GB/s of each.  Under rocprofv3 --pmc their dispatches are the
    byte counters' calibration (1 GiB read + 1 GiB written each)."""
    n_copy = 1 << 28
    src, dst = W.DeviceArray((n_copy,)), W.DeviceArray((n_copy,))
    src.fill(2.0)
    out = {}
    for entry in ("wm_copy_kernel", "wm_copy_kernel_cached"):
        op = Op(entry, lambda e=entry: W.call(e, dst.vp, src.vp, n_copy), 2 * n_copy * F32, entry, n_copy)
        for _ in range(3):
            _launch(op, kt.basis if kt.basis != "external" else "event", flush, kt)
        out[entry] = round(op.bytes / (statistics.median(op.kms or op.ms) * 1e-3) / 1e9, 1)
    src.free()
    dst.free()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--config", default="all", choices=["all"] + sorted(CONFIGS))
    ap.add_argument("--flush-mib", type=int, default=512)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline and parity legs")
    ap.add_argument("--detail", default=None, help="also write the per-op detail JSON to this path")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU; multi-GPU runs are not part of it "
              "(value is the single-GPU throughput).", file=sys.stderr)
        sys.exit(2)

    kt = KTrace()  # before the first HIP call of the process
    if not kt.ok:
        print("bench.py: dispatch tracer not registered (%s); basis %s" % (kt.err, kt.basis),
              file=sys.stderr, flush=True)
    W.call("wm_init", 0)
    cus = W.device_cus()
    flush = W.DeviceArray((args.flush_mib * (1 << 20) // 4,))
    names = ALL if args.config == "all" else [args.config]
    recs, details = {}, {}
    for nm in names:
        print(f"bench.py: {nm} ...", file=sys.stderr, flush=True)
        recs[nm], details[nm] = run_config(nm, args, flush, not args.no_cpu, kt)
        print(f"bench.py: {nm} done: {recs[nm]['value']} {recs[nm]['unit']}, parity "
              f"{recs[nm].get('parity', {}).get('pass', 'n/a')}", file=sys.stderr, flush=True)
    copies = copy_calibration(flush, kt)
    basis = kt.basis
    detail_line = json.dumps({"copy_kernel_GBps": copies, "basis": basis, "configs": details})
    print("bench.py detail: " + detail_line, file=sys.stderr, flush=True)
    if args.detail:
        with open(args.detail, "w") as f:
            f.write(detail_line + "\n")
    print(json.dumps(bench_line(recs[names[0]], recs, names, args, cus, basis, copies)), flush=True)


if __name__ == "__main__":
    main()
