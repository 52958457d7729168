"""TEST INFRASTRUCTURE ONLY: numpy front end of the CPU oracle.

Loads the three builds of oracle/wm_oracle.c (strict fp32, fp64, and the
fp64 "sum of |terms|" magnitude build) and, when present, oracle/_ref's build
of the reference's own core/tensor.cpp.  Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import this package; the product
(whitematter_amd/) never does.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
KINDS = {"f32": ("liboracle_f32.so", np.float32), "f64": ("liboracle_f64.so", np.float64),
         "abs": ("liboracle_abs.so", np.float64), "port": ("liboracle_port.so", np.float32)}
REF_PATH = os.path.join(HERE, "_ref", "libwmref.so")
# the same reference sources built without fast-math (IEEE, no contraction)
REF_IEEE_PATH = os.path.join(HERE, "_ref", "libwmref_ieee.so")

BINARY = {"add": 0, "sub": 1, "mul": 2, "div": 3, "pow": 4, "max": 5, "min": 6}
UNARY = {"relu": 0, "sigmoid": 1, "tanh": 2, "log": 3, "exp": 4, "pows": 5, "sqrt": 6,
         "abs": 7, "clamp": 8, "scale": 9}
REDUCE = {"sum": 0, "mean": 1, "max": 2, "min": 3, "argmax": 4, "argmin": 5}

_libs = {}


def _fp(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else C.c_void_p(0)


def _shape(s):
    return (C.c_int64 * max(1, len(s)))(*[int(v) for v in s]), len(s)


class Oracle:
    """One build of wm_oracle.c; outputs are numpy arrays of its REAL type."""

    def __init__(self, kind: str):
        name, dtype = KINDS[kind]
        path = os.path.join(HERE, name)
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle)")
        self.L = C.CDLL(path)
        self.dtype = np.dtype(dtype)
        self.kind = kind
        for fn in ("or_broadcast_shape", "or_binary", "or_binary_bwd", "or_unary", "or_unary_bwd",
                   "or_reduce", "or_reduce_bwd", "or_softmax", "or_log_softmax", "or_softmax_bwd",
                   "or_log_softmax_bwd", "or_f32_to_f16", "or_f16_to_f32"):
            getattr(self.L, fn).restype = C.c_int

    def broadcast_shape(self, a_shape, b_shape):
        sa, na = _shape(a_shape)
        sb, nb = _shape(b_shape)
        out = (C.c_int64 * 8)()
        nd = C.c_int()
        if self.L.or_broadcast_shape(sa, na, sb, nb, out, C.byref(nd)) != 0:
            raise ValueError("Shapes are not broadcastable")
        return tuple(out[i] for i in range(nd.value))

    def binary(self, op, a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        oshape = self.broadcast_shape(a.shape, b.shape)
        out = np.empty(oshape, self.dtype)
        sa, na = _shape(a.shape)
        sb, nb = _shape(b.shape)
        rc = self.L.or_binary(BINARY[op], _fp(out), _fp(a), sa, na, _fp(b), sb, nb)
        assert rc == 0
        return out

    def binary_bwd(self, op, g, a, b, out=None, need_a=True, need_b=True):
        g = np.ascontiguousarray(g, np.float32)
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        ga = np.zeros(a.shape, self.dtype) if need_a else None
        gb = np.zeros(b.shape, self.dtype) if need_b else None
        o = np.ascontiguousarray(out, np.float32) if out is not None else None
        sa, na = _shape(a.shape)
        sb, nb = _shape(b.shape)
        rc = self.L.or_binary_bwd(BINARY[op], _fp(g), _fp(a), sa, na, _fp(b), sb, nb, _fp(o), _fp(ga), _fp(gb))
        assert rc == 0
        return ga, gb

    def unary(self, op, x, p0=0.0, p1=0.0):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, self.dtype)
        self.L.or_unary(UNARY[op], _fp(out), _fp(x), C.c_int64(x.size), C.c_float(p0), C.c_float(p1))
        return out

    def unary_bwd(self, op, g, x, out, p0=0.0, p1=0.0):
        g = np.ascontiguousarray(g, np.float32)
        x = np.ascontiguousarray(x, np.float32) if x is not None else None
        o = np.ascontiguousarray(out, np.float32) if out is not None else None
        gx = np.zeros(g.shape, self.dtype)
        self.L.or_unary_bwd(UNARY[op], _fp(g), _fp(x), _fp(o), _fp(gx), C.c_int64(g.size),
                            C.c_float(p0), C.c_float(p1))
        return gx

    def reduce(self, op, x, outer, n, inner):
        x = np.ascontiguousarray(x, np.float32)
        val = np.empty((outer, inner), self.dtype)
        idx = np.empty((outer, inner), np.int64)
        rc = self.L.or_reduce(REDUCE[op], _fp(x), C.c_int64(outer), C.c_int64(n), C.c_int64(inner),
                              _fp(val), _fp(idx))
        assert rc == 0
        return val, idx

    def reduce_bwd(self, op, g, idx, outer, n, inner):
        g = np.ascontiguousarray(g, np.float32)
        gx = np.zeros((outer, n, inner), self.dtype)
        i = np.ascontiguousarray(idx, np.int64) if idx is not None else None
        rc = self.L.or_reduce_bwd(REDUCE[op], _fp(g), _fp(i), C.c_int64(outer), C.c_int64(n), C.c_int64(inner),
                                  _fp(gx))
        assert rc == 0
        return gx

    def softmax(self, x, log=False):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, self.dtype)
        fn = self.L.or_log_softmax if log else self.L.or_softmax
        fn(_fp(out), _fp(x), C.c_int64(x.shape[0]), C.c_int64(x.shape[1]))
        return out

    def softmax_bwd(self, g, out, log=False):
        g = np.ascontiguousarray(g, np.float32)
        o = np.ascontiguousarray(out, np.float32)
        gx = np.zeros(g.shape, self.dtype)
        fn = self.L.or_log_softmax_bwd if log else self.L.or_softmax_bwd
        fn(_fp(g), _fp(o), _fp(gx), C.c_int64(g.shape[0]), C.c_int64(g.shape[1]))
        return gx

    def f32_to_f16(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.uint16)
        self.L.or_f32_to_f16(_fp(out), _fp(x), C.c_int64(x.size))
        return out

    def f16_to_f32(self, h):
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(h.shape, np.float32)
        self.L.or_f16_to_f32(_fp(out), _fp(h), C.c_int64(h.size))
        return out

    # ---- parameter updates (float in every build); arrays are updated in
    # place, as the reference's step() does ----------------------------------

    def _optim_sigs(self):
        if getattr(self, "_optim_ready", False):
            return
        L = self.L
        L.or_bias_correction.argtypes = [C.c_float, C.c_int]
        L.or_bias_correction.restype = C.c_float
        L.or_sgd_step.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int64, C.c_float, C.c_float]
        L.or_adam_step.argtypes = [C.c_void_p] * 4 + [C.c_int64] + [C.c_float] * 7 + [C.c_int]
        L.or_rmsprop_step.argtypes = [C.c_void_p] * 4 + [C.c_int64] + [C.c_float] * 5
        L.or_grad_sumsq.argtypes = [C.c_void_p, C.c_int64]
        L.or_grad_sumsq.restype = C.c_double
        L.or_clip_grad_value.argtypes = [C.c_void_p, C.c_int64, C.c_float]
        L.or_unscale_tensor.argtypes = [C.c_void_p, C.c_int64, C.c_float]
        L.or_unscale_tensor.restype = C.c_int64
        self._optim_ready = True

    @staticmethod
    def _f32(a):
        assert a is None or (a.dtype == np.float32 and a.flags.c_contiguous), "float32 C-contiguous arrays"
        return a

    def bias_correction(self, beta, t):
        self._optim_sigs()
        return np.float32(self.L.or_bias_correction(beta, t))

    def sgd_step(self, p, g, vel, lr, momentum):
        self._optim_sigs()
        self.L.or_sgd_step(_fp(self._f32(p)), _fp(self._f32(g)), _fp(self._f32(vel)), p.size, lr, momentum)

    def adam_step(self, p, g, m, v, lr, beta1, beta2, eps, bc1, bc2, weight_decay=0.0, decoupled=False):
        self._optim_sigs()
        self.L.or_adam_step(_fp(self._f32(p)), _fp(self._f32(g)), _fp(self._f32(m)), _fp(self._f32(v)), p.size, lr,
                            beta1, beta2, eps, bc1, bc2, weight_decay, int(decoupled))

    def rmsprop_step(self, p, g, v, buf, lr, alpha, eps, momentum, weight_decay):
        self._optim_sigs()
        self.L.or_rmsprop_step(_fp(self._f32(p)), _fp(self._f32(g)), _fp(self._f32(v)), _fp(self._f32(buf)), p.size,
                               lr, alpha, eps, momentum, weight_decay)

    def grad_sumsq(self, g):
        self._optim_sigs()
        g = np.ascontiguousarray(g, np.float32)
        return self.L.or_grad_sumsq(_fp(g), g.size)

    def clip_grad_value(self, g, c):
        self._optim_sigs()
        self.L.or_clip_grad_value(_fp(self._f32(g)), g.size, c)

    def unscale_tensor(self, g, inv_scale):
        self._optim_sigs()
        return self.L.or_unscale_tensor(_fp(self._f32(g)), g.size, inv_scale)


# ---- losses (core/loss.cpp) --------------------------------------------------

LOSS_KINDS = {"smooth_l1": 0, "bce": 1, "bce_logits": 2, "kldiv": 3, "kldiv_log": 4, "binary_focal": 5}


def _loss_sigs(o):
    if getattr(o, "_loss_ready", False):
        return
    L, vp, i64, f = o.L, C.c_void_p, C.c_int64, C.c_float
    L.or_cross_entropy.argtypes = [vp, vp, i64, i64, vp]
    L.or_cross_entropy_bwd.argtypes = [vp, vp, i64, i64, f, vp]
    L.or_nll.argtypes = [vp, vp, i64, i64, vp]
    L.or_nll_bwd.argtypes = [vp, i64, i64, f, vp]
    L.or_focal.argtypes = [vp, vp, i64, i64, f, f, vp]
    L.or_focal_bwd.argtypes = [vp, vp, i64, i64, f, f, f, vp]
    L.or_pointwise_loss.argtypes = [C.c_int, vp, vp, i64, f, f, f, vp]
    L.or_pointwise_loss_bwd.argtypes = [C.c_int, vp, vp, i64, f, f, f, f, vp]
    o._loss_ready = True


def _f32c(a):
    return np.ascontiguousarray(a, np.float32)


def _loss_methods():
    """Loss entry points of an Oracle build: each forward returns the loss as
    a REAL scalar, each backward a fresh gradient array (the closure's
    contribution to a zero gradient)."""

    def cross_entropy(self, x, labels):
        _loss_sigs(self)
        x, labels = _f32c(x), _f32c(labels)
        out = np.zeros(1, self.dtype)
        self.L.or_cross_entropy(_fp(x), _fp(labels), x.shape[0], x.shape[1], _fp(out))
        return out[0]

    def cross_entropy_bwd(self, x, labels, loss_grad=1.0):
        _loss_sigs(self)
        x, labels = _f32c(x), _f32c(labels)
        gx = np.zeros(x.shape, self.dtype)
        self.L.or_cross_entropy_bwd(_fp(x), _fp(labels), x.shape[0], x.shape[1], loss_grad, _fp(gx))
        return gx

    def nll(self, x, labels):
        _loss_sigs(self)
        x, labels = _f32c(x), _f32c(labels)
        out = np.zeros(1, self.dtype)
        self.L.or_nll(_fp(x), _fp(labels), x.shape[0], x.shape[1], _fp(out))
        return out[0]

    def nll_bwd(self, shape, labels, loss_grad=1.0):
        _loss_sigs(self)
        labels = _f32c(labels)
        gx = np.zeros(shape, self.dtype)
        self.L.or_nll_bwd(_fp(labels), shape[0], shape[1], loss_grad, _fp(gx))
        return gx

    def focal(self, x, labels, gamma=2.0, alpha=-1.0):
        _loss_sigs(self)
        x, labels = _f32c(x), _f32c(labels)
        out = np.zeros(1, self.dtype)
        self.L.or_focal(_fp(x), _fp(labels), x.shape[0], x.shape[1], gamma, alpha, _fp(out))
        return out[0]

    def focal_bwd(self, x, labels, gamma=2.0, alpha=-1.0, loss_grad=1.0):
        _loss_sigs(self)
        x, labels = _f32c(x), _f32c(labels)
        gx = np.zeros(x.shape, self.dtype)
        self.L.or_focal_bwd(_fp(x), _fp(labels), x.shape[0], x.shape[1], gamma, alpha, loss_grad, _fp(gx))
        return gx

    def pointwise_loss(self, kind, x, y, p0=0.0, p1=0.0, denom=None):
        _loss_sigs(self)
        x, y = _f32c(x), _f32c(y)
        out = np.zeros(1, self.dtype)
        d = float(x.size) if denom is None else float(denom)
        self.L.or_pointwise_loss(LOSS_KINDS[kind], _fp(x), _fp(y), x.size, p0, p1, d, _fp(out))
        return out[0]

    def pointwise_loss_bwd(self, kind, x, y, p0=0.0, p1=0.0, denom=None, loss_grad=1.0):
        _loss_sigs(self)
        x, y = _f32c(x), _f32c(y)
        gx = np.zeros(x.shape, self.dtype)
        d = float(x.size) if denom is None else float(denom)
        self.L.or_pointwise_loss_bwd(LOSS_KINDS[kind], _fp(x), _fp(y), x.size, p0, p1, d, loss_grad, _fp(gx))
        return gx

    return {k: v for k, v in locals().items() if callable(v)}


for _name, _fn in _loss_methods().items():
    setattr(Oracle, _name, _fn)


# ---- normalisation layers and the attention softmax (core/layer.cpp) -----------

def _layer_sigs(o):
    if getattr(o, "_layer_ready", False):
        return
    L, vp, i64, f = o.L, C.c_void_p, C.c_int64, C.c_float
    L.or_layernorm.argtypes = [vp, vp, vp, i64, i64, f, vp, vp, vp]
    L.or_layernorm_bwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, vp, vp, vp]
    L.or_batchnorm2d.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, f, f, C.c_int, vp, vp, vp]
    L.or_batchnorm2d_bwd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, vp, vp, vp]
    L.or_attention_softmax.argtypes = [vp, vp, i64, i64, i64, i64, i64, vp]
    L.or_attention_softmax_bwd.argtypes = [vp, vp, i64, i64, vp]
    o._layer_ready = True


def _layer_methods():
    """LayerNorm / BatchNorm2d / attention-softmax entry points of an Oracle
    build.  Saved statistics come back as REAL arrays; the backward takes
    them as fp32 (the values a closure captures).  Gradients are fresh
    arrays (the closure's contribution to zero gradients)."""

    def layernorm(self, x, gamma, beta, eps=1e-5):
        _layer_sigs(self)
        x, gamma, beta = _f32c(x), _f32c(gamma), _f32c(beta)
        n = gamma.size
        rows = x.size // n
        y = np.zeros(x.shape, self.dtype)
        mean, inv = np.zeros(rows, self.dtype), np.zeros(rows, self.dtype)
        self.L.or_layernorm(_fp(x), _fp(gamma), _fp(beta), rows, n, eps, _fp(y), _fp(mean), _fp(inv))
        return y, mean, inv

    def layernorm_bwd(self, g, x, gamma, mean, inv):
        _layer_sigs(self)
        g, x, gamma, mean, inv = _f32c(g), _f32c(x), _f32c(gamma), _f32c(mean), _f32c(inv)
        n = gamma.size
        rows = x.size // n
        gx = np.zeros(x.shape, self.dtype)
        dg, db = np.zeros(n, self.dtype), np.zeros(n, self.dtype)
        self.L.or_layernorm_bwd(_fp(g), _fp(x), _fp(gamma), _fp(mean), _fp(inv), rows, n, _fp(gx), _fp(dg), _fp(db))
        return gx, dg, db

    def batchnorm2d(self, x, gamma, beta, running_mean, running_var, eps=1e-5, momentum=0.1, training=True):
        """x [B, C, H, W] (or [B, C, S]); returns (y, mean, inv_std,
        running_mean', running_var')."""
        _layer_sigs(self)
        x, gamma, beta = _f32c(x), _f32c(gamma), _f32c(beta)
        B, Cc = x.shape[0], x.shape[1]
        S = x.size // (B * Cc) if B * Cc else 0
        rm, rv = _f32c(running_mean).copy(), _f32c(running_var).copy()
        y = np.zeros(x.shape, self.dtype)
        mean, inv = np.zeros(Cc, self.dtype), np.zeros(Cc, self.dtype)
        self.L.or_batchnorm2d(_fp(x), _fp(gamma), _fp(beta), _fp(rm), _fp(rv), B, Cc, S, eps, momentum,
                              int(training), _fp(y), _fp(mean), _fp(inv))
        return y, mean, inv, rm, rv

    def batchnorm2d_bwd(self, g, x, gamma, mean, inv):
        _layer_sigs(self)
        g, x, gamma, mean, inv = _f32c(g), _f32c(x), _f32c(gamma), _f32c(mean), _f32c(inv)
        B, Cc = x.shape[0], x.shape[1]
        S = x.size // (B * Cc) if B * Cc else 0
        gx = np.zeros(x.shape, self.dtype)
        dg, db = np.zeros(Cc, self.dtype), np.zeros(Cc, self.dtype)
        self.L.or_batchnorm2d_bwd(_fp(g), _fp(x), _fp(gamma), _fp(mean), _fp(inv), B, Cc, S, _fp(gx), _fp(dg),
                                  _fp(db))
        return gx, dg, db

    def attention_softmax(self, scores, mask=None):
        """scores [B, H, tq, tk]; mask None or [Bm, 1, tq, tk]."""
        _layer_sigs(self)
        scores = _f32c(scores)
        B, H, tq, tk = scores.shape
        m = _f32c(mask) if mask is not None else None
        attn = np.zeros(scores.shape, self.dtype)
        self.L.or_attention_softmax(_fp(scores), _fp(m), m.shape[0] if m is not None else 0, B, H, tq, tk,
                                    _fp(attn))
        return attn

    def attention_softmax_bwd(self, attn, d_attn):
        _layer_sigs(self)
        attn, d_attn = _f32c(attn), _f32c(d_attn)
        tk = attn.shape[-1]
        ds = np.zeros(attn.shape, self.dtype)
        self.L.or_attention_softmax_bwd(_fp(attn), _fp(d_attn), attn.size // tk, tk, _fp(ds))
        return ds

    def dropout_mask(self, n, p, seed):
        self.L.or_dropout_mask.argtypes = [C.c_void_p, C.c_int64, C.c_float, C.c_uint64]
        mask = np.zeros(n, np.float32)
        self.L.or_dropout_mask(_fp(mask), n, p, seed)
        return mask

    return {k: v for k, v in locals().items() if callable(v)}


for _name, _fn in _layer_methods().items():
    setattr(Oracle, _name, _fn)


def _gemm_sigs(o):
    if getattr(o, "_gemm_ready", False):
        return
    L, vp, i64 = o.L, C.c_void_p, C.c_int64
    L.or_bmm.argtypes = [vp, vp, i64, i64, i64, i64, vp]
    L.or_bmm_bwd.argtypes = [vp, vp, vp, i64, i64, i64, i64, vp, vp]
    L.or_mha_forward.argtypes = [vp] * 4 + [i64] + [vp] * 8 + [i64] * 5 + [vp] * 6
    L.or_mha_backward.argtypes = [vp] * 13 + [i64] * 5 + [vp] * 11
    L.or_mha_backward.restype = C.c_int
    o._gemm_ready = True


def _gemm_methods():
    """Matrix products (Tensor::matmul / bmm) and MultiHeadAttention of an
    Oracle build.  Inputs are fp32; results are REAL arrays."""

    def bmm(self, a, b):
        """a [batch, m, k] @ b [batch, k, n] (2-D operands: one product)."""
        _gemm_sigs(self)
        a, b = _f32c(a), _f32c(b)
        two_d = a.ndim == 2
        a3, b3 = (a[None], b[None]) if two_d else (a, b)
        P, m, k = a3.shape
        n = b3.shape[2]
        c = np.zeros((P, m, n), self.dtype)
        self.L.or_bmm(_fp(a3), _fp(b3), P, m, k, n, _fp(c))
        return c[0] if two_d else c

    matmul = bmm

    def bmm_bwd(self, g, a, b, ga0=None, gb0=None, need_a=True, need_b=True):
        """(ga0 + g @ b^T, gb0 + a^T @ g) per problem; ga0 / gb0 default to 0."""
        _gemm_sigs(self)
        g, a, b = _f32c(g), _f32c(a), _f32c(b)
        two_d = a.ndim == 2
        g3, a3, b3 = (g[None], a[None], b[None]) if two_d else (g, a, b)
        P, m, k = a3.shape
        n = b3.shape[2]
        ga = (np.array(ga0, self.dtype).reshape(a3.shape) if ga0 is not None else np.zeros(a3.shape, self.dtype))
        gb = (np.array(gb0, self.dtype).reshape(b3.shape) if gb0 is not None else np.zeros(b3.shape, self.dtype))
        self.L.or_bmm_bwd(_fp(g3), _fp(a3), _fp(b3), P, m, k, n, _fp(ga) if need_a else None,
                          _fp(gb) if need_b else None)
        ga, gb = (ga[0], gb[0]) if two_d else (ga, gb)
        return (ga if need_a else None), (gb if need_b else None)

    matmul_bwd = bmm_bwd

    def mha_forward(self, q, k, v, params, heads, mask=None):
        """MultiHeadAttention::forward.  params = (Wq, Wk, Wv, Wo, bq, bk, bv,
        bo).  Returns dict(out, attn, Q, K, V, ctx).  (The abs build's values
        are not error scales here: its softmax is not a sum of terms.)"""
        _gemm_sigs(self)
        q, k, v = _f32c(q), _f32c(k), _f32c(v)
        ps = [_f32c(x) for x in params]
        B, Sq, E = q.shape
        Sk = k.shape[1]
        m = _f32c(mask) if mask is not None else None
        r = {"out": np.zeros((B, Sq, E), self.dtype), "attn": np.zeros((B, heads, Sq, Sk), self.dtype),
             "Q": np.zeros((B, Sq, E), self.dtype), "K": np.zeros((B, Sk, E), self.dtype),
             "V": np.zeros((B, Sk, E), self.dtype), "ctx": np.zeros((B, Sq, E), self.dtype)}
        self.L.or_mha_forward(_fp(q), _fp(k), _fp(v), _fp(m), m.shape[0] if m is not None else 0,
                              *[_fp(x) for x in ps], B, Sq, Sk, E, heads,
                              *[_fp(r[x]) for x in ("out", "attn", "Q", "K", "V", "ctx")])
        return r

    def mha_backward(self, dout, q, k, v, params, heads, saved, need=(True, True, True), alias=False):
        """The closure: dict of gradients (gWq, gWk, gWv, gWo, gbq, gbk, gbv,
        gbo, gq, gk, gv) added to zeros.  saved = the forward's Q, K, V, attn,
        ctx (fp32).  alias: q, k, v are one tensor (self attention), whose
        gradient collects all three contributions in 'gq'."""
        _gemm_sigs(self)
        dout, q, k, v = _f32c(dout), _f32c(q), _f32c(k), _f32c(v)
        Wq, Wk, Wv, Wo = [_f32c(x) for x in params[:4]]
        sv = [_f32c(saved[x]) for x in ("Q", "K", "V", "attn", "ctx")]
        B, Sq, E = q.shape
        Sk = k.shape[1]
        z = {n: np.zeros((E, E), self.dtype) for n in ("gWq", "gWk", "gWv", "gWo")}
        z.update({n: np.zeros(E, self.dtype) for n in ("gbq", "gbk", "gbv", "gbo")})
        z["gq"] = np.zeros(q.shape, self.dtype) if need[0] else None
        if alias:
            z["gk"] = z["gq"] if need[1] else None
            z["gv"] = z["gq"] if need[2] else None
        else:
            z["gk"] = np.zeros(k.shape, self.dtype) if need[1] else None
            z["gv"] = np.zeros(v.shape, self.dtype) if need[2] else None
        rc = self.L.or_mha_backward(_fp(dout), _fp(q), _fp(k), _fp(v), _fp(Wq), _fp(Wk), _fp(Wv), _fp(Wo),
                                    *[_fp(x) for x in sv], B, Sq, Sk, E, heads,
                                    *[_fp(z[n]) for n in ("gWq", "gWk", "gWv", "gWo", "gbq", "gbk", "gbv", "gbo",
                                                          "gq", "gk", "gv")])
        assert rc == 0
        return z

    return {k: v for k, v in locals().items() if callable(v)}


for _name, _fn in _gemm_methods().items():
    setattr(Oracle, _name, _fn)


def get(kind: str) -> Oracle:
    if kind not in _libs:
        _libs[kind] = Oracle(kind)
    return _libs[kind]


# ---- the reference itself (oracle/_ref, built from /root/reference) --------

class RefTensor:
    """A reference Tensor (core/tensor.h) behind oracle/_ref/libwmref.so."""

    def __init__(self, L, h):
        self.L, self.h = L, h

    @property
    def shape(self):
        nd = self.L.wmref_ndim(self.h)
        s = (C.c_int64 * max(1, nd))()
        self.L.wmref_shape(self.h, s)
        return tuple(s[i] for i in range(nd))

    def data(self):
        out = np.empty(self.L.wmref_numel(self.h), np.float32)
        self.L.wmref_get_data(self.h, _fp(out))
        return out.reshape(self.shape)

    def requires_grad(self) -> bool:
        return bool(self.L.wmref_requires_grad(self.h))

    def grad(self):
        out = np.empty(self.L.wmref_numel(self.h), np.float32)
        if not self.L.wmref_get_grad(self.h, _fp(out)):
            return None
        return out.reshape(self.shape)

    def run_grad_fn(self, g):
        g = np.ascontiguousarray(g, np.float32)
        return self.L.wmref_run_grad_fn(self.h, _fp(g))

    def set_grad(self, g):
        g = np.ascontiguousarray(g, np.float32)
        return self.L.wmref_set_grad(self.h, _fp(g))

    def set_data(self, v):
        v = np.ascontiguousarray(v, np.float32)
        assert v.size == self.L.wmref_numel(self.h)
        self.L.wmref_set_data(self.h, _fp(v))

    def call_grad_fn(self):
        self.L.wmref_call_grad_fn(self.h)

    def backward(self):
        self.L.wmref_backward(self.h)

    def __del__(self):
        try:
            self.L.wmref_free(self.h)
        except Exception:
            pass


class RefOptimizer:
    """A reference optimizer (core/optimizer.h) over RefTensor parameters."""

    def __init__(self, L, h, params):
        self.L, self.h, self.params = L, h, params

    def step(self):
        self.L.wmref_optim_step(self.h)

    def __del__(self):
        try:
            self.L.wmref_optim_free(self.h)
        except Exception:
            pass


class RefModule:
    """A reference Module (core/layer.h) behind oracle/_ref/libwmref.so."""

    def __init__(self, L, h):
        self.L, self.h = L, h

    def forward(self, x: RefTensor) -> RefTensor:
        return RefTensor(self.L, self.L.wmref_module_forward(self.h, x.h))

    def mha(self, q: RefTensor, k: RefTensor, v: RefTensor, mask: Optional[RefTensor] = None) -> RefTensor:
        return RefTensor(self.L, self.L.wmref_mha_forward(self.h, q.h, k.h, v.h, mask.h if mask else None))

    def params(self):
        return [RefTensor(self.L, self.L.wmref_module_param(self.h, i))
                for i in range(self.L.wmref_module_nparams(self.h))]

    def buffer(self, which=0) -> RefTensor:
        return RefTensor(self.L, self.L.wmref_module_buffer(self.h, which))

    def train(self, on=True):
        self.L.wmref_module_train(self.h, int(on))

    def __del__(self):
        try:
            self.L.wmref_module_free(self.h)
        except Exception:
            pass


class Reference:
    def __init__(self, path: str = REF_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle with /root/reference present)")
        L = C.CDLL(path)
        for fn in ("wmref_new", "wmref_binary", "wmref_unary", "wmref_reduce", "wmref_softmax", "wmref_reshape"):
            getattr(L, fn).restype = C.c_void_p
        L.wmref_new.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int]
        L.wmref_binary.argtypes = [C.c_int, C.c_void_p, C.c_void_p]
        L.wmref_matmul.restype = C.c_void_p
        L.wmref_matmul.argtypes = [C.c_int, C.c_void_p, C.c_void_p]
        L.wmref_requires_grad.argtypes = [C.c_void_p]
        L.wmref_save_tensor.argtypes = [C.c_void_p, C.c_char_p]
        L.wmref_load_tensor.argtypes = [C.c_char_p]
        L.wmref_load_tensor.restype = C.c_void_p
        for fn in ("wmref_save_model", "wmref_load_model", "wmref_save_optimizer", "wmref_load_optimizer"):
            getattr(L, fn).argtypes = [C.c_void_p, C.c_char_p]
        L.wmref_save_checkpoint.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p, C.c_int, C.c_float, C.c_float]
        L.wmref_load_checkpoint.argtypes = [C.c_char_p, C.c_void_p, C.c_void_p, C.POINTER(C.c_int),
                                            C.POINTER(C.c_float), C.POINTER(C.c_float)]
        L.wmref_unary.argtypes = [C.c_int, C.c_void_p, C.c_float, C.c_float]
        L.wmref_reduce.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_int]
        L.wmref_softmax.argtypes = [C.c_int, C.c_void_p, C.c_int]
        L.wmref_reshape.argtypes = [C.c_void_p, C.c_void_p, C.c_int]
        for fn in ("wmref_free", "wmref_backward", "wmref_zero_grad"):
            getattr(L, fn).argtypes = [C.c_void_p]
            getattr(L, fn).restype = None
        L.wmref_ndim.argtypes = [C.c_void_p]
        L.wmref_ndim.restype = C.c_int
        L.wmref_shape.argtypes = [C.c_void_p, C.c_void_p]
        L.wmref_shape.restype = None
        L.wmref_numel.argtypes = [C.c_void_p]
        L.wmref_numel.restype = C.c_int64
        L.wmref_get_data.argtypes = [C.c_void_p, C.c_void_p]
        L.wmref_get_data.restype = None
        L.wmref_get_grad.argtypes = [C.c_void_p, C.c_void_p]
        L.wmref_get_grad.restype = C.c_int
        L.wmref_run_grad_fn.argtypes = [C.c_void_p, C.c_void_p]
        L.wmref_run_grad_fn.restype = C.c_int
        L.wmref_set_grad.argtypes = [C.c_void_p, C.c_void_p]
        L.wmref_set_grad.restype = C.c_int
        L.wmref_call_grad_fn.argtypes = [C.c_void_p]
        L.wmref_call_grad_fn.restype = None
        L.wmref_set_grad_enabled.argtypes = [C.c_int]
        L.wmref_set_grad_enabled.restype = None
        L.wmref_f32_to_f16.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.wmref_f32_to_f16.restype = None
        L.wmref_f16_to_f32.argtypes = [C.c_void_p, C.c_void_p, C.c_int64]
        L.wmref_f16_to_f32.restype = None
        L.wmref_optim_new.argtypes = [C.c_int, C.c_void_p, C.c_int] + [C.c_float] * 5
        L.wmref_optim_new.restype = C.c_void_p
        for fn in ("wmref_optim_step", "wmref_optim_free"):
            getattr(L, fn).argtypes = [C.c_void_p]
            getattr(L, fn).restype = None
        L.wmref_grad_norm.argtypes = [C.c_void_p, C.c_int]
        L.wmref_grad_norm.restype = C.c_float
        L.wmref_clip_grad_norm.argtypes = [C.c_void_p, C.c_int, C.c_float]
        L.wmref_clip_grad_norm.restype = None
        L.wmref_clip_grad_value.argtypes = [C.c_void_p, C.c_int, C.c_float]
        L.wmref_clip_grad_value.restype = None
        L.wmref_unscale.argtypes = [C.c_void_p, C.c_int, C.c_float]
        L.wmref_unscale.restype = C.c_int
        L.wmref_loss.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_float, C.c_float]
        L.wmref_loss.restype = C.c_void_p
        L.wmref_module_new.argtypes = [C.c_int, C.c_void_p, C.c_int, C.c_float, C.c_float]
        L.wmref_module_new.restype = C.c_void_p
        L.wmref_module_free.argtypes = [C.c_void_p]
        L.wmref_module_free.restype = None
        L.wmref_module_train.argtypes = [C.c_void_p, C.c_int]
        L.wmref_module_train.restype = None
        L.wmref_module_forward.argtypes = [C.c_void_p, C.c_void_p]
        L.wmref_module_forward.restype = C.c_void_p
        L.wmref_mha_forward.argtypes = [C.c_void_p] * 5
        L.wmref_mha_forward.restype = C.c_void_p
        L.wmref_module_nparams.argtypes = [C.c_void_p]
        L.wmref_module_nparams.restype = C.c_int
        L.wmref_module_param.argtypes = [C.c_void_p, C.c_int]
        L.wmref_module_param.restype = C.c_void_p
        L.wmref_module_buffer.argtypes = [C.c_void_p, C.c_int]
        L.wmref_module_buffer.restype = C.c_void_p
        L.wmref_set_data.argtypes = [C.c_void_p, C.c_void_p]
        L.wmref_set_data.restype = None
        L.wmref_causal_mask.argtypes = [C.c_int64]
        L.wmref_causal_mask.restype = C.c_void_p
        self.L = L

    @staticmethod
    def _handles(params):
        return (C.c_void_p * max(1, len(params)))(*[p.h for p in params]), len(params)

    def optimizer(self, kind, params, lr, a=0.0, b=0.0, c=0.0, d=0.0):
        """kind: "sgd" (a = momentum), "adam" (a, b, c = beta1, beta2, eps),
        "adamw" (+ d = weight_decay), "rmsprop" (a = alpha, b = eps,
        c = momentum, d = weight_decay).  Returns a RefOptimizer."""
        code = {"sgd": 0, "adam": 1, "adamw": 2, "rmsprop": 3}[kind]
        hs, n = self._handles(params)
        return RefOptimizer(self.L, self.L.wmref_optim_new(code, hs, n, lr, a, b, c, d), params)

    def grad_norm(self, params):
        hs, n = self._handles(params)
        return np.float32(self.L.wmref_grad_norm(hs, n))

    def clip_grad_norm(self, params, max_norm):
        hs, n = self._handles(params)
        self.L.wmref_clip_grad_norm(hs, n, max_norm)

    def clip_grad_value(self, params, c):
        hs, n = self._handles(params)
        self.L.wmref_clip_grad_value(hs, n, c)

    def unscale(self, params, scale):
        """GradScaler(scale).unscale(...); returns True when it found inf/NaN."""
        hs, n = self._handles(params)
        return bool(self.L.wmref_unscale(hs, n, scale))

    LOSSES = {"mse": 0, "l1": 1, "smooth_l1": 2, "cross_entropy": 3, "nll": 4, "bce": 5, "bce_logits": 6,
              "kldiv": 7, "focal": 8, "binary_focal": 9}

    def loss(self, kind, pred, target, p0=0.0, p1=0.0, pred_shape=None, target_shape=None):
        """Forward and backward of the reference loss class `kind` on fresh
        tensors: returns (loss value, prediction gradient).  For "kldiv",
        p0 != 0 selects log_target; for the focal losses p0 = gamma and
        p1 = alpha; for "smooth_l1" p0 = beta."""
        tp = self.tensor(pred, True, pred_shape)
        tt = self.tensor(target, False, target_shape)
        tl = RefTensor(self.L, self.L.wmref_loss(self.LOSSES[kind], tp.h, tt.h, p0, p1))
        value = np.float32(tl.data()[0])
        tl.backward()
        return value, tp.grad()

    MODULES = {"layernorm": 0, "batchnorm2d": 1, "mha": 2, "linear": 3}

    def module(self, kind, shape, p0=1e-5, p1=0.1) -> RefModule:
        """LayerNorm(shape, eps=p0), BatchNorm2d(shape[0], eps=p0,
        momentum=p1) or MultiHeadAttention(shape[0], shape[1])."""
        sa, nd = _shape(shape)
        return RefModule(self.L, self.L.wmref_module_new(self.MODULES[kind], sa, nd, p0, p1))

    def causal_mask(self, seq_len) -> RefTensor:
        return RefTensor(self.L, self.L.wmref_causal_mask(seq_len))

    def tensor(self, data, requires_grad=False, shape: Optional[Sequence[int]] = None) -> RefTensor:
        data = np.ascontiguousarray(data, np.float32)
        s = tuple(shape) if shape is not None else data.shape
        sa, nd = _shape(s)
        return RefTensor(self.L, self.L.wmref_new(_fp(data), sa, nd, int(requires_grad)))

    def binary(self, op, a: RefTensor, b: RefTensor) -> RefTensor:
        return RefTensor(self.L, self.L.wmref_binary(BINARY[op], a.h, b.h))

    def matmul(self, a: RefTensor, b: RefTensor) -> RefTensor:
        return RefTensor(self.L, self.L.wmref_matmul(0, a.h, b.h))

    # core/serialize.h, the reference's own file writers and readers
    def save_tensor(self, t: RefTensor, path: str) -> bool:
        return bool(self.L.wmref_save_tensor(t.h, path.encode()))

    def load_tensor(self, path: str) -> Optional[RefTensor]:
        h = self.L.wmref_load_tensor(path.encode())
        return RefTensor(self.L, h) if h else None

    def save_model(self, m: "RefModule", path: str) -> bool:
        return bool(self.L.wmref_save_model(m.h, path.encode()))

    def load_model(self, m: "RefModule", path: str) -> bool:
        return bool(self.L.wmref_load_model(m.h, path.encode()))

    def save_optimizer(self, o, path: str) -> bool:
        return bool(self.L.wmref_save_optimizer(o.h, path.encode()))

    def load_optimizer(self, o, path: str) -> bool:
        return bool(self.L.wmref_load_optimizer(o.h, path.encode()))

    def save_checkpoint(self, path: str, m: "RefModule", o, epoch: int, loss: float = 0.0, acc: float = 0.0) -> bool:
        return bool(self.L.wmref_save_checkpoint(path.encode(), m.h, o.h if o else None, epoch, loss, acc))

    def load_checkpoint(self, path: str, m: "RefModule", o):
        e, l_, a = C.c_int(), C.c_float(), C.c_float()
        ok = self.L.wmref_load_checkpoint(path.encode(), m.h, o.h if o else None, C.byref(e), C.byref(l_),
                                          C.byref(a))
        return bool(ok), e.value, l_.value, a.value

    def bmm(self, a: RefTensor, b: RefTensor) -> RefTensor:
        return RefTensor(self.L, self.L.wmref_matmul(1, a.h, b.h))

    # 0 relu .. 8 clamp as in UNARY; 9 mul(s), 10 div(s), 11 neg
    def unary(self, op, x: RefTensor, p0=0.0, p1=0.0) -> RefTensor:
        code = {"mul": 9, "divs": 10, "neg": 11}.get(op, UNARY.get(op))
        return RefTensor(self.L, self.L.wmref_unary(code, x.h, p0, p1))

    def reduce(self, op, x: RefTensor, dim: int, keepdim: bool) -> RefTensor:
        return RefTensor(self.L, self.L.wmref_reduce(REDUCE[op], x.h, dim, int(keepdim)))

    def softmax(self, x: RefTensor, log=False, dim=-1) -> RefTensor:
        return RefTensor(self.L, self.L.wmref_softmax(int(log), x.h, dim))

    def reshape(self, x: RefTensor, shape) -> RefTensor:
        sa, nd = _shape(shape)
        return RefTensor(self.L, self.L.wmref_reshape(x.h, sa, nd))

    def f32_to_f16(self, x):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.uint16)
        self.L.wmref_f32_to_f16(_fp(x), _fp(out), x.size)
        return out

    def f16_to_f32(self, h):
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(h.shape, np.float32)
        self.L.wmref_f16_to_f32(_fp(h), _fp(out), h.size)
        return out


_ref = None


def reference() -> Optional[Reference]:
    """The compiled reference, or None when oracle/_ref is not built."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        _ref = Reference()
    return _ref


# ---- comparison helpers ------------------------------------------------------

def ulp_distance(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """Distance in fp32 ulps between fp32 arrays (NaN pairs count 0)."""
    xi = np.ascontiguousarray(x, np.float32).view(np.int32).astype(np.int64)
    yi = np.ascontiguousarray(y, np.float32).view(np.int32).astype(np.int64)
    # Map to a monotone integer line.
    xi = np.where(xi < 0, -(xi & 0x7FFFFFFF), xi)
    yi = np.where(yi < 0, -(yi & 0x7FFFFFFF), yi)
    d = np.abs(xi - yi)
    both_nan = np.isnan(x) & np.isnan(y)
    return np.where(both_nan, 0, d)


def ulp_vs_f64(x32: np.ndarray, ref64: np.ndarray) -> np.ndarray:
    """|x32 - ref64| in units of the fp32 ulp at ref64 (NaN/inf handled)."""
    x = np.asarray(x32, np.float64)
    r = np.asarray(ref64, np.float64)
    # Exact values beyond fp32's range round to +-inf (round-to-nearest
    # overflows at FLT_MAX + half an ulp = 2^128 - 2^103).
    r = np.where(np.abs(r) >= 2.0 ** 128 - 2.0 ** 103, np.copysign(np.inf, r), r)
    fin = np.isfinite(r)
    ar = np.where(fin, np.abs(r), 1.0).astype(np.float32)
    # fp32 ulp at |r|: spacing of the float nearest below/at |r|.
    ulp = np.spacing(ar).astype(np.float64)
    ulp = np.maximum(ulp, np.float64(np.float32(2.0 ** -149)))
    d = np.abs(x - r) / ulp
    same_special = (~fin) & ((np.isnan(r) & np.isnan(x)) | (r == x))
    d = np.where(fin, d, np.where(same_special, 0.0, np.inf))
    return d


def bit_equal(x: np.ndarray, y: np.ndarray) -> bool:
    """Bitwise equality, except that any NaN matches any NaN."""
    x = np.ascontiguousarray(x, np.float32)
    y = np.ascontiguousarray(y, np.float32)
    if x.shape != y.shape:
        return False
    xn, yn = np.isnan(x), np.isnan(y)
    if not np.array_equal(xn, yn):
        return False
    return bool(np.array_equal(x.view(np.uint32)[~xn], y.view(np.uint32)[~yn]))


def equal_modulo_zero_sign(x: np.ndarray, y: np.ndarray) -> bool:
    """bit_equal, except that -0.0 and +0.0 match.  The reference's own build
    uses -ffast-math (which includes -fno-signed-zeros), so the sign of a zero
    returned by its max/min is not defined by the source semantics."""
    x = np.where(np.asarray(x, np.float32) == 0, np.float32(0), x)
    y = np.where(np.asarray(y, np.float32) == 0, np.float32(0), y)
    return bit_equal(x, y)


def close_scaled(x, ref64, scale64, rtol=1e-5, atol=0.0):
    """|x - ref| <= rtol * max(|ref|, scale) + atol elementwise, NaN == NaN.
    Returns (ok, worst ratio)."""
    x = np.asarray(x, np.float64)
    r = np.asarray(ref64, np.float64)
    s = np.maximum(np.abs(r), np.abs(np.asarray(scale64, np.float64)))
    nan_ok = np.array_equal(np.isnan(x), np.isnan(r))
    fin = np.isfinite(r) & np.isfinite(x)
    inf_ok = np.array_equal(np.where(np.isinf(r), r, 0), np.where(np.isinf(x), x, 0))
    err = np.abs(x - r)
    lim = rtol * s + atol
    ratio = np.where(fin, err / np.maximum(lim, 1e-300), 0.0)
    worst = float(ratio.max()) if ratio.size else 0.0
    return bool(nan_ok and inf_ok and worst <= 1.0), worst
