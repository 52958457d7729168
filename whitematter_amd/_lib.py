"""ctypes binding of libwm_hip.so (the C ABI declared in include/*.h).

The library is the product: every call here launches hand-written HIP
kernels on the GPU.  There is deliberately no CPU fallback -- if the shared
library is missing or cannot be loaded, ``lib()`` raises.

Device memory is owned by the library's caching allocator (``wm_alloc``);
``DeviceArray`` wraps one allocation together with its numpy dtype and shape.
PyTorch is not used: its ROCm wheel ships its own HIP runtime, and mixing two
runtimes in one process would split device state.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libwm_hip.so")

# enum wm_binary_op
ADD, SUB, MUL, DIV, POW, MAX, MIN = range(7)
BINARY_OPS = {"add": ADD, "sub": SUB, "mul": MUL, "div": DIV, "pow": POW, "max": MAX, "min": MIN}
# enum wm_unary_op
RELU, SIGMOID, TANH, LOG, EXP, POWS, SQRT, ABS, CLAMP, SCALE = range(10)
UNARY_OPS = {"relu": RELU, "sigmoid": SIGMOID, "tanh": TANH, "log": LOG, "exp": EXP,
             "pows": POWS, "sqrt": SQRT, "abs": ABS, "clamp": CLAMP, "scale": SCALE}
# enum wm_reduce_op
R_SUM, R_MEAN, R_MAX, R_MIN, R_ARGMAX, R_ARGMIN = range(6)
REDUCE_OPS = {"sum": R_SUM, "mean": R_MEAN, "max": R_MAX, "min": R_MIN,
              "argmax": R_ARGMAX, "argmin": R_ARGMIN}

_i64p = C.POINTER(C.c_int64)
_vp = C.c_void_p
# include/wm_io.h callbacks
READ_FN = C.CFUNCTYPE(C.c_int64, C.c_void_p, C.c_void_p, C.c_int64)
WRITE_FN = C.CFUNCTYPE(C.c_int64, C.c_void_p, C.c_void_p, C.c_int64)

# name -> (restype, argtypes); every entry point returns int (status).
_SIGS = {
    "wm_init": [C.c_int],
    "wm_alloc": [C.POINTER(C.c_void_p), C.c_size_t],
    "wm_free": [_vp],
    "wm_empty_cache": [],
    "wm_h2d": [_vp, _vp, C.c_size_t],
    "wm_d2h": [_vp, _vp, C.c_size_t],
    "wm_d2d": [_vp, _vp, C.c_size_t],
    "wm_sync": [],
    "wm_device_cus": [C.POINTER(C.c_int)],
    "wm_timer_start": [],
    "wm_timer_stop": [C.POINTER(C.c_float)],
    "wm_span_begin": [],
    "wm_span_end": [C.POINTER(C.c_float), C.POINTER(C.c_float), C.POINTER(C.c_int)],
    "wm_span_kernel": [C.c_int, C.POINTER(C.c_float)],
    "wm_launch_count": [C.POINTER(C.c_int64)],
    "wm_pool_handouts": [C.POINTER(C.c_int64)],
    "wm_copy_kernel": [_vp, _vp, C.c_int64],
    "wm_gemm_library": [C.c_int],
    "wm_mha_fused": [C.c_int],
    "wm_copy_kernel_cached": [_vp, _vp, C.c_int64],
    "wm_fill": [_vp, C.c_float, C.c_int64],
    "wm_f32_to_f16_rtz": [_vp, _vp, C.c_int64],
    "wm_f16_to_f32": [_vp, _vp, C.c_int64],
    "wm_broadcast_shape": [_i64p, C.c_int, _i64p, C.c_int, _i64p, C.POINTER(C.c_int)],
    "wm_binary": [C.c_int, _vp, _vp, _i64p, C.c_int, _vp, _i64p, C.c_int],
    "wm_binary_bwd": [C.c_int, _vp, _vp, _i64p, C.c_int, _vp, _i64p, C.c_int, _vp,
                      _vp, C.c_int, _vp, C.c_int],
    "wm_unary": [C.c_int, _vp, _vp, C.c_int64, C.c_float, C.c_float],
    "wm_unary_bwd": [C.c_int, _vp, _vp, _vp, _vp, C.c_int, C.c_int64, C.c_float, C.c_float],
    "wm_reduce": [C.c_int, _vp, C.c_int64, C.c_int64, C.c_int64, _vp, _vp],
    "wm_reduce_noalloc": [C.c_int, _vp, C.c_int64, C.c_int64, C.c_int64, _vp, _vp],
    "wm_reduce_bwd": [C.c_int, _vp, _vp, C.c_int64, C.c_int64, C.c_int64, _vp, C.c_int],
    "wm_softmax_fwd": [_vp, _vp, C.c_int64, C.c_int64],
    "wm_log_softmax_fwd": [_vp, _vp, C.c_int64, C.c_int64],
    "wm_softmax_bwd": [_vp, _vp, _vp, C.c_int, C.c_int64, C.c_int64],
    "wm_log_softmax_bwd": [_vp, _vp, _vp, C.c_int, C.c_int64, C.c_int64],
    "wm_epilogue_f16_fwd": [_vp, _vp, _vp, _vp, _vp, C.c_int64, C.c_int64, C.c_float, C.c_float],
    "wm_epilogue_f16_bwd": [_vp, _vp, _vp, _vp, _vp, C.c_int, _vp, C.c_int, _vp, C.c_int,
                            C.c_int64, C.c_int64, C.c_float, C.c_float],
    # include/wm_optim.h
    "wm_sgd_step": [_vp, _vp, _vp, C.c_int64, C.c_float, C.c_float],
    "wm_adam_step": [_vp, _vp, _vp, _vp, C.c_int64] + [C.c_float] * 6,
    "wm_adamw_step": [_vp, _vp, _vp, _vp, C.c_int64] + [C.c_float] * 7,
    "wm_rmsprop_step": [_vp, _vp, _vp, _vp, C.c_int64] + [C.c_float] * 5,
    "wm_grad_sumsq_accumulate": [_vp, C.c_int64, _vp],
    "wm_clip_grad_norm_scale": [_vp, C.c_int64, _vp, C.c_float],
    "wm_clip_grad_value": [_vp, C.c_int64, C.c_float],
    "wm_grad_unscale": [C.c_int, _vp, _vp, C.c_float, C.POINTER(C.c_int)],
    "wm_sgd_step_multi": [C.c_int, _vp, _vp, _vp, _vp, C.c_float, C.c_float],
    "wm_adam_step_multi": [C.c_int, _vp, _vp, _vp, _vp, _vp] + [C.c_float] * 6,
    "wm_adamw_step_multi": [C.c_int, _vp, _vp, _vp, _vp, _vp] + [C.c_float] * 7,
    "wm_rmsprop_step_multi": [C.c_int, _vp, _vp, _vp, _vp, _vp] + [C.c_float] * 5,
    "wm_grad_sumsq_multi": [C.c_int, _vp, _vp, _vp],
    "wm_grad_sumsq_scaled_multi": [C.c_int, _vp, _vp, C.c_float, _vp],
    "wm_grads_finite_multi": [C.c_int, _vp, _vp, C.POINTER(C.c_int)],
    "wm_clip_grad_norm_scale_multi": [C.c_int, _vp, _vp, _vp, C.c_float],
    "wm_clip_grad_value_multi": [C.c_int, _vp, _vp, C.c_float],
    "wm_grad_scale_apply_multi": [C.c_int, _vp, _vp, _vp],
    "wm_sgd_step_multi_gs": [C.c_int, _vp, _vp, _vp, _vp, _vp, C.c_float, C.c_float],
    "wm_adam_step_multi_gs": [C.c_int] + [_vp] * 6 + [C.c_float] * 6,
    "wm_adamw_step_multi_gs": [C.c_int] + [_vp] * 6 + [C.c_float] * 7,
    "wm_rmsprop_step_multi_gs": [C.c_int] + [_vp] * 6 + [C.c_float] * 5,
    "wm_grad_sumsq_multi_gs": [C.c_int, _vp, _vp, _vp, C.c_float, _vp],
    "wm_grad_first_bad_multi_gs": [C.c_int, _vp, _vp, _vp, C.c_float, _vp],
    # include/wm_loss.h
    "wm_cross_entropy_fwd": [_vp, _vp, C.c_int64, C.c_int64, _vp, _vp],
    "wm_cross_entropy_bwd": [_vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int64, C.c_int64],
    "wm_nll_fwd": [_vp, _vp, C.c_int64, C.c_int64, _vp],
    "wm_nll_bwd": [_vp, _vp, _vp, C.c_int, C.c_int64, C.c_int64],
    "wm_focal_fwd": [_vp, _vp, C.c_int64, C.c_int64, C.c_float, C.c_float, _vp, _vp],
    "wm_focal_bwd": [_vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int64, C.c_int64, C.c_float, C.c_float],
    "wm_pointwise_loss_fwd": [C.c_int, _vp, _vp, C.c_int64, C.c_float, C.c_float, C.c_float, _vp],
    "wm_pointwise_loss_bwd": [C.c_int, _vp, _vp, C.c_int64, C.c_float, C.c_float, C.c_float, _vp, _vp, C.c_int],
    # include/wm_layers.h
    "wm_layernorm_fwd": [_vp, _vp, _vp, C.c_int64, C.c_int64, C.c_float, _vp, _vp, _vp],
    "wm_layernorm_bwd": [_vp, _vp, _vp, _vp, _vp, C.c_int64, C.c_int64, _vp, C.c_int, _vp, C.c_int, _vp, C.c_int],
    "wm_batchnorm2d_fwd": [_vp, _vp, _vp, _vp, _vp, C.c_int64, C.c_int64, C.c_int64, C.c_float, C.c_float, C.c_int,
                           _vp, _vp, _vp],
    "wm_batchnorm2d_bwd": [_vp, _vp, _vp, _vp, _vp, C.c_int64, C.c_int64, C.c_int64, _vp, C.c_int, _vp, C.c_int,
                           _vp, C.c_int],
    "wm_attention_softmax_fwd": [_vp, _vp, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int64, _vp],
    "wm_attention_softmax_bwd": [_vp, _vp, C.c_int64, C.c_int64, _vp],
    "wm_dropout_mask": [_vp, C.c_int64, C.c_float, C.c_uint64],
    # include/wm_gemm.h
    "wm_gemm": [C.c_int, C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_float, _vp, C.c_int64, _vp, C.c_int64,
                _vp, C.c_int64, C.c_int, _vp, C.c_int64, C.c_int64, _i64p],
    "wm_matmul": [_vp, _vp, C.c_int64, C.c_int64, C.c_int64, _vp],
    "wm_matmul_bwd": [_vp, _vp, _vp, C.c_int64, C.c_int64, C.c_int64, _vp, C.c_int, _vp, C.c_int],
    "wm_bmm": [_vp, _vp, C.c_int64, C.c_int64, C.c_int64, C.c_int64, _vp],
    "wm_bmm_bwd": [_vp, _vp, _vp, C.c_int64, C.c_int64, C.c_int64, C.c_int64, _vp, C.c_int, _vp, C.c_int],
    "wm_transpose2d": [_vp, C.c_int64, C.c_int64, _vp, C.c_int],
    # include/wm_io.h
    "wm_read_into_device": [READ_FN, _vp, _vp, C.c_int64],
    "wm_write_from_device": [WRITE_FN, _vp, _vp, C.c_int64],
    # include/wm_layers.h (MultiHeadAttention)
    "wm_mha_fwd": [_vp] * 4 + [C.c_int64] + [_vp] * 8 + [C.c_int64] * 5 + [_vp] * 6,
    "wm_mha_bwd": [_vp] * 13 + [C.c_int64] * 5 + [_vp] * 11,
}

# enum wm_pointwise_loss
L_SMOOTH_L1, L_BCE, L_BCE_LOGITS, L_KLDIV, L_KLDIV_LOG, L_BINARY_FOCAL = range(6)
CE_STATS, FOCAL_STATS = 2, 8


def ptr_array(ptrs):
    """A host array of device pointers (None -> NULL) for the multi-tensor
    entry points, as a void*."""
    arr = (C.c_void_p * max(1, len(ptrs)))(*[(p.value if isinstance(p, C.c_void_p) else p) for p in ptrs])
    return C.cast(arr, C.c_void_p), arr


class GradScale(C.Structure):
    """struct wm_grad_scale (include/wm_optim.h): a gradient's pending
    multiplications -- the first unscale_count elements by unscale, then,
    when clip_sumsq is set, every element by the clip coefficient."""
    _fields_ = [("unscale", C.c_float), ("unscale_count", C.c_int64), ("clip_sumsq", C.c_void_p),
                ("clip_max_norm", C.c_float)]


def grad_scale_array(entries):
    """A host array of wm_grad_scale, one per list position, as a void*."""
    arr = (GradScale * max(1, len(entries)))(*entries)
    return C.cast(arr, C.c_void_p), arr


def i64_array(vals):
    arr = (C.c_int64 * max(1, len(vals)))(*[int(v) for v in vals])
    return C.cast(arr, C.c_void_p), arr


class WMError(RuntimeError):
    pass


_LIB: Optional[C.CDLL] = None


def lib() -> C.CDLL:
    """Load libwm_hip.so (raises if it is not built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise WMError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        L.wm_last_error.restype = C.c_char_p
        L.wm_last_error.argtypes = []
        for name, args in _SIGS.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.restype = C.c_int
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = lib().wm_last_error().decode(errors="replace")
        raise WMError(f"{what or 'wm call'} failed (status {rc}): {msg}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def shape_arg(shape: Sequence[int]):
    arr = (C.c_int64 * max(1, len(shape)))(*[int(s) for s in shape])
    return arr, len(shape)


class DeviceArray:
    """One device allocation with a numpy dtype and shape."""

    def __init__(self, shape: Sequence[int], dtype=np.float32):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.size * self.dtype.itemsize
        p = C.c_void_p()
        call("wm_alloc", C.byref(p), max(self.nbytes, 1))
        self.ptr = p.value

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        if d.nbytes:
            call("wm_h2d", C.c_void_p(d.ptr), a.ctypes.data_as(C.c_void_p), d.nbytes)
        return d

    def to_host(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            call("wm_d2h", out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr), self.nbytes)
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        if self.nbytes:
            call("wm_h2d", C.c_void_p(self.ptr), a.ctypes.data_as(C.c_void_p), self.nbytes)

    def fill(self, v: float) -> None:
        assert self.dtype == np.float32
        call("wm_fill", C.c_void_p(self.ptr), C.c_float(v), self.size)

    @property
    def vp(self):
        return C.c_void_p(self.ptr)

    def free(self) -> None:
        if self.ptr:
            lib().wm_free(C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def nullp():
    return C.c_void_p(0)


def ptr(d: Optional[DeviceArray]):
    return d.vp if d is not None else nullp()


# ---- thin op wrappers (device in, device out) -------------------------------

def broadcast_shape(a_shape, b_shape):
    sa, na = shape_arg(a_shape)
    sb, nb = shape_arg(b_shape)
    out = (C.c_int64 * 8)()
    nd = C.c_int()
    call("wm_broadcast_shape", sa, na, sb, nb, out, C.byref(nd))
    return tuple(out[i] for i in range(nd.value))


def binary(op: int, a: DeviceArray, b: DeviceArray, out: Optional[DeviceArray] = None) -> DeviceArray:
    oshape = broadcast_shape(a.shape, b.shape)
    if out is None:
        out = DeviceArray(oshape)
    sa, na = shape_arg(a.shape)
    sb, nb = shape_arg(b.shape)
    call("wm_binary", op, out.vp, a.vp, sa, na, b.vp, sb, nb)
    return out


def binary_bwd(op, g, a, b, out, ga, ga_acc, gb, gb_acc):
    sa, na = shape_arg(a.shape)
    sb, nb = shape_arg(b.shape)
    call("wm_binary_bwd", op, g.vp, a.vp, sa, na, b.vp, sb, nb, ptr(out),
         ptr(ga), int(ga_acc), ptr(gb), int(gb_acc))


def unary(op, x, p0=0.0, p1=0.0, out=None):
    if out is None:
        out = DeviceArray(x.shape)
    call("wm_unary", op, out.vp, x.vp, x.size, C.c_float(p0), C.c_float(p1))
    return out


def unary_bwd(op, g, x, out, gx, acc, p0=0.0, p1=0.0):
    call("wm_unary_bwd", op, g.vp, ptr(x), ptr(out), gx.vp, int(acc), g.size,
         C.c_float(p0), C.c_float(p1))


def reduce(op, x, outer, n, inner, want_val=True, want_idx=False):
    val = DeviceArray((outer, inner)) if want_val else None
    idx = DeviceArray((outer, inner), np.int64) if want_idx else None
    call("wm_reduce", op, x.vp, outer, n, inner, ptr(val), ptr(idx))
    return val, idx


def reduce_bwd(op, g, idx, outer, n, inner, gx, acc):
    call("wm_reduce_bwd", op, g.vp, ptr(idx), outer, n, inner, gx.vp, int(acc))


def device_cus() -> int:
    c = C.c_int()
    call("wm_device_cus", C.byref(c))
    return c.value


def sync() -> None:
    call("wm_sync")
