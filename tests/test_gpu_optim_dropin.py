"""GPU parity of the drop-in C++ optimizers (whitematter_amd/core/optimizer.h):
SGD / Adam / AdamW / RMSprop constructed over drop-in Tensors, stepped with
fresh gradients, compared bit for bit with the strict fp32 oracle (pinned
against the reference's optimizer.cpp built with IEEE semantics) -- the
parameters and every state buffer after each step.  Also the Tensor-level
clipping helpers and zero_grad."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

o32 = oracle.get("f32")

CONFIGS = [
    ("SGD", dict(lr=0.05), ("sgd", 0.05, 0.0)),
    ("SGD", dict(lr=0.05, momentum=0.9), ("sgd", 0.05, 0.9)),
    ("Adam", dict(lr=1e-3), ("adam", 1e-3, 0.9, 0.999, 1e-8)),
    ("AdamW", dict(lr=1e-3, weight_decay=0.02), ("adamw", 1e-3, 0.9, 0.999, 1e-8, 0.02)),
    ("RMSprop", dict(lr=1e-2), ("rmsprop", 1e-2, 0.99, 1e-8, 0.0, 0.0)),
    ("RMSprop", dict(lr=1e-2, momentum=0.9, weight_decay=0.01), ("rmsprop", 1e-2, 0.99, 1e-8, 0.9, 0.01)),
]


def rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("cls,kw,spec", CONFIGS, ids=lambda v: v if isinstance(v, str) else None)
def test_dropin_optimizer_steps(wm, cls, kw, spec):
    from whitematter_amd import _tensor as T
    shapes = [(64, 33), (4096,), (7,)]
    p0 = [rng(i).standard_normal(s).astype(np.float32) for i, s in enumerate(shapes)]
    params = [T.Tensor.from_array(p, requires_grad=True) for p in p0]
    opt = getattr(T, cls)(params, **kw)
    mine = [p.ravel().copy() for p in p0]
    s1 = [np.zeros(p.size, np.float32) for p in p0]
    s2 = [np.zeros(p.size, np.float32) for p in p0]
    kind, lr = spec[0], spec[1]
    for t in range(1, 5):
        grads = [rng(10 * t + i).standard_normal(s).astype(np.float32) for i, s in enumerate(shapes)]
        for prm, g in zip(params, grads):
            prm.grad = g
        opt.step()
        for k, g in enumerate(grads):
            gf = g.ravel()
            if kind == "sgd":
                o32.sgd_step(mine[k], gf, s1[k], lr, spec[2])
            elif kind in ("adam", "adamw"):
                b1, b2, eps = spec[2], spec[3], spec[4]
                wd = spec[5] if kind == "adamw" else 0.0
                o32.adam_step(mine[k], gf, s1[k], s2[k], lr, b1, b2, eps, o32.bias_correction(b1, t),
                              o32.bias_correction(b2, t), wd, kind == "adamw")
            else:
                o32.rmsprop_step(mine[k], gf, s1[k], s2[k], lr, spec[2], spec[3], spec[4], spec[5])
        for k, prm in enumerate(params):
            assert oracle.bit_equal(np.asarray(prm.data).ravel(), mine[k]), (cls, t, k)
            for j, st in enumerate(opt.state(k)):
                assert oracle.bit_equal(st, (s1, s2)[j][k]), (cls, t, k, "state", j)
    if cls in ("Adam", "AdamW"):
        assert opt.t == 4


def test_dropin_clipping_and_zero_grad(wm):
    from whitematter_amd import _tensor as T
    grads = [rng(40 + i).standard_normal(n).astype(np.float32) * 3 for i, n in enumerate((1000, 37, 4096))]
    params = [T.Tensor.from_array(np.zeros_like(g), requires_grad=True) for g in grads]
    for p, g in zip(params, grads):
        p.grad = g
    total64 = sum(oracle.get("f64").grad_sumsq(g) for g in grads)
    norm = T.get_grad_norm(params)
    assert abs(norm - np.sqrt(total64)) <= 1e-5 * np.sqrt(total64)
    T.clip_grad_norm_(params, 1.0)
    coef = np.float32(1.0) / (np.float32(norm) + np.float32(1e-6))
    for p, g in zip(params, grads):
        assert oracle.bit_equal(np.asarray(p.grad).ravel(), g * coef)
    assert abs(T.get_grad_norm(params) - 1.0) <= 1e-5
    for p, g in zip(params, grads):
        p.grad = g
    T.clip_grad_value_(params, 2.0)
    for p, g in zip(params, grads):
        mine = g.copy()
        o32.clip_grad_value(mine, 2.0)
        assert oracle.bit_equal(np.asarray(p.grad).ravel(), mine)
    opt = T.SGD(params, 0.1)
    opt.zero_grad()
    assert all(p.grad_known_zero for p in params)
    assert T.get_grad_norm(params) == 0.0
