"""GPU parity of the drop-in loss classes (whitematter_amd/core/loss.h): every
reference loss constructed as the reference's tests construct it, run forward
and backward on drop-in Tensors, and compared with the oracle (pinned against
the reference's core/loss.cpp in test_oracle_loss.py) -- the loss value and
the prediction's gradient.  Also the graph rules: requires_grad follows the
prediction, a second backward path accumulates, and MSE / L1 stay Tensor-op
compositions."""
import numpy as np
import pytest

import oracle
from gpu_helpers import rng_normal, rng_uniform

pytestmark = pytest.mark.gpu

o64, oab = oracle.get("f64"), oracle.get("abs")


def T():
    from whitematter_amd import _tensor
    return _tensor


def close(got, ref64, scale64, atol=1e-30, rtol=1e-5):
    ok, worst = oracle.close_scaled(np.asarray(got, np.float32), ref64, scale64, rtol, atol)
    assert ok, f"{worst:.3g}x tolerance"


def run(loss, x, y, x_shape=None, y_shape=None):
    t = T()
    px = t.Tensor.from_array(x, x_shape, requires_grad=True)
    ty = t.Tensor.from_array(y, y_shape, requires_grad=False)
    out = loss(px, ty)
    value = float(np.asarray(out.data).ravel()[0])
    out.backward()
    return value, np.asarray(px.grad).reshape(x.shape)


HEADS = [("CrossEntropyLoss", {}, "cross_entropy"), ("NLLLoss", {}, "nll"),
         ("FocalLoss", {"gamma": 2.0, "alpha": -1.0}, "focal"), ("FocalLoss", {"gamma": 1.5, "alpha": 0.25}, "focal")]


@pytest.mark.parametrize("cls,kw,kind", HEADS, ids=lambda v: v if isinstance(v, str) else None)
@pytest.mark.parametrize("shape", [(32, 10), (7, 1000), (2, 40000)])
def test_dropin_heads(wm, cls, kw, kind, shape):
    x = rng_normal(shape, 1, 2.0)
    lab = np.floor(rng_uniform((shape[0],), 2, 0, shape[1])).astype(np.float32)
    value, grad = run(getattr(T(), cls)(**kw), x, lab)
    if kind == "cross_entropy":
        v64, vab, g64, gab = o64.cross_entropy(x, lab), oab.cross_entropy(x, lab), o64.cross_entropy_bwd(x, lab), \
            oab.cross_entropy_bwd(x, lab)
    elif kind == "nll":
        v64, vab, g64, gab = o64.nll(x, lab), oab.nll(x, lab), o64.nll_bwd(shape, lab), oab.nll_bwd(shape, lab)
    else:
        g, a = kw["gamma"], kw["alpha"]
        v64, vab = o64.focal(x, lab, g, a), oab.focal(x, lab, g, a)
        g64, gab = o64.focal_bwd(x, lab, g, a), oab.focal_bwd(x, lab, g, a)
    close([value], np.float64([v64]), np.float64([vab]))
    atol = 8 * 2.0 ** -24 * 4 / shape[0] if kind == "focal" else 1e-30
    close(grad, g64, gab, atol)


def test_dropin_target_as_column(wm):
    """A [batch, 1] target is accepted like a [batch] one (core/loss.cpp:69)."""
    x = rng_normal((16, 5), 3)
    lab = np.float32(np.arange(16) % 5)
    a, ga = run(T().CrossEntropyLoss(), x, lab)
    b, gb = run(T().CrossEntropyLoss(), x, lab, None, [16, 1])
    assert a == b and oracle.bit_equal(ga, gb)


POINTWISE = [("SmoothL1Loss", {"beta": 1.0}, "smooth_l1", 1.0, 0.0),
             ("SmoothL1Loss", {"beta": 0.3}, "smooth_l1", 0.3, 0.0),
             ("BCELoss", {}, "bce", 0.0, 0.0),
             ("BCEWithLogitsLoss", {}, "bce_logits", 0.0, 0.0),
             ("KLDivLoss", {}, "kldiv", 0.0, 0.0),
             ("KLDivLoss", {"log_target": True}, "kldiv_log", 0.0, 0.0),
             ("BinaryFocalLoss", {"gamma": 2.0, "alpha": 0.25}, "binary_focal", 2.0, 0.25),
             ("BinaryFocalLoss", {"gamma": 0.0, "alpha": -1.0}, "binary_focal", 0.0, -1.0)]


@pytest.mark.parametrize("cls,kw,kind,p0,p1", POINTWISE, ids=lambda v: v if isinstance(v, str) else None)
def test_dropin_pointwise(wm, cls, kw, kind, p0, p1):
    shape = (24, 50)
    if kind == "bce":
        x, y = rng_uniform(shape, 4, 0.01, 0.99), rng_uniform(shape, 5, 0, 1)
    elif kind.startswith("kldiv"):
        x = np.log(rng_uniform(shape, 4, 0.01, 1)).astype(np.float32)
        y = np.log(rng_uniform(shape, 5, 0.01, 1)).astype(np.float32) if kind == "kldiv_log" \
            else rng_uniform(shape, 5, -0.2, 1)
    elif kind == "binary_focal":
        x, y = rng_normal(shape, 4, 3.0), (rng_uniform(shape, 5, 0, 1) > 0.5).astype(np.float32)
    else:
        x, y = rng_normal(shape, 4, 2.0), rng_normal(shape, 5)
    value, grad = run(getattr(T(), cls)(**kw), x, y)
    denom = shape[0] if kind.startswith("kldiv") else None
    close([value], np.float64([o64.pointwise_loss(kind, x, y, p0, p1, denom)]),
          np.float64([oab.pointwise_loss(kind, x, y, p0, p1, denom)]))
    rtol = 1e-5
    if kind == "binary_focal":  # fp32 1 - p amplification, as in test_gpu_loss.grad_rtol
        p = 1.0 / (1.0 + np.exp(-x.astype(np.float64).ravel()))
        rtol = 1e-5 + 16 * 2.0 ** -24 / np.minimum(p, 1.0 - p)
    close(grad.ravel(), o64.pointwise_loss_bwd(kind, x, y, p0, p1, denom).ravel(),
          oab.pointwise_loss_bwd(kind, x, y, p0, p1, denom).ravel(), rtol=rtol)


def test_dropin_mse_l1_compositions(wm):
    x, y = rng_normal((8, 33), 6), rng_normal((8, 33), 7)
    xd, yd = x.astype(np.float64), y.astype(np.float64)
    v, g = run(T().MSELoss(), x, y)
    assert abs(v - np.mean((xd - yd) ** 2)) <= 1e-5 * np.mean((xd - yd) ** 2)
    # the reference's mean() gradient is the upstream gradient, unscaled
    # (core/tensor.cpp:1709-1721), so MSE's gradient is 2 (x - y)
    assert np.allclose(g, 2 * (xd - yd), rtol=1e-6, atol=1e-6)
    v, g = run(T().L1Loss(), x, y)
    assert abs(v - np.mean(np.abs(xd - yd))) <= 1e-5 * np.mean(np.abs(xd - yd))
    assert np.array_equal(np.sign(g), np.sign(xd - yd))


def test_dropin_graph_rules(wm):
    t = T()
    x = rng_normal((6, 9), 8)
    lab = np.float32(np.arange(6) % 9)
    # no grad requested: no backward closure, value still computed
    px = t.Tensor.from_array(x, requires_grad=False)
    out = t.CrossEntropyLoss()(px, t.Tensor.from_array(lab))
    assert not out.requires_grad
    # two uses of one prediction: the second closure accumulates
    px = t.Tensor.from_array(x, requires_grad=True)
    ty = t.Tensor.from_array(lab)
    total = t.CrossEntropyLoss()(px, ty) + t.FocalLoss(2.0, -1.0)(px, ty)
    total.backward()
    want = o64.cross_entropy_bwd(x, lab) + o64.focal_bwd(x, lab, 2.0, -1.0)
    scale = oab.cross_entropy_bwd(x, lab) + oab.focal_bwd(x, lab, 2.0, -1.0)
    close(np.asarray(px.grad).reshape(x.shape), want, scale, 8 * 2.0 ** -24 * 4 / 6)


def test_dropin_rejects_bad_shapes(wm):
    t = T()
    with pytest.raises(Exception):
        t.CrossEntropyLoss()(t.Tensor.from_array(np.zeros(5, np.float32)), t.Tensor.from_array(np.zeros(5, np.float32)))
    with pytest.raises(Exception):
        t.NLLLoss()(t.Tensor.from_array(np.zeros((4, 3), np.float32)), t.Tensor.from_array(np.zeros(2, np.float32)))
    with pytest.raises(Exception):
        t.BCELoss()(t.Tensor.from_array(np.zeros(4, np.float32)), t.Tensor.from_array(np.zeros(3, np.float32)))
