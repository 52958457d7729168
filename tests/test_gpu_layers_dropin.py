"""GPU parity of the drop-in modules (whitematter_amd/core/layer.h) whose
bodies run on the device: LayerNorm and BatchNorm2d (forward, running
statistics, backward into the input and both parameters, through
Tensor.backward()) against the fp64 oracle, and Dropout's mask against the
oracle's restatement of the device generator plus the reference's dropout
rules (scale 1/(1-p), eval and p = 0 are the identity, the backward
multiplies by the same mask)."""
import numpy as np
import pytest

import oracle
from gpu_helpers import rng_normal, rng_uniform

pytestmark = pytest.mark.gpu

o32, o64, oab = oracle.get("f32"), oracle.get("f64"), oracle.get("abs")


def T():
    from whitematter_amd import _tensor
    return _tensor


def close(got, ref, scale, rtol=1e-5, atol=1e-30):
    ok, worst = oracle.close_scaled(np.asarray(got, np.float32), ref, scale, rtol, atol)
    assert ok, f"{worst:.3g}x tolerance"


def backward_through_sum(t, y, w):
    """loss = sum(y * w): y's upstream gradient is w."""
    (y * t.Tensor.from_array(w)).sum().backward()


@pytest.mark.parametrize("shape", [(4, 16), (2, 3, 768), (64, 1000)])
def test_dropin_layernorm(wm, shape):
    t = T()
    n = shape[-1]
    x = rng_normal(shape, 1, 2.0) + np.float32(1.0)
    gamma, beta = rng_uniform((n,), 2, 0.5, 1.5), rng_normal((n,), 3)
    ln = t.LayerNorm(n)
    ln.gamma = t.Tensor.from_array(gamma, requires_grad=True)
    ln.beta = t.Tensor.from_array(beta, requires_grad=True)
    px = t.Tensor.from_array(x, requires_grad=True)
    y = ln(px)
    y64, mean, inv = o64.layernorm(x, gamma, beta)
    close(np.asarray(y.data), y64, oab.layernorm(x, gamma, beta)[0])
    w = rng_normal(shape, 4)
    backward_through_sum(t, y, w)
    # the closure's statistics are the device's; feed the oracle its fp32 values
    _, m32, i32 = o32.layernorm(x, gamma, beta)
    ref = o64.layernorm_bwd(w, x, gamma, m32, i32)
    scale = oab.layernorm_bwd(w, x, gamma, m32, i32)
    # the device statistics differ from the fp32 oracle's by a few ulp; that
    # moves each gradient by ~1e-7 of its scale, inside the tolerance
    close(np.asarray(px.grad).reshape(shape), ref[0], scale[0])
    close(np.asarray(ln.gamma.grad), ref[1], scale[1])
    close(np.asarray(ln.beta.grad), ref[2], scale[2])


@pytest.mark.parametrize("training", [True, False])
def test_dropin_batchnorm(wm, training):
    t = T()
    shape = (4, 8, 12, 12)
    x = rng_normal(shape, 5, 2.0) + np.float32(0.5)
    bn = t.BatchNorm2d(8)
    gamma, beta = rng_uniform((8,), 6, 0.5, 1.5), rng_normal((8,), 7)
    bn.gamma = t.Tensor.from_array(gamma, requires_grad=True)
    bn.beta = t.Tensor.from_array(beta, requires_grad=True)
    if not training:
        bn.eval()
        bn.running_mean = t.Tensor.from_array(rng_normal((8,), 8, 0.1))
        bn.running_var = t.Tensor.from_array(rng_uniform((8,), 9, 0.5, 2.0))
    rm0, rv0 = np.asarray(bn.running_mean.data).copy(), np.asarray(bn.running_var.data).copy()
    px = t.Tensor.from_array(x, requires_grad=True)
    y = bn(px)
    y64, mean, inv, rm64, rv64 = o64.batchnorm2d(x, gamma, beta, rm0, rv0, training=training)
    close(np.asarray(y.data), y64, oab.batchnorm2d(x, gamma, beta, rm0, rv0, training=training)[0])
    close(np.asarray(bn.running_mean.data), rm64, np.abs(rm64) + 0.1 * np.abs(x).mean((0, 2, 3)))
    close(np.asarray(bn.running_var.data), rv64, rv64)
    w = rng_normal(shape, 10)
    backward_through_sum(t, y, w)
    _, m32, i32, _, _ = o32.batchnorm2d(x, gamma, beta, rm0, rv0, training=training)
    ref = o64.batchnorm2d_bwd(w, x, gamma, m32, i32)
    scale = oab.batchnorm2d_bwd(w, x, gamma, m32, i32)
    close(np.asarray(px.grad).reshape(shape), ref[0], scale[0])
    close(np.asarray(bn.gamma.grad), ref[1], scale[1])
    close(np.asarray(bn.beta.grad), ref[2], scale[2])


def test_dropin_batchnorm_untracked_input_gives_no_parameter_gradient(wm):
    """Tracking follows the input (core/layer.cpp:214): with an input that
    does not require grad, gamma and beta receive no gradient."""
    t = T()
    bn = t.BatchNorm2d(3)
    y = bn(t.Tensor.from_array(rng_normal((2, 3, 4, 4), 11)))
    assert not y.requires_grad


def test_dropout_mask_matches_generator_and_rules(wm):
    from whitematter_amd import _lib as W
    n, p, seed = 1 << 20, 0.3, 12345
    m = W.DeviceArray((n,))
    W.call("wm_dropout_mask", m.vp, n, W.C.c_float(p), seed)
    got = m.to_host()
    assert oracle.bit_equal(got, o32.dropout_mask(n, p, seed))
    keep = got != 0
    assert abs(1 - keep.mean() - p) < 5 * np.sqrt(p * (1 - p) / n)
    assert np.all(got[keep] == np.float32(1) / (np.float32(1) - np.float32(p)))


# Published SplitMix64 outputs: state 1234567's first five (the Rosetta Code
# SplitMix64 task) and state 0's first.  Output k of state s is
# mix(s + k * golden); the mask's element i draws mix(seed + i + golden).
_SM64_GOLDEN = 0x9E3779B97F4A7C15
_SM64_KATS = [(1234567, k + 1, v) for k, v in enumerate(
    [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431, 16408922859458223821])] + \
    [(0, 1, 0xE220A8397B1DCDAF)]


@pytest.mark.parametrize("state,k,value", _SM64_KATS)
def test_dropout_mask_generator_known_answers(wm, state, k, value):
    """Element `offset` keeps its value iff u > p with u the top 24 bits of
    the published output: p = u drops it, p one float below u keeps it."""
    from whitematter_amd import _lib as W
    offset = 70001
    n = offset + 1
    seed = (state + k * _SM64_GOLDEN - _SM64_GOLDEN - offset) % (1 << 64)
    u = np.float32((value >> 40) * 2.0 ** -24)
    below = np.nextafter(u, np.float32(-1))
    m = W.DeviceArray((n,))
    W.call("wm_dropout_mask", m.vp, n, W.C.c_float(float(u)), seed)
    assert m.to_host()[offset] == 0.0
    W.call("wm_dropout_mask", m.vp, n, W.C.c_float(float(below)), seed)
    assert m.to_host()[offset] == np.float32(1) / (np.float32(1) - below)


def test_dropin_dropout_forward_backward(wm):
    t = T()
    x = rng_normal((32, 64), 12)
    d = t.Dropout(0.25)
    px = t.Tensor.from_array(x, requires_grad=True)
    y = np.asarray(d(px).data)
    kept = y != 0
    scale = np.float32(1) / (np.float32(1) - np.float32(0.25))
    assert np.array_equal(y[kept], x[kept] * scale) and 0.65 < kept.mean() < 0.85
    px2 = t.Tensor.from_array(x, requires_grad=True)
    out = d(px2)
    out.sum().backward()
    mask = np.asarray(out.data) != 0
    g = np.asarray(px2.grad).reshape(x.shape)
    assert np.all(g[mask] == scale) and np.all(g[~mask] == 0)
    d.eval()
    assert np.array_equal(np.asarray(d(px).data), x)
    assert np.array_equal(np.asarray(t.Dropout(0.0)(px).data), x)
