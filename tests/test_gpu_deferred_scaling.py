"""GPU tests of deferred gradient scaling (DeviceVector::defer_unscale /
defer_clip, include/wm_optim.h wm_grad_scale): GradScaler::unscale and
clip_grad_norm_ record their multiplication with the gradient instead of
writing it, and the next pass applies it as it reads -- the optimizer step,
a norm, a finiteness search -- while any other use sees the multiplied
values.

Contract: every result equals the reference's eager in-place
multiplications (core/amp.h:131-142, core/optimizer.cpp:155-164) bit for
bit: the parameters and optimizer states after a step, the gradients read
back, norms (which are sums: the same kernels, so the same bits as norms of
eagerly scaled gradients), the finiteness verdicts.  The strict fp32 oracle
(pinned against the reference's optimizer.cpp) takes the eagerly scaled
gradients.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

o32 = oracle.get("f32")
SHAPES = [(64, 33), (4096,), (7,), (1000,)]


@pytest.fixture(scope="module")
def T(wm):
    from whitematter_amd import _tensor
    return _tensor


def rng(seed):
    return np.random.default_rng(seed)


def make(T, grads, seed=0):
    ps = []
    for i, g in enumerate(grads):
        p = T.Tensor.from_array(rng(seed + i).standard_normal(g.shape).astype(np.float32), requires_grad=True)
        p.grad = g
        ps.append(p)
    return ps


def eager_clip(grads, norm, max_norm):
    coef = np.float32(max_norm) / (np.float32(norm) + np.float32(1e-6))
    return [g * coef if coef < 1 else g.copy() for g in grads]


def step_ref(kind, p, g, s1, s2, t):
    if kind == "sgd":
        o32.sgd_step(p, g, s1, 0.05, 0.9)
    elif kind == "adamw":
        o32.adam_step(p, g, s1, s2, 1e-3, 0.9, 0.999, 1e-8, o32.bias_correction(0.9, t),
                      o32.bias_correction(0.999, t), 0.02, True)
    else:
        o32.rmsprop_step(p, g, s1, s2, 1e-2, 0.99, 1e-8, 0.9, 0.01)


def optimizer(T, kind, ps):
    if kind == "sgd":
        return T.SGD(ps, 0.05, 0.9)
    if kind == "adamw":
        return T.AdamW(ps, 1e-3, 0.9, 0.999, 1e-8, 0.02)
    return T.RMSprop(ps, 1e-2, 0.99, 1e-8, 0.9, 0.01)


def check_params(ps, opt, mine, s1, s2):
    for k, p in enumerate(ps):
        assert oracle.bit_equal(np.asarray(p.data).ravel(), mine[k]), k
        for j, st in enumerate(opt.state(k)):
            assert oracle.bit_equal(st, (s1, s2)[j][k]), (k, "state", j)


@pytest.mark.parametrize("kind", ["sgd", "adamw", "rmsprop"])
def test_clip_then_steps(T, kind):
    """clip_grad_norm_ then step, twice, the gradients never read back in
    between: the step takes the clip's products as it reads the gradients."""
    ps = make(T, [np.zeros(s, np.float32) for s in SHAPES])
    opt = optimizer(T, kind, ps)
    mine = [np.asarray(p.data).ravel().copy() for p in ps]
    s1 = [np.zeros_like(m) for m in mine]
    s2 = [np.zeros_like(m) for m in mine]
    for t in (1, 2):
        grads = [rng(100 * t + i).standard_normal(s).astype(np.float32) * 4 for i, s in enumerate(SHAPES)]
        for p, g in zip(ps, grads):
            p.grad = g
        norm = T.get_grad_norm(ps)
        T.clip_grad_norm_(ps, 1.0)
        opt.step()
        for k, g in enumerate(eager_clip(grads, norm, 1.0)):
            step_ref(kind, mine[k], g.ravel(), s1[k], s2[k], t)
        check_params(ps, opt, mine, s1, s2)
    # the clipped gradients, read back after the step, are the eager products
    for p, g in zip(ps, eager_clip(grads, norm, 1.0)):
        assert oracle.bit_equal(np.asarray(p.grad).ravel(), g.ravel())


@pytest.mark.parametrize("kind", ["sgd", "adamw"])
def test_unscale_clip_step(T, kind):
    """The AMP order: unscale (deferred), clip_grad_norm_ on the unscaled
    values (deferred on top), then the step -- and the norm in between."""
    scale = 4096.0
    grads = [rng(200 + i).standard_normal(s).astype(np.float32) * np.float32(scale) for i, s in enumerate(SHAPES)]
    ps = make(T, grads)
    opt = optimizer(T, kind, ps)
    mine = [np.asarray(p.data).ravel().copy() for p in ps]
    s1 = [np.zeros_like(m) for m in mine]
    s2 = [np.zeros_like(m) for m in mine]
    scaler = T.GradScaler(scale, 2.0, 0.5, 1000)
    assert scaler.unscale(opt)
    inv = np.float32(1.0) / np.float32(scale)
    unscaled = [g * inv for g in grads]
    # a norm of the deferred values equals the norm of eagerly unscaled ones
    ref_ps = make(T, unscaled)
    norm = T.get_grad_norm(ps)
    assert norm == T.get_grad_norm(ref_ps)
    T.clip_grad_norm_(ps, 0.5)
    scaler.step(opt, True)
    for k, g in enumerate(eager_clip(unscaled, norm, 0.5)):
        step_ref(kind, mine[k], g.ravel(), s1[k], s2[k], 1)
    check_params(ps, opt, mine, s1, s2)


def test_partial_unscale_then_direct_step(T):
    """unscale stops at a non-finite product: the elements before it are
    multiplied, the rest left as they are -- a step taken anyway (the
    optimizer called directly, not through GradScaler::step) reads exactly
    that mix."""
    grads = [rng(300 + i).standard_normal(s).astype(np.float32) * 100 for i, s in enumerate(SHAPES)]
    grads[1][1234] = np.inf
    ps = make(T, grads)
    opt = optimizer(T, "sgd", ps)
    mine = [np.asarray(p.data).ravel().copy() for p in ps]
    s1 = [np.zeros_like(m) for m in mine]
    scaler = T.GradScaler(64.0, 2.0, 0.5, 1000)
    assert not scaler.unscale(opt)
    inv = np.float32(1.0) / np.float32(64.0)
    eager = [grads[0] * inv, grads[1].ravel().copy(), grads[2], grads[3]]
    eager[1][:1234] = eager[1][:1234] * inv
    assert not T.check_gradients_finite(ps)
    opt.step()
    for k, g in enumerate(eager):
        step_ref("sgd", mine[k], g.ravel(), s1[k], None, 1)
    for k, p in enumerate(ps):
        assert oracle.bit_equal(np.asarray(p.data).ravel(), mine[k]), k
    for p, g in zip(ps, eager):
        assert oracle.bit_equal(np.asarray(p.grad).ravel(), g.ravel())


def test_clip_twice_and_zero_grad(T):
    """A second clip sees the first one's products (it writes them before
    deferring its own); zero_grad drops a deferred scaling."""
    grads = [rng(400 + i).standard_normal(s).astype(np.float32) * 10 for i, s in enumerate(SHAPES)]
    ps = make(T, grads)
    n1 = T.get_grad_norm(ps)
    T.clip_grad_norm_(ps, 2.0)
    once = eager_clip(grads, n1, 2.0)
    n2 = T.get_grad_norm(ps)
    assert n2 == T.get_grad_norm(make(T, once))
    T.clip_grad_norm_(ps, 1.0)
    for p, g in zip(ps, eager_clip(once, n2, 1.0)):
        assert oracle.bit_equal(np.asarray(p.grad).ravel(), g.ravel())
    T.clip_grad_norm_(ps, 0.25)
    T.SGD(ps, 0.1).zero_grad()
    assert all(p.grad_known_zero for p in ps)
    assert T.get_grad_norm(ps) == 0.0


def test_backward_accumulates_into_a_deferred_gradient(T):
    """A closure adding to a gradient whose clip is deferred adds to the
    clipped values (the scaling is written first), as the reference's += on
    the scaled vector does; a reshape's gradient copy carries the scaling."""
    g = rng(500).standard_normal((32, 16)).astype(np.float32) * 8
    (p,) = make(T, [g])
    norm = T.get_grad_norm([p])
    T.clip_grad_norm_([p], 1.0)
    c = T.Tensor.from_array(rng(501).standard_normal((32, 16)).astype(np.float32))
    y = p.mul(c).sum().sum()
    y.backward()
    (clipped,) = eager_clip([g], norm, 1.0)
    assert oracle.bit_equal(np.asarray(p.grad), clipped + np.asarray(c.data))
    # reshape initialises its tracked result's gradient with a copy of the input's (S14)
    (q,) = make(T, [g])
    T.clip_grad_norm_([q], 1.0)
    r = q.reshape([16, 32])
    assert oracle.bit_equal(np.asarray(r.grad).ravel(), clipped.ravel())


def test_unscale_with_a_parameter_listed_twice(T):
    """A gradient listed twice is scaled twice, the second pass searching the
    first pass's products (the eager path)."""
    g0 = rng(600).standard_normal(3000).astype(np.float32) * 50
    g1 = rng(601).standard_normal(700).astype(np.float32) * 50
    ps = make(T, [g0, g1])
    opt = T.SGD([ps[0], ps[0], ps[1]], 0.1)
    scaler = T.GradScaler(16.0, 2.0, 0.5, 1000)
    assert scaler.unscale(opt)
    inv = np.float32(1.0) / np.float32(16.0)
    assert oracle.bit_equal(np.asarray(ps[0].grad), (g0 * inv) * inv)
    assert oracle.bit_equal(np.asarray(ps[1].grad), g1 * inv)


def test_overflowing_unscale_and_finite_check(T):
    """A loss scale below 1 makes unscale's products overflow: the search
    stops at the first infinite product, which check_gradients_finite then
    sees among the deferred values."""
    g = rng(700).standard_normal(5000).astype(np.float32) * 4
    ps = make(T, [g])
    opt = T.SGD(ps, 0.1)
    scale = 1e-38
    scaler = T.GradScaler(scale, 2.0, 0.5, 1000)
    assert not scaler.unscale(opt)
    inv = np.float32(1.0) / np.float32(scale)
    prod = g * inv
    stop = int(np.flatnonzero(~np.isfinite(prod))[0])
    want = g.copy()
    want[:stop] = prod[:stop]
    assert T.check_gradients_finite(ps) == bool(np.isfinite(want).all())
    assert oracle.bit_equal(np.asarray(ps[0].grad), want)


@pytest.mark.parametrize("max_norm", [-0.5, 0.0])
def test_clip_with_negative_or_zero_max_norm_and_a_zero_gradient(T, max_norm):
    """A coefficient that is negative or zero still multiplies every element
    (it is < 1), a known-zero gradient included: zeros become -0.0 under a
    negative coefficient, negative values -0.0 under a zero one, as the
    reference's float products give."""
    grads = [rng(800 + i).standard_normal(s).astype(np.float32) for i, s in enumerate(SHAPES)]
    ps = make(T, grads)
    ps[2].zero_grad()
    assert ps[2].grad_known_zero
    grads[2] = np.zeros(SHAPES[2], np.float32)
    norm = T.get_grad_norm(ps)
    T.clip_grad_norm_(ps, max_norm)
    coef = np.float32(max_norm) / (np.float32(norm) + np.float32(1e-6))
    for p, g in zip(ps, grads):
        assert oracle.bit_equal(np.asarray(p.grad), g * coef)


def test_clip_grad_norm_amp_defers_onto_scaled_gradients(T):
    """clip_grad_norm_amp measures the norm of g / scale and, when it clips,
    multiplies the still-scaled gradients by the coefficient (core/amp.h:
    303-327); the step reads them through that deferred multiplication."""
    scale = np.float32(512.0)
    grads = [(rng(900 + i).standard_normal(s) * 3).astype(np.float32) * scale for i, s in enumerate(SHAPES)]
    ps = make(T, grads)
    opt = optimizer(T, "sgd", ps)
    mine = [np.asarray(p.data).ravel().copy() for p in ps]
    s1 = [np.zeros_like(m) for m in mine]
    norm = T.clip_grad_norm_amp(ps, 1.0, float(scale))
    inv = np.float32(1.0) / scale
    ref_norm = np.sqrt(np.float32(sum(float(np.sum((g.astype(np.float64) * inv) ** 2)) for g in grads)))
    assert abs(norm - ref_norm) <= 1e-5 * ref_norm
    coef = np.float32(1.0) / (np.float32(norm) + np.float32(1e-6))
    assert coef < 1
    opt.step()
    for k, g in enumerate(grads):
        step_ref("sgd", mine[k], (g * coef).ravel(), s1[k], None, 1)
        assert oracle.bit_equal(np.asarray(ps[k].data).ravel(), mine[k]), k
    for p, g in zip(ps, grads):
        assert oracle.bit_equal(np.asarray(p.grad), g * coef)


def test_skipped_step_after_overflow_keeps_parameters(T):
    """GradScaler::step after an unscale that found an overflow leaves every
    parameter as it was; update() backs the scale off; zero_grad clears the
    partly unscaled gradients."""
    grads = [rng(1000 + i).standard_normal(s).astype(np.float32) for i, s in enumerate(SHAPES)]
    grads[3][17] = np.nan
    ps = make(T, grads)
    before = [np.asarray(p.data).copy() for p in ps]
    opt = optimizer(T, "adamw", ps)
    scaler = T.GradScaler(256.0, 2.0, 0.5, 1000)
    scaler.step(opt)
    for p, b in zip(ps, before):
        assert oracle.bit_equal(np.asarray(p.data), b)
    scaler.update()
    assert scaler.get_scale() == 128.0
    inv = np.float32(1.0) / np.float32(256.0)
    assert oracle.bit_equal(np.asarray(ps[0].grad), grads[0] * inv)
    want3 = grads[3].copy()
    want3[:17] = want3[:17] * inv
    assert oracle.bit_equal(np.asarray(ps[3].grad), want3)
    opt.zero_grad()
    assert all(p.grad_known_zero for p in ps)


def test_negative_loss_scale_flips_zero_gradients(T):
    """A negative loss scale: 1 / scale < 0 multiplies known-zero gradients
    too (+0 becomes -0), as the reference's loop over every element does."""
    grads = [rng(1100 + i).standard_normal(s).astype(np.float32) for i, s in enumerate(SHAPES)]
    ps = make(T, grads)
    ps[1].zero_grad()
    grads[1] = np.zeros(SHAPES[1], np.float32)
    opt = T.SGD(ps, 0.1)
    scaler = T.GradScaler(-2.0, 2.0, 0.5, 1000)
    assert scaler.unscale(opt)
    inv = np.float32(1.0) / np.float32(-2.0)
    for p, g in zip(ps, grads):
        assert oracle.bit_equal(np.asarray(p.grad), g * inv)
