"""CPU tests that pin the loss oracle (the or_cross_entropy / or_nll /
or_focal / or_pointwise_loss functions of oracle/wm_oracle.c and their
backward passes) before it checks the GPU loss heads:

1. the reference's own known answers (tests/test_loss.cpp:74-300);
2. the compiled reference (oracle/_ref: core/loss.cpp with core/tensor.cpp)
   in two builds of the same sources: IEEE semantics (libwmref_ieee.so), where
   the fp32 oracle agrees to a few ulp (the only difference is how the float
   exp/log/pow are rounded), and the reference's own -ffast-math build
   (libwmref.so) within the 1e-5 contract of the fp64 oracle;
3. identities between the losses that the mathematics fixes: focal loss with
   gamma = 0 is (alpha times) cross entropy, NLL of log_softmax is cross
   entropy, BCE-with-logits is BCE of the sigmoid, binary focal with gamma = 0
   and no alpha is BCE-with-logits, KL with a log target equals KL with the
   probabilities, smooth L1 with a large beta is MSE / (2 beta); closed forms
   (cross entropy = mean(logsumexp - x_label), its gradient = (softmax -
   onehot) / batch);
4. central finite differences of every fp64 loss against its fp64 gradient,
   so a dropped term, a wrong sign or a transposed index in any backward
   fails.
"""
import numpy as np
import pytest

import oracle

o32, o64, oab = oracle.get("f32"), oracle.get("f64"), oracle.get("abs")
try:
    ref = oracle.Reference()
    ref_ieee = oracle.Reference(oracle.REF_IEEE_PATH)
except FileNotFoundError:
    ref = ref_ieee = None
needs_ref = pytest.mark.skipif(ref is None, reason="oracle/_ref not built (reference sources absent)")


def rng(seed):
    return np.random.default_rng(seed)


def logits(rows, cols, seed, std=3.0):
    return (rng(seed).standard_normal((rows, cols)) * std).astype(np.float32)


def labels(rows, cols, seed):
    return rng(seed).integers(0, cols, rows).astype(np.float32)


def pointwise_inputs(kind, n, seed):
    """(pred, target, p0, p1) in each loss's natural domain."""
    r = rng(seed)
    if kind == "smooth_l1":
        return r.standard_normal(n).astype(np.float32) * 2, r.standard_normal(n).astype(np.float32), 1.0, 0.0
    if kind == "bce":
        return r.uniform(0.02, 0.98, n).astype(np.float32), r.uniform(0, 1, n).astype(np.float32), 0.0, 0.0
    if kind == "bce_logits":
        return (r.standard_normal(n) * 3).astype(np.float32), r.uniform(0, 1, n).astype(np.float32), 0.0, 0.0
    if kind == "kldiv":
        return np.log(r.uniform(0.01, 1, n)).astype(np.float32), r.uniform(-0.2, 1, n).astype(np.float32), 0.0, 0.0
    if kind == "kldiv_log":
        return (np.log(r.uniform(0.01, 1, n)).astype(np.float32), np.log(r.uniform(0.01, 1, n)).astype(np.float32),
                0.0, 0.0)
    return (r.standard_normal(n) * 3).astype(np.float32), (r.uniform(0, 1, n) > 0.5).astype(np.float32), 2.0, 0.25


POINTWISE = ["smooth_l1", "bce", "bce_logits", "kldiv", "kldiv_log", "binary_focal"]


def ref_pointwise(R, kind, x, y, p0, p1, rows):
    """The reference's loss class for `kind`, with x and y viewed as [rows, -1]."""
    shape = (rows, x.size // rows)
    if kind.startswith("kldiv"):
        return R.loss("kldiv", x, y, 1.0 if kind == "kldiv_log" else 0.0, 0.0, shape, shape)
    return R.loss(kind, x, y, p0, p1, shape, shape)


def denom_of(kind, x, rows):
    return rows if kind.startswith("kldiv") else x.size


# ---- 1. the reference's known answers ----------------------------------------

def test_known_answers_from_reference_tests():
    # test_smooth_l1_loss (test_loss.cpp:74-85): 0.8125
    assert abs(o32.pointwise_loss("smooth_l1", np.float32([0.5, 2.0]), np.float32([0, 0]), 1.0) - 0.8125) < 1e-6
    # test_nll_loss (:139-152): -log(0.7)
    pred = np.log(np.float32([[0.1, 0.7, 0.2]])).astype(np.float32)
    assert abs(o32.nll(pred, np.float32([1])) - (-np.log(np.float32(0.7)))) < 1e-6
    # test_bce_loss (:158-169): -(log 0.8 + log 0.8) / 2
    exp_bce = -(np.log(np.float32(0.8)) + np.log(np.float32(0.8))) / 2
    assert abs(o32.pointwise_loss("bce", np.float32([0.8, 0.2]), np.float32([1, 0])) - exp_bce) < 1e-6
    # test_bce_loss_perfect (:171-180): clamped, < 0.1
    assert o32.pointwise_loss("bce", np.float32([1, 0]), np.float32([1, 0])) < 0.1
    # test_bce_with_logits_gradient (:197-208): -0.5 at logit 0, target 1
    assert o32.pointwise_loss_bwd("bce_logits", np.float32([0]), np.float32([1]))[0] == np.float32(-0.5)
    # test_bce_with_logits_loss (:185-195): positive
    assert o32.pointwise_loss("bce_logits", np.float32([2, -2]), np.float32([1, 0])) > 0
    # test_kl_div_loss_same (:230-241): 0 for identical distributions (log_ adds 1e-8)
    p = np.float32([0.5, 0.3, 0.2])
    lp = np.log(p + np.float32(1e-8)).astype(np.float32)
    assert abs(o32.pointwise_loss("kldiv", lp.reshape(1, 3), p.reshape(1, 3), denom=1)) < 1e-4
    # test_kl_div_loss (:214-228): >= 0 (Gibbs)
    lq = np.log(np.float32([0.5, 0.3, 0.2])).astype(np.float32)
    assert o32.pointwise_loss("kldiv", lq.reshape(1, 3), np.float32([[0.4, 0.4, 0.2]]), denom=1) >= -1e-5
    # test_cross_entropy_loss / _perfect_prediction / _gradient (:91-134)
    x = np.float32([[1, 2, 3], [1, 2, 3]])
    assert o32.cross_entropy(x, np.float32([2, 0])) > 0
    assert o32.cross_entropy(np.float32([[-100, -100, 100]]), np.float32([2])) < 0.1
    g = o32.cross_entropy_bwd(np.float32([[1, 2, 3]]), np.float32([1]))
    assert g.shape == (1, 3) and g[0, 1] < 0 < g[0, 0] < g[0, 2]
    # test_focal_loss (:247-255), test_focal_loss_confident (:257-269)
    assert o32.focal(np.float32([[1, 2, 3]]), np.float32([2]), 2.0, -1.0) > 0
    assert o32.focal(np.float32([[-100, -100, 100]]), np.float32([2]), 2.0, -1.0) < 1e-5
    # test_binary_focal_loss (:273-281), _hard_example (:283-299)
    assert o32.pointwise_loss("binary_focal", np.float32([2, -2]), np.float32([1, 0]), 2.0, 0.25) > 0
    hard = o32.pointwise_loss("binary_focal", np.float32([-3]), np.float32([1]), 2.0, 0.5)
    easy = o32.pointwise_loss("binary_focal", np.float32([3]), np.float32([1]), 2.0, 0.5)
    assert hard > easy


# ---- 2. the compiled reference -------------------------------------------------

HEADS = [("cross_entropy", (64, 37)), ("cross_entropy", (5, 1000)), ("nll", (64, 37)), ("focal", (64, 37)),
         ("focal", (7, 300))]


def oracle_head(o, kind, x, lab, gamma=2.0, alpha=-1.0):
    if kind == "cross_entropy":
        return o.cross_entropy(x, lab), o.cross_entropy_bwd(x, lab)
    if kind == "nll":
        return o.nll(x, lab), o.nll_bwd(x.shape, lab)
    return o.focal(x, lab, gamma, alpha), o.focal_bwd(x, lab, gamma, alpha)


@needs_ref
@pytest.mark.parametrize("kind,shape", HEADS)
@pytest.mark.parametrize("gamma,alpha", [(2.0, -1.0), (0.5, 0.25)])
def test_heads_match_ieee_reference(kind, shape, gamma, alpha):
    if kind != "focal" and (gamma, alpha) != (2.0, -1.0):
        pytest.skip("gamma/alpha only parameterise the focal loss")
    x, lab = logits(*shape, 1), labels(shape[0], shape[1], 2)
    v_ref, g_ref = ref_ieee.loss(kind, x, lab, gamma, alpha)
    v, g = oracle_head(o32, kind, x, lab, gamma, alpha)
    assert oracle.ulp_distance(np.float32([v]), np.float32([v_ref])).max() <= 2
    assert oracle.ulp_distance(g, g_ref).max() <= 4
    if kind == "nll":
        assert oracle.bit_equal(g, g_ref)


@needs_ref
@pytest.mark.parametrize("kind", POINTWISE)
def test_pointwise_match_ieee_reference(kind):
    x, y, p0, p1 = pointwise_inputs(kind, 2000, 3)
    rows = 40
    v_ref, g_ref = ref_pointwise(ref_ieee, kind, x, y, p0, p1, rows)
    d = denom_of(kind, x, rows)
    v = o32.pointwise_loss(kind, x, y, p0, p1, d)
    g = o32.pointwise_loss_bwd(kind, x, y, p0, p1, d)
    assert oracle.ulp_distance(np.float32([v]), np.float32([v_ref])).max() <= 2
    assert oracle.ulp_distance(g, g_ref.ravel()).max() <= 4


@needs_ref
@pytest.mark.parametrize("kind,shape", HEADS)
def test_heads_fastmath_reference_within_contract(kind, shape):
    """The reference's own build is within 1e-5 of the fp64 oracle."""
    x, lab = logits(*shape, 4), labels(shape[0], shape[1], 5)
    v_ref, g_ref = ref.loss(kind, x, lab, 2.0, -1.0)
    v64, g64 = oracle_head(o64, kind, x, lab)
    vab, gab = oracle_head(oab, kind, x, lab)
    assert oracle.close_scaled(np.float32([v_ref]), np.float64([v64]), np.float64([vab]), 1e-5)[0]
    ok, worst = oracle.close_scaled(g_ref, g64, gab, 1e-5, atol=1e-12)
    assert ok, worst


@needs_ref
@pytest.mark.parametrize("kind", POINTWISE)
def test_pointwise_fastmath_reference_within_contract(kind):
    x, y, p0, p1 = pointwise_inputs(kind, 2000, 6)
    rows = 40
    v_ref, g_ref = ref_pointwise(ref, kind, x, y, p0, p1, rows)
    d = denom_of(kind, x, rows)
    v64 = o64.pointwise_loss(kind, x, y, p0, p1, d)
    vab = oab.pointwise_loss(kind, x, y, p0, p1, d)
    assert oracle.close_scaled(np.float32([v_ref]), np.float64([v64]), np.float64([vab]), 1e-5)[0]
    g64 = o64.pointwise_loss_bwd(kind, x, y, p0, p1, d)
    gab = oab.pointwise_loss_bwd(kind, x, y, p0, p1, d)
    # The fast-math build's reciprocal-based division costs a few ulp of each
    # term of the gradient formula.
    ok, worst = oracle.close_scaled(g_ref.ravel(), g64, gab, 1e-5, atol=1e-12)
    assert ok, worst


# ---- 3. identities and closed forms --------------------------------------------

def test_focal_gamma_zero_is_cross_entropy():
    """Forward: focal loss with gamma = 0 is alpha * cross entropy.  Backward:
    the reference's closure (core/loss.cpp:307-318) writes +(1-p_t)^gamma
    where the derivative of its forward has -(1-p_t)^gamma (see
    focal_closure_discrepancy), so at gamma = 0 its gradient is exactly the
    negated cross-entropy gradient.  Parity is with the reference."""
    x, lab = logits(50, 40, 7), labels(50, 40, 8)
    ce, gce = o64.cross_entropy(x, lab), o64.cross_entropy_bwd(x, lab)
    for alpha in (-1.0, 0.3):
        a = 1.0 if alpha < 0 else float(np.float32(alpha))
        fl, gfl = o64.focal(x, lab, 0.0, alpha), o64.focal_bwd(x, lab, 0.0, alpha)
        assert abs(fl - a * ce) <= 1e-12 * abs(ce)
        assert np.allclose(gfl, -a * gce, rtol=0, atol=1e-14)


def focal_closure_discrepancy(x, lab, gamma, alpha, loss_grad=1.0):
    """The reference's focal closure minus the derivative of its forward:
    2 (1-p_t)^gamma (onehot - p) * alpha * loss_grad / batch, from
      closure, label:  p_t (gamma log(p_t) q^g - q^g) + q^g
      derivative:      gamma p_t q^g log(p_t) - q^(g+1)
      closure, other:  -p_c q^(g-1) (gamma p_t log(p_t) + q)
      derivative:      -p_c q^(g-1) (gamma p_t log(p_t) - q)
    with q = 1 - p_t (p_t clamped at 1e-7, inactive here)."""
    xd = x.astype(np.float64)
    p = np.exp(xd - xd.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    rows = x.shape[0]
    li = lab.astype(np.int64)
    q = 1 - p[np.arange(rows), li]
    onehot = np.zeros_like(p)
    onehot[np.arange(rows), li] = 1
    a = 1.0 if alpha < 0 else float(np.float32(alpha))
    return 2 * (q ** gamma)[:, None] * (onehot - p) * a * loss_grad / rows


def test_cross_entropy_closed_form_and_nll_of_log_softmax():
    x, lab = logits(30, 25, 9), labels(30, 25, 10)
    xd = x.astype(np.float64)
    lse = np.log(np.exp(xd - xd.max(1, keepdims=True)).sum(1)) + xd.max(1)
    li = lab.astype(np.int64)
    want = np.mean(lse - xd[np.arange(30), li])
    assert abs(o64.cross_entropy(x, lab) - want) <= 1e-12 * want
    p = np.exp(xd - lse[:, None])
    onehot = np.zeros_like(p)
    onehot[np.arange(30), li] = 1
    assert np.allclose(o64.cross_entropy_bwd(x, lab), (p - onehot) / 30, rtol=0, atol=1e-15)
    assert np.allclose(o64.cross_entropy_bwd(x, lab, 2.5), 2.5 * (p - onehot) / 30, rtol=0, atol=1e-15)
    ls = o32.softmax(x, log=True)
    assert abs(o64.nll(ls, lab) - want) <= 1e-6 * want


def test_bce_logits_is_bce_of_sigmoid_and_binary_focal_gamma_zero():
    r = rng(11)
    x = (r.standard_normal(500) * 3).astype(np.float32)
    y = r.uniform(0, 1, 500).astype(np.float32)
    s = (1 / (1 + np.exp(-x.astype(np.float64))))
    yd = y.astype(np.float64)
    # BCE on the sigmoid in fp64 (no fp32 rounding of the probability)
    bce = -np.mean(yd * np.log(s) + (1 - yd) * np.log(1 - s))
    assert abs(o64.pointwise_loss("bce_logits", x, y) - bce) <= 1e-12 * bce
    assert np.allclose(o64.pointwise_loss_bwd("bce_logits", x, y), (s - yd) / 500, rtol=1e-12, atol=1e-18)
    # binary focal, gamma = 0 and no alpha: BCE-with-logits for 0/1 targets
    # (its p_t form needs y in {0, 1}) where the probability clamp is inactive
    yb = (y > 0.5).astype(np.float32)
    bf = o64.pointwise_loss("binary_focal", x, yb, 0.0, -1.0)
    assert abs(bf - o64.pointwise_loss("bce_logits", x, yb)) <= 1e-12 * bf
    assert np.allclose(o64.pointwise_loss_bwd("binary_focal", x, yb, 0.0, -1.0),
                       o64.pointwise_loss_bwd("bce_logits", x, yb), rtol=1e-10, atol=0)


def test_kldiv_log_target_and_smooth_l1_large_beta():
    r = rng(12)
    x = np.log(r.uniform(0.01, 1, 300)).astype(np.float32)
    t = r.uniform(0.01, 1, 300).astype(np.float32)
    lt = np.log(t.astype(np.float64)).astype(np.float32)
    a, b = o64.pointwise_loss("kldiv", x, t, denom=3), o64.pointwise_loss("kldiv_log", x, lt, denom=3)
    assert abs(a - b) <= 1e-6 * abs(a)  # t and exp(log t) differ by fp32 rounding of log t
    # KL of a distribution with itself: 0
    assert abs(o64.pointwise_loss("kldiv", np.log(t.astype(np.float64)).astype(np.float32), t)) < 1e-7
    p, q = r.standard_normal(300).astype(np.float32), r.standard_normal(300).astype(np.float32)
    beta = 100.0
    mse = np.mean((p.astype(np.float64) - q) ** 2)
    assert abs(o64.pointwise_loss("smooth_l1", p, q, beta) - 0.5 * mse / beta) <= 1e-12 * mse


def test_label_reading_rules():
    """Labels truncate toward zero like static_cast<size_t>; anything that is
    not a class gives a NaN term, a NaN cross-entropy row gradient and no NLL
    scatter."""
    x = logits(4, 5, 13)
    base = o64.cross_entropy(x, np.float32([0, 1, 2, 4]))
    assert o64.cross_entropy(x, np.float32([-0.5, 1.9, 2.2, 4.99])) == base
    for bad in (5.0, -1.0, np.nan, 1e30):
        lab = np.float32([0, 1, bad, 4])
        assert np.isnan(o64.cross_entropy(x, lab)) and np.isnan(o64.focal(x, lab)) and np.isnan(o64.nll(x, lab))
        g = o64.cross_entropy_bwd(x, lab)
        assert np.isnan(g[2]).all() and np.isfinite(np.delete(g, 2, 0)).all()
        assert np.isnan(o64.focal_bwd(x, lab)[2]).all()
        gn = o64.nll_bwd(x.shape, lab)
        assert (gn[2] == 0).all() and gn[0, 0] == -0.25


# ---- 4. finite differences -------------------------------------------------------

def fd_check(f, grad, x, idx, h=1e-2, rtol=2e-4):
    """Central differences of f (an fp64 loss of an fp32 array) at the flat
    positions idx, against grad.  The fp32 step is exactly representable."""
    g = grad.ravel()
    for i in idx:
        xp, xm = x.copy(), x.copy()
        xp.flat[i] += np.float32(h)
        xm.flat[i] -= np.float32(h)
        hh = (np.float64(xp.flat[i]) - np.float64(xm.flat[i]))
        num = (f(xp) - f(xm)) / hh
        assert abs(num - g[i]) <= rtol * max(abs(num), 1e-3 * np.abs(g).max()), (i, num, g[i])


@pytest.mark.parametrize("gamma,alpha", [(2.0, -1.0), (1.5, 0.25), (0.0, -1.0)])
def test_head_gradients_finite_differences(gamma, alpha):
    x, lab = logits(6, 9, 14, 1.5), labels(6, 9, 15)
    idx = list(range(0, x.size, 5)) + [int(r * 9 + lab[r]) for r in range(6)]
    fd_check(lambda z: o64.cross_entropy(z, lab), o64.cross_entropy_bwd(x, lab), x, idx)
    fd_check(lambda z: o64.nll(z, lab), o64.nll_bwd(x.shape, lab), x, idx)
    # The focal closure is the reference's: the derivative of the forward
    # plus the closed-form sign discrepancy of its (1-p_t)^gamma term.
    g = o64.focal_bwd(x, lab, gamma, alpha)
    fd_check(lambda z: o64.focal(z, lab, gamma, alpha), g - focal_closure_discrepancy(x, lab, gamma, alpha), x, idx)
    assert np.abs(focal_closure_discrepancy(x, lab, gamma, alpha)).max() > 1e-3  # the discrepancy is real


@pytest.mark.parametrize("kind", POINTWISE)
def test_pointwise_gradients_finite_differences(kind):
    x, y, p0, p1 = pointwise_inputs(kind, 64, 16)
    if kind == "smooth_l1":  # keep clear of the |d| = beta kink
        d = x - y
        x = np.where(np.abs(np.abs(d) - 1.0) < 0.05, x + np.float32(0.2), x).astype(np.float32)
    h = 1e-4 if kind in ("bce", "kldiv", "kldiv_log") else 1e-2
    g = o64.pointwise_loss_bwd(kind, x, y, p0, p1)
    if kind == "kldiv":
        # The reference's closure (core/loss.cpp:244-253) gives every element
        # -target * scale, but its forward skips targets <= 0 (:229-231), so
        # for a negative target the closure is not the loss's derivative.
        neg = y < 0
        assert neg.any() and np.all(g[neg] == -y[neg].astype(np.float64) / x.size)
        g = np.where(neg, 0.0, g)
    fd_check(lambda z: o64.pointwise_loss(kind, z, y, p0, p1), g, x, range(0, 64, 3), h)
