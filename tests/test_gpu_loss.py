"""GPU parity of the loss heads (include/wm_loss.h) through the C ABI.

Reference: core/loss.cpp (CrossEntropyLoss :67-97, NLLLoss :99-127,
FocalLoss :260-331, the element-wise losses :21-65 and :130-418), restated by
the oracle (pinned in test_oracle_loss.py).  Contract:
  - cross entropy: the per-row label term equals wm_log_softmax_fwd's entry
    bit for bit, and the fused backward equals the composition it replaces
    (the label scatter, then wm_log_softmax_bwd) bit for bit;
  - NLL backward: bit-exact against the fp32 oracle;
  - losses and gradients: within 1e-5 of the fp64 oracle relative to the sum
    of |terms| (the abs oracle), for the focal gradient plus the fp32
    representation floor of p (a few ulp of the scale: the gradient's
    sensitivity to p is bounded by gamma + 2).
"""
import numpy as np
import pytest

import oracle
from gpu_helpers import (ce_bwd, ce_fwd, dev, focal_bwd, focal_fwd, nll_bwd, nll_fwd, pw_bwd, pw_fwd, rng_normal,
                         rng_uniform, softmax_bwd, softmax_fwd)
from whitematter_amd import _lib as W
from whitematter_amd import synth

pytestmark = pytest.mark.gpu

o32, o64, oab = oracle.get("f32"), oracle.get("f64"), oracle.get("abs")

# register-tile rows (<= 32768 columns) and the online long-row path
SHAPES = [(1, 1), (4, 3), (33, 100), (16, 1000), (8, 2048), (4, 2049), (3, 10001), (2, 32000), (2, 32768),
          (2, 40000), (2, 50257), (300, 37)]


def logits(shape, seed):
    x = rng_normal(shape, seed, 3.0)
    return synth.spikes(x, seed, 0.01, 20.0)


def labels(rows, cols, seed):
    return np.floor(rng_uniform((rows,), seed, 0, cols)).clip(0, cols - 1).astype(np.float32)


def scalar_ok(got, ref64, scale64, rtol=1e-5):
    ok, worst = oracle.close_scaled(np.float32([got]), np.float64([ref64]), np.float64([scale64]), rtol)
    return ok, worst


# ---- cross entropy ---------------------------------------------------------------

@pytest.mark.parametrize("shape", SHAPES)
def test_cross_entropy_forward(wm, shape):
    x, lab = logits(shape, shape[1]), labels(shape[0], shape[1], 1)
    loss, stats = ce_fwd(x, lab)
    ok, worst = scalar_ok(loss, o64.cross_entropy(x, lab), oab.cross_entropy(x, lab))
    assert ok, f"{worst:.3g}x tolerance"
    li = lab.astype(np.int64)
    if shape[1] <= 32768:  # same row kernel as log_softmax
        lp = softmax_fwd(x, log=True)
        assert oracle.bit_equal(stats[:, 1], lp[np.arange(shape[0]), li])
    # mean of the per-row terms, negated: the same sum in fp64
    assert abs(np.float64(loss) + stats[:, 1].astype(np.float64).mean()) <= 1e-6 * abs(loss) + 1e-30


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("loss_grad", [1.0, 0.37])
@pytest.mark.parametrize("shape", [(4, 3), (33, 100), (8, 2048), (3, 10001), (2, 32000), (2, 40000), (1, 50257),
                                   (300, 37)])
def test_cross_entropy_backward(wm, shape, loss_grad, accumulate):
    x, lab = logits(shape, 3), labels(shape[0], shape[1], 4)
    g0 = rng_normal(shape, 5) if accumulate else None
    got = ce_bwd(x, lab, loss_grad, g0)
    ref = o64.cross_entropy_bwd(x, lab, loss_grad)
    scale = oab.cross_entropy_bwd(x, lab, loss_grad)
    if accumulate:
        ref, scale = ref + g0, scale + np.abs(g0)
    ok, worst = oracle.close_scaled(got, ref, scale, 1e-5, atol=1e-30)
    assert ok, f"{worst:.3g}x tolerance"
    if shape[1] <= 32768:
        # the composition the fused pass replaces: scatter -scale at the
        # labels, then log_softmax's backward on the stored log-probabilities
        rows = shape[0]
        sc = np.float32(loss_grad) / np.float32(rows)
        g = np.zeros(shape, np.float32)
        g[np.arange(rows), lab.astype(np.int64)] = np.float32(0) - sc
        comp = softmax_bwd(g, softmax_fwd(x, log=True), g0, log=True)
        assert oracle.bit_equal(got, comp)


def test_cross_entropy_rows_sum_to_zero_and_match_softmax(wm):
    """Each gradient row is (softmax - onehot) * scale: it sums to ~0 and its
    off-label entries are the softmax kernel's probabilities times scale."""
    shape = (64, 4096)
    x, lab = logits(shape, 6), labels(64, 4096, 7)
    g = ce_bwd(x, lab).astype(np.float64) * 64
    assert np.all(np.abs(g.sum(1)) <= 4096 * 2.0 ** -22)
    p = softmax_fwd(x).astype(np.float64)
    mask = np.ones(shape, bool)
    mask[np.arange(64), lab.astype(np.int64)] = False
    assert np.allclose(g[mask], p[mask], rtol=1e-5, atol=1e-30)


# ---- NLL -------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(1, 1), (4, 3), (300, 37), (1000, 1000), (70000, 3)])
def test_nll_forward(wm, shape):
    x, lab = rng_normal(shape, 8, 2.0), labels(shape[0], shape[1], 9)
    ok, worst = scalar_ok(nll_fwd(x, lab), o64.nll(x, lab), oab.nll(x, lab))
    assert ok, f"{worst:.3g}x tolerance"


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("shape", [(1, 1), (4, 3), (300, 37), (64, 1001), (1000, 1000)])
def test_nll_backward_bit_exact(wm, shape, accumulate):
    lab = labels(shape[0], shape[1], 10)
    g0 = rng_normal(shape, 11) if accumulate else None
    got = nll_bwd(shape, lab, 0.75, g0)
    want = o32.nll_bwd(shape, lab, 0.75)
    if accumulate:
        want = g0 + want  # the reference's grad -= scale at the labels
    assert oracle.bit_equal(got, want)


# ---- focal -------------------------------------------------------------------------

FOCAL = [(2.0, -1.0), (0.5, 0.25), (0.0, -1.0), (3.0, 0.75)]


def focal_floor(gamma, alpha, loss_grad, rows):
    a = 1.0 if alpha < 0 else alpha
    return 8 * 2.0 ** -24 * (gamma + 2) * a * abs(loss_grad) / rows


@pytest.mark.parametrize("gamma,alpha", FOCAL)
@pytest.mark.parametrize("shape", [(1, 1), (4, 3), (33, 100), (16, 1000), (4, 2049), (2, 32000), (2, 40000),
                                   (300, 37)])
def test_focal_forward(wm, shape, gamma, alpha):
    x, lab = rng_normal(shape, 12, 1.5), labels(shape[0], shape[1], 13)
    loss, _ = focal_fwd(x, lab, gamma, alpha)
    ok, worst = scalar_ok(loss, o64.focal(x, lab, gamma, alpha), oab.focal(x, lab, gamma, alpha))
    assert ok, f"{worst:.3g}x tolerance"


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("gamma,alpha", FOCAL)
@pytest.mark.parametrize("shape", [(4, 3), (33, 100), (8, 2048), (3, 10001), (2, 40000), (300, 37)])
def test_focal_backward(wm, shape, gamma, alpha, accumulate):
    x, lab = rng_normal(shape, 14, 1.5), labels(shape[0], shape[1], 15)
    g0 = rng_normal(shape, 16) if accumulate else None
    got = focal_bwd(x, lab, gamma, alpha, 0.6, g0)
    ref = o64.focal_bwd(x, lab, gamma, alpha, 0.6)
    scale = oab.focal_bwd(x, lab, gamma, alpha, 0.6)
    if accumulate:
        ref, scale = ref + g0, scale + np.abs(g0)
    ok, worst = oracle.close_scaled(got, ref, scale, 1e-5, atol=focal_floor(gamma, alpha, 0.6, shape[0]))
    assert ok, f"{worst:.3g}x tolerance"


def test_focal_confident_rows(wm):
    """The reference's confident-prediction case (test_loss.cpp:257-269) and
    spiked rows where p_t is within an ulp or two of 1."""
    x = np.float32([[-100, -100, 100], [0, 0, 30], [1, 2, 3]])
    lab = np.float32([2, 2, 0])
    loss, _ = focal_fwd(x, lab, 2.0, -1.0)
    ok, worst = scalar_ok(loss, o64.focal(x, lab), oab.focal(x, lab))
    assert ok, worst
    g = focal_bwd(x, lab, 2.0, -1.0)
    ok, worst = oracle.close_scaled(g, o64.focal_bwd(x, lab), oab.focal_bwd(x, lab), 1e-5,
                                    atol=focal_floor(2.0, -1.0, 1.0, 3))
    assert ok, worst


# ---- element-wise losses ------------------------------------------------------------

def pw_inputs(kind, n, seed):
    if kind == "smooth_l1":
        return rng_normal((n,), seed, 2.0), rng_normal((n,), seed + 1), 1.0, 0.0
    if kind == "bce":
        return rng_uniform((n,), seed, -0.05, 1.05), rng_uniform((n,), seed + 1, 0, 1), 0.0, 0.0
    if kind == "bce_logits":
        return rng_normal((n,), seed, 4.0), rng_uniform((n,), seed + 1, 0, 1), 0.0, 0.0
    if kind == "kldiv":
        return (np.log(rng_uniform((n,), seed, 0.01, 1)).astype(np.float32), rng_uniform((n,), seed + 1, -0.2, 1),
                0.0, 0.0)
    if kind == "kldiv_log":
        return (np.log(rng_uniform((n,), seed, 0.01, 1)).astype(np.float32),
                np.log(rng_uniform((n,), seed + 1, 0.01, 1)).astype(np.float32), 0.0, 0.0)
    return rng_normal((n,), seed, 3.0), (rng_uniform((n,), seed + 1, 0, 1) > 0.5).astype(np.float32), 2.0, 0.25


KINDS = ["smooth_l1", "bce", "bce_logits", "kldiv", "kldiv_log", "binary_focal"]


def grad_rtol(kind, x):
    """1e-5, except for the binary focal gradient.  That formula (core/loss.cpp:
    375-414) forms 1 - p and 1 - (1 - p) from the fp32 sigmoid p, so any fp32
    evaluation of it -- the reference's included -- carries a relative error
    of about 2^-24 / min(p, 1 - p) in those factors; the tolerance adds that
    amplification (16 ulp of it) element by element."""
    if kind != "binary_focal":
        return 1e-5
    p = 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))
    return 1e-5 + 16 * 2.0 ** -24 / np.maximum(np.minimum(p, 1.0 - p), 1e-300)


@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("n", [1, 7, 1000, 4099, 1 << 20])
@pytest.mark.parametrize("kind", KINDS)
def test_pointwise_forward(wm, kind, n, offset):
    x, y, p0, p1 = pw_inputs(kind, n, n % 97)
    denom = 10.0 if kind.startswith("kldiv") else None
    got = pw_fwd(kind, x, y, p0, p1, denom, offset)
    ok, worst = scalar_ok(got, o64.pointwise_loss(kind, x, y, p0, p1, denom),
                          oab.pointwise_loss(kind, x, y, p0, p1, denom))
    assert ok, f"{worst:.3g}x tolerance"


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("n", [1, 7, 4099, 1 << 18])
@pytest.mark.parametrize("kind", KINDS)
def test_pointwise_backward(wm, kind, n, offset, accumulate):
    x, y, p0, p1 = pw_inputs(kind, n, n % 89)
    g0 = rng_normal((n,), 17) if accumulate else None
    got = pw_bwd(kind, x, y, p0, p1, None, 0.8, g0, offset)
    ref = o64.pointwise_loss_bwd(kind, x, y, p0, p1, None, 0.8)
    scale = oab.pointwise_loss_bwd(kind, x, y, p0, p1, None, 0.8)
    if accumulate:
        ref, scale = ref + g0, scale + np.abs(g0)
    ok, worst = oracle.close_scaled(got, ref, scale, grad_rtol(kind, x), atol=1e-30)
    assert ok, f"{worst:.3g}x tolerance"


def test_pointwise_gamma_zero_binary_focal_and_special_values(wm):
    """gamma = 0 takes the closure's other branch (core/loss.cpp:396-398);
    NaN inputs propagate through the reference's std::max / std::min clamp."""
    x = np.float32([0.5, -3.0, np.nan, 2.0])
    y = np.float32([1.0, 0.0, 1.0, 0.0])
    for kind, p0, p1 in (("binary_focal", 0.0, -1.0), ("bce", 0.0, 0.0), ("bce_logits", 0.0, 0.0)):
        xx = np.clip(x, 0, 1) if kind == "bce" else x.copy()
        xx[2] = np.nan
        assert np.isnan(pw_fwd(kind, xx, y, p0, p1))
        g = pw_bwd(kind, xx, y, p0, p1)
        ref = o64.pointwise_loss_bwd(kind, xx, y, p0, p1)
        assert np.array_equal(np.isnan(g), np.isnan(ref))
        fin = ~np.isnan(ref)
        rt = grad_rtol(kind, xx)
        rt = rt[fin] if np.ndim(rt) else rt
        assert np.all(np.abs(g[fin] - ref[fin]) <= rt * np.abs(ref[fin]) + 1e-30)


# ---- edge cases ------------------------------------------------------------------

def test_invalid_labels_poison_rows(wm):
    x = logits((4, 50), 18)
    for bad in (50.0, -1.0, np.nan, 1e30):
        lab = np.float32([0, 1, bad, 49])
        loss, _ = ce_fwd(x, lab)
        assert np.isnan(loss) and np.isnan(focal_fwd(x, lab, 2.0, -1.0)[0]) and np.isnan(nll_fwd(x, lab))
        g = ce_bwd(x, lab)
        assert np.isnan(g[2]).all() and np.isfinite(np.delete(g, 2, 0)).all()
        gf = focal_bwd(x, lab, 2.0, -1.0)
        assert np.isnan(gf[2]).all() and np.isfinite(np.delete(gf, 2, 0)).all()
        gn = nll_bwd(x.shape, lab)
        assert (gn[2] == 0).all() and gn[0, 0] == np.float32(-0.25)
    # truncation toward zero, as static_cast<size_t>
    a, _ = ce_fwd(x, np.float32([0, 1, 2, 49]))
    b, _ = ce_fwd(x, np.float32([-0.5, 1.9, 2.2, 49.99]))
    assert a == b


def test_empty_batch_is_nan(wm):
    """The reference divides the empty sum by batch_size = 0."""
    x = np.zeros((0, 5), np.float32)
    assert np.isnan(ce_fwd(x, np.zeros(0, np.float32))[0])
    assert np.isnan(nll_fwd(x, np.zeros(0, np.float32)))
    assert np.isnan(focal_fwd(x, np.zeros(0, np.float32), 2.0, -1.0)[0])
    assert np.isnan(pw_fwd("bce_logits", np.zeros(0, np.float32), np.zeros(0, np.float32)))


def test_bad_arguments_rejected(wm):
    with pytest.raises(W.WMError):
        W.call("wm_cross_entropy_fwd", W.nullp(), W.nullp(), -1, 3, W.nullp(), W.nullp())
    with pytest.raises(W.WMError):
        W.call("wm_pointwise_loss_fwd", 99, W.nullp(), W.nullp(), 0, 0.0, 0.0, 1.0, dev(np.zeros(1, np.float32)).vp)
    x = dev(np.zeros((2, 0), np.float32))
    with pytest.raises(W.WMError):  # no class can be valid
        W.call("wm_cross_entropy_fwd", x.vp, dev(np.zeros(2, np.float32)).vp, 2, 0,
               dev(np.zeros(4, np.float32)).vp, dev(np.zeros(1, np.float32)).vp)


def test_deterministic(wm):
    x, lab = logits((512, 4096), 19), labels(512, 4096, 20)
    assert ce_fwd(x, lab)[0] == ce_fwd(x, lab)[0]
    assert oracle.bit_equal(focal_bwd(x, lab, 2.0, -1.0), focal_bwd(x, lab, 2.0, -1.0))


def test_full_size_cross_entropy(wm):
    """logits [8192, 32000] (the softmax config's shape): the fused forward's
    terms equal log_softmax's entries at the labels bit for bit, the loss is
    their mean, and the fused backward equals the composition bit for bit."""
    rows, cols = 8192, 32000
    x = synth.spikes(synth.normal((rows, cols), synth.seed_for(4, 0), 0.0, 3.0), synth.seed_for(4, 1))
    lab = labels(rows, cols, 21)
    loss, stats = ce_fwd(x, lab)
    lp = softmax_fwd(x, log=True)
    li = lab.astype(np.int64)
    assert oracle.bit_equal(stats[:, 1], lp[np.arange(rows), li])
    want = -lp[np.arange(rows), li].astype(np.float64).mean()
    assert abs(loss - want) <= 1e-6 * abs(want)
    g = np.zeros((rows, cols), np.float32)
    g[np.arange(rows), li] = np.float32(0) - np.float32(1.0) / np.float32(rows)
    comp = softmax_bwd(g, lp, None, log=True)
    del g, lp
    assert oracle.bit_equal(ce_bwd(x, lab), comp)
