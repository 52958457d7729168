"""CPU tests that pin the parameter-update oracle (the or_*_step, clipping and
unscaling functions of oracle/wm_oracle.c) before it checks the GPU kernels:

1. the reference's own known answers (tests/test_optimizer.cpp:266-313 for
   clip_grad_value_ / get_grad_norm);
2. the compiled reference (oracle/_ref: core/optimizer.cpp and core/amp.h's
   GradScaler) in two builds of the same sources: with IEEE semantics
   (libwmref_ieee.so) bit for bit over several steps, and with the
   reference's own -ffast-math flags (libwmref.so) within 1e-5 of the update
   terms, since that build's reciprocal division and contracted updates
   differ from IEEE in the last bits;
3. closed forms the update rules fix: SGD with momentum under a constant
   gradient, Adam's first step (|update| = lr |g| / (|g| + eps)), RMSprop's
   first step, AdamW's decay with a zero gradient.
"""
import numpy as np
import pytest

import oracle

o32 = oracle.get("f32")
try:
    ref = oracle.Reference()
    ref_ieee = oracle.Reference(oracle.REF_IEEE_PATH)
except FileNotFoundError:
    ref = ref_ieee = None
needs_ref = pytest.mark.skipif(ref is None, reason="oracle/_ref not built (reference sources absent)")

CONFIGS = [
    ("sgd", dict(lr=0.05, a=0.0)),
    ("sgd", dict(lr=0.05, a=0.9)),
    ("adam", dict(lr=1e-3, a=0.9, b=0.999, c=1e-8)),
    ("adamw", dict(lr=1e-3, a=0.9, b=0.999, c=1e-8, d=0.01)),
    ("rmsprop", dict(lr=1e-2, a=0.99, b=1e-8, c=0.0, d=0.0)),
    ("rmsprop", dict(lr=1e-2, a=0.9, b=1e-6, c=0.9, d=0.05)),
]


def rng(seed):
    return np.random.default_rng(seed)


class OracleOptimizer:
    """The oracle's update functions driven the way the reference's step()
    drives its loops: state zero-initialised, Adam's t incremented first."""

    def __init__(self, kind, params, lr, a=0.0, b=0.0, c=0.0, d=0.0):
        self.kind, self.params, self.lr, self.h = kind, params, lr, (a, b, c, d)
        z = [np.zeros_like(p) for p in params]
        self.s1 = z
        self.s2 = [np.zeros_like(p) for p in params]
        self.t = 0

    def step(self, grads):
        a, b, c, d = self.h
        if self.kind in ("adam", "adamw"):
            self.t += 1
            bc1, bc2 = o32.bias_correction(a, self.t), o32.bias_correction(b, self.t)
        for p, g, s1, s2 in zip(self.params, grads, self.s1, self.s2):
            if self.kind == "sgd":
                o32.sgd_step(p, g, s1, self.lr, a)
            elif self.kind in ("adam", "adamw"):
                o32.adam_step(p, g, s1, s2, self.lr, a, b, c, bc1, bc2, d, self.kind == "adamw")
            else:
                o32.rmsprop_step(p, g, s1, s2, self.lr, a, b, c, d)


@needs_ref
@pytest.mark.parametrize("kind,hp", CONFIGS, ids=lambda v: v if isinstance(v, str) else "-".join(map(str, v.values())))
def test_steps_match_reference(kind, hp):
    shapes = [(37,), (16, 9), (1000,)]
    params = [rng(i).standard_normal(s).astype(np.float32) for i, s in enumerate(shapes)]
    tps = [ref.tensor(p, True) for p in params]
    ropt = ref.optimizer(kind, tps, **hp)
    mine = [p.copy() for p in params]
    oopt = OracleOptimizer(kind, mine, **hp)
    for step in range(4):
        grads = [rng(100 + 10 * step + i).standard_normal(p.shape).astype(np.float32) for i, p in enumerate(params)]
        before = [p.copy() for p in mine]
        for tp, g in zip(tps, grads):
            tp.set_grad(g)
        ropt.step()
        oopt.step(grads)
        for tp, g, p0, p1 in zip(tps, grads, before, mine):
            # The reference contracts p - lr * u into one fused multiply-add
            # (its new p may differ by the rounding of p itself), and its
            # fast-math division / square root differ from IEEE by ~1e-7 of
            # the terms, which momentum buffers can cancel; so the bound is
            # relative to lr * (1 + |g|), the size of those terms.  A wrong
            # term, sign or order of operations moves p by O(lr).
            d_ref = tp.data().astype(np.float64) - p0
            d_or = p1.astype(np.float64) - p0
            lim = 1e-5 * (np.abs(d_or) + hp["lr"] * (1 + np.abs(g))) + 2 * np.spacing(np.abs(p1)).astype(np.float64)
            assert np.all(np.abs(d_ref - d_or) <= lim), (kind, step)


@needs_ref
@pytest.mark.parametrize("kind,hp", CONFIGS, ids=lambda v: v if isinstance(v, str) else "-".join(map(str, v.values())))
def test_steps_match_reference_ieee_bitexact(kind, hp):
    """The reference source compiled without fast-math gives the oracle's
    parameters and state bit for bit over several steps."""
    shapes = [(37,), (16, 9), (1000,)]
    params = [rng(i).standard_normal(s).astype(np.float32) for i, s in enumerate(shapes)]
    tps = [ref_ieee.tensor(p, True) for p in params]
    ropt = ref_ieee.optimizer(kind, tps, **hp)
    mine = [p.copy() for p in params]
    oopt = OracleOptimizer(kind, mine, **hp)
    for step in range(5):
        grads = [rng(300 + 10 * step + i).standard_normal(p.shape).astype(np.float32) for i, p in enumerate(params)]
        for tp, g in zip(tps, grads):
            tp.set_grad(g)
        ropt.step()
        oopt.step(grads)
        for tp, p1 in zip(tps, mine):
            assert oracle.bit_equal(tp.data(), p1), (kind, step)


def test_sgd_momentum_constant_gradient_closed_form():
    """v_k = g (1 - mu^k) / (1 - mu);  p_k = p_0 - lr sum_i v_i."""
    p0 = rng(1).standard_normal(64).astype(np.float32)
    g = rng(2).standard_normal(64).astype(np.float32)
    lr, mu = np.float32(0.1), np.float32(0.5)
    p, v = p0.copy(), np.zeros_like(p0)
    for _ in range(6):
        o32.sgd_step(p, g, v, lr, mu)
    k = np.arange(1, 7)
    vk = g[None, :].astype(np.float64) * ((1 - 0.5 ** k) / 0.5)[:, None]
    assert np.allclose(v, vk[-1], rtol=1e-6)
    assert np.allclose(p, p0 - 0.1 * vk.sum(axis=0), rtol=1e-5, atol=1e-6)


def test_adam_first_step_closed_form():
    """m_hat = g and v_hat = g^2 on step 1, so p_1 = p_0 - lr g / (|g| + eps)."""
    p0 = rng(3).standard_normal(256).astype(np.float32)
    g = (rng(4).standard_normal(256) * np.logspace(-6, 2, 256)).astype(np.float32)
    lr, eps = 1e-2, 1e-8
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    o32.adam_step(p, g, m, v, lr, 0.9, 0.999, eps, o32.bias_correction(0.9, 1), o32.bias_correction(0.999, 1))
    g64 = g.astype(np.float64)
    expect = p0 - lr * g64 / (np.abs(g64) + eps)
    assert np.allclose(p, expect, rtol=1e-6, atol=1e-7)
    omb1, omb2 = np.float32(1) - np.float32(0.9), np.float32(1) - np.float32(0.999)
    assert np.allclose(m, float(omb1) * g64, rtol=1e-6) and np.allclose(v, float(omb2) * g64 * g64, rtol=1e-6)


def test_bias_correction_is_double_pow():
    """1.0f - std::pow(beta, t) goes through the double pow (core/optimizer.cpp:48)."""
    for beta in (0.9, 0.999, 0.5):
        for t in (1, 2, 10, 1000):
            b32 = np.float32(beta)
            assert o32.bias_correction(b32, t) == np.float32(1.0 - float(b32) ** t)


def test_adamw_decay_only():
    """With g = 0, AdamW reduces to p_1 = p_0 - lr * wd * p_0 (m = v = 0)."""
    p0 = rng(5).standard_normal(100).astype(np.float32)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    o32.adam_step(p, np.zeros_like(p0), m, v, 0.1, 0.9, 0.999, 1e-8, o32.bias_correction(0.9, 1),
                  o32.bias_correction(0.999, 1), 0.01, True)
    assert np.allclose(p, p0 - 0.1 * 0.01 * p0.astype(np.float64), rtol=1e-6)


def test_rmsprop_first_step_closed_form():
    """v_1 = (1 - a) g^2, so p_1 = p_0 - lr g / (sqrt(1 - a) |g| + eps)."""
    p0 = rng(6).standard_normal(128).astype(np.float32)
    g = rng(7).standard_normal(128).astype(np.float32)
    p, v = p0.copy(), np.zeros_like(p0)
    o32.rmsprop_step(p, g, v, None, 0.01, 0.99, 1e-8, 0.0, 0.0)
    g64 = g.astype(np.float64)
    assert np.allclose(p, p0 - 0.01 * g64 / (np.sqrt(0.01) * np.abs(g64) + 1e-8), rtol=1e-5, atol=1e-7)


def test_clip_value_and_norm_kats():
    """tests/test_optimizer.cpp:284-313: clip 10 -> 8, -20 -> -8, 5 kept;
    ||[1,2,2]|| = 3, ||[0,0,0,4]|| = 4."""
    g = np.array([10.0, -20.0, 5.0, np.nan], np.float32)
    o32.clip_grad_value(g, 8.0)
    assert g[0] == 8.0 and g[1] == -8.0 and g[2] == 5.0 and np.isnan(g[3])
    assert np.sqrt(o32.grad_sumsq(np.array([1.0, 2.0, 2.0], np.float32))) == 3.0
    assert np.sqrt(o32.grad_sumsq(np.array([0.0, 0.0, 0.0, 4.0], np.float32))) == 4.0


@needs_ref
def test_clipping_matches_reference():
    grads = [rng(10 + i).standard_normal(n).astype(np.float32) * 3 for i, n in enumerate((50, 200, 7))]
    tps = [ref.tensor(np.zeros_like(g), True) for g in grads]
    for tp, g in zip(tps, grads):
        tp.set_grad(g)
    total = sum(oracle.get("f64").grad_sumsq(g) for g in grads)
    assert abs(float(ref.grad_norm(tps)) - np.sqrt(total)) <= 1e-5 * np.sqrt(total)
    ref.clip_grad_value(tps, 1.5)
    for tp, g in zip(tps, grads):
        mine = g.copy()
        o32.clip_grad_value(mine, 1.5)
        assert oracle.bit_equal(tp.grad(), mine)


def _unscale_case(bad, R):
    scale = 0.25 if bad == (1, 3, 3e38) else 1024.0
    grads = [rng(20 + i).standard_normal(n).astype(np.float32) * 100 for i, n in enumerate((30, 40, 9))]
    if bad is not None:
        grads[bad[0]][bad[1]] = bad[2]
    tps = [R.tensor(np.zeros_like(g), True) for g in grads]
    for tp, g in zip(tps, grads):
        tp.set_grad(g)
    found = R.unscale(tps, scale)
    mine = [g.copy() for g in grads]
    inv = np.float32(1.0) / np.float32(scale)
    found_or = False
    for gm in mine:
        if o32.unscale_tensor(gm, inv) < gm.size:
            found_or = True
            break
    return found, found_or, tps, mine


BAD = [None, (1, 17, np.inf), (0, 0, np.nan), (2, 6, -np.inf), (1, 3, 3e38)]


@needs_ref
@pytest.mark.parametrize("bad", BAD)
def test_unscale_matches_reference_ieee(bad):
    """GradScaler::unscale stops at the first non-finite product and leaves the
    rest as they were (core/amp.h:134-142); 3e38 * 4 overflows to inf."""
    found, found_or, tps, mine = _unscale_case(bad, ref_ieee)
    assert found == found_or == (bad is not None)
    for tp, gm in zip(tps, mine):
        assert oracle.bit_equal(tp.grad(), gm)


@needs_ref
@pytest.mark.parametrize("bad", BAD)
def test_unscale_fast_math_build_never_stops(bad):
    """The reference's own build (-ffast-math implies -ffinite-math-only) folds
    std::isfinite to true: it reports no overflow and scales every element.
    The drop-in follows the source (the IEEE build above); this pins the
    artefact so the difference is on record."""
    found, _, tps, _ = _unscale_case(bad, ref)
    assert found is False
    scale = 0.25 if bad == (1, 3, 3e38) else 1024.0
    grads = [rng(20 + i).standard_normal(n).astype(np.float32) * 100 for i, n in enumerate((30, 40, 9))]
    if bad is not None:
        grads[bad[0]][bad[1]] = bad[2]
    for tp, g in zip(tps, grads):
        assert oracle.bit_equal(tp.grad(), g * (np.float32(1.0) / np.float32(scale)))
