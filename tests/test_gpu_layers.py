"""GPU parity of the LayerNorm, BatchNorm2d and attention-softmax kernels
(include/wm_layers.h) through the C ABI.

Reference: core/layer.cpp (LayerNorm :395-504, BatchNorm2d :202-374,
MultiHeadAttention's mask add and softmax :1198-1237, backward :1343-1360),
restated by the oracle and pinned bit for bit against the reference's IEEE
build in test_oracle_layers.py.  Contract: within 1e-5 of the fp64 oracle
relative to the abs oracle's sum of |terms| (sums, statistics, softmax and
every gradient).  The backward tests feed the statistics the GPU forward
saved to both sides, as the reference's closures use the captured values.
"""
import numpy as np
import pytest

import oracle
from gpu_helpers import (attn_softmax_bwd, attn_softmax_fwd, batchnorm_bwd, batchnorm_fwd, layernorm_bwd,
                         layernorm_fwd, rng_normal, rng_uniform)

pytestmark = pytest.mark.gpu

o64, oab = oracle.get("f64"), oracle.get("abs")


def close(got, ref, scale, rtol=1e-5, atol=1e-30):
    ok, worst = oracle.close_scaled(got, ref, scale, rtol, atol)
    assert ok, f"{worst:.3g}x tolerance"


# ---- LayerNorm -------------------------------------------------------------------

LN_SHAPES = [(1, 1), (4, 3), (33, 100), (7, 256), (5, 257), (3, 512), (9, 768), (4, 1000), (6, 2048), (3, 4096),
             (2, 5000), (2, 8192), (2, 8193), (3, 20000), (1000, 64), (4096, 256), (3000, 1000)]


def ln_inputs(rows, n, seed):
    return (rng_normal((rows, n), seed, 2.0) + np.float32(1.0), rng_uniform((n,), seed + 1, 0.5, 1.5),
            rng_normal((n,), seed + 2))


@pytest.mark.parametrize("shape", LN_SHAPES)
def test_layernorm_forward(wm, shape):
    x, gamma, beta = ln_inputs(*shape, 1)
    y, mean, inv = layernorm_fwd(x, gamma, beta)
    y64, m64, i64 = o64.layernorm(x, gamma, beta)
    close(y, y64, oab.layernorm(x, gamma, beta)[0])
    close(mean, m64, oab.layernorm(np.abs(x), gamma, beta)[1])  # scale: mean of |x|
    close(inv, i64, i64)


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("shape", LN_SHAPES)
def test_layernorm_backward(wm, shape, accumulate):
    x, gamma, beta = ln_inputs(*shape, 2)
    g = rng_normal(shape, 5)
    _, mean, inv = layernorm_fwd(x, gamma, beta)
    n = shape[1]
    g0 = (rng_normal(shape, 6), rng_normal((n,), 7), rng_normal((n,), 8)) if accumulate else (None, None, None)
    got = layernorm_bwd(g, x, gamma, mean, inv, *g0)
    ref = o64.layernorm_bwd(g, x, gamma, mean, inv)
    scale = oab.layernorm_bwd(g, x, gamma, mean, inv)
    for k in range(3):
        r, s = ref[k], scale[k]
        if accumulate:
            r, s = r + g0[k], s + np.abs(g0[k])
        close(got[k], r, s)


@pytest.mark.parametrize("rows,n", [(64, 768), (4096, 256), (130, 9000)])
@pytest.mark.parametrize("want", [(True, False, False), (False, True, True), (False, True, False),
                                  (False, False, True), (True, False, True)])
def test_layernorm_backward_subsets(wm, want, rows, n):
    """Each subset of (dx, dgamma, dbeta); [4096, 256] takes the two-stage
    parameter column sum (more than 64 partial rows), [130, 9000] the
    long-row kernels."""
    x, gamma, beta = ln_inputs(rows, n, 3)
    g = rng_normal(x.shape, 9)
    _, mean, inv = layernorm_fwd(x, gamma, beta)
    got = layernorm_bwd(g, x, gamma, mean, inv, want=want)
    ref = o64.layernorm_bwd(g, x, gamma, mean, inv)
    scale = oab.layernorm_bwd(g, x, gamma, mean, inv)
    for k in range(3):
        if want[k]:
            close(got[k], ref[k], scale[k])
        else:
            assert got[k] is None


# ---- BatchNorm2d -------------------------------------------------------------------

BN_SHAPES = [(1, 1, 1, 1), (3, 4, 5, 6), (2, 3, 7, 7), (4, 8, 16, 16), (8, 64, 28, 28), (2, 3, 1, 1),
             (2, 2, 100, 100), (32, 16, 56, 56)]


def bn_inputs(shape, seed):
    C = shape[1]
    return (rng_normal(shape, seed, 2.0) + np.float32(0.5), rng_uniform((C,), seed + 1, 0.5, 1.5),
            rng_normal((C,), seed + 2), rng_normal((C,), seed + 3, 0.1), rng_uniform((C,), seed + 4, 0.5, 2.0))


@pytest.mark.parametrize("training", [True, False])
@pytest.mark.parametrize("shape", BN_SHAPES)
def test_batchnorm_forward(wm, shape, training):
    x, gamma, beta, rm, rv = bn_inputs(shape, 10)
    y, mean, inv, rm1, rv1 = batchnorm_fwd(x, gamma, beta, rm, rv, training)
    y64, m64, i64, rm64, rv64 = o64.batchnorm2d(x, gamma, beta, rm, rv, training=training)
    close(y, y64, oab.batchnorm2d(x, gamma, beta, rm, rv, training=training)[0])
    xs = np.abs(x)
    close(mean, m64, o64.batchnorm2d(xs, gamma, beta, np.abs(rm), rv, training=training)[1])
    close(inv, i64, i64)
    if training:
        close(rm1, rm64, 0.9 * np.abs(rm) + 0.1 * np.abs(xs).mean((0, 2, 3)))
        close(rv1, rv64, rv64)
    else:
        assert oracle.bit_equal(rm1, rm) and oracle.bit_equal(rv1, rv)


# Larger tensors: several workgroups per channel (the statistics from chunk
# partials, combined by every workgroup of the second pass itself), channel
# counts below and above the grid's rows, odd plane sizes.
BN_LARGE_SHAPES = [(64, 64, 32, 32), (256, 24, 28, 28), (20, 300, 28, 28), (128, 3, 112, 112), (4, 1100, 32, 32),
                   (64, 256, 56, 56), (16, 40, 33, 35)]


@pytest.mark.parametrize("shape", BN_LARGE_SHAPES)
def test_batchnorm_large(wm, shape):
    x, gamma, beta, rm, rv = bn_inputs(shape, 20)
    y, mean, inv, rm1, rv1 = batchnorm_fwd(x, gamma, beta, rm, rv, True)
    y64, m64, i64, rm64, rv64 = o64.batchnorm2d(x, gamma, beta, rm, rv, training=True)
    close(y, y64, oab.batchnorm2d(x, gamma, beta, rm, rv, training=True)[0])
    xs = np.abs(x)
    close(mean, m64, o64.batchnorm2d(xs, gamma, beta, np.abs(rm), rv, training=True)[1])
    close(inv, i64, i64)
    close(rm1, rm64, 0.9 * np.abs(rm) + 0.1 * np.abs(xs).mean((0, 2, 3)))
    close(rv1, rv64, rv64)
    # a second launch gives the same bits (fixed-order combines)
    y2, mean2, inv2, rm2, rv2 = batchnorm_fwd(x, gamma, beta, rm, rv, True)
    for a, b in ((y, y2), (mean, mean2), (inv, inv2), (rm1, rm2), (rv1, rv2)):
        assert oracle.bit_equal(a, b)
    g = rng_normal(shape, 21)
    got = batchnorm_bwd(g, x, gamma, mean, inv)
    ref = o64.batchnorm2d_bwd(g, x, gamma, mean, inv)
    scale = oab.batchnorm2d_bwd(g, x, gamma, mean, inv)
    for k in range(3):
        close(got[k], ref[k], scale[k])


@pytest.mark.parametrize("accumulate", [False, True])
@pytest.mark.parametrize("shape", BN_SHAPES)
def test_batchnorm_backward(wm, shape, accumulate):
    x, gamma, beta, rm, rv = bn_inputs(shape, 11)
    g = rng_normal(shape, 12)
    _, mean, inv, _, _ = batchnorm_fwd(x, gamma, beta, rm, rv, True)
    C = shape[1]
    g0 = (rng_normal(shape, 13), rng_normal((C,), 14), rng_normal((C,), 15)) if accumulate else (None, None, None)
    got = batchnorm_bwd(g, x, gamma, mean, inv, *g0)
    ref = o64.batchnorm2d_bwd(g, x, gamma, mean, inv)
    scale = oab.batchnorm2d_bwd(g, x, gamma, mean, inv)
    for k in range(3):
        r, s = ref[k], scale[k]
        if accumulate:
            r, s = r + g0[k], s + np.abs(g0[k])
        close(got[k], r, s)


def test_batchnorm_eval_backward_and_subsets(wm):
    x, gamma, beta, rm, rv = bn_inputs((4, 8, 16, 16), 16)
    g = rng_normal(x.shape, 17)
    _, mean, inv, _, _ = batchnorm_fwd(x, gamma, beta, rm, rv, False)
    ref = o64.batchnorm2d_bwd(g, x, gamma, mean, inv)
    scale = oab.batchnorm2d_bwd(g, x, gamma, mean, inv)
    for want in ((True, True, True), (True, False, False), (False, True, True)):
        got = batchnorm_bwd(g, x, gamma, mean, inv, want=want)
        for k in range(3):
            if want[k]:
                close(got[k], ref[k], scale[k])
            else:
                assert got[k] is None


def test_batchnorm_constant_channel(wm):
    """A constant channel has variance exactly 0 (the one-pass fp64 moments
    cancel exactly), so inv_std = 1/sqrt(eps) and y = beta."""
    x = np.full((4, 2, 8, 8), 3.25, np.float32)
    x[:, 1] = rng_normal((4, 8, 8), 18)
    gamma, beta = np.float32([1.5, 1.0]), np.float32([0.25, 0.0])
    y, mean, inv, _, rv = batchnorm_fwd(x, gamma, beta, np.zeros(2, np.float32), np.ones(2, np.float32))
    assert mean[0] == np.float32(3.25) and inv[0] == np.float32(1.0) / np.sqrt(np.float32(1e-5))
    assert np.all(y[:, 0] == np.float32(0.25)) and rv[0] == np.float32(0.9)


# ---- attention softmax ---------------------------------------------------------------

def causal(t, big=-1e9):
    return np.where(np.triu(np.ones((t, t)), 1) > 0, big, 0).astype(np.float32)[None, None]


ATT = [((1, 1, 1, 1), None), ((2, 3, 5, 7), None), ((2, 4, 16, 16), "causal"), ((1, 2, 8, 33), "batch"),
       ((2, 8, 128, 128), "causal"), ((1, 1, 4, 2048), None), ((2, 2, 3, 4099), "batch"), ((1, 1, 2, 40000), None),
       ((1, 2, 3, 40000), "batch")]


def att_inputs(shape, mask_kind, seed):
    s = rng_normal(shape, seed, 3.0)
    B, H, tq, tk = shape
    if mask_kind == "causal" and tq == tk:
        m = causal(tq)
    elif mask_kind == "batch":
        m = np.where(rng_uniform((B, 1, tq, tk), seed + 1, 0, 1) < 0.3, np.float32(-1e9), np.float32(0))
        m = m.astype(np.float32)
    else:
        m = None
    return s, m


@pytest.mark.parametrize("shape,mask_kind", ATT, ids=str)
def test_attention_softmax_forward(wm, shape, mask_kind):
    s, m = att_inputs(shape, mask_kind, 20)
    got = attn_softmax_fwd(s, m)
    ref = o64.attention_softmax(s, m)
    close(got, ref, ref, atol=3e-45)
    assert np.allclose(got.astype(np.float64).sum(-1), 1.0, atol=1e-5)
    if mask_kind == "causal":
        assert np.all(got[..., np.triu(np.ones(shape[2:], bool), 1)] == 0)


@pytest.mark.parametrize("shape,mask_kind", ATT, ids=str)
def test_attention_softmax_backward(wm, shape, mask_kind):
    s, m = att_inputs(shape, mask_kind, 21)
    a = attn_softmax_fwd(s, m)
    d = rng_normal(shape, 22)
    got = attn_softmax_bwd(a, d)
    close(got, o64.attention_softmax_bwd(a, d), oab.attention_softmax_bwd(a, d), atol=1e-30)


def test_attention_softmax_special_rows(wm):
    """A fully masked (-inf) row is NaN (exp(-inf) sums to 0), a NaN score
    makes its row NaN, a +inf score too; -1e9 masks give exact zeros."""
    s = rng_normal((1, 1, 4, 64), 23, 2.0)
    m = np.zeros((1, 1, 4, 64), np.float32)
    m[0, 0, 0] = -np.inf
    s[0, 0, 1, 5] = np.nan
    s[0, 0, 2, 7] = np.inf
    m[0, 0, 3, 10:] = -1e9
    got = attn_softmax_fwd(s, m)
    ref = o64.attention_softmax(s, m)
    assert np.isnan(got[0, 0, :3]).all() and np.isnan(ref[0, 0, :3]).all()
    assert np.all(got[0, 0, 3, 10:] == 0)
    close(got[0, 0, 3], ref[0, 0, 3], ref[0, 0, 3])
