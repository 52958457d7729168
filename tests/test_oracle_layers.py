"""CPU tests that pin the normalisation / attention-softmax oracle
(or_layernorm, or_batchnorm2d, or_attention_softmax and their backward passes
in oracle/wm_oracle.c) before it checks the GPU kernels:

1. the compiled reference's own modules (oracle/_ref: core/layer.cpp's
   LayerNorm, BatchNorm2d, MultiHeadAttention) -- with IEEE semantics the
   fp32 oracle equals LayerNorm and BatchNorm2d bit for bit (forward,
   running statistics, all three gradients); the attention softmax is
   checked against MultiHeadAttention's stored attention weights, with the
   scores recomputed in the reference's float order; the reference's
   fast-math build within the contract;
2. the reference's known answers (tests/test_layers.cpp: layernorm_forward,
   batchnorm2d_forward / _train_eval, mha_attention_weights_sum,
   mha_causal_mask_structure);
3. identities: normalised outputs have zero mean and variance var/(var+eps),
   the attention softmax without a mask is the Tensor softmax, its backward
   is the Tensor softmax's Jacobian closure, rows of the LayerNorm input
   gradient sum to zero;
4. central finite differences of the fp64 forwards against the fp64
   backwards (BatchNorm2d in training mode; in eval mode the reference's
   closure keeps the batch-statistics terms, pinned as a closed form).
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


def f32(a):
    return np.asarray(a, np.float32)


def ln_case(rows, n, seed):
    r = rng(seed)
    return (f32(r.standard_normal((rows, n)) * 2 + 1), f32(r.uniform(0.5, 1.5, n)), f32(r.standard_normal(n)),
            f32(r.standard_normal((rows, n))))


def bn_case(shape, seed):
    r = rng(seed)
    C = shape[1]
    return (f32(r.standard_normal(shape) * 2 + 0.5), f32(r.uniform(0.5, 1.5, C)), f32(r.standard_normal(C)),
            f32(r.standard_normal(shape)))


# ---- 1. the compiled reference ---------------------------------------------------

def ref_layernorm(R, x, gamma, beta, g):
    m = R.module("layernorm", [x.shape[-1]], 1e-5)
    p = m.params()
    p[0].set_data(gamma)
    p[1].set_data(beta)
    tx = R.tensor(x, True)
    ty = m.forward(tx)
    y = ty.data()
    ty.run_grad_fn(g)
    return y, tx.grad(), p[0].grad(), p[1].grad()


def ref_batchnorm(R, x, gamma, beta, g, training=True, rm=None, rv=None):
    C = x.shape[1]
    m = R.module("batchnorm2d", [C], 1e-5, 0.1)
    m.train(training)
    p = m.params()
    p[0].set_data(gamma)
    p[1].set_data(beta)
    if rm is not None:
        m.buffer(0).set_data(rm)
        m.buffer(1).set_data(rv)
    tx = R.tensor(x, True)
    ty = m.forward(tx)
    y = ty.data()
    ty.run_grad_fn(g)
    return y, tx.grad(), p[0].grad(), p[1].grad(), m.buffer(0).data(), m.buffer(1).data()


@needs_ref
@pytest.mark.parametrize("rows,n", [(1, 1), (6, 10), (33, 100), (4, 1000)])
def test_layernorm_bit_exact_vs_ieee_reference(rows, n):
    x, gamma, beta, g = ln_case(rows, n, 1)
    y_r, gx_r, dg_r, db_r = ref_layernorm(ref_ieee, x, gamma, beta, g)
    y, mean, inv = o32.layernorm(x, gamma, beta)
    assert oracle.bit_equal(y, y_r)
    gx, dg, db = o32.layernorm_bwd(g, x, gamma, mean, inv)
    assert oracle.bit_equal(gx, gx_r) and oracle.bit_equal(dg, dg_r) and oracle.bit_equal(db, db_r)


@needs_ref
@pytest.mark.parametrize("training", [True, False])
@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (3, 4, 5, 6), (2, 3, 7, 7), (4, 8, 16, 16)])
def test_batchnorm_bit_exact_vs_ieee_reference(shape, training):
    x, gamma, beta, g = bn_case(shape, 2)
    C = shape[1]
    rm0, rv0 = f32(rng(3).standard_normal(C) * 0.1), f32(rng(4).uniform(0.5, 2, C))
    y_r, gx_r, dg_r, db_r, rm_r, rv_r = ref_batchnorm(ref_ieee, x, gamma, beta, g, training, rm0, rv0)
    y, mean, inv, rm, rv = o32.batchnorm2d(x, gamma, beta, rm0, rv0, training=training)
    assert oracle.bit_equal(y, y_r)
    assert oracle.bit_equal(rm, rm_r) and oracle.bit_equal(rv, rv_r)
    gx, dg, db = o32.batchnorm2d_bwd(g, x, gamma, mean, inv)
    assert oracle.bit_equal(gx, gx_r) and oracle.bit_equal(dg, dg_r) and oracle.bit_equal(db, db_r)


@needs_ref
def test_norms_fastmath_reference_within_contract():
    x, gamma, beta, g = ln_case(33, 100, 5)
    y_r, gx_r, dg_r, db_r = ref_layernorm(ref, x, gamma, beta, g)
    y64, mean, inv = o64.layernorm(x, gamma, beta)
    yab = oab.layernorm(x, gamma, beta)[0]
    assert oracle.close_scaled(y_r, y64, yab, 1e-5)[0]
    gx64, dg64, db64 = o64.layernorm_bwd(g, x, gamma, f32(mean), f32(inv))
    gxa, dga, dba = oab.layernorm_bwd(g, x, gamma, f32(mean), f32(inv))
    for a, b, c in ((gx_r, gx64, gxa), (dg_r, dg64, dga), (db_r, db64, dba)):
        ok, worst = oracle.close_scaled(a, b, c, 1e-5)
        assert ok, worst
    xb, gb, bb, gg = bn_case((4, 8, 16, 16), 6)
    y_r, gx_r, dg_r, db_r, _, _ = ref_batchnorm(ref, xb, gb, bb, gg)
    y64, mean, inv, _, _ = o64.batchnorm2d(xb, gb, bb, np.zeros(8, np.float32), np.ones(8, np.float32))
    assert oracle.close_scaled(y_r, y64, oab.batchnorm2d(xb, gb, bb, np.zeros(8), np.ones(8))[0], 1e-5)[0]
    gx64, dg64, db64 = o64.batchnorm2d_bwd(gg, xb, gb, f32(mean), f32(inv))
    gxa, dga, dba = oab.batchnorm2d_bwd(gg, xb, gb, f32(mean), f32(inv))
    for a, b, c in ((gx_r, gx64, gxa), (dg_r, dg64, dga), (db_r, db64, dba)):
        ok, worst = oracle.close_scaled(a, b, c, 1e-5)
        assert ok, worst


def mha_scores_like_reference(params, q, k, v, heads):
    """The reference's projections and scaled dot products (core/layer.cpp:
    1127-1208), in its float operation order: sum = b[d]; sum += x[k] * W[d, k]
    for k in order; dot accumulated over d in order; dot * (1 / sqrt(hd))."""
    W_q, W_k, W_v, W_o, b_q, b_k, b_v, b_o = [p.data() for p in params]
    E = W_q.shape[0]
    hd = E // heads

    def proj(x, W, b):
        s = np.broadcast_to(b, x.shape[:-1] + (E,)).astype(np.float32).copy()
        for kk in range(E):
            s = f32(s + f32(x[..., kk:kk + 1] * W[:, kk]))
        return s

    Q, K = proj(q, W_q, b_q), proj(k, W_k, b_k)
    B, tq, tk = q.shape[0], q.shape[1], k.shape[1]
    scale = f32(1.0) / np.sqrt(f32(hd), dtype=np.float32)
    dot = np.zeros((B, heads, tq, tk), np.float32)
    for h in range(heads):
        for d in range(hd):
            c = h * hd + d
            dot[:, h] = f32(dot[:, h] + f32(Q[:, :, None, c] * K[:, None, :, c]))
    return f32(dot * scale)


@needs_ref
@pytest.mark.parametrize("masked", [False, True])
def test_attention_softmax_vs_reference_mha(masked):
    R = ref_ieee
    B, T, E, H = 2, 5, 8, 2
    mha = R.module("mha", [E, H])
    r = rng(7)
    q, k, v = (f32(r.standard_normal((B, T, E))) for _ in range(3))
    mask = R.causal_mask(T) if masked else None
    mha.mha(R.tensor(q), R.tensor(k), R.tensor(v), mask)
    attn_r = mha.buffer(0).data()
    scores = mha_scores_like_reference(mha.params(), q, k, v, H)
    m = mask.data() if masked else None
    attn = o32.attention_softmax(scores, m)
    assert oracle.ulp_distance(attn, attn_r).max() <= 2
    if masked:
        upper = np.triu(np.ones((T, T), bool), 1)
        assert np.all(attn_r[:, :, upper] == 0)


# ---- 2. the reference's known answers ------------------------------------------------

def test_known_answers_from_reference_layer_tests():
    # layernorm_forward / batchnorm2d_forward: normalised output (gamma 1,
    # beta 0) has mean ~0 and variance ~1 per instance / channel
    x = f32(rng(8).standard_normal((4, 16)) * 3 + 2)
    y, _, _ = o64.layernorm(x, np.ones(16, np.float32), np.zeros(16, np.float32))
    assert np.allclose(y.mean(1), 0, atol=1e-6) and np.allclose(y.var(1), 1, atol=1e-4)
    xb = f32(rng(9).standard_normal((8, 3, 4, 4)) * 2 + 1)
    y, _, _, rm, rv = o64.batchnorm2d(xb, np.ones(3), np.zeros(3), np.zeros(3), np.ones(3))
    assert np.allclose(y.mean((0, 2, 3)), 0, atol=1e-6) and np.allclose(y.var((0, 2, 3)), 1, atol=1e-4)
    # batchnorm2d_train_eval: eval uses the running statistics, no update
    ye, _, _, rm2, rv2 = o64.batchnorm2d(xb, np.ones(3), np.zeros(3), rm, rv, training=False)
    assert np.array_equal(rm2, rm) and np.array_equal(rv2, rv)
    assert np.allclose(ye, (xb - rm[None, :, None, None]) / np.sqrt(rv[None, :, None, None] + 1e-5), atol=1e-6)
    # mha_attention_weights_sum / mha_causal_mask_structure
    s = f32(rng(10).standard_normal((2, 3, 4, 4)) * 2)
    causal = np.where(np.triu(np.ones((4, 4)), 1) > 0, -1e9, 0).astype(np.float32)[None, None]
    a = o64.attention_softmax(s, causal)
    assert np.allclose(a.sum(-1), 1, atol=1e-12) and np.all(a[..., np.triu(np.ones((4, 4), bool), 1)] == 0)


# ---- 3. identities --------------------------------------------------------------------

def test_attention_softmax_is_tensor_softmax():
    s = f32(rng(11).standard_normal((2, 3, 5, 17)) * 3)
    a = o64.attention_softmax(s)
    assert np.allclose(a.reshape(-1, 17), o64.softmax(s.reshape(-1, 17)), rtol=1e-14, atol=0)
    d = f32(rng(12).standard_normal(s.shape))
    af = f32(a)
    assert np.allclose(o64.attention_softmax_bwd(af, d).reshape(-1, 17),
                       o64.softmax_bwd(d.reshape(-1, 17), af.reshape(-1, 17)), rtol=1e-12, atol=1e-15)
    # masked rows: all -inf gives NaN (0 / 0 after max -FLT_MAX), as the reference
    m = np.zeros((1, 1, 5, 17), np.float32)
    m[0, 0, 2] = -np.inf
    assert np.isnan(o64.attention_softmax(s, m)[:, :, 2]).all()


def test_layernorm_gradient_rows_sum_to_zero():
    x, gamma, beta, g = ln_case(20, 64, 13)
    _, mean, inv = o64.layernorm(x, gamma, beta)
    gx, _, _ = o64.layernorm_bwd(g, x, gamma, f32(mean), f32(inv))
    assert np.all(np.abs(gx.sum(1)) <= 1e-5 * np.abs(gx).sum(1))


# ---- 4. finite differences ------------------------------------------------------------

def fd(f, x, idx, h=1e-3):
    out = []
    for i in idx:
        xp, xm = x.copy(), x.copy()
        xp.flat[i] += np.float32(h)
        xm.flat[i] -= np.float32(h)
        out.append((f(xp) - f(xm)) / (np.float64(xp.flat[i]) - np.float64(xm.flat[i])))
    return np.array(out)


def test_layernorm_finite_differences():
    x, gamma, beta, g = ln_case(3, 12, 14)
    w = g.astype(np.float64)

    def loss_x(z):
        return (o64.layernorm(z, gamma, beta)[0] * w).sum()

    _, mean, inv = o64.layernorm(x, gamma, beta)
    # the closure reads the captured fp32 mean / inv_std; in fp64 they are the
    # rounded true values, a relative perturbation of ~1e-7
    gx, dg, db = o64.layernorm_bwd(g, x, gamma, f32(mean), f32(inv))
    idx = list(range(0, x.size, 3))
    assert np.allclose(fd(loss_x, x, idx), gx.flat[idx], rtol=1e-4, atol=1e-6)
    assert np.allclose(fd(lambda z: (o64.layernorm(x, z, beta)[0] * w).sum(), gamma, range(12)), dg, rtol=1e-4,
                       atol=1e-6)
    assert np.allclose(fd(lambda z: (o64.layernorm(x, gamma, z)[0] * w).sum(), beta, range(12)), db, rtol=1e-4,
                       atol=1e-6)


def test_batchnorm_finite_differences_and_eval_closure():
    x, gamma, beta, g = bn_case((3, 2, 4, 5), 15)
    w = g.astype(np.float64)
    z2 = np.zeros(2, np.float32)
    o2 = np.ones(2, np.float32)

    def loss_x(z):
        return (o64.batchnorm2d(z, gamma, beta, z2, o2)[0] * w).sum()

    _, mean, inv, _, _ = o64.batchnorm2d(x, gamma, beta, z2, o2)
    gx, dg, db = o64.batchnorm2d_bwd(g, x, gamma, f32(mean), f32(inv))
    idx = list(range(0, x.size, 7))
    assert np.allclose(fd(loss_x, x, idx), gx.flat[idx], rtol=1e-4, atol=1e-6)
    assert np.allclose(fd(lambda z: (o64.batchnorm2d(x, z, beta, z2, o2)[0] * w).sum(), gamma, range(2)), dg,
                       rtol=1e-4)
    assert np.allclose(fd(lambda z: (o64.batchnorm2d(x, gamma, z, z2, o2)[0] * w).sum(), beta, range(2)), db,
                       rtol=1e-4)
    # eval mode: the forward is affine in x (running statistics), but the
    # reference's closure (core/layer.cpp:287-374) is the same batch-
    # statistics formula; closure - derivative = dvar*2(x-m)/n + dmean/n
    rm, rv = f32([0.3, -0.2]), f32([1.5, 0.7])
    _, me, ie, _, _ = o64.batchnorm2d(x, gamma, beta, rm, rv, training=False)
    ge, _, _ = o64.batchnorm2d_bwd(g, x, gamma, f32(me), f32(ie))
    deriv = (g.astype(np.float64) * gamma[None, :, None, None]) * f32(ie).astype(np.float64)[None, :, None, None]
    n = 3 * 20
    xm = x.astype(np.float64) - f32(me)[None, :, None, None]
    gg = g.astype(np.float64) * gamma[None, :, None, None]
    iv = f32(ie).astype(np.float64)[None, :, None, None]
    dvar = (gg * xm * -0.5 * iv ** 3).sum((0, 2, 3), keepdims=True)
    dmean = (gg * -iv).sum((0, 2, 3), keepdims=True) + dvar * (-2 * xm).sum((0, 2, 3), keepdims=True) / n
    assert np.allclose(ge - deriv, dvar * 2 * xm / n + dmean / n, rtol=1e-9, atol=1e-12)
    assert np.abs(dmean).max() > 1e-3  # the extra terms are real


def test_attention_softmax_finite_differences():
    s = f32(rng(16).standard_normal((1, 2, 3, 7)))
    w = rng(17).standard_normal(s.shape)
    a = o64.attention_softmax(s)
    ds = o64.attention_softmax_bwd(f32(a), f32(w))
    idx = list(range(s.size))
    num = fd(lambda z: (o64.attention_softmax(z) * f32(w)).sum(), s, idx, 1e-3)
    assert np.allclose(num, ds.flat[idx], rtol=1e-4, atol=1e-6)


# Published SplitMix64 outputs (Vigna's generator): the sequence for state
# 1234567 (6457827717110365317, ...; the Rosetta Code SplitMix64 task) and
# the first output for state 0.  Output k of state s is mix(s + k * golden).
_SM64_GOLDEN = 0x9E3779B97F4A7C15
_SM64_KATS = [(1234567, k + 1, v) for k, v in enumerate(
    [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431, 16408922859458223821])] + \
    [(0, 1, 0xE220A8397B1DCDAF)]


@pytest.mark.parametrize("offset", [0, 5, 1000003])
@pytest.mark.parametrize("state,k,value", _SM64_KATS)
def test_dropout_mask_generator_known_answers(state, k, value, offset):
    """The dropout mask draws u = top 24 bits of mix(seed + i + golden) for
    element i and keeps the element when u > p (core/layer.cpp:59).  Choosing
    seed so that seed + i + golden is the state of a published output pins
    the mix and the counter: with p = u the element is dropped (u > u is
    false), with p one float below u it is kept, so u equals those 24 bits."""
    o32 = oracle.get("f32")
    n = offset + 1
    seed = (state + k * _SM64_GOLDEN - _SM64_GOLDEN - offset) % (1 << 64)
    u = np.float32((value >> 40) * 2.0 ** -24)
    drop = o32.dropout_mask(n, u, seed)
    keep = o32.dropout_mask(n, np.nextafter(u, np.float32(-1)), seed)
    assert drop[offset] == 0.0
    assert keep[offset] == np.float32(1.0) / (np.float32(1.0) - np.nextafter(u, np.float32(-1)))
