"""CPU tests that pin the matrix-product and MultiHeadAttention oracle
(or_bmm, or_bmm_bwd, or_mha_forward, or_mha_backward in oracle/wm_oracle.c)
before it checks the GPU kernels:

1. the compiled reference (oracle/_ref): with IEEE semantics the fp32 oracle
   equals Tensor::matmul / Tensor::bmm and their closures bit for bit
   (core/tensor.cpp:783-895), and MultiHeadAttention's forward and closure
   (core/layer.cpp:1103-1437) -- the softmax's exp aside, which the oracle
   rounds from double (a few ulp from the reference's expf): the backward is
   bit-exact when fed the reference's own attention weights; the reference's
   fast-math build (AVX dot products in matmul's closure) within the contract;
2. the reference's known answers (tests/test_tensor.cpp matmul_2d,
   matmul_batch; tests/test_autograd.cpp matmul_grad; tests/test_layers.cpp
   mha_attention_weights_sum, mha_causal_mask_structure);
3. mathematics: the fp64 oracle against numpy's float64 matmul, identities
   (A @ I = A, permutations move rows), small-integer products exact in
   every build, the closures against the transposed products, central
   finite differences of the fp64 MHA forward against its backward.
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


SHAPES = [(1, 1, 1), (2, 3, 2), (3, 5, 7), (33, 65, 17), (64, 31, 129), (5, 1, 4), (7, 40, 1)]


def mm_case(m, k, n, seed, batch=None):
    r = rng(seed)
    pre = (batch,) if batch else ()
    return f32(r.standard_normal(pre + (m, k))), f32(r.standard_normal(pre + (k, n))), f32(
        r.standard_normal(pre + (m, n)))


# ---- 1. the compiled reference -------------------------------------------------------

@needs_ref
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("batched", [False, True])
def test_matmul_bit_exact_vs_reference_ieee(shape, batched):
    R = ref_ieee
    m, k, n = shape
    a, b, g = mm_case(m, k, n, 1, 3 if batched else None)
    ta, tb = R.tensor(a, True), R.tensor(b, True)
    y = R.bmm(ta, tb) if batched else R.matmul(ta, tb)
    assert oracle.bit_equal(y.data(), o32.bmm(a, b))
    y.run_grad_fn(g)
    ga, gb = o32.bmm_bwd(g, a, b)
    assert oracle.bit_equal(ta.grad(), ga) and oracle.bit_equal(tb.grad(), gb)


@needs_ref
@pytest.mark.parametrize("shape", SHAPES)
def test_matmul_fast_math_reference_within_contract(shape):
    R = ref
    m, k, n = shape
    a, b, g = mm_case(m, k, n, 2)
    ta, tb = R.tensor(a, True), R.tensor(b, True)
    y = R.matmul(ta, tb)
    assert oracle.close_scaled(y.data(), o64.matmul(a, b), oab.matmul(a, b), 1e-5)[0]
    y.run_grad_fn(g)
    ga, gb = o64.matmul_bwd(g, a, b)
    sa, sb = oab.matmul_bwd(g, a, b)
    assert oracle.close_scaled(ta.grad(), ga, sa, 1e-5)[0]
    assert oracle.close_scaled(tb.grad(), gb, sb, 1e-5)[0]


def mha_params(R, E, H):
    m = R.module("mha", [E, H])
    return m, [p.data() for p in m.params()]


def ctx_like_reference(attn, V, heads):
    """context[b, i, h*hd + d] = sum_j attn[b, h, i, j] * V[b, j, h*hd + d],
    j ascending, in fp32 (core/layer.cpp:1242-1259)."""
    B, H, Sq, Sk = attn.shape
    E = V.shape[2]
    hd = E // heads
    Vh = V.reshape(B, Sk, H, hd).transpose(0, 2, 1, 3)  # [B, H, Sk, hd]
    s = np.zeros((B, H, Sq, hd), np.float32)
    for j in range(Sk):
        s = f32(s + f32(attn[:, :, :, j:j + 1] * Vh[:, :, None, j, :]))
    return np.ascontiguousarray(s.transpose(0, 2, 1, 3).reshape(B, Sq, E))


@needs_ref
@pytest.mark.parametrize("case", [(2, 5, 5, 8, 2, None), (1, 4, 6, 12, 3, "batch"), (2, 6, 6, 16, 4, "causal"),
                                  (1, 3, 3, 8, 1, None)])
def test_mha_vs_reference_ieee(case):
    """Forward within a few fp32 roundings (exp), backward bit for bit when
    the oracle gets the reference's attention weights."""
    R = ref_ieee
    B, Sq, Sk, E, H, mk = case
    mod, params = mha_params(R, E, H)
    r = rng(3)
    q = f32(r.standard_normal((B, Sq, E)))
    k = f32(r.standard_normal((B, Sk, E)))
    v = f32(r.standard_normal((B, Sk, E)))
    if mk == "causal":
        mask = R.causal_mask(Sq)
        m = mask.data()
    elif mk == "batch":
        m = np.where(r.uniform(size=(B, 1, Sq, Sk)) < 0.3, np.float32(-1e9), np.float32(0)).astype(np.float32)
        mask = R.tensor(m)
    else:
        mask, m = None, None
    tq, tk, tv = R.tensor(q, True), R.tensor(k, True), R.tensor(v, True)
    out = mod.mha(tq, tk, tv, mask)
    attn_r = mod.buffer(0).data()
    f = o32.mha_forward(q, k, v, params, H, m)
    assert oracle.ulp_distance(f["attn"], attn_r).max() <= 4
    # output: same operation order; only the exp roundings differ
    s = oracle.get("f64").mha_forward(q, k, v, params, H, m)
    scale = np.abs(s["ctx"]).reshape(-1, E) @ np.abs(params[3]).T + np.abs(params[7])
    scale = scale.reshape(out.data().shape) + np.abs(s["out"])
    assert oracle.close_scaled(out.data(), f["out"], scale, 1e-6)[0]

    dout = f32(r.standard_normal((B, Sq, E)))
    out.run_grad_fn(dout)
    saved = {"Q": f["Q"], "K": f["K"], "V": f["V"], "attn": attn_r, "ctx": ctx_like_reference(attn_r, f["V"], H)}
    g = o32.mha_backward(dout, q, k, v, params, H, saved)
    got = [p.grad() for p in mod.params()]
    for name, gr in zip(("gWq", "gWk", "gWv", "gWo", "gbq", "gbk", "gbv", "gbo"), got):
        assert oracle.bit_equal(gr, g[name]), name
    for name, t in (("gq", tq), ("gk", tk), ("gv", tv)):
        assert oracle.bit_equal(t.grad(), g[name]), name


@needs_ref
def test_mha_self_attention_input_gradient_collects_three_paths():
    R = ref_ieee
    B, S, E, H = 2, 4, 8, 2
    mod, params = mha_params(R, E, H)
    x = f32(rng(4).standard_normal((B, S, E)))
    tx = R.tensor(x, True)
    out = mod.mha(tx, tx, tx, None)
    attn_r = mod.buffer(0).data()
    f = o32.mha_forward(x, x, x, params, H)
    dout = f32(rng(5).standard_normal((B, S, E)))
    out.run_grad_fn(dout)
    saved = {"Q": f["Q"], "K": f["K"], "V": f["V"], "attn": attn_r, "ctx": ctx_like_reference(attn_r, f["V"], H)}
    g = o32.mha_backward(dout, x, x, x, params, H, saved, alias=True)
    assert oracle.bit_equal(tx.grad(), g["gq"])


# ---- 2. the reference's known answers ----------------------------------------------

@pytest.mark.parametrize("o", [o32, o64])
def test_known_answers(o):
    # test_tensor.cpp:152-165 matmul_2d
    a = f32([1, 2, 3, 4, 5, 6]).reshape(2, 3)
    b = f32([1, 2, 3, 4, 5, 6]).reshape(3, 2)
    assert np.array_equal(o.matmul(a, b), [[22, 28], [49, 64]])
    # test_tensor.cpp:167-174 matmul_batch: [2, 2, 3] x [2, 3, 2] -> [2, 2, 2]
    x, y, _ = mm_case(2, 3, 2, 6, batch=2)
    assert o.bmm(x, y).shape == (2, 2, 2)
    # test_autograd.cpp:184-200 matmul_grad: d sum(AB)/dA = 1 @ B^T, /dB = A^T @ 1
    A = f32([1, 2, 3, 4]).reshape(2, 2)
    B = f32([5, 6, 7, 8]).reshape(2, 2)
    ga, gb = o.matmul_bwd(np.ones((2, 2), np.float32), A, B)
    assert np.array_equal(ga, [[11, 15], [11, 15]]) and np.array_equal(gb, [[4, 4], [6, 6]])


def test_known_answers_mha():
    # test_layers.cpp mha_attention_weights_sum / mha_causal_mask_structure
    E, H, B, S = 16, 4, 2, 5
    r = rng(7)
    params = [f32(r.standard_normal((E, E)) * 0.3) for _ in range(4)] + [f32(r.standard_normal(E)) for _ in range(4)]
    x = f32(r.standard_normal((B, S, E)))
    causal = np.where(np.triu(np.ones((S, S)), 1) > 0, -1e9, 0).astype(np.float32)[None, None]
    f = o64.mha_forward(x, x, x, params, H, causal)
    assert np.allclose(f["attn"].sum(-1), 1.0, atol=1e-12)
    assert np.all(f["attn"][:, :, np.triu(np.ones((S, S), bool), 1)] == 0)
    assert f["out"].shape == (B, S, E)


# ---- 3. mathematics ------------------------------------------------------------------

@pytest.mark.parametrize("shape", SHAPES)
def test_f64_oracle_is_numpy_float64_matmul(shape):
    m, k, n = shape
    a, b, g = mm_case(m, k, n, 8, batch=2)
    a64, b64, g64 = (x.astype(np.float64) for x in (a, b, g))
    scale = np.abs(a64) @ np.abs(b64)
    assert oracle.close_scaled(o64.bmm(a, b), a64 @ b64, scale, 1e-14)[0]
    assert np.allclose(oab.bmm(a, b), scale, rtol=1e-14, atol=0)
    ga, gb = o64.bmm_bwd(g, a, b)
    assert oracle.close_scaled(ga, g64 @ b64.transpose(0, 2, 1), np.abs(g64) @ np.abs(b64).transpose(0, 2, 1),
                               1e-14)[0]
    assert oracle.close_scaled(gb, a64.transpose(0, 2, 1) @ g64, np.abs(a64).transpose(0, 2, 1) @ np.abs(g64),
                               1e-14)[0]


def test_identities_and_exact_integer_products():
    r = rng(9)
    a = f32(r.standard_normal((6, 9)))
    assert np.array_equal(o32.matmul(a, np.eye(9, dtype=np.float32)), a)
    perm = np.eye(6, dtype=np.float32)[[3, 0, 5, 1, 4, 2]]
    assert np.array_equal(o32.matmul(perm, a), a[[3, 0, 5, 1, 4, 2]])
    # small integers: every partial sum is exact in fp32, so all builds agree
    ai = f32(r.integers(-8, 9, (17, 23)))
    bi = f32(r.integers(-8, 9, (23, 11)))
    exact = ai.astype(np.int64) @ bi.astype(np.int64)
    for o in (o32, o64):
        assert np.array_equal(o.matmul(ai, bi), exact)
    gi = f32(r.integers(-4, 5, (17, 11)))
    ga, gb = o32.matmul_bwd(gi, ai, bi)
    assert np.array_equal(ga, gi.astype(np.int64) @ bi.astype(np.int64).T)
    assert np.array_equal(gb, ai.astype(np.int64).T @ gi.astype(np.int64))
    # accumulation into existing gradients
    ga0, gb0 = f32(r.integers(-3, 4, ai.shape)), f32(r.integers(-3, 4, bi.shape))
    ga2, gb2 = o32.matmul_bwd(gi, ai, bi, ga0, gb0)
    assert np.array_equal(ga2, ga + ga0) and np.array_equal(gb2, gb + gb0)


def test_mha_backward_matches_finite_differences():
    """The fp64 closure against central differences of the fp64 forward, for
    a scalar loss sum(out * w), with respect to inputs and parameters."""
    E, H, B, Sq, Sk = 8, 2, 2, 3, 4
    r = rng(10)
    params = [r.standard_normal((E, E)) * 0.5 for _ in range(4)] + [r.standard_normal(E) * 0.1 for _ in range(4)]
    q, k, v = r.standard_normal((B, Sq, E)), r.standard_normal((B, Sk, E)), r.standard_normal((B, Sk, E))
    w = r.standard_normal((B, Sq, E))
    mask = np.where(r.uniform(size=(B, 1, Sq, Sk)) < 0.25, -1e9, 0.0)

    # fp64 throughout: the oracle takes fp32 inputs, so work on values exactly
    # representable in fp32 and difference with steps that stay so
    def as32(x):
        return np.asarray(x, np.float32)

    params = [as32(p) for p in params]
    q, k, v, w, mask = as32(q), as32(k), as32(v), as32(w), as32(mask)

    def loss(qq, kk, vv, ps):
        return float((o64.mha_forward(qq, kk, vv, ps, H, mask)["out"] * w).sum())

    f = o64.mha_forward(q, k, v, params, H, mask)
    saved = {n: as32(f[n]) for n in ("Q", "K", "V", "attn", "ctx")}
    # the closure reads fp32 copies of the intermediates; differences of the
    # fp64 forward are compared at a tolerance that absorbs that rounding
    g = o64.mha_backward(w, q, k, v, params, H, saved)
    h = np.float32(2 ** -8)

    def fd(x, idx, fn):
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        return (fn(xp) - fn(xm)) / (2 * float(h))

    picks = [("gq", q, (0, 1, 3)), ("gk", k, (1, 2, 5)), ("gv", v, (0, 3, 7))]
    for name, x, idx in picks:
        def fn(xx, name=name):
            args = {"gq": (xx, k, v), "gk": (q, xx, v), "gv": (q, k, xx)}[name]
            return loss(*args, params)
        assert abs(fd(x, idx, fn) - g[name][idx]) <= 2e-3 * (1 + abs(g[name][idx])), name
    for pi, name, idx in ((0, "gWq", (1, 2)), (1, "gWk", (3, 4)), (2, "gWv", (5, 0)), (3, "gWo", (2, 6)),
                          (4, "gbq", (3,)), (6, "gbv", (1,)), (7, "gbo", (4,))):
        def fn(pp, pi=pi):
            ps = list(params)
            ps[pi] = pp
            return loss(q, k, v, ps)
        assert abs(fd(params[pi], idx, fn) - g[name][idx]) <= 2e-3 * (1 + abs(g[name][idx])), name
    # bk's gradient is zero in exact arithmetic: softmax is invariant to a
    # per-row shift of the scores, and q . bk is one
    assert np.all(np.abs(g["gbk"]) < 1e-5)
