"""CPU tests that pin the oracle (oracle/wm_oracle.c) before it is trusted as
the GPU path's checker:

1. the reference's own known-answer tests (tests/golden/ref_kats.json);
2. the compiled reference itself (oracle/_ref/libwmref.so, built from the
   reference's core/tensor.cpp; skipped where it is not built) on seeded
   inputs -- bit-exact for the IEEE-exact ops, within a few ulp / 1e-5 for
   the rest;
3. the committed golden vectors produced by that reference build
   (tests/golden/ref_vectors.npz), so the pinning survives where the
   reference sources are absent;
4. invariants the mathematics fixes (closed forms, sums of quantised values,
   softmax rows summing to 1, the Jacobian's null vector), chosen so that a
   dropped term, a wrong sign or a transposed index fails one of them.
"""
import os

import numpy as np
import pytest

import oracle
from kat_runner import KATS, OracleEngine, check_forward, check_grads
from whitematter_amd import synth

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "ref_vectors.npz")


@pytest.fixture(scope="module")
def eng():
    return OracleEngine()


# ---- 1. reference KATs ------------------------------------------------------

@pytest.mark.parametrize("case", KATS["forward"], ids=lambda c: c["id"])
def test_oracle_forward_kats(eng, case):
    err = check_forward(case, eng.forward(case))
    assert err is None, err


@pytest.mark.parametrize("case", KATS["autograd"], ids=lambda c: c["id"])
def test_oracle_autograd_kats(eng, case):
    err = check_grads(case, eng.autograd(case))
    assert err is None, err


# ---- 2. the compiled reference (this container) -----------------------------

ref = oracle.reference()
needs_ref = pytest.mark.skipif(ref is None, reason="oracle/_ref not built (reference sources absent)")


def _seeded(shape, seed, kind="normal"):
    if kind == "normal":
        return synth.normal(shape, 0xAB000000 + seed)
    return synth.uniform(shape, 0xAB000000 + seed, 0.5, 2.0)


BIN_SHAPES = [((6, 5), (6, 5)), ((6, 5), (5,)), ((6, 5), (6, 1)), ((3, 1, 4), (1, 5, 1)), ((7,), (1,))]


@needs_ref
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "pow", "max", "min"])
@pytest.mark.parametrize("sa,sb", BIN_SHAPES)
def test_oracle_matches_reference_binary(op, sa, sb):
    a = _seeded(sa, 1)
    b = _seeded(sb, 2, "uniform" if op in ("div", "pow") else "normal")
    if op == "pow":
        a = np.abs(a) + np.float32(0.5)
    if op in ("max", "min"):
        a, b = np.rint(a * 2) / 2, np.rint(b * 2) / 2  # ties
        a, b = a.astype(np.float32), b.astype(np.float32)
    ta, tb = ref.tensor(a, True), ref.tensor(b, True)
    ty = ref.binary(op, ta, tb)
    y_ref = ty.data()
    y32 = oracle.get("f32").binary(op, a, b)
    same_shape = tuple(sa) == tuple(sb)
    if op in ("add", "sub", "mul") or (op == "div" and not same_shape):
        assert oracle.bit_equal(y32, y_ref), op
    elif op in ("max", "min"):
        assert oracle.equal_modulo_zero_sign(y32, y_ref), op
    else:
        # same-shape div is vrcpps-based and pow goes through libmvec in the
        # fast-math reference build: a few ulp from IEEE / fp64
        u = oracle.ulp_distance(y32, y_ref)
        assert u.max() <= 4, (op, u.max())
    g = _seeded(y_ref.shape, 3)
    ty.run_grad_fn(g)
    ga64, gb64 = oracle.get("f64").binary_bwd(op, g, a, b, y_ref)
    sa64, sb64 = oracle.get("abs").binary_bwd(op, g, a, b, y_ref)
    assert oracle.close_scaled(ta.grad(), ga64, sa64, 1e-5)[0], "grad a"
    assert oracle.close_scaled(tb.grad(), gb64, sb64, 1e-5)[0], "grad b"


@needs_ref
def test_oracle_pow_grad_exponent_minus_one_is_float():
    """d/da of pow reads pow(a, b - 1.0f) with b - 1.0f rounded in float
    (core/tensor.cpp:1405-1406, :1377-1378): for b = -1.0000001f that is
    exactly -2, so a negative base still has a finite gradient.  Computing
    b - 1 in double would give a non-integer exponent and NaN."""
    a = np.array([-2.0, -0.5, -3.0, 2.0], np.float32)
    b = np.full(4, -1.0000001, np.float32)
    assert np.float32(b[0] - np.float32(1.0)) == np.float32(-2.0)
    ta, tb = ref.tensor(a, True), ref.tensor(b, False)
    ty = ref.binary("pow", ta, tb)
    g = np.ones(4, np.float32)
    ty.run_grad_fn(g)
    ga64, _ = oracle.get("f64").binary_bwd("pow", g, a, b, ty.data())
    assert np.all(np.isfinite(ga64))
    assert np.allclose(ga64, ta.grad(), rtol=1e-6)
    # pow(Tensor, float) likewise
    tx = ref.tensor(a, True)
    tyu = ref.unary("pows", tx, float(b[0]), 0.0)
    tyu.run_grad_fn(g)
    gx64 = oracle.get("f64").unary_bwd("pows", g, a, tyu.data(), float(b[0]))
    assert np.all(np.isfinite(gx64))
    assert np.allclose(gx64, tx.grad(), rtol=1e-6)


UNARY = [("relu", 0, 0), ("sigmoid", 0, 0), ("tanh", 0, 0), ("log", 0, 0), ("exp", 0, 0), ("pows", 2.5, 0),
         ("sqrt", 0, 0), ("abs", 0, 0), ("clamp", -0.5, 0.75)]


@needs_ref
@pytest.mark.parametrize("op,p0,p1", UNARY)
def test_oracle_matches_reference_unary(op, p0, p1):
    x = _seeded((4099,), 7) * np.float32(2.0)
    if op in ("log", "sqrt", "pows"):
        x = np.abs(x) + np.float32(1e-3)
    tx = ref.tensor(x, True)
    ty = ref.unary(op, tx, p0, p1)
    y_ref = ty.data()
    if op in ("relu", "abs", "clamp"):
        assert oracle.bit_equal(oracle.get("f32").unary(op, x, p0, p1), y_ref)
    else:
        # The reference build (-ffast-math, libmvec, rcp/rsqrt) is itself up to
        # a few ulp from the exact value the fp64 oracle computes.
        u = oracle.ulp_vs_f64(y_ref, oracle.get("f64").unary(op, x, p0, p1))
        assert u.max() <= 6, (op, u.max())
    g = _seeded(x.shape, 8)
    ty.run_grad_fn(g)
    r = oracle.get("f64").unary_bwd(op, g, x, y_ref, p0, p1)
    s = oracle.get("abs").unary_bwd(op, g, x, y_ref, p0, p1)
    assert oracle.close_scaled(tx.grad(), r, s, 1e-5, atol=1e-30)[0]


@needs_ref
@pytest.mark.parametrize("op", ["sum", "mean", "max", "min", "argmax", "argmin"])
@pytest.mark.parametrize("dim", [-1, 0, 1])
@pytest.mark.parametrize("keepdim", [False, True])
def test_oracle_matches_reference_reduce(op, dim, keepdim):
    x = synth.quantize(_seeded((37, 53), 9))
    tx = ref.tensor(x, op not in ("argmax", "argmin"))
    ty = ref.reduce(op, tx, dim, keepdim)
    if op in ("argmax", "argmin"):
        d = dim if dim >= 0 else 2 + dim
        view = (1, 37, 53) if d == 0 else (37, 53, 1)
    else:
        view = (1, x.size, 1) if dim == -1 else ((1, 37, 53) if dim == 0 else (37, 53, 1))
    v32, idx = oracle.get("f32").reduce(op, x, *view)
    if op in ("sum", "mean"):
        v64, _ = oracle.get("f64").reduce(op, x, *view)
        assert np.allclose(ty.data().ravel(), v64.ravel(), rtol=1e-6, atol=1e-6)
    else:
        assert oracle.bit_equal(ty.data().ravel(), v32.ravel())
    # output shapes: sum/mean(-1) -> [1] whatever keepdim; max/min(-1, keepdim) keep rank
    if op in ("sum", "mean") and dim == -1:
        assert ty.shape == (1,)
    if op in ("max", "min") and dim == -1:
        assert ty.shape == ((1, 1) if keepdim else (1,))
    if op in ("argmax", "argmin"):
        return
    g = _seeded(ty.shape, 10)
    ty.run_grad_fn(g)
    gx = oracle.get("f64").reduce_bwd("sum" if op == "mean" else op, g.reshape(view[0], view[2]),
                                      idx if op in ("max", "min") else None, *view)
    assert np.allclose(tx.grad().ravel(), gx.ravel(), rtol=1e-6, atol=1e-6)


@needs_ref
@pytest.mark.parametrize("log", [False, True])
def test_oracle_matches_reference_softmax(log):
    x = synth.spikes(_seeded((5, 40), 11) * np.float32(3.0), 11, 0.05)
    tx = ref.tensor(x, True)
    ty = ref.softmax(tx, log)
    r64 = oracle.get("f64").softmax(x, log)
    s64 = oracle.get("abs").softmax(x, log)
    assert oracle.close_scaled(ty.data(), r64, s64, 1e-5)[0]
    g = _seeded(x.shape, 12)
    ty.run_grad_fn(g)
    gr = oracle.get("f64").softmax_bwd(g, ty.data(), log)
    gs = oracle.get("abs").softmax_bwd(g, ty.data(), log)
    assert oracle.close_scaled(tx.grad(), gr, gs, 1e-5, atol=1e-30)[0]


@needs_ref
def test_oracle_matches_reference_fp16():
    x = np.concatenate([_seeded((5000,), 13) * np.float32(1000.0),
                        np.array([0.0, -0.0, 65504.0, 65520.0, 1e5, -1e5, 6e-8, 3e-8, 1e-40, np.inf, -np.inf,
                                  np.nan], np.float32)]).astype(np.float32)
    h_ref = ref.f32_to_f16(x)
    assert np.array_equal(oracle.get("f32").f32_to_f16(x), h_ref)
    allh = np.arange(65536, dtype=np.uint16)
    assert oracle.bit_equal(oracle.get("f32").f16_to_f32(allh), ref.f16_to_f32(allh))


# ---- 3. golden vectors from the reference build -------------------------------

golden = np.load(GOLDEN) if os.path.exists(GOLDEN) else None


@pytest.mark.skipif(golden is None, reason="tests/golden/ref_vectors.npz missing")
def test_oracle_matches_golden_vectors():
    """Every case in ref_vectors.npz: inputs, the reference's outputs/grads."""
    cases = sorted({k.split("/")[0] for k in golden.files})
    assert cases
    o32, o64, oab = oracle.get("f32"), oracle.get("f64"), oracle.get("abs")
    for c in cases:
        kind = str(golden[c + "/kind"])
        if kind == "binary":
            op = str(golden[c + "/op"])
            a, b = golden[c + "/a"], golden[c + "/b"]
            y = golden[c + "/y"]
            if op in ("add", "sub", "mul") or (op == "div" and a.shape != b.shape):
                assert oracle.bit_equal(o32.binary(op, a, b), y), c
            elif op in ("max", "min"):
                assert oracle.equal_modulo_zero_sign(o32.binary(op, a, b), y), c
            else:
                assert oracle.ulp_distance(o32.binary(op, a, b), y).max() <= 4, c
            ga, gb = o64.binary_bwd(op, golden[c + "/g"], a, b, y)
            sa, sb = oab.binary_bwd(op, golden[c + "/g"], a, b, y)
            assert oracle.close_scaled(golden[c + "/ga"], ga, sa, 1e-5)[0], c
            assert oracle.close_scaled(golden[c + "/gb"], gb, sb, 1e-5)[0], c
        elif kind == "reduce":
            op = str(golden[c + "/op"])
            x, view = golden[c + "/x"], tuple(int(v) for v in golden[c + "/view"])
            v32, _ = o32.reduce(op, x, *view)
            if op in ("sum", "mean"):
                v64, _ = o64.reduce(op, x, *view)
                assert np.allclose(golden[c + "/y"].ravel(), v64.ravel(), rtol=1e-6, atol=1e-6), c
            else:
                assert oracle.bit_equal(golden[c + "/y"].ravel(), v32.ravel()), c
        elif kind == "softmax":
            log = bool(golden[c + "/log"])
            x = golden[c + "/x"]
            assert oracle.close_scaled(golden[c + "/y"], o64.softmax(x, log), oab.softmax(x, log), 1e-5)[0], c
            g, y = golden[c + "/g"], golden[c + "/y"]
            assert oracle.close_scaled(golden[c + "/gx"], o64.softmax_bwd(g, y, log),
                                       oab.softmax_bwd(g, y, log), 1e-5, atol=1e-30)[0], c


# ---- 4. invariants fixed by the mathematics -----------------------------------

def test_broadcast_shape_rules():
    o = oracle.get("f64")
    assert o.broadcast_shape((1024, 1024), (1024,)) == (1024, 1024)
    assert o.broadcast_shape((3, 1, 5), (4, 1)) == (3, 4, 5)
    assert o.broadcast_shape((1,), (2, 3)) == (2, 3)
    with pytest.raises(ValueError):
        o.broadcast_shape((2, 3), (3, 2))


def test_broadcast_grad_is_column_and_row_sum():
    """add's broadcast gradient equals numpy's column / row sums of g (fp64)."""
    g = synth.normal((33, 17), 5)
    a = synth.normal((33, 17), 6)
    ga, gr = oracle.get("f64").binary_bwd("add", g, a, synth.normal((17,), 7))
    assert np.allclose(gr, g.astype(np.float64).sum(axis=0), rtol=1e-12, atol=1e-12)
    assert np.array_equal(ga, g.astype(np.float64))
    _, gc = oracle.get("f64").binary_bwd("mul", g, a, synth.normal((33, 1), 8))
    assert np.allclose(gc.ravel(), (g.astype(np.float64) * a).sum(axis=1), rtol=1e-12, atol=1e-12)
    # sub flips the sign of the second operand's gradient; div's is -g*a/b^2
    b = synth.uniform((17,), 9, 0.5, 2.0)
    _, gs = oracle.get("f64").binary_bwd("sub", g, a, b)
    assert np.allclose(gs, -g.astype(np.float64).sum(axis=0))
    _, gd = oracle.get("f64").binary_bwd("div", g, a, b)
    want = -(g.astype(np.float64) * a / (b.astype(np.float64) ** 2)).sum(axis=0)
    assert np.allclose(gd, want, rtol=1e-12)


def test_quantised_sums_exact():
    """Sums of multiples of 1/64 are exact in fp32 below 2^18: the fp32
    oracle's sequential sum equals the fp64 one bit for bit."""
    x = synth.config3(256, 512)
    for view in ((1, 256, 512), (256, 512, 1), (1, x.size, 1)):
        v32, _ = oracle.get("f32").reduce("sum", x, *view)
        v64, _ = oracle.get("f64").reduce("sum", x, *view)
        assert np.array_equal(v32.astype(np.float64), v64)


def test_first_index_ties_and_nan_rule():
    o = oracle.get("f32")
    x = np.array([1, 3, 3, 2, 3], np.float32)
    assert o.reduce("argmax", x, 1, 5, 1)[1][0, 0] == 1
    assert o.reduce("argmin", np.array([2, 1, 1], np.float32), 1, 3, 1)[1][0, 0] == 1
    nan_first = np.array([np.nan, 5, 1], np.float32)
    v, i = o.reduce("max", nan_first, 1, 3, 1)
    assert np.isnan(v[0, 0]) and i[0, 0] == 0
    nan_later = np.array([1, np.nan, 5], np.float32)
    v, i = o.reduce("max", nan_later, 1, 3, 1)
    assert v[0, 0] == 5 and i[0, 0] == 2


def test_softmax_invariants():
    x = synth.normal((6, 50), 21) * np.float32(3)
    y = oracle.get("f64").softmax(x)
    assert np.allclose(y.sum(axis=1), 1.0, atol=1e-12)
    ly = oracle.get("f64").softmax(x, log=True)
    assert np.allclose(np.exp(ly).sum(axis=1), 1.0, atol=1e-12)
    g = synth.normal(x.shape, 22)
    gx = oracle.get("f64").softmax_bwd(g, y.astype(np.float32))
    # J^T g is orthogonal to the ones vector, and equals the closed form
    assert np.allclose(gx.sum(axis=1), 0.0, atol=1e-7)
    y32 = y.astype(np.float32).astype(np.float64)
    closed = y32 * (g - (g * y32).sum(axis=1, keepdims=True))
    assert np.allclose(gx, closed, atol=1e-12)


def test_mean_gradient_is_sums():
    """mean's backward reuses sum's closure: the gradient is not divided by n."""
    g = np.array([[2.0]], np.float32)
    gx = oracle.get("f64").reduce_bwd("mean", g, None, 1, 4, 1)
    assert np.array_equal(gx.ravel(), [2.0, 2.0, 2.0, 2.0])


def test_unary_closed_forms():
    o = oracle.get("f64")
    x = np.array([-1.5, -0.0, 0.0, 0.5, 2.0], np.float32)
    assert np.allclose(o.unary("sigmoid", x), 1 / (1 + np.exp(-x.astype(np.float64))))
    assert o.unary("log", np.array([1.0], np.float32))[0] == 0.0  # 1 + 1e-8f rounds to 1 in fp32
    assert np.array_equal(o.unary("relu", x), [0, 0, 0, 0.5, 2.0])
    assert np.array_equal(o.unary("clamp", x, -1.0, 1.0), [-1, -0.0, 0, 0.5, 1.0])
    gx = o.unary_bwd("abs", np.ones(5, np.float32), x, None)
    assert np.array_equal(gx, [-1, 0, 0, 1, 1])
    gx = o.unary_bwd("pows", np.ones(1, np.float32), np.array([3.0], np.float32), None, 2.0)
    assert gx[0] == 6.0


def test_fp16_truncation_rules():
    o = oracle.get("f32")
    h = o.f32_to_f16(np.array([1.0, 65504.0, 65536.0, 1.0009765625 + 2 ** -12, -2.0, 1e-10],
                              np.float32))
    assert h.tolist() == [0x3C00, 0x7BFF, 0x7C00, 0x3C01, 0xC000, 0x0000]
    back = o.f16_to_f32(np.array([0x0001, 0x03FF, 0x3C00, 0xFC00], np.uint16))
    assert back[0] == np.float32(2.0 ** -24) and back[1] == np.float32(1023 * 2.0 ** -24)
    assert back[2] == 1.0 and np.isneginf(back[3])
