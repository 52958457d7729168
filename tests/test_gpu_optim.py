"""GPU parity: parameter updates through the C ABI (include/wm_optim.h).

Contract: the optimizer steps (SGD with/without momentum, Adam, AdamW,
RMSprop with/without weight decay and momentum), clip_grad_value_ and
GradScaler::unscale are bit-exact against the strict fp32 oracle (the
reference's source evaluated with IEEE arithmetic, pinned bit for bit against
the reference built without fast-math) over several steps, for the vector
path (16-byte aligned, n % 4 == 0) and the scalar path.  The gradient norm's
sum of squares is within 1e-5 of the fp64 oracle; clip_grad_norm_ scales by
the coefficient of that norm exactly.
"""
import ctypes as C

import numpy as np
import pytest

import oracle
from whitematter_amd import _lib as W

pytestmark = pytest.mark.gpu

o32 = oracle.get("f32")

CONFIGS = [
    ("sgd", dict(lr=0.05, a=0.0)),
    ("sgd", dict(lr=0.05, a=0.9)),
    ("adam", dict(lr=1e-3, a=0.9, b=0.999, c=1e-8)),
    ("adamw", dict(lr=1e-3, a=0.9, b=0.999, c=1e-8, d=0.01)),
    ("rmsprop", dict(lr=1e-2, a=0.99, b=1e-8, c=0.0, d=0.0)),
    ("rmsprop", dict(lr=1e-2, a=0.9, b=1e-6, c=0.9, d=0.0)),
    ("rmsprop", dict(lr=1e-2, a=0.9, b=1e-6, c=0.0, d=0.05)),
    ("rmsprop", dict(lr=1e-2, a=0.9, b=1e-6, c=0.9, d=0.05)),
]


def rng(seed):
    return np.random.default_rng(seed)


class Slot:
    """A device copy of a float32 array, optionally placed 4 bytes past a
    16-byte boundary to force the scalar kernels."""

    def __init__(self, a, misalign=False):
        self.n = a.size
        self.off = 1 if misalign else 0
        self.d = W.DeviceArray((self.n + self.off,))
        host = np.zeros(self.n + self.off, np.float32)
        host[self.off:] = a.ravel()
        self.d.upload(host)

    @property
    def vp(self):
        return C.c_void_p(self.d.ptr + 4 * self.off)

    def get(self):
        return self.d.to_host()[self.off:]


def gpu_step(kind, hp, p, g, s1, s2, t):
    lr, a, b, c, d = hp["lr"], hp.get("a", 0.0), hp.get("b", 0.0), hp.get("c", 0.0), hp.get("d", 0.0)
    n = p.n
    if kind == "sgd":
        W.call("wm_sgd_step", p.vp, g.vp, s1.vp if a > 0 else None, n, lr, a)
    elif kind in ("adam", "adamw"):
        bc1, bc2 = o32.bias_correction(a, t), o32.bias_correction(b, t)
        if kind == "adam":
            W.call("wm_adam_step", p.vp, g.vp, s1.vp, s2.vp, n, lr, a, b, c, bc1, bc2)
        else:
            W.call("wm_adamw_step", p.vp, g.vp, s1.vp, s2.vp, n, lr, a, b, c, bc1, bc2, d)
    else:
        W.call("wm_rmsprop_step", p.vp, g.vp, s1.vp, s2.vp if c > 0 else None, n, lr, a, b, c, d)


def oracle_step(kind, hp, p, g, s1, s2, t):
    lr, a, b, c, d = hp["lr"], hp.get("a", 0.0), hp.get("b", 0.0), hp.get("c", 0.0), hp.get("d", 0.0)
    if kind == "sgd":
        o32.sgd_step(p, g, s1, lr, a)
    elif kind in ("adam", "adamw"):
        o32.adam_step(p, g, s1, s2, lr, a, b, c, o32.bias_correction(a, t), o32.bias_correction(b, t), d,
                      kind == "adamw")
    else:
        o32.rmsprop_step(p, g, s1, s2, lr, a, b, c, d)


@pytest.mark.parametrize("n,misalign", [(4096, False), (1001, False), (1000, True), (3, False)])
@pytest.mark.parametrize("kind,hp", CONFIGS, ids=lambda v: v if isinstance(v, str) else "-".join(map(str, v.values())))
def test_steps_bitexact(wm, kind, hp, n, misalign):
    p0 = rng(n).standard_normal(n).astype(np.float32)
    mine = [p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)]
    dev = [Slot(x, misalign) for x in mine]
    for t in range(1, 5):
        g = (rng(1000 * t + n).standard_normal(n) * (10.0 ** rng(t).uniform(-3, 1, n))).astype(np.float32)
        dg = Slot(g, misalign)
        gpu_step(kind, hp, dev[0], dg, dev[1], dev[2], t)
        oracle_step(kind, hp, mine[0], g, mine[1], mine[2], t)
        for name, dv, hv in zip(("p", "state1", "state2"), dev, mine):
            assert oracle.bit_equal(dv.get(), hv), f"{kind} step {t}: {name} differs"


def test_empty_and_null_state(wm):
    W.call("wm_sgd_step", None, None, None, 0, 0.1, 0.0)          # n == 0 is a no-op
    p = Slot(np.ones(8, np.float32))
    g = Slot(np.ones(8, np.float32))
    with pytest.raises(W.WMError):
        W.call("wm_sgd_step", p.vp, g.vp, None, 8, 0.1, 0.9)      # momentum needs a velocity buffer
    with pytest.raises(W.WMError):
        W.call("wm_rmsprop_step", p.vp, g.vp, None, None, 8, 0.1, 0.9, 1e-8, 0.0, 0.0)


def test_grad_norm_and_clip(wm):
    sizes = (1000, 37, 4096, 1)
    grads = [(rng(50 + i).standard_normal(n) * 3).astype(np.float32) for i, n in enumerate(sizes)]
    total = W.DeviceArray((1,))
    total.fill(0.0)
    dgs = [Slot(g) for g in grads]
    for dg, g in zip(dgs, grads):
        W.call("wm_grad_sumsq_accumulate", dg.vp, g.size, total.vp)
    t_gpu = np.float32(total.to_host()[0])
    t64 = sum(oracle.get("f64").grad_sumsq(g) for g in grads)
    assert abs(float(t_gpu) - t64) <= 1e-5 * t64
    for max_norm in (1.0, 1e6):                                    # clips / leaves alone
        ds = [Slot(g) for g in grads]
        for d, g in zip(ds, grads):
            W.call("wm_clip_grad_norm_scale", d.vp, g.size, total.vp, max_norm)
        coef = np.float32(max_norm) / (np.sqrt(t_gpu, dtype=np.float32) + np.float32(1e-6))
        for d, g in zip(ds, grads):
            expect = g * coef if coef < 1 else g
            assert oracle.bit_equal(d.get(), expect)


def test_clip_value(wm):
    g = np.concatenate([rng(60).standard_normal(5000).astype(np.float32) * 10,
                        np.array([np.nan, np.inf, -np.inf, 8.0, -8.0, -0.0], np.float32)])
    d = Slot(g)
    W.call("wm_clip_grad_value", d.vp, g.size, 8.0)
    mine = g.copy()
    o32.clip_grad_value(mine, 8.0)
    assert oracle.bit_equal(d.get(), mine)


@pytest.mark.parametrize("bad", [None, (1, 17, np.inf), (0, 0, np.nan), (2, 6, -np.inf), (1, 3, 3e38),
                                 (2, 70000, np.nan)])
def test_unscale(wm, bad):
    scale = 0.25 if bad == (1, 3, 3e38) else 1024.0
    sizes = (30, 4000, 100003)
    grads = [(rng(70 + i).standard_normal(n) * 100).astype(np.float32) for i, n in enumerate(sizes)]
    if bad is not None:
        grads[bad[0]][bad[1]] = bad[2]
    ds = [Slot(g) for g in grads]
    ptrs = (C.c_void_p * 3)(*[d.vp.value for d in ds])
    ns = (C.c_int64 * 3)(*sizes)
    found = C.c_int(-1)
    inv = np.float32(1.0) / np.float32(scale)
    W.call("wm_grad_unscale", 3, C.cast(ptrs, C.c_void_p), C.cast(ns, C.c_void_p), float(inv), C.byref(found))
    mine = [g.copy() for g in grads]
    found_or = 0
    for gm in mine:
        if o32.unscale_tensor(gm, inv) < gm.size:
            found_or = 1
            break
    assert found.value == found_or == (0 if bad is None else 1)
    for d, gm in zip(ds, mine):
        assert oracle.bit_equal(d.get(), gm)


# ---- multi-tensor entry points --------------------------------------------

MULTI_SIZES = [(4096, False), (0, False), (7, False), (200003, False), (1000, True), (65536, False), (131077, True)]


def _ptrs(slots):
    return W.ptr_array([s.vp if s is not None else None for s in slots])


@pytest.mark.parametrize("kind,hp", CONFIGS, ids=lambda v: v if isinstance(v, str) else "-".join(map(str, v.values())))
def test_multi_steps_bitexact(wm, kind, hp):
    """One launch over a list of tensors (empty, tiny, multi-chunk, misaligned)
    equals the single-tensor update of each: bit-exact against the oracle."""
    lr, a, b, c, d = hp["lr"], hp.get("a", 0.0), hp.get("b", 0.0), hp.get("c", 0.0), hp.get("d", 0.0)
    mine, dev = [], []
    for i, (n, mis) in enumerate(MULTI_SIZES):
        arrs = [rng(7 * i).standard_normal(n).astype(np.float32), np.zeros(n, np.float32), np.zeros(n, np.float32)]
        mine.append(arrs)
        dev.append([Slot(x, mis) for x in arrs])
    ns, _ns = W.i64_array([n for n, _ in MULTI_SIZES])
    for t in range(1, 4):
        gs = [(rng(100 * t + i).standard_normal(n) * 10.0 ** rng(t + i).uniform(-3, 1, n)).astype(np.float32)
              for i, (n, _) in enumerate(MULTI_SIZES)]
        dgs = [Slot(g, mis) for g, (_, mis) in zip(gs, MULTI_SIZES)]
        P, _p = _ptrs([x[0] for x in dev])
        G, _g = _ptrs(dgs)
        S1, _s1 = _ptrs([x[1] for x in dev])
        S2, _s2 = _ptrs([x[2] for x in dev])
        cnt = len(MULTI_SIZES)
        if kind == "sgd":
            W.call("wm_sgd_step_multi", cnt, P, G, S1 if a > 0 else None, ns, lr, a)
        elif kind == "adam":
            W.call("wm_adam_step_multi", cnt, P, G, S1, S2, ns, lr, a, b, c, o32.bias_correction(a, t),
                   o32.bias_correction(b, t))
        elif kind == "adamw":
            W.call("wm_adamw_step_multi", cnt, P, G, S1, S2, ns, lr, a, b, c, o32.bias_correction(a, t),
                   o32.bias_correction(b, t), d)
        else:
            W.call("wm_rmsprop_step_multi", cnt, P, G, S1, S2 if c > 0 else None, ns, lr, a, b, c, d)
        for arrs, g in zip(mine, gs):
            oracle_step(kind, hp, arrs[0], g, arrs[1], arrs[2], t)
        for i, (arrs, slots) in enumerate(zip(mine, dev)):
            for j in range(3):
                assert oracle.bit_equal(slots[j].get(), arrs[j]), (kind, t, i, j)


def test_multi_many_tensors_and_unscale(wm):
    """A list long enough that the element-wise passes' chunk -> tensor lookup
    crosses many coarse-index blocks, several of them holding dozens of small
    tensors: AdamW bit-exact against the oracle for every tensor, then an
    unscale whose first non-finite value sits in a late small tensor."""
    r = rng(4242)
    sizes = [int(v) for v in r.integers(1, 3000, 300)] + [300001, 4, 70000] + [int(v) for v in r.integers(1, 600, 200)]
    mis = [i % 7 == 3 for i in range(len(sizes))]
    hp = dict(lr=1e-3, a=0.9, b=0.999, c=1e-8, d=0.01)
    mine = [[rng(5 * i).standard_normal(n).astype(np.float32), np.zeros(n, np.float32), np.zeros(n, np.float32)]
            for i, n in enumerate(sizes)]
    dev = [[Slot(x, m) for x in arrs] for arrs, m in zip(mine, mis)]
    gs = [(rng(900 + i).standard_normal(n)).astype(np.float32) for i, n in enumerate(sizes)]
    dgs = [Slot(g, m) for g, m in zip(gs, mis)]
    ns, _ns = W.i64_array(sizes)
    P, _p = _ptrs([x[0] for x in dev])
    G, _g = _ptrs(dgs)
    S1, _s1 = _ptrs([x[1] for x in dev])
    S2, _s2 = _ptrs([x[2] for x in dev])
    W.call("wm_adamw_step_multi", len(sizes), P, G, S1, S2, ns, hp["lr"], hp["a"], hp["b"], hp["c"],
           o32.bias_correction(hp["a"], 1), o32.bias_correction(hp["b"], 1), hp["d"])
    for arrs, g in zip(mine, gs):
        oracle_step("adamw", hp, arrs[0], g, arrs[1], arrs[2], 1)
    for i, (arrs, slots) in enumerate(zip(mine, dev)):
        for j in range(3):
            assert oracle.bit_equal(slots[j].get(), arrs[j]), (i, sizes[i], j)
    # unscale: the first non-finite product is in tensor `bad`
    bad = len(sizes) - 40
    gs2 = [g * np.float32(64.0) for g in gs]
    gs2[bad][sizes[bad] // 2] = np.float32(np.inf)
    gs2[-3][0] = np.float32(np.nan)  # later: must stay untouched
    d2 = [Slot(g, m) for g, m in zip(gs2, mis)]
    G2, _g2 = _ptrs(d2)
    found = W.C.c_int(-1)
    W.call("wm_grad_unscale", len(sizes), G2, ns, W.C.c_float(1.0 / 64.0), W.C.byref(found))
    assert found.value == 1
    for i, (d_, g) in enumerate(zip(d2, gs2)):
        want = g.copy()
        if i < bad:
            want = want * np.float32(1.0 / 64.0)
        elif i == bad:
            k = sizes[bad] // 2
            want[:k] = want[:k] * np.float32(1.0 / 64.0)
        assert oracle.bit_equal(d_.get(), want), i


def test_multi_norm_clip_value(wm):
    gs = [(rng(80 + i).standard_normal(n) * 3).astype(np.float32) for i, (n, _) in enumerate(MULTI_SIZES)]
    ds = [Slot(g, mis) for g, (_, mis) in zip(gs, MULTI_SIZES)]
    G, _g = _ptrs(ds)
    ns, _ns = W.i64_array([n for n, _ in MULTI_SIZES])
    total = W.DeviceArray((1,))
    total.fill(123.0)                                   # overwritten, not accumulated
    W.call("wm_grad_sumsq_multi", len(gs), G, ns, total.vp)
    t_gpu = np.float32(total.to_host()[0])
    t64 = sum(oracle.get("f64").grad_sumsq(g) for g in gs)
    assert abs(float(t_gpu) - t64) <= 1e-5 * t64
    W.call("wm_clip_grad_norm_scale_multi", len(gs), G, ns, total.vp, 10.0)
    coef = np.float32(10.0) / (np.sqrt(t_gpu, dtype=np.float32) + np.float32(1e-6))
    assert coef < 1
    for d_, g in zip(ds, gs):
        assert oracle.bit_equal(d_.get(), g * coef)
    W.call("wm_clip_grad_value_multi", len(gs), G, ns, 0.5)
    for d_, g in zip(ds, gs):
        mine = g * coef
        o32.clip_grad_value(mine, 0.5)
        assert oracle.bit_equal(d_.get(), mine)


@pytest.mark.parametrize("kind,hp", CONFIGS, ids=lambda v: v if isinstance(v, str) else "-".join(map(str, v.values())))
def test_multi_duplicated_parameter(wm, kind, hp):
    """A parameter listed twice (one module added to a list twice) is
    updated twice, one update after the other, each listing with its own
    state, as the reference's loop over the list does
    (core/optimizer.cpp:22-138); the multi-tensor launch must not let two
    workgroups update it at once."""
    lr, a, b, c, d = hp["lr"], hp.get("a", 0.0), hp.get("b", 0.0), hp.get("c", 0.0), hp.get("d", 0.0)
    n0, n1 = 70001, 4096
    p0 = rng(11).standard_normal(n0).astype(np.float32)
    p1 = rng(12).standard_normal(n1).astype(np.float32)
    # list: [p0, p1, p0] with separate state per listing
    mine_p = [p0.copy(), p1.copy()]
    states = [[np.zeros(n, np.float32), np.zeros(n, np.float32)] for n in (n0, n1, n0)]
    dp = [Slot(p0), Slot(p1)]
    ds = [[Slot(s[0]), Slot(s[1])] for s in states]
    for t in range(1, 3):
        g0 = (rng(20 + t).standard_normal(n0)).astype(np.float32)
        g1 = (rng(30 + t).standard_normal(n1)).astype(np.float32)
        dg = [Slot(g0), Slot(g1)]
        P, _p = _ptrs([dp[0], dp[1], dp[0]])
        G, _g = _ptrs([dg[0], dg[1], dg[0]])
        S1, _s1 = _ptrs([x[0] for x in ds])
        S2, _s2 = _ptrs([x[1] for x in ds])
        ns, _ns = W.i64_array([n0, n1, n0])
        if kind == "sgd":
            W.call("wm_sgd_step_multi", 3, P, G, S1 if a > 0 else None, ns, lr, a)
        elif kind == "adam":
            W.call("wm_adam_step_multi", 3, P, G, S1, S2, ns, lr, a, b, c, o32.bias_correction(a, t),
                   o32.bias_correction(b, t))
        elif kind == "adamw":
            W.call("wm_adamw_step_multi", 3, P, G, S1, S2, ns, lr, a, b, c, o32.bias_correction(a, t),
                   o32.bias_correction(b, t), d)
        else:
            W.call("wm_rmsprop_step_multi", 3, P, G, S1, S2 if c > 0 else None, ns, lr, a, b, c, d)
        for which, g, st in ((0, g0, states[0]), (1, g1, states[1]), (0, g0, states[2])):
            oracle_step(kind, hp, mine_p[which], g, st[0], st[1], t)
        assert oracle.bit_equal(dp[0].get(), mine_p[0]), (kind, t)
        assert oracle.bit_equal(dp[1].get(), mine_p[1]), (kind, t)


def test_multi_duplicated_gradient_clip_and_unscale(wm):
    """clip_grad_value_ / clip_grad_norm_'s scaling and GradScaler::unscale
    over a list holding one gradient twice: applied twice in list order."""
    n = 50000
    g = (rng(40).standard_normal(n) * 3).astype(np.float32)
    d = Slot(g)
    G, _g = _ptrs([d, d])
    ns, _ns = W.i64_array([n, n])
    W.call("wm_clip_grad_value_multi", 2, G, ns, 0.5)
    mine = g.copy()
    o32.clip_grad_value(mine, 0.5)
    o32.clip_grad_value(mine, 0.5)
    assert oracle.bit_equal(d.get(), mine)
    total = W.DeviceArray.from_host(np.float32([400.0]))
    W.call("wm_clip_grad_norm_scale_multi", 2, G, ns, total.vp, 2.0)
    coef = np.float32(2.0) / (np.sqrt(np.float32(400.0)) + np.float32(1e-6))
    mine = (mine * coef) * coef
    assert oracle.bit_equal(d.get(), mine)
    found = C.c_int(-1)
    inv = np.float32(1.0) / np.float32(4.0)
    W.call("wm_grad_unscale", 2, G, ns, float(inv), C.byref(found))
    assert found.value == 0
    assert oracle.bit_equal(d.get(), (mine * inv) * inv)


# ---- deferred scalings (wm_grad_scale) ---------------------------------------

def _eager(g, gsv, sumsq):
    """The reference's in-place multiplications on a copy of g: unscale's
    prefix (core/amp.h:131-142), then clip_grad_norm_'s coefficient
    (core/optimizer.cpp:155-164), each product rounded to fp32."""
    v = g.copy()
    k = gsv.unscale_count
    v[:k] = v[:k] * np.float32(gsv.unscale)
    if gsv.clip_sumsq:
        c = np.float32(gsv.clip_max_norm) / (np.sqrt(np.float32(sumsq)) + np.float32(1e-6))
        if c < 1:
            v = v * c
    return v


@pytest.mark.parametrize("kind,hp", CONFIGS, ids=lambda v: v if isinstance(v, str) else "-".join(map(str, v.values())))
def test_multi_steps_with_deferred_scaling(wm, kind, hp):
    """The *_multi_gs steps read each gradient through its pending unscale
    prefix and clip coefficient: bit-exact against the oracle's steps on the
    eagerly multiplied gradients, per-entry scalings differing (full, partial
    and no unscale; clip or none), the clip's sum of squares a device float
    written by wm_grad_sumsq_multi_gs over the unscaled values."""
    lr, a, b, c, d = hp["lr"], hp.get("a", 0.0), hp.get("b", 0.0), hp.get("c", 0.0), hp.get("d", 0.0)
    sizes = [n for n, _ in MULTI_SIZES]
    mine, dev = [], []
    for i, (n, mis) in enumerate(MULTI_SIZES):
        arrs = [rng(17 * i).standard_normal(n).astype(np.float32), np.zeros(n, np.float32), np.zeros(n, np.float32)]
        mine.append(arrs)
        dev.append([Slot(x, mis) for x in arrs])
    ns, _ns = W.i64_array(sizes)
    inv = float(np.float32(1.0) / np.float32(1024.0))
    counts = [n if i % 3 != 2 else n // 3 for i, n in enumerate(sizes)]
    counts[3] = 0
    total = W.DeviceArray((1,))
    for t in range(1, 4):
        gs = [(rng(300 * t + i).standard_normal(n) * 1024.0).astype(np.float32) for i, n in enumerate(sizes)]
        dgs = [Slot(g, mis) for g, (_, mis) in zip(gs, MULTI_SIZES)]
        G, _g = _ptrs(dgs)
        unscale = [W.GradScale(inv, k, None, 0.0) for k in counts]
        GS, _gs = W.grad_scale_array(unscale)
        W.call("wm_grad_sumsq_multi_gs", len(sizes), G, GS, ns, 1.0, total.vp)
        sumsq = np.float32(total.to_host()[0])
        entries = [W.GradScale(inv, k, None if i == 5 else total.ptr, 1.0) for i, k in enumerate(counts)]
        GS, _gs = W.grad_scale_array(entries)
        P, _p = _ptrs([x[0] for x in dev])
        S1, _s1 = _ptrs([x[1] for x in dev])
        S2, _s2 = _ptrs([x[2] for x in dev])
        cnt = len(sizes)
        if kind == "sgd":
            W.call("wm_sgd_step_multi_gs", cnt, P, G, GS, S1 if a > 0 else None, ns, lr, a)
        elif kind == "adam":
            W.call("wm_adam_step_multi_gs", cnt, P, G, GS, S1, S2, ns, lr, a, b, c, o32.bias_correction(a, t),
                   o32.bias_correction(b, t))
        elif kind == "adamw":
            W.call("wm_adamw_step_multi_gs", cnt, P, G, GS, S1, S2, ns, lr, a, b, c, o32.bias_correction(a, t),
                   o32.bias_correction(b, t), d)
        else:
            W.call("wm_rmsprop_step_multi_gs", cnt, P, G, GS, S1, S2 if c > 0 else None, ns, lr, a, b, c, d)
        eager = [_eager(g, e, sumsq) for g, e in zip(gs, entries)]
        for arrs, v in zip(mine, eager):
            oracle_step(kind, hp, arrs[0], v, arrs[1], arrs[2], t)
        for i, (arrs, slots) in enumerate(zip(mine, dev)):
            for j in range(3):
                assert oracle.bit_equal(slots[j].get(), arrs[j]), (kind, t, i, j)
        for dg, g in zip(dgs, gs):                       # the steps only read the gradients
            assert oracle.bit_equal(dg.get(), g)


def test_deferred_scaling_norm_search_and_apply(wm):
    """wm_grad_sumsq_multi_gs equals wm_grad_sumsq_multi over the eagerly
    multiplied gradients bit for bit (same reduction order); the finiteness
    search finds the first non-finite v * scale; wm_grad_scale_apply_multi
    writes exactly the eager products."""
    sizes = [n for n, _ in MULTI_SIZES]
    ns, _ns = W.i64_array(sizes)
    gs = [(rng(500 + i).standard_normal(n) * 300.0).astype(np.float32) for i, n in enumerate(sizes)]
    counts = [n // 2 if i % 2 else n for i, n in enumerate(sizes)]
    clip_total = W.DeviceArray.from_host(np.float32([2.5e9]))
    entries = [W.GradScale(0.125, k, clip_total.ptr if i != 1 else None, 3000.0) for i, k in enumerate(counts)]
    GS, _gs = W.grad_scale_array(entries)
    eager = [_eager(g, e, np.float32(2.5e9)) for g, e in zip(gs, entries)]
    dgs = [Slot(g, mis) for g, (_, mis) in zip(gs, MULTI_SIZES)]
    des = [Slot(v, mis) for v, (_, mis) in zip(eager, MULTI_SIZES)]
    G, _g = _ptrs(dgs)
    E, _e = _ptrs(des)
    t_gs, t_eager = W.DeviceArray((1,)), W.DeviceArray((1,))
    W.call("wm_grad_sumsq_multi_gs", len(sizes), G, GS, ns, 1.0, t_gs.vp)
    W.call("wm_grad_sumsq_multi", len(sizes), E, ns, t_eager.vp)
    assert oracle.bit_equal(t_gs.to_host(), t_eager.to_host())
    W.call("wm_grad_sumsq_multi_gs", len(sizes), G, GS, ns, 0.5, t_gs.vp)
    W.call("wm_grad_sumsq_scaled_multi", len(sizes), E, ns, 0.5, t_eager.vp)
    assert oracle.bit_equal(t_gs.to_host(), t_eager.to_host())
    where = (C.c_int64 * 2)(-1, -1)
    W.call("wm_grad_first_bad_multi_gs", len(sizes), G, GS, ns, 1.0, C.cast(where, C.c_void_p))
    assert list(where) == [len(sizes), 0]
    # a value finite as stored but not once multiplied: the search sees v
    big = np.float32(3e38)
    gs[5][77] = big
    dgs[5] = Slot(gs[5], MULTI_SIZES[5][1])
    G, _g = _ptrs(dgs)
    ent = list(entries)
    ent[5] = W.GradScale(4.0, 100, None, 0.0)
    GS, _gs = W.grad_scale_array(ent)
    W.call("wm_grad_first_bad_multi_gs", len(sizes), G, GS, ns, 1.0, C.cast(where, C.c_void_p))
    assert list(where) == [5, 77]
    W.call("wm_grad_scale_apply_multi", len(sizes), G, GS, ns)
    for dg, g, e in zip(dgs, gs, ent):
        assert oracle.bit_equal(dg.get(), _eager(g, e, np.float32(2.5e9)))
