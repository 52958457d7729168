"""GPU parity of MultiHeadAttention's forward and closure (wm_mha_fwd /
wm_mha_bwd, include/wm_layers.h) through the C ABI, against the oracle's
restatement of core/layer.cpp:1103-1437 (pinned bit-exact against the
reference's IEEE build in test_oracle_gemm.py).

Contract: within 1e-5 of the fp64 oracle relative to the first-order error
scale of each value -- for the forward composed here from the fp64 values
(sum of |terms| of each product, an attention weight's sensitivity to its
row's scores, carried through the context and output products); for the
backward the abs oracle's closure fed the same fp32 intermediates the GPU
forward saved, as the reference's closure reads what its forward stored.
"""
import numpy as np
import pytest

import oracle
from gpu_helpers import mha_bwd, mha_forward_scales, mha_fwd, rng_normal, rng_uniform

pytestmark = pytest.mark.gpu

o64, oab = oracle.get("f64"), oracle.get("abs")


@pytest.fixture(autouse=True, params=[1, 0], ids=["route-fused", "route-two-pass"])
def route(request, wm):
    """Every test under both routes of the per-head score products
    (wm_mha_fused): the fused score / softmax kernels where the shape fits
    (keys <= 1024, head width <= 128 and a multiple of 4), and the two-pass
    route (product into a scores buffer, then the attention softmax)."""
    from whitematter_amd import _lib as W
    before = W.lib().wm_mha_fused(-1)
    W.lib().wm_mha_fused(request.param)
    yield request.param
    W.lib().wm_mha_fused(before)


def close(got, ref, scale, rtol=1e-5, atol=1e-30):
    ok, worst = oracle.close_scaled(got, ref, scale, rtol, atol)
    assert ok, f"{worst:.3g}x tolerance"


def params_for(E, seed):
    s = 1.0 / np.sqrt(E)
    return ([rng_normal((E, E), seed + i, s) for i in range(4)] + [rng_normal((E,), seed + 4 + i, 0.1)
                                                                     for i in range(4)])


CASES = [(2, 5, 5, 8, 2, None), (1, 4, 6, 12, 3, "batch"), (2, 6, 6, 16, 4, "causal"), (1, 3, 3, 8, 1, None),
         (2, 64, 64, 64, 4, "causal"), (1, 33, 47, 96, 3, "batch"), (2, 128, 128, 128, 8, None),
         (1, 200, 130, 64, 2, None), (2, 256, 256, 256, 8, "causal"),
         # ragged query blocks against longer key rows (softmax tiles of 2, 4
         # and more than 8 float4 per thread)
         (1, 37, 300, 32, 1, "causal"), (2, 40, 700, 64, 2, "batch"), (1, 20, 1100, 32, 2, None),
         # the fused kernels' edges: 1024 keys (eight 128-key chunks) at head
         # width 64; widths 128 (four k stages), 100 (zero-filled k) and 36;
         # past the fused limits (1025 keys, width 132: the two-pass route)
         (2, 70, 1024, 128, 2, "causal"), (1, 50, 257, 256, 2, "batch"), (1, 33, 129, 200, 2, None),
         (1, 40, 90, 72, 2, "batch"), (2, 96, 1025, 64, 1, "causal"), (1, 17, 64, 264, 2, None),
         # one key, one query row, width 128 at E = 1024, and workgroup counts
         # that are (16, 72) and are not (1, 4, 6, 27) multiples of the 8 XCDs
         (3, 1, 1, 8, 2, None), (1, 2, 1, 4, 1, "batch"), (1, 1, 300, 64, 4, "causal"),
         (1, 40, 70, 1024, 8, "causal"), (3, 70, 200, 96, 8, "batch"), (3, 65, 128, 48, 3, None),
         # past 1024 keys: the two-pass forward with the fused backward, whose
         # chunk loop has no key limit
         (1, 33, 2100, 64, 2, "batch"), (2, 40, 1500, 96, 3, "causal")]


def case_inputs(case, seed):
    B, Sq, Sk, E, H, mk = case
    q, k, v = rng_normal((B, Sq, E), seed), rng_normal((B, Sk, E), seed + 1), rng_normal((B, Sk, E), seed + 2)
    if mk == "causal":
        m = np.where(np.triu(np.ones((Sq, Sk)), 1) > 0, -1e9, 0).astype(np.float32)[None, None]
    elif mk == "batch":
        m = np.where(rng_uniform((B, 1, Sq, Sk), seed + 3, 0, 1) < 0.3, np.float32(-1e9), np.float32(0))
        m = m.astype(np.float32)
    else:
        m = None
    return q, k, v, m, params_for(E, seed + 10)


@pytest.mark.parametrize("case", CASES, ids=str)
def test_mha_forward(wm, case):
    q, k, v, m, params = case_inputs(case, 1)
    H = case[4]
    got = mha_fwd(q, k, v, params, H, m)
    ref = o64.mha_forward(q, k, v, params, H, m)
    sc = mha_forward_scales(q, k, v, params, H, ref)
    for name in ("Q", "K", "V", "attn", "ctx", "out"):
        close(got[name], ref[name], sc[name])
    assert np.allclose(got["attn"].astype(np.float64).sum(-1), 1.0, atol=1e-5)
    if case[5] == "causal":
        assert np.all(got["attn"][..., np.triu(np.ones(case[1:3], bool), 1)] == 0)


@pytest.mark.parametrize("case", CASES, ids=str)
def test_mha_backward(wm, case):
    q, k, v, m, params = case_inputs(case, 2)
    H = case[4]
    saved = mha_fwd(q, k, v, params, H, m)
    dout = rng_normal(q.shape, 30)
    got = mha_bwd(dout, q, k, v, params, H, saved)
    ref = o64.mha_backward(dout, q, k, v, params, H, saved)
    scale = oab.mha_backward(dout, q, k, v, params, H, saved)
    for name in ref:
        close(got[name], ref[name], scale[name])


def test_mha_backward_self_attention_accumulates(wm):
    """One buffer for q = k = v collects the three input gradients on top of
    its starting value; parameter gradients add to theirs."""
    B, S, E, H = 2, 16, 32, 4
    x = rng_normal((B, S, E), 40)
    params = params_for(E, 41)
    saved = mha_fwd(x, x, x, params, H)
    dout = rng_normal(x.shape, 42)
    start = {"gq": rng_normal(x.shape, 43), "gWq": rng_normal((E, E), 44), "gbo": rng_normal((E,), 45)}
    got = mha_bwd(dout, x, x, x, params, H, saved, alias=True, start=start)
    ref = o64.mha_backward(dout, x, x, x, params, H, saved, alias=True)
    scale = oab.mha_backward(dout, x, x, x, params, H, saved, alias=True)
    for name in ("gq", "gWq", "gbo"):
        close(got[name], ref[name] + start[name], scale[name] + np.abs(start[name]))
    for name in ("gWk", "gWv", "gWo", "gbq", "gbk", "gbv"):
        close(got[name], ref[name], scale[name])


@pytest.mark.parametrize("need", [(False, False, False), (True, False, True)])
def test_mha_backward_without_some_input_gradients(wm, need):
    q, k, v, m, params = case_inputs((2, 9, 11, 24, 3, "batch"), 50)
    saved = mha_fwd(q, k, v, params, 3, m)
    dout = rng_normal(q.shape, 51)
    got = mha_bwd(dout, q, k, v, params, 3, saved, need=need)
    ref = o64.mha_backward(dout, q, k, v, params, 3, saved, need=need)
    scale = oab.mha_backward(dout, q, k, v, params, 3, saved, need=need)
    for name in ref:
        if ref[name] is None:
            assert name not in got
        else:
            close(got[name], ref[name], scale[name])


@pytest.mark.parametrize("Sk", [7, 300])
def test_mha_fully_masked_rows(wm, Sk):
    """A row whose mask is -inf everywhere: the reference's max stays at
    -FLT_MAX, every exp is 0 and the row becomes 0 / 0 = NaN (core/layer.cpp:
    1213-1236); the other rows are unaffected."""
    B, Sq, E, H = 1, 5, 16, 2
    q, k, v = rng_normal((B, Sq, E), 60), rng_normal((B, Sk, E), 61), rng_normal((B, Sk, E), 62)
    m = np.zeros((1, 1, Sq, Sk), np.float32)
    m[0, 0, 2, :] = -np.inf
    params = params_for(E, 63)
    got = mha_fwd(q, k, v, params, H, m)
    assert np.all(np.isnan(got["attn"][:, :, 2, :]))
    rest = np.delete(got["attn"], 2, axis=2)
    assert np.all(np.isfinite(rest))
    assert np.allclose(rest.astype(np.float64).sum(-1), 1.0, atol=1e-5)


def test_mha_routes_agree_at_width_64(wm):
    """The fused kernels against the two-pass route at the bench's head width
    and key length (16 heads of 64, 1024 keys, causal): the same products in
    the same k order, so the weights differ only by the softmax sums' order
    and the score gradients by the row dot's form."""
    from whitematter_amd import _lib as W
    B, Sq, Sk, E, H = 1, 64, 1024, 1024, 16
    q, k, v = rng_normal((B, Sq, E), 70), rng_normal((B, Sk, E), 71), rng_normal((B, Sk, E), 72)
    m = np.where(np.triu(np.ones((Sq, Sk)), 1) > 0, -1e9, 0).astype(np.float32)[None, None]
    params = params_for(E, 73)
    dout = rng_normal(q.shape, 74)
    res = {}
    for mode in (1, 0):
        W.lib().wm_mha_fused(mode)
        saved = mha_fwd(q, k, v, params, H, m)
        res[mode] = (saved, mha_bwd(dout, q, k, v, params, H, saved))
    (f1, g1), (f0, g0) = res[1], res[0]
    for name in ("Q", "K", "V"):
        assert np.array_equal(f1[name], f0[name])
    ref = o64.mha_forward(q, k, v, params, H, m)
    sc = mha_forward_scales(q, k, v, params, H, ref)
    for name in ("attn", "ctx", "out"):
        close(f1[name], f0[name], sc[name])
    scale = oab.mha_backward(dout, q, k, v, params, H, f0)
    for name in g0:
        close(g1[name], g0[name], scale[name])
