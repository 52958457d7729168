"""GPU parity of the fp32 matrix products (include/wm_gemm.h) through the C
ABI: Tensor::matmul / Tensor::bmm and their closures (core/tensor.cpp:
783-895) and the general strided product.

Contract: within 1e-5 of the fp64 oracle (or_bmm / or_bmm_bwd, pinned in
test_oracle_gemm.py) relative to the abs oracle's sum_k |a_ik * b_kj| (plus
|C| and |bias| where they are added); bit-exact where every partial sum is
exact in fp32 (small integers).  Sizes past the oracle's seconds are checked
against numpy's float64 product, which test_oracle_gemm.py pins to the fp64
oracle.
"""
import numpy as np
import pytest

import oracle
from gpu_helpers import gemm, matmul, matmul_bwd, rng_normal, rng_uniform

pytestmark = pytest.mark.gpu

o64, oab = oracle.get("f64"), oracle.get("abs")


def close(got, ref, scale, rtol=1e-5):
    ok, worst = oracle.close_scaled(got, ref, scale, rtol, 1e-30)
    assert ok, f"{worst:.3g}x tolerance"


@pytest.fixture(autouse=True, params=[1, 0], ids=["route-default", "route-mfma-kernel"])
def route(request, wm):
    """Every test under both routes of the plain large products
    (wm_gemm_library): rocBLAS where it is faster, and this library's MFMA
    kernels for everything."""
    from whitematter_amd import _lib as W
    before = W.lib().wm_gemm_library(-1)
    W.lib().wm_gemm_library(request.param)
    yield request.param
    W.lib().wm_gemm_library(before)


SHAPES = [(1, 1, 1), (2, 3, 2), (3, 5, 7), (33, 65, 17), (64, 31, 129), (5, 1, 4), (7, 40, 1), (128, 32, 128),
          (128, 64, 256), (129, 33, 127), (256, 100, 200), (300, 513, 257)]


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_matmul_forward(wm, shape):
    m, k, n = shape
    a, b = rng_normal((m, k), 1), rng_normal((k, n), 2)
    close(matmul(a, b), o64.matmul(a, b), oab.matmul(a, b))


@pytest.mark.parametrize("shape", SHAPES, ids=str)
@pytest.mark.parametrize("accumulate", [False, True])
def test_matmul_backward(wm, shape, accumulate):
    m, k, n = shape
    a, b, g = rng_normal((m, k), 3), rng_normal((k, n), 4), rng_normal((m, n), 5)
    ga0 = rng_normal((m, k), 6) if accumulate else None
    gb0 = rng_normal((k, n), 7) if accumulate else None
    ga, gb = matmul_bwd(g, a, b, ga0, gb0)
    ra, rb = o64.matmul_bwd(g, a, b, ga0, gb0)
    sa, sb = oab.matmul_bwd(g, a, b, None if ga0 is None else np.abs(ga0), None if gb0 is None else np.abs(gb0))
    close(ga, ra, sa)
    close(gb, rb, sb)


@pytest.mark.parametrize("need", [(True, False), (False, True)])
def test_matmul_backward_one_side(wm, need):
    a, b, g = rng_normal((40, 24), 8), rng_normal((24, 56), 9), rng_normal((40, 56), 10)
    ga, gb = matmul_bwd(g, a, b, need_a=need[0], need_b=need[1])
    ra, rb = o64.matmul_bwd(g, a, b)
    sa, sb = oab.matmul_bwd(g, a, b)
    assert (ga is None) != need[0] and (gb is None) != need[1]
    if need[0]:
        close(ga, ra, sa)
    else:
        close(gb, rb, sb)


@pytest.mark.parametrize("shape", [(1, 2, 3, 2), (2, 2, 3, 2), (4, 33, 17, 65), (3, 128, 64, 128), (6, 70, 129, 40)],
                         ids=str)
def test_bmm_forward_backward(wm, shape):
    P, m, k, n = shape
    a, b, g = rng_normal((P, m, k), 11), rng_normal((P, k, n), 12), rng_normal((P, m, n), 13)
    close(matmul(a, b), o64.bmm(a, b), oab.bmm(a, b))
    ga0, gb0 = rng_normal((P, m, k), 14), rng_normal((P, k, n), 15)
    ga, gb = matmul_bwd(g, a, b, ga0, gb0)
    ra, rb = o64.bmm_bwd(g, a, b, ga0, gb0)
    sa, sb = oab.bmm_bwd(g, a, b, np.abs(ga0), np.abs(gb0))
    close(ga, ra, sa)
    close(gb, rb, sb)


def test_known_answer_and_small_integers_exact(wm):
    a = np.float32([1, 2, 3, 4, 5, 6]).reshape(2, 3)
    assert np.array_equal(matmul(a, a.reshape(3, 2)), [[22, 28], [49, 64]])  # test_tensor.cpp matmul_2d
    for m, k, n, seed in ((17, 23, 11, 20), (130, 70, 129, 21), (256, 256, 256, 22)):
        r = np.random.default_rng(seed)
        ai = r.integers(-8, 9, (m, k)).astype(np.float32)
        bi = r.integers(-8, 9, (k, n)).astype(np.float32)
        gi = r.integers(-4, 5, (m, n)).astype(np.float32)
        exact = ai.astype(np.int64) @ bi.astype(np.int64)
        assert np.array_equal(matmul(ai, bi), exact)
        ga, gb = matmul_bwd(gi, ai, bi)
        assert np.array_equal(ga, gi.astype(np.int64) @ bi.astype(np.int64).T)
        assert np.array_equal(gb, ai.astype(np.int64).T @ gi.astype(np.int64))


def op_store(x, trans, ld):
    """Row-major storage of op(X) = x (trans: store x^T) with row stride ld."""
    s = x.T if trans else x
    buf = np.full((s.shape[0], ld), np.nan, np.float32)
    buf[:, :s.shape[1]] = s
    return buf


@pytest.mark.parametrize("trans", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=lambda t: "NT"[t[0]] + "NT"[t[1]])
@pytest.mark.parametrize("mnk", [(1, 1, 1), (5, 3, 7), (128, 128, 32), (130, 129, 33), (257, 64, 100),
                                 (64, 300, 513)], ids=str)
@pytest.mark.parametrize("pad", [0, 3, 4])
def test_gemm_transposes_strides_alpha_accumulate_bias(wm, trans, mnk, pad):
    ta, tb = trans
    m, n, k = mnk
    A, B = rng_normal((m, k), 30), rng_normal((k, n), 31)
    C0, bias = rng_normal((m, n), 32), rng_normal((n,), 33)
    sa, sb = op_store(A, ta, (m if ta else k) + pad), op_store(B, tb, (k if tb else n) + pad)
    ldc = n + pad
    c0 = np.full((m, ldc), 7.0, np.float32)
    c0[:, :n] = C0
    alpha = 0.375
    got = gemm(ta, tb, m, n, k, alpha, sa, sa.shape[1], sb, sb.shape[1], c0, ldc, True, bias)
    ref = alpha * o64.matmul(A, B) + C0 + bias
    scale = alpha * oab.matmul(A, B) + np.abs(C0) + np.abs(bias)
    close(got[:, :n], ref, scale)
    assert np.all(got[:, n:] == 7.0)  # the row padding of C is untouched
    # overwrite, no bias
    got = gemm(ta, tb, m, n, k, 1.0, sa, sa.shape[1], sb, sb.shape[1], c0, ldc, False)
    close(got[:, :n], o64.matmul(A, B), oab.matmul(A, B))


def test_gemm_k_zero_and_empty(wm):
    c0 = rng_normal((3, 4), 40)
    bias = rng_normal((4,), 41)
    got = gemm(0, 0, 3, 4, 0, 1.0, np.zeros(1, np.float32), 1, np.zeros(1, np.float32), 4, c0, 4, True, bias)
    assert np.array_equal(got, c0 + bias)
    got = gemm(0, 0, 3, 4, 0, 1.0, np.zeros(1, np.float32), 1, np.zeros(1, np.float32), 4, c0, 4, False)
    assert np.array_equal(got, np.zeros((3, 4), np.float32))
    assert matmul(np.zeros((0, 5), np.float32), rng_normal((5, 3), 42)).shape == (0, 3)


@pytest.mark.parametrize("mnk", [(128, 128, 1), (130, 140, 100), (200, 129, 256), (128, 256, 257)], ids=str)
def test_gemm_one_level_batch_padded_alpha_accumulate(wm, mnk):
    """One-level batches of untransposed products with padded rows and
    problem strides, alpha and accumulation (the shapes up to k = 256 with
    m, n >= 128 take rocBLAS's strided-batched route by default, k = 257
    this library's kernel); the padding of C stays untouched."""
    m, n, k = mnk
    P, pad, gap = 3, 3, 11
    lda, ldb, ldc = k + pad, n + pad, n + pad
    sa, sb, sc = m * lda + gap, k * ldb + gap, m * ldc + gap
    A, B = rng_normal((P, m, k), 45), rng_normal((P, k, n), 46)
    C0 = rng_normal((P, m, n), 47)
    a = np.zeros(P * sa, np.float32)
    b = np.zeros(P * sb, np.float32)
    c0 = np.full(P * sc, 7.0, np.float32)
    for p in range(P):
        a[p * sa:p * sa + m * lda].reshape(m, lda)[:, :k] = A[p]
        b[p * sb:p * sb + k * ldb].reshape(k, ldb)[:, :n] = B[p]
        c0[p * sc:p * sc + m * ldc].reshape(m, ldc)[:, :n] = C0[p]
    alpha = 0.625
    got = gemm(0, 0, m, n, k, alpha, a, lda, b, ldb, c0, ldc, True, None, P, 1, (sa, 0, sb, 0, sc, 0))
    for p in range(P):
        gp = got[p * sc:p * sc + m * ldc].reshape(m, ldc)
        close(gp[:, :n], alpha * o64.matmul(A[p], B[p]) + C0[p], alpha * oab.matmul(A[p], B[p]) + np.abs(C0[p]))
        assert np.all(gp[:, n:] == 7.0)
        if p + 1 < P:
            assert np.all(got[p * sc + m * ldc:(p + 1) * sc] == 7.0)  # the gap between problems


@pytest.mark.parametrize("case", [(2, 128, 128, 64, False), (5, 256, 384, 192, True), (3, 384, 128, 1024, False),
                                  (17, 1024, 1024, 64, True), (16, 1024, 512, 128, False)], ids=str)
def test_gemm_dma_batches(wm, case):
    """One-level batches whose tiles are all interior (m, n multiples of 128,
    k of 64, 16-byte rows) run on the direct-to-LDS kernel (untransposed here):
    k = 64 and 192 (one and three rounds of its four stage buffers), 1024;
    17 problems of 64 tiles take two problems per workgroup with a last
    workgroup of one; padded rows (pad 4 keeps the rows 16-byte aligned) and
    gaps between problems stay untouched; alpha, accumulation and a bias."""
    P, m, n, k, with_bias = case
    pad, gap = 4, 8
    lda, ldb, ldc = k + pad, n + pad, n + pad
    sa, sb, sc = m * lda + gap, k * ldb + gap, m * ldc + gap
    A, B = rng_normal((P, m, k), 80), rng_uniform((P, k, n), 81, -1.0, 1.0)
    C0 = rng_normal((P, m, n), 82)
    bias = rng_normal((n,), 83) if with_bias else None
    a = np.zeros(P * sa, np.float32)
    b = np.zeros(P * sb, np.float32)
    c0 = np.full(P * sc, 7.0, np.float32)
    for q in range(P):
        a[q * sa:q * sa + m * lda].reshape(m, lda)[:, :k] = A[q]
        b[q * sb:q * sb + k * ldb].reshape(k, ldb)[:, :n] = B[q]
        c0[q * sc:q * sc + m * ldc].reshape(m, ldc)[:, :n] = C0[q]
    alpha = 0.625
    got = gemm(0, 0, m, n, k, alpha, a, lda, b, ldb, c0, ldc, True, bias, P, 1, (sa, 0, sb, 0, sc, 0))
    bias64 = np.zeros(n) if bias is None else bias.astype(np.float64)
    for q in range(P):
        gq = got[q * sc:q * sc + m * ldc].reshape(m, ldc)
        a64, b64 = A[q].astype(np.float64), B[q].astype(np.float64)
        ref = alpha * (a64 @ b64) + C0[q] + bias64
        scale = alpha * (np.abs(a64) @ np.abs(b64)) + np.abs(C0[q]) + np.abs(bias64)
        close(gq[:, :n], ref, scale)
        assert np.all(gq[:, n:] == 7.0)
        if q + 1 < P:
            assert np.all(got[q * sc + m * ldc:(q + 1) * sc] == 7.0)


@pytest.mark.parametrize("trans", [(0, 1), (1, 0), (1, 1)], ids=lambda t: "NT"[t[0]] + "NT"[t[1]])
@pytest.mark.parametrize("case", [(3, 128, 256, 64), (2, 256, 128, 192), (4, 256, 256, 384), (3, 1024, 128, 1024),
                                  (17, 1024, 1024, 64)], ids=str)
def test_gemm_dma_transposed(wm, trans, case):
    """The direct-to-LDS kernels with transposed operands (A stored k x m,
    B stored n x k): the k-contiguous and row-contiguous stagings swap sides;
    k <= 256 on the three-buffer kernel, k = 384 on the four-buffer one.
    Padded leading dimensions and gaps between problems, alpha, accumulation
    and a bias; 17 problems of 64 tiles take two problems per workgroup."""
    ta, tb = trans
    P, m, n, k = case
    pad, gap = 4, 8
    ar, ac = (k, m) if ta else (m, k)
    br, bc = (n, k) if tb else (k, n)
    lda, ldb, ldc = ac + pad, bc + pad, n + pad
    sa, sb, sc = ar * lda + gap, br * ldb + gap, m * ldc + gap
    A, B = rng_normal((P, ar, ac), 90), rng_uniform((P, br, bc), 91, -1.0, 1.0)
    C0 = rng_normal((P, m, n), 92)
    bias = rng_normal((n,), 93)
    a = np.zeros(P * sa, np.float32)
    b = np.zeros(P * sb, np.float32)
    c0 = np.full(P * sc, 7.0, np.float32)
    for q in range(P):
        a[q * sa:q * sa + ar * lda].reshape(ar, lda)[:, :ac] = A[q]
        b[q * sb:q * sb + br * ldb].reshape(br, ldb)[:, :bc] = B[q]
        c0[q * sc:q * sc + m * ldc].reshape(m, ldc)[:, :n] = C0[q]
    alpha = -1.25
    got = gemm(ta, tb, m, n, k, alpha, a, lda, b, ldb, c0, ldc, True, bias, P, 1, (sa, 0, sb, 0, sc, 0))
    b64 = bias.astype(np.float64)
    for q in range(P):
        gq = got[q * sc:q * sc + m * ldc].reshape(m, ldc)
        oa = (A[q].T if ta else A[q]).astype(np.float64)
        ob = (B[q].T if tb else B[q]).astype(np.float64)
        ref = alpha * (oa @ ob) + C0[q] + b64
        scale = abs(alpha) * (np.abs(oa) @ np.abs(ob)) + np.abs(C0[q]) + np.abs(b64)
        close(gq[:, :n], ref, scale)
        assert np.all(gq[:, n:] == 7.0)
        if q + 1 < P:
            assert np.all(got[q * sc + m * ldc:(q + 1) * sc] == 7.0)


@pytest.mark.parametrize("shape", [(4, 1024, 128, 1024), (64, 256, 128, 256), (8, 512, 128, 512)], ids=str)
def test_bmm_backward_on_dma_kernel(wm, shape):
    """bmm's closure at attention-like shapes: its two products (g b^T and
    a^T g) run on the direct-to-LDS kernel; both gradients, overwritten and
    accumulated."""
    P, t, hd, t2 = shape
    a, b = rng_normal((P, t, hd), 94), rng_normal((P, hd, t2), 95)
    g = rng_normal((P, t, t2), 96)
    a64, b64, g64 = a.astype(np.float64), b.astype(np.float64), g.astype(np.float64)
    ga, gb = matmul_bwd(g, a, b)
    close(ga, g64 @ np.swapaxes(b64, 1, 2), np.abs(g64) @ np.abs(np.swapaxes(b64, 1, 2)))
    close(gb, np.swapaxes(a64, 1, 2) @ g64, np.abs(np.swapaxes(a64, 1, 2)) @ np.abs(g64))
    ga0, gb0 = rng_normal((P, t, hd), 97), rng_normal((P, hd, t2), 98)
    ga, gb = matmul_bwd(g, a, b, ga0, gb0)
    close(ga, ga0 + g64 @ np.swapaxes(b64, 1, 2), np.abs(ga0) + np.abs(g64) @ np.abs(np.swapaxes(b64, 1, 2)))
    close(gb, gb0 + np.swapaxes(a64, 1, 2) @ g64, np.abs(gb0) + np.abs(np.swapaxes(a64, 1, 2)) @ np.abs(g64))


@pytest.mark.parametrize("kind", ["ctx", "dv", "scores"])
@pytest.mark.parametrize("hd", [64, 128])
def test_gemm_two_level_per_head_interior(wm, kind, hd):
    """Per-head products of [B, S, H * hd] activations as MultiHeadAttention
    issues them (two-level batches) at sizes whose tiles are all interior:
    ctx = attn V (NN), dV = attn^T dctx (TN; with 64-wide heads on the
    32-k direct-to-LDS kernel), scores = alpha Q K^T (NT), for 64- and
    128-wide heads."""
    B, S, H = 2, 256, 4
    E = H * hd
    attn = rng_normal((B * H, S, S), 100)
    X, Y = rng_normal((B, S, E), 101), rng_normal((B, S, E), 102)
    heads = lambda Z: Z.reshape(B, S, H, hd).transpose(0, 2, 1, 3).reshape(B * H, S, hd).astype(np.float64)
    a64 = attn.astype(np.float64)
    if kind == "scores":
        alpha = 0.125
        out = np.full((B, H, S, S), np.nan, np.float32)
        got = gemm(0, 1, S, S, hd, alpha, X, E, Y, E, out, S, False, None, B * H, H,
                   (S * E, hd, S * E, hd, H * S * S, S * S)).reshape(B * H, S, S)
        ref = alpha * (heads(X) @ np.swapaxes(heads(Y), 1, 2))
        scale = alpha * (np.abs(heads(X)) @ np.abs(np.swapaxes(heads(Y), 1, 2)))
        close(got, ref, scale)
        return
    ta = 1 if kind == "dv" else 0
    out = np.full((B, S, E), np.nan, np.float32)
    got = gemm(ta, 0, S, hd, S, 1.0, attn, S, X, E, out, E, False, None, B * H, H,
               (H * S * S, S * S, S * E, hd, S * E, hd))
    oa = np.swapaxes(a64, 1, 2) if ta else a64
    ref, scale = oa @ heads(X), np.abs(oa) @ np.abs(heads(X))
    close(heads(got), ref, scale)


@pytest.mark.parametrize("case", [(129, 1024, 32), (5, 256, 96), (3, 384, 1024)], ids=str)
def test_gemm_dma32_transposed_a(wm, case):
    """op(A) = A^T with n = 64 (the attention backward's dV and dK) on the
    32-k direct-to-LDS kernel: one stage (k = 32), three stages rotating over
    the three buffers (k = 96), k = 1024; 129 problems of 8 tiles take two
    problems per workgroup with a last one of one; padded rows, gaps between
    problems, alpha, accumulation and a bias."""
    P, m, k = case
    n, pad, gap = 64, 4, 8
    lda, ldb, ldc = m + pad, n + pad, n + pad
    sa, sb, sc = k * lda + gap, k * ldb + gap, m * ldc + gap
    A, B = rng_normal((P, k, m), 110), rng_uniform((P, k, n), 111, -1.0, 1.0)
    C0 = rng_normal((P, m, n), 112)
    bias = rng_normal((n,), 113)
    a = np.zeros(P * sa, np.float32)
    b = np.zeros(P * sb, np.float32)
    c0 = np.full(P * sc, 7.0, np.float32)
    for q in range(P):
        a[q * sa:q * sa + k * lda].reshape(k, lda)[:, :m] = A[q]
        b[q * sb:q * sb + k * ldb].reshape(k, ldb)[:, :n] = B[q]
        c0[q * sc:q * sc + m * ldc].reshape(m, ldc)[:, :n] = C0[q]
    alpha = 0.75
    got = gemm(1, 0, m, n, k, alpha, a, lda, b, ldb, c0, ldc, True, bias, P, 1, (sa, 0, sb, 0, sc, 0))
    b64 = bias.astype(np.float64)
    for q in range(P):
        gq = got[q * sc:q * sc + m * ldc].reshape(m, ldc)
        oa, ob = A[q].T.astype(np.float64), B[q].astype(np.float64)
        close(gq[:, :n], alpha * (oa @ ob) + C0[q] + b64,
              alpha * (np.abs(oa) @ np.abs(ob)) + np.abs(C0[q]) + np.abs(b64))
        assert np.all(gq[:, n:] == 7.0)
        if q + 1 < P:
            assert np.all(got[q * sc + m * ldc:(q + 1) * sc] == 7.0)


@pytest.mark.parametrize("mnk_lda", [(128, 128, 96, 96), (130, 128, 64, 64), (128, 128, 64, 66)], ids=str)
def test_gemm_dma_near_misses(wm, mnk_lda):
    """Shapes one step outside the direct-to-LDS kernel's conditions (k not a
    multiple of 64, a partial row tile, rows of A not 16-byte aligned) take
    the other kernels with the same results."""
    m, n, k, lda = mnk_lda
    P = 3
    A, B = rng_normal((P, m, k), 84), rng_normal((P, k, n), 85)
    a = np.zeros((P, m, lda), np.float32)
    a[:, :, :k] = A
    got = gemm(0, 0, m, n, k, 1.0, a.ravel(), lda, B.ravel(), n, np.zeros(P * m * n, np.float32), n, False, None, P,
               1, (m * lda, 0, k * n, 0, m * n, 0)).reshape(P, m, n)
    close(got, o64.bmm(A, B), oab.bmm(A, B))


def test_bmm_dma_consecutive_calls(wm):
    """Two products in a row on the direct-to-LDS kernel, the first with two
    problems per workgroup, the second smaller (one problem per workgroup):
    each equals its float64 product."""
    for P, m, n, k, seed in ((20, 1024, 1024, 128, 86), (2, 128, 256, 64, 88)):
        a, b = rng_normal((P, m, k), seed), rng_normal((P, k, n), seed + 1)
        a64, b64 = a.astype(np.float64), b.astype(np.float64)
        close(matmul(a, b), a64 @ b64, np.abs(a64) @ np.abs(b64))


def test_gemm_batch_sharing_one_output(wm):
    """A batch whose problems all write one C (stride 0) overwrites it with
    one problem's product, whichever route: every problem here is the same
    product, so the result is that product."""
    m, n, k, P = 128, 128, 64, 4
    A, B = rng_normal((m, k), 48), rng_normal((k, n), 49)
    got = gemm(0, 0, m, n, k, 1.0, A, k, B, n, np.zeros((m, n), np.float32), n, False, None, P, 1, (0, 0, 0, 0, 0, 0))
    close(got, o64.matmul(A, B), oab.matmul(A, B))


def test_gemm_two_level_batch_per_head_slices(wm):
    """scores[b, h] = Q[b, :, h] @ K[b, :, h]^T * alpha on [B, S, H * hd]
    activations, as MultiHeadAttention slices its heads."""
    B, Sq, Sk, H, hd = 3, 37, 45, 4, 16
    E = H * hd
    Q, K = rng_normal((B, Sq, E), 43), rng_normal((B, Sk, E), 44)
    out = np.full((B, H, Sq, Sk), np.nan, np.float32)
    alpha = 0.25
    got = gemm(0, 1, Sq, Sk, hd, alpha, Q, E, K, E, out, Sk, False, None, B * H, H,
               (Sq * E, hd, Sk * E, hd, H * Sq * Sk, Sq * Sk))
    Qh = Q.reshape(B, Sq, H, hd).transpose(0, 2, 1, 3).reshape(B * H, Sq, hd)
    Kh = K.reshape(B, Sk, H, hd).transpose(0, 2, 3, 1).reshape(B * H, hd, Sk)
    ref = alpha * o64.bmm(np.ascontiguousarray(Qh), np.ascontiguousarray(Kh))
    scale = alpha * oab.bmm(np.ascontiguousarray(Qh), np.ascontiguousarray(Kh))
    close(got.reshape(B * H, Sq, Sk), ref, scale)


@pytest.mark.parametrize("shape", [(2048, 2048, 2048), (1500, 900, 1700), (4096, 1024, 4096)], ids=str)
def test_matmul_large_vs_float64(wm, shape):
    m, k, n = shape
    a, b = rng_normal((m, k), 50), rng_uniform((k, n), 51, -1.0, 1.0)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    close(matmul(a, b), a64 @ b64, np.abs(a64) @ np.abs(b64))


def test_bmm_more_problems_than_one_grid_dimension(wm):
    """70,000 tiny problems: more than the 65,535 the launch's second grid
    dimension holds, so workgroups walk the batch in strides."""
    P, m, k, n = 70000, 2, 3, 5
    a, b = rng_normal((P, m, k), 60), rng_normal((P, k, n), 61)
    close(matmul(a, b), o64.bmm(a, b), oab.bmm(a, b))


@pytest.mark.parametrize("trans", [(0, 0), (0, 1), (1, 0), (1, 1)], ids=lambda t: "NT"[t[0]] + "NT"[t[1]])
@pytest.mark.parametrize("mnk", [(70, 130, 5000), (256, 256, 8192), (200, 40, 3000), (1, 1, 1024)], ids=str)
@pytest.mark.parametrize("pad", [0, 3])
def test_gemm_split_k(wm, trans, mnk, pad):
    """Few output tiles and a long k: the product runs as k slices whose
    partial products a second pass adds (ragged last slice, narrow tiles,
    unaligned rows, accumulate and bias in the second pass)."""
    ta, tb = trans
    m, n, k = mnk
    A, B = rng_normal((m, k), 34), rng_normal((k, n), 35)
    C0, bias = rng_normal((m, n), 36), rng_normal((n,), 37)
    sa, sb = op_store(A, ta, (m if ta else k) + pad), op_store(B, tb, (k if tb else n) + pad)
    ldc = n + pad
    c0 = np.full((m, ldc), 7.0, np.float32)
    c0[:, :n] = C0
    A64, B64 = A.astype(np.float64), B.astype(np.float64)
    alpha = 0.375
    got = gemm(ta, tb, m, n, k, alpha, sa, sa.shape[1], sb, sb.shape[1], c0, ldc, True, bias)
    close(got[:, :n], alpha * (A64 @ B64) + C0 + bias, alpha * (np.abs(A64) @ np.abs(B64)) + np.abs(C0) +
          np.abs(bias))
    assert np.all(got[:, n:] == 7.0)
    got = gemm(ta, tb, m, n, k, 1.0, sa, sa.shape[1], sb, sb.shape[1], c0, ldc, False)
    close(got[:, :n], A64 @ B64, np.abs(A64) @ np.abs(B64))


def test_gemm_split_k_two_level_batch(wm):
    """Per-head weight-gradient-shaped products (hd x hd over a long k) on
    [rows, H * hd] activations: split k across a two-level batch."""
    B, R, H, hd = 2, 2100, 3, 64
    E = H * hd
    X, G = rng_normal((B, R, E), 38), rng_normal((B, R, E), 39)
    out = np.full((B, H, hd, hd), np.nan, np.float32)
    got = gemm(1, 0, hd, hd, R, 1.0, X, E, G, E, out, hd, False, None, B * H, H,
               (R * E, hd, R * E, hd, H * hd * hd, hd * hd))
    Xh = X.astype(np.float64).reshape(B, R, H, hd).transpose(0, 2, 3, 1)
    Gh = G.astype(np.float64).reshape(B, R, H, hd).transpose(0, 2, 1, 3)
    close(got, Xh @ Gh, np.abs(Xh) @ np.abs(Gh))


def test_matmul_weight_gradient_split_k(wm):
    """matmul's closure for a Linear-shaped product: gb = a^T g over 8192
    rows (split k) and ga = g b^T (not split), against float64."""
    m, k, n = 8192, 512, 256
    a, b, g = rng_normal((m, k), 62), rng_normal((k, n), 63), rng_normal((m, n), 64)
    gb0 = rng_normal((k, n), 65)
    ga, gb = matmul_bwd(g, a, b, None, gb0)
    a64, b64, g64 = a.astype(np.float64), b.astype(np.float64), g.astype(np.float64)
    close(ga, g64 @ b64.T, np.abs(g64) @ np.abs(b64).T)
    close(gb, gb0 + a64.T @ g64, np.abs(gb0) + np.abs(a64).T @ np.abs(g64))
