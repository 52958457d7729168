"""GPU tests of the drop-in amp.h (whitematter_amd/core/amp.h, amp.cpp):
HalfTensor's device conversions, GradScaler::unscale / step / update,
check_gradients_finite and clip_grad_norm_amp (reference core/amp.h:96-327),
and the reference's own mixed-precision program (examples/test_amp.cpp)
built against the drop-in headers.

Contract: HalfTensor bit-exact with the oracle's fp16 formulas (pinned
against the reference); unscale bit-exact with fp32 g * (1 / scale) up to
the first non-finite product and untouched from there on, as the reference's
loop (core/amp.h:131-142); the clipping norm is a sum (1e-5 of the fp64
value), the clipped gradients g * coef bit for bit.
"""
import os
import re
import subprocess

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
AMP_BIN = os.path.join(ROOT, "oracle", "_ref", "run_ref_amp")


@pytest.fixture(scope="module")
def T(wm):
    from whitematter_amd import _tensor
    return _tensor


def tensor(T, a, rg=False):
    a = np.ascontiguousarray(a, np.float32)
    return T.Tensor.from_array(a, list(a.shape), rg)


def test_half_tensor_round_trip(T):
    x = np.random.default_rng(1).standard_normal((300, 77)).astype(np.float32) * np.float32(3000)
    x.ravel()[:12] = [0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 6e-8, 2.9e-8, np.inf, -np.inf, np.nan, 1e-40]
    t = tensor(T, x)
    h = T.HalfTensor(t)
    o32 = oracle.get("f32")
    ref = o32.f32_to_f16(x)
    assert np.array_equal(np.asarray(h.data).reshape(x.shape), ref)
    assert list(h.shape) == [300, 77] and h.size() == x.size and h.memory_saved() == 2 * x.size
    back = h.to_float(True)
    assert list(back.shape) == [300, 77] and back.requires_grad
    assert oracle.bit_equal(np.asarray(back.data).reshape(x.shape), o32.f16_to_f32(ref))


def params_with_grads(T, grads):
    ps = []
    for g in grads:
        p = tensor(T, np.zeros_like(g), True)
        p.grad = g
        ps.append(p)
    return ps


def test_grad_scaler_unscale_stops_at_first_non_finite(T):
    rng = np.random.default_rng(2)
    grads = [rng.standard_normal(n).astype(np.float32) * np.float32(1000) for n in (5000, 7000, 3000)]
    grads[1][4321] = np.inf
    ps = params_with_grads(T, grads)
    opt = T.SGD(ps, 0.1)
    scaler = T.GradScaler(1024.0, 2.0, 0.5, 3)
    assert not scaler.unscale(opt)
    inv = np.float32(1.0) / np.float32(1024.0)
    assert np.array_equal(np.asarray(ps[0].grad), grads[0] * inv)
    assert np.array_equal(np.asarray(ps[1].grad)[:4321], grads[1][:4321] * inv)
    assert np.array_equal(np.asarray(ps[1].grad)[4321:], grads[1][4321:])  # the inf and after: untouched
    assert np.array_equal(np.asarray(ps[2].grad), grads[2])
    scaler.step(opt, True)                     # skipped after an overflow
    assert all(not np.asarray(p.data).any() for p in ps)
    scaler.update()
    assert scaler.get_scale() == 512.0 and scaler.growth_tracker() == 0


def test_grad_scaler_finite_step_and_growth(T):
    g = np.random.default_rng(3).standard_normal(4096).astype(np.float32)
    ps = params_with_grads(T, [g])
    opt = T.SGD(ps, 0.5)
    scaler = T.GradScaler(8.0, 2.0, 0.5, 2)
    for i in range(2):
        ps[0].grad = g
        scaler.step(opt)                       # unscale inside, then the optimizer step
        scaler.update()
    assert scaler.get_scale() == 16.0          # grew after growth_interval = 2 clean steps
    gs = g * (np.float32(1.0) / np.float32(8.0))
    assert np.array_equal(np.asarray(ps[0].data), -(np.float32(0.5) * gs) - np.float32(0.5) * gs)
    loss = tensor(T, np.float32([3.0]), True)
    assert float(np.asarray(scaler.scale(loss).data)[0]) == 48.0
    off = T.GradScaler(8.0, 2.0, 0.5, 2, False)
    assert off.get_scale() == 1.0 and off.unscale(opt)


def test_check_gradients_finite(T):
    g = np.random.default_rng(4).standard_normal((64, 33)).astype(np.float32)
    ps = params_with_grads(T, [g, g.copy()])
    ps.append(tensor(T, np.zeros(10, np.float32), True))   # a gradient never written (known zero)
    assert T.check_gradients_finite(ps)
    assert np.array_equal(np.asarray(ps[0].grad), g)     # values untouched
    bad = g.copy()
    bad[7, 3] = np.nan
    ps[1].grad = bad
    assert not T.check_gradients_finite(ps)
    assert np.array_equal(np.asarray(ps[1].grad)[:7], bad[:7])


@pytest.mark.parametrize("max_norm", [1e9, 5.0])
def test_clip_grad_norm_amp(T, max_norm):
    rng = np.random.default_rng(5)
    grads = [rng.standard_normal(n).astype(np.float32) * np.float32(256) for n in (10000, 333)]
    ps = params_with_grads(T, grads)
    scale = 256.0
    norm = T.clip_grad_norm_amp(ps, max_norm, scale)
    g64 = np.concatenate(grads).astype(np.float64) / scale
    ref = np.sqrt((g64 * g64).sum())
    assert abs(norm - ref) <= 1e-5 * ref
    coef = np.float32(max_norm) / (np.float32(norm) + np.float32(1e-6))
    for p, g in zip(ps, grads):
        want = g * coef if coef < 1 else g
        assert np.array_equal(np.asarray(p.grad), want)


@pytest.mark.skipif(not os.path.exists(AMP_BIN), reason="oracle/_ref/run_ref_amp not built")
def test_reference_amp_program_against_drop_in():
    """examples/test_amp.cpp (fp16 conversion, HalfTensor, GradScaler, a
    scaled training loop, overflow back-off) built against the drop-in
    headers: every one of its five checks passes."""
    r = subprocess.run([AMP_BIN], capture_output=True, text=True, timeout=300)
    out = r.stdout + r.stderr
    print(out[-3000:])
    assert r.returncode == 0, out[-2000:]
    assert len(re.findall(r"^\s+PASSED", out, re.M)) == 5 and "FAILED" not in out, out[-2000:]
    assert "All tests completed!" in out


def test_clip_grad_norm_amp_large_scaled_gradients(T):
    """Each element is scaled before it is squared (core/amp.h:306-312): with
    scale 2^32 and an unscaled norm near 1e10, g^2 alone would overflow fp32,
    the reference's sum does not."""
    rng = np.random.default_rng(6)
    scale = 2.0 ** 32
    grads = [(rng.standard_normal(n) * 3e7 * scale).astype(np.float32) for n in (100000, 4097)]
    assert np.isfinite(np.concatenate(grads)).all()
    ps = params_with_grads(T, grads)
    norm = T.clip_grad_norm_amp(ps, 1.0, scale)
    inv = np.float32(1.0) / np.float32(scale)
    g64 = np.concatenate([g * inv for g in grads]).astype(np.float64)
    ref = np.sqrt((g64 * g64).sum())
    assert np.isfinite(norm) and abs(norm - ref) <= 1e-5 * ref
    coef = np.float32(1.0) / (np.float32(norm) + np.float32(1e-6))
    for p, g in zip(ps, grads):
        assert np.array_equal(np.asarray(p.grad), g * coef)


def test_unscale_with_zero_scale_reports_overflow(T):
    """inv_scale = 1 / 0 = inf makes every product non-finite, zeros included
    (0 * inf = NaN): the reference reports an overflow as soon as any
    parameter has a gradient, even an all-zero one, and changes nothing."""
    z = tensor(T, np.zeros(16, np.float32), True)           # known-zero gradient
    opt = T.SGD([z], 0.1)
    scaler = T.GradScaler(1.0, 2.0, 0.5, 3)
    scaler.set_scale(0.0)
    assert not scaler.unscale(opt)
    assert not np.asarray(z.grad).any()


def test_check_gradients_finite_leaves_device_values(T):
    """The finite check is read-only: values are unchanged afterwards,
    including a huge finite value that any rescaling would disturb."""
    g = np.float32([3e38, -1.5, 0.0, 7.0] * 256)
    ps = params_with_grads(T, [g])
    assert T.check_gradients_finite(ps)
    assert np.array_equal(np.asarray(ps[0].grad), g)
