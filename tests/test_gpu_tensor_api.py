"""GPU tests of the drop-in C++ Tensor (whitematter_amd/core, through the
whitematter_amd._tensor module): the reference's known-answer tests, the
config-1 chain end to end, and the reference behaviours a drop-in must keep
(full-reduction shapes, unscaled mean gradient, first-index ties, reshape's
gradient copy, accumulation, no-grad mode, host/device coherence)."""
import numpy as np
import pytest

import oracle
from kat_runner import KATS, TensorEngine, check_forward, check_grads
from whitematter_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def T(wm):
    from whitematter_amd import _tensor
    return _tensor.Tensor


@pytest.fixture(scope="module")
def eng(wm):
    return TensorEngine()


def tensor(T, a, rg=False):
    a = np.ascontiguousarray(a, np.float32)
    return T.from_array(a, list(a.shape), rg)


@pytest.mark.parametrize("case", KATS["forward"], ids=lambda c: c["id"])
def test_forward_kats(eng, case):
    err = check_forward(case, eng.forward(case))
    assert err is None, err


@pytest.mark.parametrize("case", KATS["autograd"], ids=lambda c: c["id"])
def test_autograd_kats(eng, case):
    err = check_grads(case, eng.autograd(case))
    assert err is None, err


def test_config1_chain(T):
    """y = relu(a + b).sum(1).sum(); y.backward() on a[1024,1024], b[1024]."""
    a_np, b_np = synth.config1()
    a, b = tensor(T, a_np, True), tensor(T, b_np, True)
    t = a.add(b)
    r = t.relu()
    s1 = r.sum(1)
    y = s1.sum()
    assert list(s1.shape) == [1024] and list(y.shape) == [1]
    y.backward()
    o32, o64, oab = oracle.get("f32"), oracle.get("f64"), oracle.get("abs")
    t_ref = o32.binary("add", a_np, b_np)
    assert oracle.bit_equal(t.data, t_ref)
    r_ref = o32.unary("relu", t_ref)
    assert oracle.bit_equal(r.data, r_ref)
    s_ref, _ = o64.reduce("sum", r_ref, 1024, 1024, 1)
    s_abs, _ = oab.reduce("sum", r_ref, 1024, 1024, 1)
    assert oracle.close_scaled(s1.data, s_ref.ravel(), s_abs.ravel(), 1e-5)[0]
    assert abs(float(y.data[0]) - s_ref.sum()) <= 1e-5 * s_abs.sum()
    mask = (r_ref > 0).astype(np.float32)
    assert np.array_equal(a.grad, mask)
    assert np.array_equal(b.grad.astype(np.float64), mask.astype(np.float64).sum(axis=0))
    # the graph is released after backward, as in the reference
    assert not y.has_grad_fn and y.num_parents == 0


def test_reduction_shapes(T):
    x = tensor(T, synth.normal((4, 6), 1), True)
    assert list(x.sum().shape) == [1]
    assert list(x.sum(-1, True).shape) == [1]          # keepdim ignored for the full sum
    assert list(x.mean(-1, True).shape) == [1]
    assert list(x.sum(0, True).shape) == [1, 6]
    assert list(x.sum(1).shape) == [4]
    assert list(x.sum(5).shape) == [4]                 # any dim other than 0 reduces columns
    assert list(x.max(-1, True).shape) == [1, 1]       # max/min keep the rank
    assert list(x.max(-1).shape) == [1]
    assert list(x.min(0, True).shape) == [1, 6]
    assert list(x.argmax(-1).shape) == [4]             # -1 is the last axis for arg*
    assert list(x.argmax(0, True).shape) == [1, 6]
    y = tensor(T, synth.normal((2, 3, 5), 2))
    assert list(y.argmin(1).shape) == [2, 5]
    assert list(tensor(T, np.ones(7, np.float32)).argmax(0).shape) == [1]


def test_mean_backward_is_unscaled(T):
    x = tensor(T, synth.normal((3, 4), 3), True)
    x.mean().backward()
    assert np.array_equal(x.grad, np.ones((3, 4), np.float32))
    x2 = tensor(T, synth.normal((3, 4), 3), True)
    x2.mean(0).sum().backward()
    assert np.array_equal(x2.grad, np.ones((3, 4), np.float32))


def test_softmax_ignores_dim(T):
    x = tensor(T, synth.normal((3, 7), 4))
    assert np.array_equal(x.softmax(0).data, x.softmax(-1).data)
    assert np.array_equal(x.log_softmax(0).data, x.log_softmax(1).data)


def test_argmax_ties_and_values(T):
    x = tensor(T, np.array([[1, 3, 3], [2, 2, 1]], np.float32))
    assert x.argmax(1).data.tolist() == [1.0, 0.0]
    assert x.argmin(1).data.tolist() == [0.0, 2.0]
    assert x.argmax(0).data.tolist() == [1.0, 0.0, 0.0]


def test_max_backward_routes_to_first_winner(T):
    x = tensor(T, np.array([[1, 5, 5], [7, 2, 7]], np.float32), True)
    x.max(1).sum().backward()
    assert x.grad.tolist() == [[0, 1, 0], [1, 0, 0]]
    z = tensor(T, np.array([[1, 5, 5], [7, 2, 7]], np.float32), True)
    z.min(-1).backward()
    assert z.grad.tolist() == [[1, 0, 0], [0, 0, 0]]


def test_elementwise_max_routes_ties_to_self(T):
    a = tensor(T, np.array([1, 2, 3], np.float32), True)
    b = tensor(T, np.array([1, 3, 2], np.float32), True)
    a.maximum(b).sum().backward()
    assert a.grad.tolist() == [1, 0, 1] and b.grad.tolist() == [0, 1, 0]


def test_reshape_copies_grad(T):
    """reshape's result starts with a copy of the input's gradient, which its
    closure then adds back: a.grad = 2*g0 + 1 after r.sum().backward()."""
    a = tensor(T, synth.normal((2, 6), 5), True)
    g0 = synth.normal((2, 6), 6)
    a.grad = g0
    r = a.reshape([3, 4])
    assert np.array_equal(r.grad.ravel(), g0.ravel())
    r.sum().backward()
    assert np.allclose(a.grad, 2 * g0 + 1, atol=1e-6)


def test_accumulation_and_zero_grad(T):
    a = tensor(T, synth.normal((64, 64), 7), True)
    assert a.grad_known_zero
    a.mul(2.0).sum().backward()
    assert not a.grad_known_zero
    a.mul(3.0).sum().backward()
    assert np.array_equal(a.grad, np.full((64, 64), 5.0, np.float32))
    a.zero_grad()
    assert a.grad_known_zero and not a.grad.any()


def test_shared_operand_mul(T):
    x = synth.normal((8, 8), 8)
    a = tensor(T, x, True)
    a.mul(a).sum().backward()
    assert np.allclose(a.grad, 2 * x, rtol=1e-6)


def test_no_grad_mode(T):
    from whitematter_amd import _tensor
    a = tensor(T, synth.normal((4,), 9), True)
    _tensor.set_grad_enabled(False)
    try:
        b = a.mul(3.0)
        assert not b.has_grad_fn and not b.requires_grad
    finally:
        _tensor.set_grad_enabled(True)
    assert a.mul(3.0).has_grad_fn


def test_host_writes_reach_the_device(T):
    a = tensor(T, np.zeros((2, 3), np.float32))
    b = tensor(T, np.ones((3,), np.float32))
    assert np.array_equal(a.add(b).data, np.ones((2, 3)))
    a.data = np.full((2, 3), 4.0, np.float32)   # host-side rewrite after a device op
    assert np.array_equal(a.add(b).data, np.full((2, 3), 5.0))


def test_broadcast_ops_through_tensor(T):
    """c2 layouts at a reduced size through the Tensor API: forward bit-exact,
    broadcast gradients within tolerance."""
    A, c, r, G = synth.config2(256, 1024)
    o32, o64, oab = oracle.get("f32"), oracle.get("f64"), oracle.get("abs")
    for op, other in (("add", r), ("mul", c), ("div", r), ("sub", c)):
        tA, to = tensor(T, A, True), tensor(T, other, True)
        y = getattr(tA, op)(to)
        assert oracle.bit_equal(y.data, o32.binary(op, A, other)), op
        y.run_grad_fn(G)
        ga, gb = o64.binary_bwd(op, G, A, other)
        sa, sb = oab.binary_bwd(op, G, A, other)
        assert oracle.close_scaled(tA.grad, ga, sa, 1e-5)[0], op
        assert oracle.close_scaled(to.grad, gb, sb, 1e-5)[0], op


def test_matrix_ops_through_the_api(T):
    """matmul and transpose are in the build (matrix cores / a tiled copy);
    the ops still outside it throw "not part of" (checked by the reference's
    own suites in test_gpu_ref_suites.py)."""
    x = np.float32([[1, 2], [3, 4]])
    a = tensor(T, x)
    assert np.array_equal(np.asarray(a.matmul(a).data).reshape(2, 2), x @ x)
    assert np.array_equal(np.asarray(a.transpose().data).reshape(2, 2), x.T)
    with pytest.raises(ValueError):
        a.matmul(tensor(T, np.ones((3, 2), np.float32)))


def test_host_pointer_contract(tmp_path):
    """The drop-in's host-pointer contract, through the reference's class
    API in C++: a non-const data() / begin() pointer is valid until the next
    device operation on the vector."""
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    wm = os.path.join(root, "whitematter_amd")
    exe = str(tmp_path / "host_pointer_contract")
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(wm, "core"), "-I", os.path.join(root, "include"),
                    os.path.join(root, "tests", "cpp", "host_pointer_contract.cpp"), "-L", wm, "-lwm_tensor",
                    "-lwm_hip", "-Wl,-rpath," + wm, "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0 and "CONTRACT HOLDS" in r.stdout, r.stdout + r.stderr
