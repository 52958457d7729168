"""Runs the reference's known-answer tests (tests/golden/ref_kats.json)
against an engine: the CPU oracle (OracleEngine) or the C++ Tensor on the GPU
(TensorEngine, tests/test_gpu_tensor_api.py)."""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "ref_kats.json")))

UNARY_SCALAR = {"mul_scalar", "div_scalar", "neg"}


def check_forward(case, got):
    """Compare one forward KAT result (flat float array); returns an error
    string or None."""
    got = np.asarray(got, np.float64).ravel()
    tol = case.get("tol", 0.0)
    if "expect" in case:
        exp = np.asarray(case["expect"], np.float64)
        if got.shape != exp.shape or not np.all(np.abs(got - exp) <= tol):
            return f"{case['id']}: got {got.tolist()} expected {exp.tolist()}"
    if "expect_first" in case and not abs(got[0] - case["expect_first"]) <= tol:
        return f"{case['id']}: got {got[0]} expected {case['expect_first']}"
    if "expect_gt" in case and not np.all(got > np.asarray(case["expect_gt"])):
        return f"{case['id']}: {got.tolist()} not > {case['expect_gt']}"
    if "expect_lt" in case and not np.all(got < np.asarray(case["expect_lt"])):
        return f"{case['id']}: {got.tolist()} not < {case['expect_lt']}"
    if "expect_sum" in case and not abs(got.sum() - case["expect_sum"]) <= tol:
        return f"{case['id']}: sum {got.sum()}"
    if case.get("expect_increasing") and not np.all(np.diff(got) > 0):
        return f"{case['id']}: not increasing {got.tolist()}"
    return None


def check_grads(case, grads):
    tol = case["tol"]
    for name, exp in case.get("expect_grad", {}).items():
        g = np.asarray(grads[name], np.float64).ravel()
        if not np.all(np.abs(g - np.asarray(exp)) <= tol):
            return f"{case['id']}: grad {name} = {g.tolist()} expected {exp}"
    for name in case.get("expect_grad_all_equal_nonzero", []):
        g = np.asarray(grads[name], np.float64).ravel()
        if not (abs(g[0]) > 1e-6 and np.all(np.abs(g - g[0]) <= tol)):
            return f"{case['id']}: grad {name} = {g.tolist()} not equal/non-zero"
    return None


class TensorEngine:
    """The C++ Tensor through whitematter_amd._tensor."""

    def __init__(self):
        from whitematter_amd import _tensor
        self.T = _tensor.Tensor

    def tensor(self, data, shape, rg=False):
        return self.T.from_array(np.asarray(data, np.float32), list(shape), rg)

    def forward(self, case):
        k = case["kind"]
        if k == "binary":
            a, b = self.tensor(case["a"], case["a_shape"]), self.tensor(case["b"], case["b_shape"])
            return getattr(a, case["op"])(b).data
        if k == "unary":
            x = self.tensor(case["x"], case["shape"])
            return self.apply_unary(x, case["op"], case.get("p0", 0.0), case.get("p1", 0.0)).data
        if k == "softmax":
            return self.tensor(case["x"], case["shape"]).softmax(-1).data
        if k == "reduce":
            x = self.tensor(case["x"], case["shape"])
            y = getattr(x, case["op"])(case["dim"], case["keepdim"])
            assert list(y.shape) == case["expect_shape"], (case["id"], y.shape)
            return y.data
        raise ValueError(k)

    def apply_unary(self, x, op, p0=0.0, p1=0.0):
        if op == "mul_scalar":
            return x.mul(p0)
        if op == "div_scalar":
            return x.div(p0)
        if op == "neg":
            return x.neg()
        if op == "pows":
            return x.pow(p0)
        if op == "clamp":
            return x.clamp(p0, p1)
        return getattr(x, {"tanh": "tanh_", "exp": "exp_", "log": "log_"}.get(op, op))()

    def autograd(self, case):
        env = {n: self.tensor(d, s, True) for n, (d, s) in case["tensors"].items()}
        last = None
        for step in case["program"]:
            if step[0] == "!backward":
                env[step[1]].backward()
                continue
            if step[0] == "!zero_grad":
                env[step[1]].zero_grad()
                continue
            out, op, src = step[0], step[1], step[2]
            x = env[src]
            if op in ("add", "sub", "mul", "div"):
                env[out] = getattr(x, op)(env[step[3]])
            elif op in ("sum", "mean"):
                env[out] = getattr(x, op)()
            else:
                env[out] = self.apply_unary(x, op, *(step[3:] or [0.0]))
            last = out
        if not case.get("no_final_backward"):
            env[last].backward()
        return {n: env[n].grad for n in case["tensors"]}


class OracleEngine:
    """The CPU oracle, with a minimal tape autograd over its backward
    functions (forward in strict fp32, backward in fp64)."""

    def __init__(self):
        import oracle
        self.o32 = oracle.get("f32")
        self.o64 = oracle.get("f64")

    def unary(self, op, x, p0=0.0, p1=0.0):
        if op == "mul_scalar":
            return self.o32.unary("scale", x, p0), ("scale", p0)
        if op == "div_scalar":
            s = float(np.float32(1.0) / np.float32(p0))
            return self.o32.unary("scale", x, s), ("scale", s)
        if op == "neg":
            return self.o32.unary("scale", x, -1.0), ("scale", -1.0)
        return self.o32.unary(op, x, p0, p1), (op, p0, p1)

    def reduce_view(self, shape, dim):
        if dim == -1:
            return 1, int(np.prod(shape)), 1
        rows, cols = shape
        return (1, rows, cols) if dim == 0 else (rows, cols, 1)

    def forward(self, case):
        k = case["kind"]
        if k == "binary":
            a = np.asarray(case["a"], np.float32).reshape(case["a_shape"])
            b = np.asarray(case["b"], np.float32).reshape(case["b_shape"])
            return self.o32.binary(case["op"], a, b)
        if k == "unary":
            return self.unary(case["op"], np.asarray(case["x"], np.float32), case.get("p0", 0.0),
                              case.get("p1", 0.0))[0]
        if k == "softmax":
            return self.o32.softmax(np.asarray(case["x"], np.float32).reshape(case["shape"]))
        if k == "reduce":
            x = np.asarray(case["x"], np.float32)
            v, _ = self.o32.reduce(case["op"], x, *self.reduce_view(case["shape"], case["dim"]))
            return v
        raise ValueError(k)

    def autograd(self, case):
        vals = {n: np.asarray(d, np.float32).reshape(s) for n, (d, s) in case["tensors"].items()}
        grads = {n: np.zeros(v.shape, np.float64) for n, v in vals.items()}
        tape = []

        def backward(root):
            g = {root: np.ones(vals[root].shape, np.float64)}
            for out, op, srcs, extra in reversed(tape):
                if out not in g:
                    continue
                go = g[out].astype(np.float32)
                if op in ("add", "sub", "mul", "div"):
                    ga, gb = self.o64.binary_bwd(op, go, vals[srcs[0]], vals[srcs[1]], vals[out])
                    contrib = [(srcs[0], ga), (srcs[1], gb)]
                elif op in ("sum", "mean"):
                    x = vals[srcs[0]]
                    gx = self.o64.reduce_bwd("sum", go.reshape(1, 1), None, 1, x.size, 1).reshape(x.shape)
                    contrib = [(srcs[0], gx)]
                else:
                    x = vals[srcs[0]]
                    gx = self.o64.unary_bwd(extra[0], go, x, vals[out], *extra[1:])
                    contrib = [(srcs[0], gx)]
                for name, c in contrib:
                    if name in grads:
                        grads[name] += c
                    else:
                        g[name] = g.get(name, 0) + c
            tape.clear()

        last = None
        for step in case["program"]:
            if step[0] == "!backward":
                backward(step[1])
                continue
            if step[0] == "!zero_grad":
                grads[step[1]][...] = 0
                continue
            out, op, src = step[0], step[1], step[2]
            if op in ("add", "sub", "mul", "div"):
                vals[out] = self.o32.binary(op, vals[src], vals[step[3]])
                tape.append((out, op, (src, step[3]), None))
            elif op in ("sum", "mean"):
                v, _ = self.o32.reduce(op, vals[src], 1, vals[src].size, 1)
                vals[out] = v.reshape(1)
                tape.append((out, op, (src,), None))
            else:
                vals[out], extra = self.unary(op, vals[src], *(step[3:] or [0.0]))
                tape.append((out, op, (src,), extra))
            last = out
        if not case.get("no_final_backward"):
            backward(last)
        return grads
