"""Writes tests/golden/ref_vectors.npz: small input/output vectors produced by
the reference's own core/tensor.cpp (compiled by oracle/Makefile into
oracle/_ref/libwmref.so with the reference's Makefile flags).

Run in the build container, where the reference sources are present:
    make -C oracle && python tests/golden/make_golden.py
The vectors are data (inputs, outputs, gradients); tests/test_oracle.py and
the GPU tests compare against them.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from whitematter_amd import synth  # noqa: E402


def main():
    ref = oracle.reference()
    if ref is None:
        raise SystemExit("oracle/_ref/libwmref.so is not built")
    out = {}
    n = 0

    def seeded(shape, seed, lo=None, hi=None):
        if lo is None:
            return synth.normal(shape, 0x60D0000 + seed)
        return synth.uniform(shape, 0x60D0000 + seed, lo, hi)

    # binary ops, fwd + bwd (config-like layouts at small sizes)
    layouts = [((16, 32), (32,)), ((16, 32), (1, 32)), ((16, 32), (16, 1)), ((16, 32), (16, 32)),
               ((2, 3, 8), (3, 1)), ((5,), (1,))]
    for op in ("add", "sub", "mul", "div", "pow", "max", "min"):
        for sa, sb in layouts:
            a = seeded(sa, n)
            b = seeded(sb, n + 1, 0.5, 2.0) if op in ("div", "pow") else seeded(sb, n + 1)
            if op == "pow":
                a = np.abs(a) + np.float32(0.25)
            if op in ("max", "min"):
                a, b = (np.rint(a * 2) / 2).astype(np.float32), (np.rint(b * 2) / 2).astype(np.float32)
            ta, tb = ref.tensor(a, True), ref.tensor(b, True)
            ty = ref.binary(op, ta, tb)
            g = seeded(ty.shape, n + 2)
            ty.run_grad_fn(g)
            key = f"b{n:03d}"
            out.update({key + "/kind": "binary", key + "/op": op, key + "/a": a, key + "/b": b, key + "/y": ty.data(),
                        key + "/g": g, key + "/ga": ta.grad(), key + "/gb": tb.grad()})
            n += 3
    # reductions through the reference API (quantised inputs: ties)
    x = synth.quantize(seeded((24, 40), 900))
    for op in ("sum", "mean", "max", "min", "argmax", "argmin"):
        for dim in (-1, 0, 1):
            tx = ref.tensor(x, False)
            ty = ref.reduce(op, tx, dim, False)
            if op in ("argmax", "argmin"):
                d = dim if dim >= 0 else 1
                view = (1, 24, 40) if d == 0 else (24, 40, 1)
            else:
                view = (1, x.size, 1) if dim == -1 else ((1, 24, 40) if dim == 0 else (24, 40, 1))
            key = f"r{op}{dim + 1}"
            out.update({key + "/kind": "reduce", key + "/op": op, key + "/x": x, key + "/view": np.array(view),
                        key + "/y": ty.data()})
    # softmax / log_softmax with spikes, fwd + bwd
    for log in (False, True):
        xs = synth.spikes(seeded((6, 64), 950) * np.float32(3.0), 950, 0.05)
        tx = ref.tensor(xs, True)
        ty = ref.softmax(tx, log)
        g = seeded(xs.shape, 951)
        ty.run_grad_fn(g)
        key = f"s{int(log)}"
        out.update({key + "/kind": "softmax", key + "/log": np.array(log), key + "/x": xs, key + "/y": ty.data(),
                    key + "/g": g, key + "/gx": tx.grad()})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_vectors.npz")
    np.savez_compressed(path, **{k: np.asarray(v) for k, v in out.items()})
    print(f"wrote {path}: {len(out)} arrays")


if __name__ == "__main__":
    main()
