"""CPU tests that pin the byte-level restatement of whitematter's file
formats (oracle/wmt.py) against the reference's own serializer
(core/serialize.cpp, compiled into oracle/_ref):

1. every writer -- save_tensor, save_model, save_optimizer (SGD, Adam),
   save_checkpoint (with and without optimizer state) -- produces exactly
   the restatement's bytes, for ragged shapes including 0-d and empty
   tensors and state after real optimizer steps;
2. the reference loads the restatement's files to the same values, and the
   restatement parses the reference's;
3. the reference's failure rules the drop-in must keep: bad magic, a
   truncated payload, a parameter count or shape mismatch, an optimizer of
   the other kind.
"""
import os

import numpy as np
import pytest

import oracle
from oracle import wmt

try:
    R = oracle.Reference()
except FileNotFoundError:
    R = None
pytestmark = pytest.mark.skipif(R is None, reason="oracle/_ref not built (reference sources absent)")

SHAPES = [(3,), (2, 3), (1, 1, 1), (4, 0, 2), (5, 7, 3), ()]


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


def read(path):
    with open(path, "rb") as f:
        return f.read()


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_tensor_file_bytes_and_round_trip(tmp_path, shape):
    a = rnd(shape, 1) if shape != () else np.float32([2.5]).reshape(())
    p = str(tmp_path / "t.wmt")
    t = R.tensor(a.reshape(-1) if a.ndim else a.reshape(1), shape=shape)
    assert R.save_tensor(t, p)
    assert read(p) == wmt.tensor_file(a)
    assert np.array_equal(wmt.read_tensor_file(read(p)), a)
    q = str(tmp_path / "u.wmt")
    with open(q, "wb") as f:
        f.write(wmt.tensor_file(a))
    back = R.load_tensor(q)
    assert back is not None and back.shape == tuple(shape)
    assert np.array_equal(back.data().reshape(shape), a)
    assert back.requires_grad()  # load_tensor creates with requires_grad = true (:96)


def test_tensor_file_failures(tmp_path):
    a = rnd((4, 5), 2)
    good = wmt.tensor_file(a)
    cases = {"magic": b"XXXX" + good[4:], "truncated": good[:-3], "header_only": good[:12], "empty": b""}
    for name, data in cases.items():
        p = str(tmp_path / (name + ".wmt"))
        with open(p, "wb") as f:
            f.write(data)
        assert R.load_tensor(p) is None, name
    assert R.load_tensor(str(tmp_path / "missing.wmt")) is None


def linear(seed):
    m = R.module("linear", [6, 4])
    for i, prm in enumerate(m.params()):
        prm.set_data(rnd(prm.shape, seed + i))
    return m


def test_model_file_bytes_and_load(tmp_path):
    m = linear(3)
    params = [p.data() for p in m.params()]
    p = str(tmp_path / "m.wmm")
    assert R.save_model(m, p)
    assert read(p) == wmt.model_file(params)
    # load into a fresh module: values replaced
    m2 = linear(10)
    assert R.load_model(m2, p)
    for a, b in zip(m2.params(), params):
        assert np.array_equal(a.data(), b)
    # count and shape mismatches refuse the file
    other = R.module("linear", [6, 5])
    assert not R.load_model(other, p)
    q = str(tmp_path / "short.wmm")
    with open(q, "wb") as f:
        f.write(wmt.model_file(params[:1]))
    assert not R.load_model(m2, q)


def stepped_optimizer(kind, seed):
    m = linear(seed)
    params = m.params()
    opt = R.optimizer(kind, params, 0.01, 0.9, 0.999, 1e-8) if kind == "adam" else R.optimizer(kind, params, 0.05,
                                                                                                  0.9)
    for s in range(2):
        for i, prm in enumerate(params):
            prm.set_grad(rnd(prm.shape, 100 * seed + 10 * s + i))
        opt.step()
    return m, opt


@pytest.mark.parametrize("kind", ["sgd", "adam"])
def test_optimizer_and_checkpoint_files(tmp_path, kind):
    m, opt = stepped_optimizer(kind, 4)
    p = str(tmp_path / "o.wmo")
    assert R.save_optimizer(opt, p)
    data = read(p)
    r = wmt.Reader(data)
    assert r.u32() == wmt.OPTIM_MAGIC
    name, st = wmt.read_optimizer_block(r)
    assert name == kind and r.o == len(data)
    if kind == "sgd":
        block = wmt.sgd_block(st["lr"], st["momentum"], st["velocity"])
        assert np.float32(st["lr"]) == np.float32(0.05) and np.float32(st["momentum"]) == np.float32(0.9)
        assert any(np.any(v) for v in st["velocity"])
    else:
        block = wmt.adam_block(st["lr"], st["beta1"], st["beta2"], st["eps"], st["t"], st["m"], st["v"])
        assert st["t"] == 2 and any(np.any(v) for v in st["v"])
    assert data == wmt.optimizer_file(block)
    # a fresh optimizer of the same kind takes the state; the other kind refuses
    m2, opt2 = stepped_optimizer(kind, 5)
    assert R.load_optimizer(opt2, p)
    q = str(tmp_path / "o2.wmo")
    assert R.save_optimizer(opt2, q) and read(q) == data
    _, wrong = stepped_optimizer("adam" if kind == "sgd" else "sgd", 6)
    assert not R.load_optimizer(wrong, p)
    # checkpoint: header, parameters, optimizer block
    c = str(tmp_path / "c.ckpt")
    assert R.save_checkpoint(c, m, opt, 7, 0.25, 0.75)
    params = [x.data() for x in m.params()]
    assert read(c) == wmt.checkpoint_file(7, 0.25, 0.75, params, block)
    ok, epoch, loss, acc = R.load_checkpoint(c, m2, opt2)
    assert ok and epoch == 7 and loss == np.float32(0.25) and acc == np.float32(0.75)
    for a, b in zip(m2.params(), params):
        assert np.array_equal(a.data(), b)
    # without optimizer state
    d = str(tmp_path / "d.ckpt")
    assert R.save_checkpoint(d, m, None, 1)
    assert read(d) == wmt.checkpoint_file(1, 0.0, 0.0, params, None)
    # a checkpoint of the other optimizer kind loads its parameters and skips the state
    ok, *_ = R.load_checkpoint(c, m2, wrong)
    assert ok
