"""GPU parity of the drop-in serializer (whitematter_amd/core/serialize.h,
payloads through include/wm_io.h straight between the file and HBM) against
the byte-level restatement of the reference's formats (oracle/wmt.py,
pinned against the reference's own writer in test_oracle_wmt.py) and, where
oracle/_ref is built, against files the reference itself wrote.

Bar: bit-exact -- every file the drop-in writes is byte-identical to the
restatement's (and the reference's), every file it loads reproduces the
values bit for bit, and the reference's failure rules hold.
"""
import os

import numpy as np
import pytest

import oracle
from gpu_helpers import rng_normal
from oracle import wmt

pytestmark = pytest.mark.gpu

try:
    R = oracle.Reference()
except FileNotFoundError:
    R = None


def T():
    from whitematter_amd import _tensor
    return _tensor


def read(path):
    with open(path, "rb") as f:
        return f.read()


def write(path, data):
    with open(path, "wb") as f:
        f.write(data)


# shapes spanning 0-d, empty, ragged, and payloads of several 8 MiB staging chunks
SHAPES = [(3,), (2, 3), (1, 1, 1), (4, 0, 2), (5, 7, 3), (), (2097152,), (5000003,), (3, 1024, 1025)]


def sample(shape, seed):
    if shape == ():
        return np.float32(-1.75).reshape(())
    return rng_normal(shape, seed)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_save_tensor_bytes(wm, tmp_path, shape):
    t = T()
    a = sample(shape, 1)
    x = t.Tensor.from_array(a.reshape(-1), shape=list(shape), requires_grad=True)
    p = str(tmp_path / "t.wmt")
    assert t.save_tensor(x, p)
    assert read(p) == wmt.tensor_file(a)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_load_tensor_values(wm, tmp_path, shape):
    t = T()
    a = sample(shape, 2)
    p = str(tmp_path / "t.wmt")
    write(p, wmt.tensor_file(a))
    x = t.load_tensor(p)
    assert x is not None and list(x.shape) == list(shape) and x.requires_grad
    assert np.array_equal(np.asarray(x.data).reshape(shape), a)
    # the loaded tensor is device-resident: a kernel reads it directly
    y = x * 2.0
    assert np.array_equal(np.asarray(y.data).reshape(shape), a * np.float32(2))


def test_load_tensor_failures(wm, tmp_path):
    t = T()
    good = wmt.tensor_file(rng_normal((1000, 5000), 3))  # 20 MB: three staging chunks
    assert len(good) > (8 << 20) + 100
    for name, data in {"magic": b"WMT?" + good[4:], "truncated_one_chunk": good[:-1],
                       "truncated_mid_chunk": good[:(8 << 20) + 100], "header_only": good[:12], "empty": b""}.items():
        p = str(tmp_path / (name + ".wmt"))
        write(p, data)
        assert t.load_tensor(p) is None, name
    assert t.load_tensor(str(tmp_path / "missing.wmt")) is None
    assert not t.save_tensor(t.Tensor.from_array(np.ones(3, np.float32)), str(tmp_path / "no_dir" / "x.wmt"))


@pytest.mark.skipif(R is None, reason="oracle/_ref not built")
def test_reference_files_load_and_rewrite_identically(wm, tmp_path):
    t = T()
    for i, shape in enumerate([(7,), (33, 65), (2, 3, 4), (4, 0, 2)]):
        a = rng_normal(shape, 10 + i)
        p = str(tmp_path / f"r{i}.wmt")
        assert R.save_tensor(R.tensor(a.reshape(-1), shape=shape), p)
        x = t.load_tensor(p)
        assert np.array_equal(np.asarray(x.data).reshape(shape), a)
        q = str(tmp_path / f"w{i}.wmt")
        assert t.save_tensor(x, q)
        assert read(q) == read(p)


def mha(t, E, H, seed):
    m = t.MultiHeadAttention(E, H)
    for j, name in enumerate(("W_q", "W_k", "W_v", "W_o", "b_q", "b_k", "b_v", "b_o")):
        shape = (E, E) if name[0] == "W" else (E,)
        setattr(m, name, t.Tensor.from_array(rng_normal(shape, seed + j), requires_grad=True))
    return m


def params_of(m):
    return [np.asarray(p.data).reshape(p.shape) for p in m.parameters()]


def test_model_files(wm, tmp_path):
    t = T()
    m = mha(t, 64, 4, 20)
    p = str(tmp_path / "m.wmm")
    assert t.save_model(m, p)
    assert read(p) == wmt.model_file(params_of(m))
    m2 = mha(t, 64, 4, 40)
    assert t.load_model(m2, p)
    for a, b in zip(params_of(m2), params_of(m)):
        assert np.array_equal(a, b)
    # mismatches are refused (count, shape), files written elsewhere load
    assert not t.load_model(t.Linear(64, 64), p)
    assert not t.load_model(mha(t, 32, 4, 60), p)
    q = str(tmp_path / "lin.wmm")
    lin_params = [rng_normal((5, 3), 70), rng_normal((3,), 71)]
    write(q, wmt.model_file(lin_params))
    lin = t.Linear(5, 3)
    assert t.load_model(lin, q)
    assert np.array_equal(np.asarray(lin.weight.data).reshape(5, 3), lin_params[0])
    assert np.array_equal(np.asarray(lin.bias.data).reshape(3), lin_params[1])


def stepped(t, kind, seed, shapes=((64, 32), (32,), (1000, 7))):
    ps = [t.Tensor.from_array(rng_normal(s, seed + i), requires_grad=True) for i, s in enumerate(shapes)]
    opt = t.SGD(ps, 0.05, 0.9) if kind == "sgd" else t.Adam(ps, 0.01)
    for s in range(2):
        for i, p in enumerate(ps):
            p.grad = rng_normal(p.shape, 100 * seed + 10 * s + i)
        opt.step()
    return ps, opt


class Holder:
    """A stand-in module for save_checkpoint: the parameters of a list."""


@pytest.mark.parametrize("kind", ["sgd", "adam"])
def test_optimizer_files_round_trip(wm, tmp_path, kind):
    t = T()
    ps, opt = stepped(t, kind, 1)
    p = str(tmp_path / "o.wmo")
    assert t.save_optimizer(opt, p)
    data = read(p)
    r = wmt.Reader(data)
    assert r.u32() == wmt.OPTIM_MAGIC
    name, st = wmt.read_optimizer_block(r)
    assert name == kind and r.o == len(data)
    bufs = st["velocity"] if kind == "sgd" else st["m"]
    for i in range(len(ps)):
        state = opt.state(i)
        assert np.array_equal(bufs[i], state[0].reshape(-1))
        if kind == "adam":
            assert np.array_equal(st["v"][i], state[1].reshape(-1)) and st["t"] == opt.t == 2
    # a fresh optimizer takes the state and writes the same bytes back
    ps2, opt2 = stepped(t, kind, 5)
    assert t.load_optimizer(opt2, p)
    q = str(tmp_path / "o2.wmo")
    assert t.save_optimizer(opt2, q) and read(q) == data
    # the other kind refuses, a wrong buffer count refuses
    _, wrong = stepped(t, "adam" if kind == "sgd" else "sgd", 6)
    assert not t.load_optimizer(wrong, p)
    _, fewer = stepped(t, kind, 7, shapes=((64, 32),))
    assert not t.load_optimizer(fewer, p)


@pytest.mark.skipif(R is None, reason="oracle/_ref not built")
@pytest.mark.parametrize("kind", ["sgd", "adam"])
def test_reference_optimizer_and_checkpoint_files_round_trip(wm, tmp_path, kind):
    """Files the reference wrote (its Linear + optimizer after two steps) load
    into the drop-in's Linear + optimizer, which then writes identical bytes."""
    t = T()
    m = R.module("linear", [6, 4])
    params = m.params()
    opt = R.optimizer(kind, params, 0.01, 0.9, 0.999, 1e-8) if kind == "adam" else R.optimizer(kind, params, 0.05, 0.9)
    for s in range(2):
        for i, prm in enumerate(params):
            prm.set_grad(rng_normal(prm.shape, 30 + 10 * s + i))
        opt.step()
    po, pc = str(tmp_path / "ref.wmo"), str(tmp_path / "ref.ckpt")
    assert R.save_optimizer(opt, po) and R.save_checkpoint(pc, m, opt, 3, 0.5, 0.25)
    lin = t.Linear(6, 4)
    dopt = t.SGD(lin.parameters(), 0.1, 0.5) if kind == "sgd" else t.Adam(lin.parameters(), 0.1)
    assert t.load_optimizer(dopt, po)
    qo = str(tmp_path / "drop.wmo")
    assert t.save_optimizer(dopt, qo) and read(qo) == read(po)
    ok, epoch, loss, acc = t.load_checkpoint(pc, lin, dopt)
    assert ok and (epoch, loss, acc) == (3, np.float32(0.5), np.float32(0.25))
    qc = str(tmp_path / "drop.ckpt")
    assert t.save_checkpoint(qc, lin, dopt, epoch, loss, acc) and read(qc) == read(pc)


def test_checkpoint_without_optimizer_and_mismatch(wm, tmp_path):
    t = T()
    m = mha(t, 16, 2, 80)
    p = str(tmp_path / "c.ckpt")
    assert t.save_checkpoint(p, m, None, 9, 1.5, 0.5)
    assert read(p) == wmt.checkpoint_file(9, 1.5, 0.5, params_of(m), None)
    m2 = mha(t, 16, 2, 90)
    ok, epoch, loss, acc = t.load_checkpoint(p, m2, None)
    assert ok and epoch == 9 and loss == 1.5 and acc == 0.5
    for a, b in zip(params_of(m2), params_of(m)):
        assert np.array_equal(a, b)
    bad = str(tmp_path / "bad.ckpt")
    data = bytearray(read(p))
    data[4] = 2  # version 2
    write(bad, bytes(data))
    assert not t.load_checkpoint(bad, m2, None)[0]


def test_checkpoint_state_rules_and_messages(wm, tmp_path, capfd):
    """Checkpoints take optimizer state as it comes (core/serialize.cpp:
    459-500): state of the other kind is skipped with a warning and the load
    succeeds, an unknown kind tag is ignored, and a short state buffer list
    is not compared.  WMO files refuse the same cases (:255-312) with the
    reference's messages."""
    t = T()
    lin = t.Linear(6, 4)
    params = [np.asarray(p.data).reshape(p.shape) for p in lin.parameters()]
    vel = [rng_normal(p.shape, 200 + i).reshape(-1) for i, p in enumerate(params)]
    sgd = wmt.sgd_block(0.25, 0.5, vel)
    adam = wmt.adam_block(0.01, 0.9, 0.999, 1e-8, 3, vel, vel)
    capfd.readouterr()
    # Adam state into an SGD optimizer: skipped with a warning, load succeeds
    p = str(tmp_path / "a.ckpt")
    write(p, wmt.checkpoint_file(4, 0.75, 0.5, params, adam))
    opt = t.SGD(lin.parameters(), 0.1, 0.9)
    ok, epoch, loss, acc = t.load_checkpoint(p, lin, opt)
    err = capfd.readouterr().err
    assert ok and epoch == 4 and "Warning: Checkpoint has Adam state but optimizer is not Adam, skipping" in err
    assert opt.lr == np.float32(0.1)
    # an unknown kind tag is ignored
    write(p, wmt.checkpoint_file(4, 0.75, 0.5, params, struct_u32(7)))
    assert t.load_checkpoint(p, lin, opt)[0]
    # the checkpoint reads each buffer's own size whatever count the file states
    bad_count = bytearray(sgd)
    bad_count[12] = 9  # the velocity count word
    write(p, wmt.checkpoint_file(4, 0.75, 0.5, params, bytes(bad_count)))
    assert t.load_checkpoint(p, lin, opt)[0]
    assert opt.lr == np.float32(0.25) and opt.momentum == np.float32(0.5)
    for i in range(len(params)):
        assert np.array_equal(opt.state(i)[0].reshape(-1), vel[i])
    # the same block in a WMO file is refused on the count, with its message
    q = str(tmp_path / "o.wmo")
    capfd.readouterr()
    write(q, wmt.optimizer_file(bytes(bad_count)))
    assert not t.load_optimizer(opt, q)
    assert "Error: Velocity buffer count mismatch" in capfd.readouterr().err
    write(q, wmt.optimizer_file(adam))
    assert not t.load_optimizer(opt, q)
    assert "Error: File contains Adam state but optimizer is not Adam" in capfd.readouterr().err
    write(q, wmt.optimizer_file(struct_u32(7)))
    assert not t.load_optimizer(opt, q)
    assert "Error: Unknown optimizer type in file: 7" in capfd.readouterr().err
    # a size mismatch in the WMO file refuses too
    short = [v[:-1] for v in vel]
    write(q, wmt.optimizer_file(wmt.sgd_block(0.25, 0.5, short)))
    assert not t.load_optimizer(opt, q)
    assert "Error: Velocity buffer size mismatch" in capfd.readouterr().err


def struct_u32(v):
    import struct
    return struct.pack("<I", v)
