"""TEST INFRASTRUCTURE ONLY: a byte-level restatement of whitematter's file
formats (reference core/serialize.h:9-12, core/serialize.cpp:1-507), used by
tests/ to check the drop-in serializer's files byte for byte and to write
inputs for its loaders.  The product (whitematter_amd/) never imports it.

All integers are little-endian 4-byte words (the reference writes raw
uint32 / int / float values on x86); float payloads are raw fp32.

  WMT file   = u32 TENSOR_MAGIC, tensor body                    (:59-70)
  tensor body = u32 ndim, ndim x u32 dims, prod(dims) x f32     (:36-56)
  WMM file   = u32 MODEL_MAGIC, u32 count, count x tensor body  (:111-135)
  WMO file   = u32 OPTIM_MAGIC, optimizer block                 (:184-229)
  SGD block  = u32 1, f32 lr, f32 momentum, u32 n, n x (u32 size, size x f32)
  Adam block = u32 2, f32 lr, beta1, beta2, eps, i32 t, u32 n,
               n x (u32 size, size x f32) [m], n x (u32 size, size x f32) [v]
  checkpoint = u32 MODEL_MAGIC, u32 1, i32 epoch, f32 loss, f32 accuracy,
               u32 count, count x tensor body, u32 has_optimizer,
               [optimizer block]                                (:319-400)
"""
from __future__ import annotations

import struct
from typing import List, Optional, Sequence, Tuple

import numpy as np

TENSOR_MAGIC = 0x574D5400  # "WMT\0"
MODEL_MAGIC = 0x574D4D00   # "WMM\0"
OPTIM_MAGIC = 0x574D4F00   # "WMO\0"


def _u32(v: int) -> bytes:
    return struct.pack("<I", v & 0xFFFFFFFF)


def _i32(v: int) -> bytes:
    return struct.pack("<i", v)


def _f32(v: float) -> bytes:
    return struct.pack("<f", v)


def tensor_body(a: np.ndarray) -> bytes:
    a = np.asarray(a, np.float32, order="C")  # keeps 0-d arrays 0-d
    return _u32(a.ndim) + b"".join(_u32(d) for d in a.shape) + a.astype("<f4").tobytes()


def tensor_file(a: np.ndarray) -> bytes:
    return _u32(TENSOR_MAGIC) + tensor_body(a)


def model_file(params: Sequence[np.ndarray]) -> bytes:
    return _u32(MODEL_MAGIC) + _u32(len(params)) + b"".join(tensor_body(p) for p in params)


def _buffers(bufs: Sequence[np.ndarray]) -> bytes:
    return b"".join(_u32(b.size) + np.ascontiguousarray(b, "<f4").tobytes() for b in bufs)


def sgd_block(lr: float, momentum: float, velocity: Sequence[np.ndarray]) -> bytes:
    return _u32(1) + _f32(lr) + _f32(momentum) + _u32(len(velocity)) + _buffers(velocity)


def adam_block(lr, beta1, beta2, eps, t, m: Sequence[np.ndarray], v: Sequence[np.ndarray]) -> bytes:
    return (_u32(2) + _f32(lr) + _f32(beta1) + _f32(beta2) + _f32(eps) + _i32(t) + _u32(len(m)) + _buffers(m) +
            _buffers(v))


def optimizer_file(block: bytes) -> bytes:
    return _u32(OPTIM_MAGIC) + block


def checkpoint_file(epoch: int, loss: float, accuracy: float, params: Sequence[np.ndarray],
                    block: Optional[bytes]) -> bytes:
    head = _u32(MODEL_MAGIC) + _u32(1) + _i32(epoch) + _f32(loss) + _f32(accuracy)
    body = _u32(len(params)) + b"".join(tensor_body(p) for p in params)
    return head + body + (_u32(1) + block if block is not None else _u32(0))


class Reader:
    """Sequential reader over a byte string, failing like the reference's
    ifstream reads: a short read raises EOFError."""

    def __init__(self, data: bytes):
        self.d, self.o = data, 0

    def take(self, n: int) -> bytes:
        if self.o + n > len(self.d):
            raise EOFError(f"need {n} bytes at {self.o}, have {len(self.d) - self.o}")
        b = self.d[self.o:self.o + n]
        self.o += n
        return b

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def i32(self) -> int:
        return struct.unpack("<i", self.take(4))[0]

    def f32(self) -> float:
        return struct.unpack("<f", self.take(4))[0]

    def floats(self, n: int) -> np.ndarray:
        return np.frombuffer(self.take(4 * n), "<f4").astype(np.float32)

    def tensor(self) -> np.ndarray:
        nd = self.u32()
        shape = tuple(self.u32() for _ in range(nd))
        return self.floats(int(np.prod(shape, dtype=np.int64))).reshape(shape)


def read_tensor_file(data: bytes) -> np.ndarray:
    r = Reader(data)
    if r.u32() != TENSOR_MAGIC:
        raise ValueError("Invalid tensor file format")
    return r.tensor()


def read_model_file(data: bytes) -> List[np.ndarray]:
    r = Reader(data)
    if r.u32() != MODEL_MAGIC:
        raise ValueError("Invalid model file format")
    return [r.tensor() for _ in range(r.u32())]


def read_optimizer_block(r: Reader) -> Tuple[str, dict]:
    kind = r.u32()
    if kind == 1:
        lr, mom, n = r.f32(), r.f32(), r.u32()
        return "sgd", {"lr": lr, "momentum": mom, "velocity": [r.floats(r.u32()) for _ in range(n)]}
    if kind == 2:
        lr, b1, b2, eps, t, n = r.f32(), r.f32(), r.f32(), r.f32(), r.i32(), r.u32()
        m = [r.floats(r.u32()) for _ in range(n)]
        v = [r.floats(r.u32()) for _ in range(n)]
        return "adam", {"lr": lr, "beta1": b1, "beta2": b2, "eps": eps, "t": t, "m": m, "v": v}
    raise ValueError(f"Unknown optimizer type in file: {kind}")
