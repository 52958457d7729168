"""Seeded synthetic inputs for the parity tests and the bench.

One host generator feeds the GPU path, the CPU oracle and the reference CPU
baseline, so all of them see byte-identical fp32 inputs:

  splitmix64 counter stream (state_i = seed + (i+1) * 0x9E3779B97F4A7C15)
  -> uniform doubles -> Box-Muller (cos branch) in fp64 -> fp32.

Seeds are ``0x5EED0000 + 16 * config + tensor_id``.  Uniform U[a,b] uses the
top 24 bits; quantisation rounds half-to-even; spikes come from an
independent Bernoulli stream.  Work is chunked so multi-GiB tensors do not
need multi-GiB temporaries.
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def seed_for(config: int, tensor_id: int) -> int:
    return 0x5EED0000 + 16 * int(config) + int(tensor_id)


def _splitmix(seed: int, start: int, count: int) -> np.ndarray:
    i = np.arange(start + 1, start + 1 + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _u53(z: np.ndarray) -> np.ndarray:
    """(0, 1] doubles from the top 53 bits."""
    return ((z >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)


def _chunks(n: int, fill) -> None:
    """Run fill(start, count) over n elements in _CHUNK pieces.  The
    generator is a counter stream, so the pieces are independent; large
    tensors spread them over threads (numpy releases the GIL in these
    element-wise passes), and the bytes do not depend on the thread count."""
    starts = range(0, n, _CHUNK)
    workers = min(len(starts), 16, os.cpu_count() or 1)
    if workers <= 1:
        for s in starts:
            fill(s, min(_CHUNK, n - s))
        return
    with ThreadPoolExecutor(workers) as ex:
        list(ex.map(lambda s: fill(s, min(_CHUNK, n - s)), starts))


def normal(shape, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, np.float32)

    def fill(s, c):
        z = _splitmix(seed, 2 * s, 2 * c)
        u1, u2 = _u53(z[0::2]), _u53(z[1::2])
        v = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        out[s:s + c] = (mean + std * v).astype(np.float32)

    _chunks(n, fill)
    return out.reshape(shape)


def uniform(shape, seed: int, lo: float, hi: float) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, np.float32)

    def fill(s, c):
        u24 = (_splitmix(seed, s, c) >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)
        out[s:s + c] = (lo + (hi - lo) * u24).astype(np.float32)

    _chunks(n, fill)
    return out.reshape(shape)


def quantize(x: np.ndarray, step_inv: float = 64.0) -> np.ndarray:
    """Round to multiples of 1/step_inv (half to even)."""
    return (np.rint(x.astype(np.float64) * step_inv) / step_inv).astype(np.float32)


def spikes(x: np.ndarray, seed: int, p: float = 0.01, value: float = 20.0) -> np.ndarray:
    """Set an independent Bernoulli(p) subset of x to +value."""
    flat = x.reshape(-1).copy()

    def fill(s, c):
        u = (_splitmix(seed ^ 0x5B1CE, s, c) >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)
        flat[s:s + c][u < p] = np.float32(value)

    _chunks(flat.size, fill)
    return flat.reshape(x.shape)


# ---- the five BASELINE configurations ---------------------------------------

def config1(scale: int = 1):
    """c1: a[1024,1024] ~N(0,1), b[1024] ~N(0,1)."""
    r = 1024 // scale
    a = normal((r, 1024), seed_for(1, 0))
    b = normal((1024,), seed_for(1, 1))
    return a, b


def config2(rows: int = 8192, cols: int = 8192):
    """c2: A ~N(0,1); c[rows,1], r[1,cols] ~U[0.5,2]; upstream G ~N(0,1)."""
    A = normal((rows, cols), seed_for(2, 0))
    c = uniform((rows, 1), seed_for(2, 1), 0.5, 2.0)
    r = uniform((1, cols), seed_for(2, 2), 0.5, 2.0)
    G = normal((rows, cols), seed_for(2, 3))
    return A, c, r, G


def config3(rows: int = 16384, cols: int = 4096):
    """c3: X ~N(0,1) quantised to multiples of 1/64; upstream g ~N(0,1)."""
    X = quantize(normal((rows, cols), seed_for(3, 0)))
    return X


def config4(rows: int = 8192, cols: int = 32000):
    """c4: logits ~N(0,3) with 1% +20 spikes; upstream G ~N(0,1)."""
    L = spikes(normal((rows, cols), seed_for(4, 0), 0.0, 3.0), seed_for(4, 1))
    G = normal((rows, cols), seed_for(4, 2))
    return L, G


def config5(b: int = 32, t: int = 1024, c: int = 4096):
    """c5: h, residual ~N(0,1) (fp32, to be stored as fp16), g[c] ~U[0.8,1.2],
    upstream dm[b,t,1] ~N(0,1)."""
    h = normal((b, t, c), seed_for(5, 0))
    res = normal((b, t, c), seed_for(5, 1))
    g = uniform((c,), seed_for(5, 2), 0.8, 1.2)
    dm = normal((b, t, 1), seed_for(5, 3))
    return h, res, g, dm
