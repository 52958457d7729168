"""The drop-in amp.h's host fp16 conversions (whitematter_amd/core/amp.h;
reference core/amp.h:15-90) against the oracle's restatement of the
reference's bit formulas (pinned bit for bit against the compiled reference
in test_oracle.py): every fp16 pattern back to fp32, and fp32 patterns
covering every exponent with random mantissas, signs and NaN payloads.
No GPU: these are host functions."""
import numpy as np
import pytest

import oracle


@pytest.fixture(scope="module")
def T():
    from whitematter_amd import _tensor
    return _tensor


def test_half_to_float_every_pattern(T):
    h = np.arange(1 << 16, dtype=np.uint16)
    assert oracle.bit_equal(T.from_half(h), oracle.get("f32").f16_to_f32(h))
    # the scalar form (quiet NaNs only: a Python float quiets a signalling one)
    for v in (0, 0x8000, 1, 0x3FF, 0x400, 0x3C00, 0x7BFF, 0x7C00, 0xFC00, 0x7E00):
        ref = oracle.get("f32").f16_to_f32(np.uint16([v]))[0]
        assert np.float32(T.half_to_float(v)).view(np.uint32) == ref.view(np.uint32)


def test_float_to_half_bit_patterns(T):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 1 << 32, 1 << 24, dtype=np.uint64).astype(np.uint32)
    # every exponent, both signs, NaN payloads only in the low 13 bits
    edge = np.array([e << 23 | m for e in range(256) for m in (0, 1, 0x1FFF, 0x2000, 0x400000, 0x7FFFFF)],
                    np.uint32)
    bits = np.concatenate([bits, edge, edge | 0x80000000])
    x = bits.view(np.float32)
    got = T.to_half(x)
    assert np.array_equal(got, oracle.get("f32").f32_to_f16(x))
    for v in (0.0, -0.0, 1.0, 65504.0, 65519.99, 65536.0, 6e-8, 2.98e-8, float("inf"), float("nan")):
        assert T.float_to_half(v) == int(oracle.get("f32").f32_to_f16(np.float32([v]))[0])
