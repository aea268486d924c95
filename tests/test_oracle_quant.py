"""Pins the oracle quantizer (reference draftkv/compress.py:21-46) without
retyping its formula: closed forms, special cases, a scalar brute force in
IEEE float32 built from Python's ``struct`` rounding, and the reference's own
test expectations (tests/test_math.py:58-64)."""

import math
import struct

import numpy as np
import pytest

from oracle.quant import dequantize, quantize, quantize_codes


def f32(x: float) -> float:
    """Round a Python float (binary64) to the nearest binary32."""
    return struct.unpack("<f", struct.pack("<f", x))[0]


def brute(row, bits, group):
    """Scalar restatement in binary32 arithmetic: each operation on two
    binary32 values is done exactly in binary64 and then rounded once to
    binary32 (exact for +, -, *, / of binary32 operands)."""
    d = len(row)
    pad = (-d) % group
    vals = [f32(v) for v in row] + [0.0] * pad
    levels = (1 << bits) - 1
    codes, deq = [], []
    for g0 in range(0, len(vals), group):
        g = vals[g0:g0 + group]
        lo, hi = min(g), max(g)
        scale = max(f32(f32(hi - lo) / levels), f32(1e-8))
        for x in g:
            t = f32(f32(x - lo) / scale)
            q = float(round(t))               # Python round: half to even
            q = min(max(q, 0.0), float(levels))
            codes.append(int(q))
            deq.append(f32(f32(q * scale) + lo))
    return codes[:d], deq[:d]


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("group,d", [(64, 16), (64, 64), (32, 128), (64, 80), (32, 40)])
def test_matches_scalar_brute_force(bits, group, d):
    rng = np.random.default_rng(bits * 100 + d)
    x = (rng.standard_normal((3, d)) * rng.choice([0.01, 1.0, 30.0])).astype(np.float32)
    codes, scale, lo, deq = quantize_codes(x, bits, group)
    for r in range(x.shape[0]):
        bc, bd = brute(x[r].tolist(), bits, group)
        assert codes[r].tolist() == bc
        assert np.array_equal(deq[r], np.array(bd, np.float32))


def test_bits16_is_identity_and_error_monotone():        # reference tests/test_math.py:58-64
    x = np.random.default_rng(0).standard_normal((16, 8, 64)).astype(np.float32)
    errs = [np.abs(quantize(x, b) - x).mean() for b in (2, 3, 4, 8)]
    assert errs == sorted(errs, reverse=True)
    assert np.array_equal(quantize(x, 16), x)


def test_integer_ramp_is_exact():
    # lo=0, hi=15 at 4 bits -> scale exactly 1, codes are the values themselves
    x = np.arange(16, dtype=np.float32).reshape(1, 16)
    codes, scale, lo, deq = quantize_codes(x, 4, 16)
    assert codes.tolist() == [list(range(16))]
    assert scale.item() == 1.0 and lo.item() == 0.0
    assert np.array_equal(deq, x)


def test_constant_group_uses_floor_scale():
    x = np.full((2, 64), 3.25, np.float32)
    codes, scale, lo, deq = quantize_codes(x, 4, 64)
    assert (codes == 0).all()
    assert np.all(scale == np.float32(1e-8))
    assert np.array_equal(deq, x)


def test_padding_joins_last_group():
    # d=16 < group=64: 48 zeros take part in min/max, so an all-positive row
    # gets lo=0 (not its own minimum)
    x = np.linspace(1.0, 2.0, 16, dtype=np.float32).reshape(1, 16)
    codes, scale, lo, deq = quantize_codes(x, 8, 64)
    assert lo.item() == 0.0
    assert scale.item() == np.float32(np.float32(2.0) / 255)


def test_codes_and_meta_reconstruct_deq():
    x = np.random.default_rng(1).standard_normal((5, 3, 128)).astype(np.float32)
    for meta in ("f32", "f16"):
        codes, scale, lo, deq = quantize_codes(x, 4, 32, meta)
        assert np.array_equal(dequantize(codes, scale, lo, 32), deq)
        assert codes.max() <= 15


def test_f16_meta_stores_half_values():
    x = np.random.default_rng(2).standard_normal((7, 64)).astype(np.float32)
    codes, scale, lo, deq = quantize_codes(x, 4, 32, "f16")
    assert np.array_equal(scale.astype(np.float16).astype(np.float32), scale)
    assert np.array_equal(lo.astype(np.float16).astype(np.float32), lo)
    # error stays within ~one step of the grid (a wrong lo/scale pairing would not)
    gi = np.arange(64) // 32
    assert np.all(np.abs(deq - x) <= scale[:, gi] * 0.5 + np.abs(lo[:, gi]) * 2e-3 + 1e-6)


def test_rounding_is_half_to_even():
    # values landing exactly on .5 of a step: 0.5 -> 0, 1.5 -> 2, 2.5 -> 2
    x = np.array([[0.0, 0.5, 1.5, 2.5, 3.0]], np.float32)
    codes, scale, lo, _ = quantize_codes(x, 2, 5)
    assert scale.item() == 1.0
    assert codes.tolist() == [[0, 0, 2, 2, 3]]
    assert math.isclose(float(scale.item()), 1.0)
