"""CPU: pin the oracle's fp16 conversions (src/quant.cc:32-101).

fp16 -> fp32 is checked exhaustively against numpy's IEEE binary16 decoder.
fp32 -> fp16 is checked against numpy (round-to-nearest-even) on inputs that
are not exact ties, where the two rules coincide, and against exact rational
rounding on ties and boundaries (tests/golden/reference_vectors.json), which
is where the reference's ties-away-from-zero rule differs from RNE.
"""
from __future__ import annotations

import json
import os
from fractions import Fraction

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")


def test_fp16_to_f32_exhaustive(oracle):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = oracle.fp16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@np.errstate(over="ignore")
def _is_tie(f32: np.ndarray) -> np.ndarray:
    """True where the value lies exactly halfway between two fp16 values."""
    h = f32.astype(np.float16)
    out = np.zeros(f32.shape, bool)
    for i, (x, hv) in enumerate(zip(f32.tolist(), h.tolist())):
        if not np.isfinite(x) or not np.isfinite(hv):
            continue
        lo = np.nextafter(np.float16(hv), np.float16(-np.inf))
        hi = np.nextafter(np.float16(hv), np.float16(np.inf))
        fx = Fraction(x)
        for nb in (lo, hi):
            if np.isfinite(nb) and Fraction(float(nb)) + Fraction(float(hv)) == 2 * fx:
                out[i] = True
    return out


@pytest.mark.parametrize("scale", [1e-7, 1e-5, 3e-3, 1.0, 300.0, 6e4])
def test_f32_to_fp16_matches_numpy_off_ties(oracle, scale):
    rng = np.random.default_rng(int(scale * 1e7) % 2**31)
    x = (rng.standard_normal(20000) * scale).astype(np.float32)
    got = oracle.f32_to_fp16(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    diff = got != ref
    # every disagreement must be an exact tie (RNE vs ties-away)
    assert not np.any(diff & ~_is_tie(x))


def test_f32_to_fp16_all_fp16_values_roundtrip(oracle):
    """Every finite fp16 value converts back to itself."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    vals = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(vals)
    got = oracle.f32_to_fp16(vals[finite])
    exp = bits[finite].copy()
    assert np.array_equal(got, exp)


def test_f32_to_fp16_ties_and_specials(oracle):
    with open(GOLDEN) as f:
        cases = json.load(f)["fp16_rounding"]
    src = np.array([c["f32_bits"] for c in cases], np.uint32).view(np.float32)
    exp = np.array([c["fp16_bits"] for c in cases], np.uint16)
    assert np.array_equal(oracle.f32_to_fp16(src), exp)


def test_f32_to_fp16_ties_go_away_from_zero(oracle):
    """A plausible mistake (RNE) fails here: 1 + 2^-11 is the midpoint of
    1.0 and 1 + 2^-10; RNE keeps 1.0 (even), the reference rounds up."""
    x = np.array([1.0 + 2.0 ** -11, -(1.0 + 2.0 ** -11), 2.0 ** -25], np.float32)
    assert oracle.f32_to_fp16(x).tolist() == [0x3C01, 0xBC01, 0x0001]
