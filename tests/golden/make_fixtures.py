#!/usr/bin/env python3
"""Writes tests/golden/reference_vectors.json.

Two kinds of fixtures, neither produced by the oracle under test:
 1. Known-answer data transcribed from the reference's own tests (inputs and
    the expected values / bounds their assertions state):
      tests/test_quant.cc:11-303 and tests/test_cuda.cc:68-132, 679-743.
 2. float -> fp16 rounding vectors computed with exact rational arithmetic
    (fractions.Fraction) under the rounding rule of src/quant.cc:32-70 read
    as a textbook rule: round to nearest, ties away from zero; results below
    half of the smallest subnormal flush to signed zero; overflow and NaN go
    to signed infinity.
The reference itself is not built or run (it needs spdlog / nlohmann_json /
GTest / CUDA, none of which exist here); its test literals are data.
"""
from __future__ import annotations

import json
import math
import os
import struct
from fractions import Fraction

HERE = os.path.dirname(os.path.abspath(__file__))


def f32_bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


def bits_f32(b: int) -> float:
    return struct.unpack("<f", struct.pack("<I", b))[0]


def fp16_value(h: int) -> Fraction:
    """Exact value of a finite fp16 bit pattern."""
    sign = -1 if h & 0x8000 else 1
    e = (h >> 10) & 0x1F
    m = h & 0x3FF
    if e == 0:
        return sign * Fraction(m, 1 << 24)
    return sign * Fraction(1024 + m, 1 << 10) * Fraction(2) ** (e - 15)


POS_FINITE = [fp16_value(h) for h in range(0x7C00)]  # 0 .. 65504, increasing


def round_ties_away(x: float) -> int:
    """Exact textbook rounding of an fp32 value to fp16 bits."""
    if math.isnan(x):
        return 0x7C00 | (0x8000 if f32_bits(x) >> 31 else 0)
    sign = 0x8000 if (f32_bits(x) >> 31) else 0
    if math.isinf(x):
        return sign | 0x7C00
    a = abs(Fraction(x))
    max_h = POS_FINITE[-1]
    half_ulp_top = Fraction(16)  # ulp at 32768..65504 is 32
    if a >= max_h + half_ulp_top:
        return sign | 0x7C00
    # binary search the largest fp16 <= a
    lo, hi = 0, len(POS_FINITE) - 1
    while lo < hi:
        mid = (lo + hi + 1) // 2
        if POS_FINITE[mid] <= a:
            lo = mid
        else:
            hi = mid - 1
    below = lo
    if POS_FINITE[below] == a or below == len(POS_FINITE) - 1:
        return sign | below
    above = below + 1
    d_lo = a - POS_FINITE[below]
    d_hi = POS_FINITE[above] - a
    return sign | (above if d_hi <= d_lo else below)  # tie -> away from zero


def tie_vectors():
    cases = []
    # exact midpoints between consecutive fp16 values (normal and subnormal,
    # even and odd lower neighbours), both signs
    picks = [0x0000, 0x0001, 0x0002, 0x0003, 0x01FF, 0x03FE, 0x03FF, 0x0400,
             0x0401, 0x3BFF, 0x3C00, 0x3C01, 0x3C02, 0x4000, 0x57FF, 0x5800,
             0x7BFE]
    for h in picks:
        mid = (fp16_value(h) + fp16_value(h + 1)) / 2
        v = float(mid)
        assert Fraction(v) == mid  # exactly representable in fp32
        v = bits_f32(f32_bits(v))
        for s in (1.0, -1.0):
            cases.append({"f32_bits": f32_bits(s * v),
                          "fp16_bits": round_ties_away(s * v)})
    # overflow boundary and specials
    for v in [65504.0, 65519.0, 65520.0, 65536.0, 1e10, float("inf"),
              2.0 ** -24, 2.0 ** -25, bits_f32(f32_bits(2.0 ** -25) - 1),
              2.0 ** -26, 1e-30, 0.0, 5.960464477539063e-08, 6.103515625e-05,
              6.097555160522461e-05]:
        for s in (1.0, -1.0):
            cases.append({"f32_bits": f32_bits(s * v),
                          "fp16_bits": round_ties_away(s * v)})
    cases.append({"f32_bits": 0x7FC00000, "fp16_bits": 0x7C00})  # NaN -> inf
    cases.append({"f32_bits": 0xFFC00000, "fp16_bits": 0xFC00})
    return cases


def reference_test_vectors():
    v = {}
    # tests/test_quant.cc:231-248 (q4_1 dequantize known values)
    v["q4_1_dequant_known"] = {
        "block": {"d": 0x3800, "m": 0xBC00,
                  "qs": [i | ((15 - i) << 4) for i in range(16)]},
        "expected": [-1.0 + 0.5 * i for i in range(16)] +
                    [-1.0 + 0.5 * (15 - i) for i in range(16)],
        "tol": 1e-6,
    }
    # tests/test_quant.cc:250-263 (q4_1 linear known value)
    v["q4_1_linear_known"] = {
        "block": {"d": 0x3C00, "m": 0x0000, "qs": [0x11] * 16},
        "x": [2.0] * 32, "w_shape": [1, 32], "expected": [64.0], "tol": 1e-6,
    }
    # tests/test_quant.cc:20-79 (q8_0 round trips), 196-229 (q4_0)
    v["q8_0_roundtrip"] = {"x": [i * 0.1 for i in range(32)], "blocks": 1,
                           "max_err": 6e-2}
    v["q8_0_multiblock"] = {"x": [i * 0.05 for i in range(100)], "blocks": 4,
                            "max_err": 6e-2}
    v["q8_0_zeros"] = {"n": 64, "blocks": 2, "tol": 1e-6}
    v["q4_0_roundtrip"] = {"x": [i * 0.1 for i in range(32)], "blocks": 1,
                           "max_err": 3e-1}
    v["q4_0_zeros"] = {"n": 64, "blocks": 2, "tol": 1e-6}
    # tests/test_quant.cc:95-128 (matmulQ80 vs F32, 2e-1)
    v["matmul_q8_0"] = {"a": [[1, 2, 3], [4, 5, 6]], "b": [[1, 2], [3, 4], [5, 6]],
                        "tol": 2e-1}
    # tests/test_quant.cc:130-144 (compareMatmulError < 1e-1)
    v["compare_matmul_error"] = {"a_scale": 0.01, "a_offset": -1.0,
                                 "b_scale": 0.01, "b_offset": -0.5,
                                 "shape": [16, 16], "max_err": 1e-1}
    # tests/test_quant.cc:265-286 (q4_0 linear vs F32 within 2.0)
    v["q4_0_linear_vs_f32"] = {"w_scale": 0.05, "w_offset": -1.0, "w_shape": [4, 32],
                               "x_scale": 0.1, "x_offset": -0.4, "tol": 2.0}
    # tests/test_quant.cc:288-303 (compareQ40Error < 2.0)
    v["compare_q40_error"] = {"w_scale": 0.01, "w_offset": -1.0, "w_shape": [8, 32],
                              "x_scale": 0.01, "x_offset": -0.5, "max_err": 2.0}
    # tests/test_cuda.cc:679-743 (GPU vs CPU inputs; 1e-4 absolute)
    v["cuda_linear_inputs"] = {
        "w_scale": 0.05, "w_offset": -1.0, "w_shape": [4, 32],
        "x_scale": 0.1, "x_offset": -0.4, "x2_scale": 0.07, "x2_offset": -0.3,
        "x2_shape": [2, 32], "bias_scale": 0.2, "bias_offset": -0.1,
        "q4_1_block": {"d": 0x3800, "m": 0x0000,
                       "qs": [((i * 3 + 1) & 0xF) | (((i * 5 + 2) & 0xF) << 4)
                              for i in range(16)]},
        "tol_host": 1e-4, "tol_device_variants": 1e-5,
    }
    # block sizes (tests/test_quant.cc:11-15, 184-194)
    v["block_bytes"] = {"q8_0": 34, "q4_0": 18, "q4_1": 20, "elements": 32}
    return v


def main():
    data = {"_source": "reference tests/test_quant.cc and tests/test_cuda.cc "
                       "literals; fp16 ties by exact rational rounding",
            "reference_tests": reference_test_vectors(),
            "fp16_rounding": tie_vectors()}
    path = os.path.join(HERE, "reference_vectors.json")
    with open(path, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {path}: {len(data['fp16_rounding'])} fp16 vectors")


if __name__ == "__main__":
    main()
