"""Seeded synthetic workloads with the value distributions of the benchmark
configurations (numpy only; fp16 fields via numpy's IEEE binary16 rounding).

  q8_0: q ~ U{-127..127}, d = |N(0, 0.02)| / 127        (value = q*d)
  q4_0: nibbles ~ U{0..15}, d = |N(0, 0.02)| / 8         (value = (q-8)*d)
  q4_1: nibbles ~ U{0..15}, d = |N(0, 0.02)| / 15,
        m ~ N(0, 0.01)                                   (value = q*d + m)
  activations: fp32 ~ N(0, 1)
Blocks are GGUF AoS structured arrays (34 / 18 / 20 bytes each).
"""
from __future__ import annotations

import numpy as np

BLOCK_DTYPES = {
    "q8_0": np.dtype([("d", "<u2"), ("qs", "i1", (32,))]),
    "q4_0": np.dtype([("d", "<u2"), ("qs", "u1", (16,))]),
    "q4_1": np.dtype([("d", "<u2"), ("m", "<u2"), ("qs", "u1", (16,))]),
}


def f16_bits(values) -> np.ndarray:
    return np.asarray(values, np.float32).astype(np.float16).view(np.uint16)


def make_blocks(qtype: str, n: int, k: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    count = n * ((k + 31) // 32)
    out = np.empty(count, BLOCK_DTYPES[qtype])
    if qtype == "q8_0":
        out["qs"] = rng.integers(-127, 128, (count, 32), dtype=np.int8)
        out["d"] = f16_bits(np.abs(rng.normal(0.0, 0.02, count)) / 127.0)
    elif qtype == "q4_0":
        out["qs"] = rng.integers(0, 256, (count, 16), dtype=np.uint8)
        out["d"] = f16_bits(np.abs(rng.normal(0.0, 0.02, count)) / 8.0)
    elif qtype == "q4_1":
        out["qs"] = rng.integers(0, 256, (count, 16), dtype=np.uint8)
        out["d"] = f16_bits(np.abs(rng.normal(0.0, 0.02, count)) / 15.0)
        out["m"] = f16_bits(rng.normal(0.0, 0.01, count))
    else:
        raise ValueError(qtype)
    return out


def make_x(m: int, k: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((m, k), dtype=np.float32)
