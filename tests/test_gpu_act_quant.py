"""GPU q8_0 activation quantizer (mlq_quantize_act_q8_0) against the oracle's
restatement of quantizeToQ80 (src/quant.cc:130-190): bit-exact block bytes.

The cases pin the rules that a plausible kernel mistake would break: the
reference's fp16 rounding of the scale (a tie rounds up, where
round-to-nearest-even would not), round half away from zero of the codes,
the clamp, zero / underflowing / overflowing scales, the zero padding of a
partial last block, and non-finite elements.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _check(pkg, oracle, cuda, x):
    import torch
    got = pkg.quantize_act_q8_0(torch.from_numpy(np.ascontiguousarray(x)).to(cuda))
    torch.cuda.synchronize()
    ref = oracle.quantize(x, "q8_0").view(np.uint8)
    got = got.cpu().numpy()
    assert got.size == ref.size
    bad = np.flatnonzero(got != ref)
    assert bad.size == 0, f"{bad.size} bytes differ, first at block {bad[0] // 34}"


@pytest.mark.parametrize("rows,k", [(1, 32), (1, 100), (3, 4096), (7, 33), (2, 1),
                                    (5, 18944), (512, 4096)])
def test_random_rows(pkg, oracle, cuda, rows, k):
    _case(test="act_q8_0", rows=rows, k=k)
    rng = np.random.default_rng(rows * 7919 + k)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x *= np.float32(2.0) ** rng.integers(-12, 12, size=(rows, 1)).astype(np.float32)
    _check(pkg, oracle, cuda, x)


def test_one_dimensional_input(pkg, oracle, cuda):
    _case(test="act_q8_0_1d", k=1000)
    x = np.random.default_rng(3).standard_normal(1000).astype(np.float32)
    _check(pkg, oracle, cuda, x)


def _blocks(*rows):
    """One row of 32-element blocks from the given 32-value lists."""
    return np.concatenate([np.asarray(r, np.float32) for r in rows])[None, :]


def test_scale_rounding_and_code_rounding(pkg, oracle, cuda):
    _case(test="act_q8_0_rounding")
    blocks = []
    # amax / 127 = 1 + 2^-11 exactly: a tie between fp16 1.0 and its next
    # value; the reference rounds up (0x3c01), round-to-nearest-even would not
    for e in (-20, -3, 0, 5):
        t = np.float32((1 + 2.0 ** -11) * 2.0 ** e)
        b = np.zeros(32, np.float32)
        b[0] = np.float32(127) * t
        b[1:] = np.linspace(-1, 1, 31, dtype=np.float32) * b[0]
        blocks.append(b)
    # amax 127 -> d = 1 exactly: quotients k + 0.5 round away from zero
    b = np.array([127, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]
                 + [0.49999997, -0.49999997] + [3.0] * 21, np.float32)
    blocks.append(b)
    # a block of one value per sign and the clamp edge
    blocks.append(np.array([-127.0] + [127.0] * 31, np.float32))
    blocks.append(np.full(32, 1e-3, np.float32))
    _check(pkg, oracle, cuda, _blocks(*blocks))


def test_zero_underflow_overflow_scales(pkg, oracle, cuda):
    _case(test="act_q8_0_scales")
    z = np.zeros(32, np.float32)
    neg0 = np.full(32, -0.0, np.float32)
    tiny = np.full(32, 1e-9, np.float32)            # d underflows to 0
    sub = np.linspace(-3e-6, 3e-6, 32, dtype=np.float32)  # subnormal fp16 d
    huge = np.linspace(-3e38, 3e38, 32, dtype=np.float32)  # d overflows to inf
    edge = np.full(32, np.float32(127 * 65504.0))     # largest finite d
    _check(pkg, oracle, cuda, _blocks(z, neg0, tiny, sub, huge, edge))


def test_partial_last_block_padding(pkg, oracle, cuda):
    _case(test="act_q8_0_padding")
    rng = np.random.default_rng(9)
    for k in (31, 33, 47, 63, 65):
        _check(pkg, oracle, cuda, rng.standard_normal((3, k)).astype(np.float32))


def test_non_finite_elements(pkg, oracle, cuda):
    """NaN never becomes the block maximum; an element with no integer
    quotient (NaN, or inf under an infinite scale) stores -127, the x86
    conversion the reference's (int)std::round compiles to."""
    _case(test="act_q8_0_nonfinite")
    a = np.linspace(-2, 2, 32, dtype=np.float32)
    a[3] = np.nan
    b = np.full(32, np.nan, np.float32)
    c = np.linspace(-2, 2, 32, dtype=np.float32)
    c[5] = np.inf
    d = np.linspace(-2, 2, 32, dtype=np.float32)
    d[7] = -np.inf
    _check(pkg, oracle, cuda, _blocks(a, b, c, d))
