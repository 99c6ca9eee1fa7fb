"""CPU: pin the oracle's quantizers, dequantizers and quantized Linear
(src/quant.cc:130-650, src/ops.cc:28-40, src/threadpool.cc:26-57).

Checks are chosen so that a plausible restatement mistake fails one of them:
  - the reference tests' own known answers and bounds (tests/test_quant.cc);
  - per-element invariants of the quantizers;
  - closed-form dequantization (d*q is exact in fp32);
  - exact-arithmetic Linear cases: small-integer codes, power-of-two scales
    and dyadic activations make every product and partial sum exactly
    representable, so the fp32 result must equal the integer result; a
    dropped term, wrong nibble order, swapped index or transposed weight
    changes it;
  - float64 brute force within the standard fp32 dot-product error bound;
  - the thread partition and the AVX2 build against the scalar build.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.json")
TYPES = ["q8_0", "q4_0", "q4_1"]


@pytest.fixture(scope="module")
def ref():
    with open(GOLDEN) as f:
        return json.load(f)["reference_tests"]


def fill_linear(n, scale, offset):
    return (offset + scale * np.arange(n, dtype=np.float32)).astype(np.float32)


# ---------------------------------------------------------------------------
# reference known answers (tests/test_quant.cc)
# ---------------------------------------------------------------------------
def test_block_sizes(oracle, ref):
    for t in TYPES:
        assert oracle.BLOCK_DTYPES[t].itemsize == ref["block_bytes"][t]


@pytest.mark.parametrize("name,qtype", [("q8_0_roundtrip", "q8_0"),
                                        ("q8_0_multiblock", "q8_0"),
                                        ("q4_0_roundtrip", "q4_0")])
def test_roundtrip_bounds(oracle, ref, name, qtype):
    case = ref[name]
    x = np.array(case["x"], np.float32)
    blocks = oracle.quantize(x, qtype)
    assert blocks.size == case["blocks"]
    back = oracle.dequantize(blocks, x.shape, qtype)
    assert np.max(np.abs(back - x)) < case["max_err"]


@pytest.mark.parametrize("name,qtype", [("q8_0_zeros", "q8_0"), ("q4_0_zeros", "q4_0")])
def test_all_zeros(oracle, ref, name, qtype):
    case = ref[name]
    x = np.zeros(case["n"], np.float32)
    blocks = oracle.quantize(x, qtype)
    assert blocks.size == case["blocks"]
    assert np.all(blocks["d"] == 0)
    assert np.all(np.abs(oracle.dequantize(blocks, x.shape, qtype)) <= case["tol"])


def test_q4_1_dequant_known_values(oracle, ref):
    case = ref["q4_1_dequant_known"]
    b = np.zeros(1, oracle.BLOCK_Q4_1)
    b["d"], b["m"] = case["block"]["d"], case["block"]["m"]
    b["qs"] = np.array(case["block"]["qs"], np.uint8)
    got = oracle.dequantize(b, (32,), "q4_1")
    assert np.max(np.abs(got - np.array(case["expected"]))) <= case["tol"]


@pytest.mark.parametrize("flavor", ["scalar", "avx2"])
def test_q4_1_linear_known_value(oracle, ref, flavor):
    if not oracle.flavor_available(flavor):
        pytest.skip("no AVX2/FMA on this host")
    case = ref["q4_1_linear_known"]
    b = np.zeros(1, oracle.BLOCK_Q4_1)
    b["d"], b["m"] = case["block"]["d"], case["block"]["m"]
    b["qs"] = np.array(case["block"]["qs"], np.uint8)
    y = oracle.linear(np.array(case["x"], np.float32), b, case["w_shape"], "q4_1",
                      flavor=flavor)
    assert y.shape == (1,)
    assert abs(y[0] - case["expected"][0]) <= case["tol"]


def test_matmul_q8_0_matches_f32(oracle, ref):
    case = ref["matmul_q8_0"]
    a = np.array(case["a"], np.float32)
    b = np.array(case["b"], np.float32)
    qa = oracle.quantize(a, "q8_0")
    deq = oracle.dequantize(qa, a.shape, "q8_0")
    assert np.max(np.abs(deq @ b - a @ b)) <= case["tol"]


def test_compare_matmul_error(oracle, ref):
    case = ref["compare_matmul_error"]
    a = fill_linear(256, case["a_scale"], case["a_offset"]).reshape(16, 16)
    b = fill_linear(256, case["b_scale"], case["b_offset"]).reshape(16, 16)
    deq = oracle.dequantize(oracle.quantize(a, "q8_0"), a.shape, "q8_0")
    err = np.max(np.abs(deq @ b - a @ b))
    assert 0 <= err < case["max_err"]


@pytest.mark.parametrize("name", ["q4_0_linear_vs_f32", "compare_q40_error"])
def test_q4_0_linear_vs_f32(oracle, ref, name):
    case = ref[name]
    n, k = case["w_shape"]
    w = fill_linear(n * k, case["w_scale"], case["w_offset"]).reshape(n, k)
    x = fill_linear(k, case["x_scale"], case["x_offset"])
    y = oracle.linear(x, oracle.quantize(w, "q4_0"), (n, k), "q4_0")
    bound = case.get("tol", case.get("max_err"))
    assert np.max(np.abs(y - w @ x)) < bound


# ---------------------------------------------------------------------------
# quantizer invariants
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("k", [32, 100, 4096, 33])
def test_q8_0_quantizer_invariants(oracle, k):
    rng = np.random.default_rng(k)
    x = (rng.standard_normal((7, k)) * rng.uniform(1e-3, 10, (7, 1))).astype(np.float32)
    x[3, :] = 0.0
    blocks = oracle.quantize(x, "q8_0")
    nb = (k + 31) // 32
    assert blocks.size == 7 * nb
    d = oracle.fp16_to_f32(blocks["d"]).reshape(7, nb)
    q = blocks["qs"].reshape(7, nb, 32).astype(np.int32)
    assert q.min() >= -127 and q.max() <= 127
    xp = np.zeros((7, nb * 32), np.float32)
    xp[:, :k] = x
    xb = xp.reshape(7, nb, 32)
    amax = np.abs(xb).max(axis=2)
    # scale = fp16(amax / 127) with the reference rounding
    assert np.array_equal(blocks["d"].reshape(7, nb),
                          oracle.f32_to_fp16((amax / np.float32(127)).astype(np.float32)))
    # reconstruction error at most half a step (plus fp16 scale rounding)
    err = np.abs(xb - d[..., None] * q)
    assert np.all(err <= 0.5 * d[..., None] * (1 + 1e-3) + 1e-30)
    # padding of the partial last block is zero; zero rows give d = 0
    if k % 32:
        assert np.all(q[:, -1, k % 32:] == 0)
    assert np.all(blocks["d"].reshape(7, nb)[3] == 0)


@pytest.mark.parametrize("k", [32, 96, 50])
def test_q4_0_quantizer_invariants(oracle, k):
    rng = np.random.default_rng(k + 1)
    x = rng.standard_normal((5, k)).astype(np.float32)
    blocks = oracle.quantize(x, "q4_0")
    nb = (k + 31) // 32
    qs = blocks["qs"].reshape(5, nb, 16)
    codes = np.concatenate([qs & 0xF, qs >> 4], axis=2).astype(np.int32)
    d = oracle.fp16_to_f32(blocks["d"]).reshape(5, nb)
    xp = np.zeros((5, nb * 32), np.float32)
    xp[:, :k] = x
    xb = xp.reshape(5, nb, 32)
    rec = d[..., None] * (codes - 8)
    # the clamp to 15 costs up to one extra step at the positive extreme
    assert np.all(np.abs(xb - rec) <= 1.0 * d[..., None] * (1 + 1e-3))
    if k % 32:
        assert np.all(codes[:, -1, k % 32:] == 8)  # padding quantizes 0 -> 8


# ---------------------------------------------------------------------------
# dequantization closed form (exact products)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_closed_form(oracle, qtype):
    from conftest import make_blocks
    n, k = 9, 200
    blocks = make_blocks(qtype, n, k, seed=3)
    got = oracle.dequantize(blocks, (n, k), qtype)
    nb = (k + 31) // 32
    d = blocks["d"].view(np.float16).astype(np.float64).reshape(n, nb, 1)
    if qtype == "q8_0":
        q = blocks["qs"].astype(np.float64).reshape(n, nb, 32)
        val = d * q
    else:
        qs = blocks["qs"].reshape(n, nb, 16)
        q = np.concatenate([qs & 0xF, qs >> 4], axis=2).astype(np.float64)
        if qtype == "q4_0":
            val = d * (q - 8)
        else:
            m = blocks["m"].view(np.float16).astype(np.float64).reshape(n, nb, 1)
            # d*q is exact in fp32; the add rounds once, like the reference
            val = (d * q).astype(np.float32) + m.astype(np.float32)
    exp = np.asarray(val, np.float32).reshape(n, nb * 32)[:, :k]
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


# ---------------------------------------------------------------------------
# Linear: exact arithmetic
# ---------------------------------------------------------------------------
def _exact_blocks(qtype, n, k, rng):
    """Blocks with power-of-two scales (and mins) and integer codes."""
    nb = (k + 31) // 32
    b = np.zeros(n * nb, oracle_dtype(qtype))
    exps = rng.integers(-4, 3, n * nb)
    b["d"] = (2.0 ** exps).astype(np.float16).view(np.uint16)
    if qtype == "q8_0":
        b["qs"] = rng.integers(-127, 128, (n * nb, 32))
    else:
        b["qs"] = rng.integers(0, 256, (n * nb, 16))
    if qtype == "q4_1":
        b["m"] = (rng.integers(-3, 4, n * nb) * 2.0 ** rng.integers(-3, 1, n * nb)
                  ).astype(np.float16).view(np.uint16)
    return b


def oracle_dtype(qtype):
    import oracle
    return oracle.BLOCK_DTYPES[qtype]


def _exact_reference(qtype, blocks, x, n, k):
    """Integer-exact y = W x (Python ints / float64 on dyadic values)."""
    from fractions import Fraction
    nb = (k + 31) // 32
    d = blocks["d"].view(np.float16).astype(np.float64).reshape(n, nb)
    if qtype == "q8_0":
        codes = blocks["qs"].astype(np.int64).reshape(n, nb, 32)
    else:
        qs = blocks["qs"].reshape(n, nb, 16).astype(np.int64)
        codes = np.concatenate([qs & 0xF, qs >> 4], axis=2)
        if qtype == "q4_0":
            codes = codes - 8
    w = d[..., None] * codes
    if qtype == "q4_1":
        w = w + blocks["m"].view(np.float16).astype(np.float64).reshape(n, nb, 1)
    w = w.reshape(n, nb * 32)[:, :k]
    out = np.zeros((x.shape[0], n))
    for r in range(x.shape[0]):
        for j in range(n):
            out[r, j] = float(sum(Fraction(a) * Fraction(b)
                                  for a, b in zip(w[j].tolist(), x[r].tolist())))
    return out


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("m,n,k", [(1, 3, 32), (2, 4, 70), (3, 2, 256), (1, 1, 33)])
@pytest.mark.parametrize("flavor", ["scalar", "avx2"])
def test_linear_exact_arithmetic(oracle, qtype, m, n, k, flavor):
    if not oracle.flavor_available(flavor):
        pytest.skip("no AVX2/FMA on this host")
    rng = np.random.default_rng(m * 100 + n * 10 + k)
    blocks = _exact_blocks(qtype, n, k, rng)
    x = (rng.integers(-16, 17, (m, k)) / 8.0).astype(np.float32)
    exp = _exact_reference(qtype, blocks, x.astype(np.float64), n, k)
    # magnitudes stay far below 2^24 ulps: every fp32 partial sum is exact
    got = oracle.linear(x, blocks, (n, k), qtype, flavor=flavor)
    assert np.array_equal(got.astype(np.float64), exp)


def test_linear_exact_detects_wrong_nibble_order(oracle):
    """Swapping the low/high nibble halves (a plausible mistake) changes the
    exact result; the oracle keeps element i<16 in the low nibble."""
    b = np.zeros(1, oracle.BLOCK_Q4_0)
    b["d"] = 0x3C00
    b["qs"] = np.array([(i & 0xF) | (((15 - i) & 0xF) << 4) for i in range(16)], np.uint8)
    x = np.zeros(32, np.float32)
    x[0] = 1.0   # element 0 -> low nibble of qs[0] = 0 -> value -8
    x[16] = 1.0  # element 16 -> high nibble of qs[0] = 15 -> value 7
    x[5] = 2.0   # element 5 -> low nibble of qs[5] = 5 -> value -3
    y = oracle.linear(x, b, (1, 32), "q4_0")
    assert y[0] == -8.0 + 7.0 + 2.0 * -3.0


# ---------------------------------------------------------------------------
# Linear: float64 brute force, threads, flavours, validation
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("qtype", TYPES)
def test_linear_float64_bound(oracle, qtype):
    from conftest import make_blocks
    n, k, m = 24, 1000, 3
    blocks = make_blocks(qtype, n, k, seed=9)
    rng = np.random.default_rng(10)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = oracle.dequantize(blocks, (n, k), qtype).astype(np.float64)
    exact = x.astype(np.float64) @ w.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(w).T
    u = 2.0 ** -24
    gamma = k * u / (1 - k * u)
    got = oracle.linear(x, blocks, (n, k), qtype)
    assert np.all(np.abs(got - exact) <= gamma * mag)


@pytest.mark.parametrize("qtype", TYPES)
def test_linear_threads_do_not_change_results(oracle, qtype):
    from conftest import make_blocks
    n, k, m = 300, 256, 2  # 600 outputs: threaded for <= 37 threads
    blocks = make_blocks(qtype, n, k, seed=4)
    x = np.random.default_rng(5).standard_normal((m, k)).astype(np.float32)
    y1 = oracle.linear(x, blocks, (n, k), qtype, threads=1)
    for t in (2, 3, 7, 16):
        assert np.array_equal(oracle.linear(x, blocks, (n, k), qtype, threads=t), y1)


def test_avx2_q8_0_close_to_scalar(oracle):
    if not oracle.flavor_available("avx2"):
        pytest.skip("no AVX2/FMA on this host")
    from conftest import make_blocks
    n, k = 64, 4096
    blocks = make_blocks("q8_0", n, k, seed=12)
    x = np.random.default_rng(13).standard_normal(k).astype(np.float32)
    ys = oracle.linear(x, blocks, (n, k), "q8_0", flavor="scalar")
    ya = oracle.linear(x, blocks, (n, k), "q8_0", flavor="avx2")
    w = oracle.dequantize(blocks, (n, k), "q8_0").astype(np.float64)
    mag = np.abs(w) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(ys - ya) <= 2 * k * 2.0 ** -24 * mag)
    assert not np.array_equal(ys, ya)  # different summation order really runs


def test_avx2_q8_0_inf_in_widened_window_gives_nan(oracle):
    """The reference AVX2 loop multiplies zero weights by x[k+4..k+11]
    (quant.cc:598-604); for the last step of a row that window reaches into
    the next row of x, so an infinity there turns this row's output into NaN
    while the scalar build returns the finite sum."""
    if not oracle.flavor_available("avx2"):
        pytest.skip("no AVX2/FMA on this host")
    w = np.zeros(1, oracle.BLOCK_Q8_0)
    w["d"] = 0x3C00  # 1.0
    w["qs"] = 1
    x = np.ones((2, 32), np.float32)
    x[1, 2] = np.inf  # flat index 34, inside row 0's last window x[28..35]
    ya = oracle.linear(x, w, (1, 32), "q8_0", flavor="avx2")
    ys = oracle.linear(x, w, (1, 32), "q8_0", flavor="scalar")
    assert np.isnan(ya[0, 0]) and np.isinf(ya[1, 0])
    assert ys[0, 0] == 32.0 and np.isinf(ys[1, 0])


@pytest.mark.parametrize("qtype", TYPES)
def test_linear_validation(oracle, qtype):
    from conftest import make_blocks
    blocks = make_blocks(qtype, 4, 64, seed=1)
    x = np.zeros(64, np.float32)
    assert oracle.linear_raw(x, blocks, 4, 64, qtype) == oracle.REF_OK
    assert oracle.linear_raw(x, blocks, 4, 32, qtype) == oracle.REF_ERR_SHAPE
    assert oracle.linear_raw(x, blocks[:-1], 4, 64, qtype) == oracle.REF_ERR_BLOCKS
    with pytest.raises(ValueError):
        oracle.dequantize(blocks[:-1], (4, 64), qtype)
