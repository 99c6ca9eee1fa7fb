"""GPU parity of the HIP quantized-Linear path against the CPU oracle.

Everything here calls libmlq through its C ABI (ctypes); the oracle
(restated reference CPU path, src/quant.cc:192-650) is the checker.
  - dequantization: bit-exact (integer/byte work and exact d*q products);
  - Linear outputs: the stated tolerance (tests/conftest.py), plus the
    reference CUDA tests' 1e-4 absolute bound on their own inputs;
  - full benchmark shapes: every output against the oracle.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import error_report, make_blocks, make_x, tolerance_ok

pytestmark = pytest.mark.gpu

TYPES = ["q8_0", "q4_0", "q4_1"]


def _torch():
    import torch
    return torch


def _dev(a, cuda):
    return _torch().from_numpy(np.ascontiguousarray(a)).to(cuda)


def _print_case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


# --------------------------------------------------------------------------
# dequantization: bit-exact
# --------------------------------------------------------------------------
@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("n,k", [(1, 32), (16, 128), (17, 100), (40, 1000),
                                 (33, 4096)])
def test_dequant_bit_exact(pkg, oracle, cuda, qtype, n, k):
    _print_case(test="dequant", qtype=qtype, n=n, k=k)
    blocks = make_blocks(qtype, n, k, seed=11 * n + k)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    got = pkg.dequantize(tw).cpu().numpy()
    ref = oracle.dequantize(blocks, (n, k), qtype)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_subnormal_and_special_scales(pkg, oracle, cuda, qtype):
    """Every fp16 scale class: subnormals, zero, negative zero, max normal."""
    n, k = 64, 256
    blocks = make_blocks(qtype, n, k, seed=5)
    specials = np.array([0x0001, 0x03ff, 0x0200, 0x0000, 0x8000, 0x8001,
                         0x7bff, 0x0400, 0x3c00, 0xbc00], np.uint16)
    blocks["d"][: specials.size * 10] = np.repeat(specials, 10)
    if qtype == "q4_1":
        blocks["m"][::7] = 0x8123  # negative subnormal mins
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    got = pkg.dequantize(tw).cpu().numpy()
    ref = oracle.dequantize(blocks, (n, k), qtype)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("qtype,n,k", [("q8_0", 4096, 4096), ("q4_0", 18944, 3584),
                                       ("q4_1", 4096, 14336)])
def test_dequant_bit_exact_config_rows(pkg, oracle, cuda, qtype, n, k):
    """Benchmark shapes: rows spread over the whole weight, incl. the last."""
    _print_case(test="dequant_config", qtype=qtype, n=n, k=k)
    blocks = make_blocks(qtype, n, k, seed=3)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    nb = (k + 31) // 32
    for row0 in (0, n // 3 + 5, n - 7):
        got = pkg.dequantize(tw, row0, 7).cpu().numpy()
        sub = blocks[row0 * nb:(row0 + 7) * nb]
        ref = oracle.dequantize(sub, (7, k), qtype)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), row0


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("n,k", [(16, 128), (45, 300), (100, 4096), (16, 2080)])
def test_device_repack_equals_host_repack(pkg, cuda, qtype, n, k):
    """The device repack writes every byte of the tiled image (alignment
    gaps zeroed), equal to the host repack's; the destination starts out
    filled with 0xAB so an unwritten byte shows."""
    import ctypes
    torch = _torch()
    blocks = make_blocks(qtype, n, k, seed=n + k)
    host = pkg.upload(qtype, blocks, n, k, device=cuda)
    aos = pkg.upload_aos(blocks, device=cuda)
    lay = pkg.weight_layout(qtype, n, k)
    buf = torch.full((int(lay.bytes),), 0xAB, dtype=torch.uint8, device=cuda)
    st = pkg.lib().mlq_repack_device(pkg.TYPES[qtype], aos.data_ptr(),
                                     aos.numel() // pkg.BLOCK_BYTES[qtype], n, k,
                                     buf.data_ptr(), buf.numel(), pkg._stream())
    assert st == 0
    torch.cuda.synchronize()
    assert torch.equal(buf, host.buffer)


# --------------------------------------------------------------------------
# Linear: reference CUDA-test inputs at the reference's 1e-4 bound
# --------------------------------------------------------------------------
def _fill_linear(n, scale, offset):
    return (offset + scale * np.arange(n, dtype=np.float32)).astype(np.float32)


def _ref_q41_blocks(out_features, in_features):
    """tests/test_cuda.cc:116-132 makeQ41Blocks (d = 0.5, m = 0)."""
    import oracle as o
    bpr = (in_features + 31) // 32
    b = np.zeros(out_features * bpr, o.BLOCK_Q4_1)
    b["d"] = 0x3800
    b["m"] = 0
    i = np.arange(16)
    b["qs"] = (((i * 3 + 1) & 0xF) | (((i * 5 + 2) & 0xF) << 4)).astype(np.uint8)
    return b


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("path", [1, 2])  # GEMV, MFMA GEMM
def test_reference_cuda_test_inputs(pkg, oracle, cuda, qtype, path):
    """tests/test_cuda.cc:679-743 inputs: W[4,32] fillLinear(0.05,-1),
    x[32] fillLinear(0.1,-0.4), x2[2,32] fillLinear(0.07,-0.3)."""
    w = _fill_linear(128, 0.05, -1.0).reshape(4, 32)
    if qtype == "q4_1":
        blocks = _ref_q41_blocks(4, 32)
    else:
        blocks = oracle.quantize(w, qtype)
    x = _fill_linear(32, 0.1, -0.4)
    x2 = _fill_linear(64, 0.07, -0.3).reshape(2, 32)
    tw = pkg.upload(qtype, blocks, 4, 32, device=cuda)
    for xv in (x, x2):
        ref = oracle.linear(xv, blocks, (4, 32), qtype)
        got = pkg.linear(tw, _dev(xv, cuda), path=path).cpu().numpy()
        if path == 1:
            # GEMV is fp32-class: the reference's own 1e-4 absolute bound
            assert np.max(np.abs(got - ref)) <= 1e-4, (got, ref)
        else:
            assert tolerance_ok(got, ref, np.atleast_2d(xv), 32).all(), (got, ref)


# --------------------------------------------------------------------------
# Linear: random shapes, both kernel families, all types
# --------------------------------------------------------------------------
SHAPES = [(1, 16, 32), (1, 17, 33), (1, 100, 1000), (1, 300, 4096),
          (2, 64, 256), (3, 48, 200), (4, 130, 640), (8, 64, 2048),
          (5, 33, 4096), (16, 256, 512), (64, 128, 1024), (130, 70, 300),
          # skinny GEMM: rows not a multiple of 16, k not a multiple of 128
          (33, 48, 1001), (50, 17, 4000), (9, 300, 33),
          # skinny GEMM with 2 and 4 weight tiles per workgroup, the last
          # workgroup partly past N
          (16, 8200, 256), (40, 16400, 300),
          (257, 300, 256),
          # one-wave workgroups with m > 4 (fewer threads than m*16 outputs)
          (5, 100, 512), (8, 40, 256), (6, 20, 100)]


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_linear_matches_oracle(pkg, oracle, cuda, qtype, m, n, k):
    _print_case(test="linear", qtype=qtype, m=m, n=n, k=k)
    blocks = make_blocks(qtype, n, k, seed=m * 1000 + n + k)
    x = make_x(m, k, seed=m + 7 * k)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    xd = _dev(x, cuda)
    ref = oracle.linear(x, blocks, (n, k), qtype, threads=8)
    paths = [0, 2] + ([1] if m <= 8 else [])
    for path in paths:
        got = pkg.linear(tw, xd, path=path).cpu().numpy()
        ok = tolerance_ok(got, ref, x, k)
        assert ok.all(), (path, error_report(got, ref, x, k))
        if path == 1:
            # decode path is fp32-class: far inside the stated tolerance
            rep = error_report(got, ref, x, k)
            assert rep["max_abs_over_atol"] < 0.05, rep


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("split", [0, 1, 2, 4, 8, 16])
def test_gemv_every_split(pkg, oracle, cuda, qtype, split):
    """Every GEMV K split on shapes that take each code path: slices of
    1..8 groups all in flight, slices longer than the in-flight budget (the
    refill ring), a shorter last slice (groups % split != 0), k % 4 != 0
    (element-wise activation loads), slices of 9 and 10 groups in flight
    (one activation row) and 1, 2, 3 and 8 activation rows."""
    _print_case(test="gemv_split", qtype=qtype, split=split)
    pkg.set_gemv_split(split)
    try:
        for m, n, k in [(1, 48, 4000), (3, 40, 2100), (8, 17, 1500),
                        (2, 20, 1001), (1, 33, 9000), (1, 20, 5000)]:
            blocks = make_blocks(qtype, n, k, seed=n + k + m)
            x = make_x(m, k, seed=k + 3)
            tw = pkg.upload(qtype, blocks, n, k, device=cuda)
            got = pkg.linear(tw, _dev(x, cuda), path=pkg.PATH_GEMV).cpu().numpy()
            ref = oracle.linear(x, blocks, (n, k), qtype, threads=8)
            rep = error_report(got, ref, x, k)
            assert np.isfinite(got).all() and rep["max_abs_over_atol"] < 0.05, (m, n, k, rep)
    finally:
        pkg.set_gemv_split(0)


@pytest.mark.parametrize("qtype", TYPES)
def test_one_row_gemv_long_k(pkg, oracle, cuda, qtype):
    """One activation row at 70B-class K (Qwen2-72B's down projection, K =
    29568: 231 groups, slices longer than the in-flight budget, the refill
    ring) stays on the decode GEMV (a forced GEMV path raises when the
    planner cannot fit a shape) and meets the stated tolerance."""
    n, k = 40, 29568
    _print_case(test="gemv_long_k", qtype=qtype, n=n, k=k)
    blocks = make_blocks(qtype, n, k, seed=n + k)
    x = make_x(1, k, seed=k + 1)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    got = pkg.linear(tw, _dev(x[0], cuda), path=pkg.PATH_GEMV).cpu().numpy()
    ref = oracle.linear(x, blocks, (n, k), qtype, threads=8)[0]
    assert tolerance_ok(got, ref, x, k).all(), error_report(got, ref, x, k)


@pytest.mark.parametrize("qtype", ["q4_0", "q4_1"])
@pytest.mark.parametrize("split", [0, 1, 4])
def test_one_row_gemv_block_sums_exact(pkg, oracle, cuda, qtype, split):
    """The one-row GEMV carries activations as integers in three fp16
    digits and removes the codes' fp16 bias on the matrix core; every
    product and partial sum of a block is an integer below 2^24, so a block
    sum is exact. Pinned bit for bit: unit block scales (q4_1 mins 0) and
    integer activations that are non-zero in one 32-element block only (at
    every block position of a group, in several groups and K slices; the
    slice's largest |x| from 2^3 to 2^22 - 1, so its exponent moves from
    scaling up to none), where every output must equal the exact integer
    dot product rounded once to fp32. A wrong digit, sign, bias constant or
    lane-quarter sum breaks the equality. (K = 896: seven groups, so even
    one K slice holds every group in flight, the path that stages digits;
    ring slices keep fp16 hi/lo pairs.)"""
    n, k = 48, 896
    blocks = make_blocks(qtype, n, k, seed=97)
    blocks["d"] = 0x3C00  # 1.0
    if qtype == "q4_1":
        blocks["m"] = 0
    w = oracle.dequantize(blocks, (n, k), qtype).astype(np.int64)  # q - 8 / q
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    rng = np.random.default_rng(5)
    pkg.set_gemv_split(split)
    try:
        for blk in [0, 1, 2, 3, 5, 14, 22, 27]:
            for top in [2 ** 3, 2 ** 12, 2 ** 22 - 1]:
                _print_case(test="block_sums_exact", qtype=qtype, split=split, blk=blk, top=top)
                xi = np.zeros(k, np.int64)
                xi[32 * blk:32 * blk + 32] = rng.integers(-top, top + 1, 32)
                xi[32 * blk + 7] = top
                want = (w @ xi).astype(np.float32)
                got = pkg.linear(tw, _dev(xi.astype(np.float32), cuda),
                                 path=pkg.PATH_GEMV).cpu().numpy()
                assert np.array_equal(got, want), (blk, top, np.abs(got - want).max())
    finally:
        pkg.set_gemv_split(0)


@pytest.mark.parametrize("qtype", TYPES)
def test_linear_1d_input_and_aos_path(pkg, oracle, cuda, qtype):
    n, k = 80, 544
    blocks = make_blocks(qtype, n, k, seed=21)
    x = make_x(1, k, seed=22)[0]
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    y_tiled = pkg.linear(tw, _dev(x, cuda)).cpu().numpy()
    assert y_tiled.shape == (n,)
    y_aos = pkg.linear_aos(qtype, pkg.upload_aos(blocks, device=cuda), n, k,
                           _dev(x, cuda)).cpu().numpy()
    ref = oracle.linear(x, blocks, (n, k), qtype)
    assert tolerance_ok(y_tiled, ref, x[None], k).all()
    assert tolerance_ok(y_aos, ref, x[None], k).all()


AOS_SHAPES = [  # (m, n, k): direct GEMV (m <= 8, x fits LDS) and repack fallback
    (1, 80, 544), (3, 17, 1001), (1, 4096, 4096), (1, 33, 18944), (8, 70, 300),
    (8, 40, 3000), (2, 300, 97), (8, 40, 4000), (9, 40, 256)]


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("m,n,k", AOS_SHAPES)
def test_aos_direct_gemv(pkg, oracle, cuda, qtype, m, n, k):
    """Raw GGUF blocks (the reference's `const void*` device weight,
    src/cuda_quant.cu:300-361): up to 8 rows whose x fits in LDS read the
    blocks as they are (no workspace), with the reference's fp32
    per-element arithmetic in another order: within 1e-5 of max|y| of the
    oracle, and the stated bar; rows that start at any 2-byte offset (odd
    block counts, a base pointer 2 / 6 / 10 bytes past alignment); larger
    shapes take the repack and match the tiled kernels bit for bit."""
    torch = _torch()
    _print_case(test="aos_direct", qtype=qtype, m=m, n=n, k=k)
    blocks = make_blocks(qtype, n, k, seed=3 * n + k + m)
    x = make_x(m, k, seed=k + 5)
    xd = _dev(x if m > 1 else x[0], cuda)
    ref = oracle.linear(x, blocks, (n, k), qtype, threads=8)
    need = pkg.aos_workspace_bytes(qtype, n, k, m)
    direct = m <= 8 and need == 0
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    for lead in (0, 2, 6, 10):
        buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device=cuda)
        buf[lead:lead + raw.size] = torch.from_numpy(raw).to(cuda)
        aos = buf[lead:lead + raw.size]
        y = np.atleast_2d(pkg.linear_aos(qtype, aos, n, k, xd).cpu().numpy())
        assert tolerance_ok(y, ref, x, k).all(), (lead, error_report(y, ref, x, k))
        if direct:
            scale = np.abs(ref).max() + 1e-30
            assert np.abs(y - ref).max() <= 1e-5 * scale, (lead, np.abs(y - ref).max() / scale)
        else:
            tw = pkg.upload(qtype, blocks, n, k, device=cuda)
            want = np.atleast_2d(pkg.linear(tw, xd, path=pkg.PATH_AUTO,
                                            workspace=None).cpu().numpy())
            assert np.array_equal(y, want), lead
        again = np.atleast_2d(pkg.linear_aos(qtype, aos, n, k, xd).cpu().numpy())
        assert np.array_equal(y, again)
    if m <= 8 and k <= 3000:
        assert direct, (m, n, k, need)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("m,n,k", [(9, 40, 200), (130, 70, 300), (64, 256, 4096),
                                   (300, 100, 1001), (33, 48, 1001), (50, 17, 4000),
                                   (16, 8200, 256), (61, 16400, 300), (1030, 8200, 256)])
def test_gemm_workspace_path_matches_direct(pkg, oracle, cuda, qtype, m, n, k):
    """mlq_linear_ws (fp16 copy of x made by a pre-pass) and the direct GEMM
    (x converted inside) round x to fp16 identically, so they must agree bit
    for bit (also when the grid exceeds the CU count and the workspace path
    runs two workgroups per CU); the workspace contract is enforced. 9..16
    rows with k <= 6144 take the skinny kernel that reads fp32 x itself
    and need no workspace."""
    torch = _torch()
    _print_case(test="gemm_ws", qtype=qtype, m=m, n=n, k=k)
    blocks = make_blocks(qtype, n, k, seed=m + n + k)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    xd = _dev(make_x(m, k, seed=k), cuda)
    need = pkg.workspace_bytes(tw, m)
    x32 = m <= 16 and k % 4 == 0 and k <= 6144  # skinny kernel reading fp32 x itself
    if x32:
        # no copy of x and no workspace; x is rounded per (row, 128-k group)
        # instead of per row, so the bar is the stated one against the
        # oracle, and repeat calls are bit-identical
        assert need == 0
        got = pkg.linear(tw, xd).cpu().numpy()
        x = make_x(m, k, seed=k)
        ref = oracle.linear(x, blocks, (n, k), qtype)
        assert tolerance_ok(got, ref, x, k).all(), error_report(got, ref, x, k)
        assert np.array_equal(got, pkg.linear(tw, xd).cpu().numpy())
        return
    assert need >= m * k * 2
    ws = torch.empty(need, dtype=torch.uint8, device=cuda)
    got_ws = pkg.linear(tw, xd, workspace=ws).cpu().numpy()
    got_direct = pkg.linear(tw, xd, path=pkg.PATH_MFMA).cpu().numpy()
    if m > 64:
        # the planner may split K (another fp32 summation order); one K
        # range per tile must reproduce the direct GEMM bit for bit
        x = make_x(m, k, seed=k)
        atol = 1e-3 * np.linalg.norm(x, axis=1, keepdims=True) * np.sqrt(k / 4096)
        assert np.all(np.abs(got_ws - got_direct) <= 1e-3 * atol)
        pkg.set_gemm_split(1)
        try:
            got_one = pkg.linear(tw, xd, workspace=ws).cpu().numpy()
        finally:
            pkg.set_gemm_split(0)
        assert np.array_equal(got_one, got_direct)
    else:
        # 9..64 rows take the skinny GEMM: same fp16 operands, another fp32
        # summation order
        x = make_x(m, k, seed=k)
        atol = 1e-3 * np.linalg.norm(x, axis=1, keepdims=True) * np.sqrt(k / 4096)
        assert np.all(np.abs(got_ws - got_direct) <= 1e-3 * atol)
    with pytest.raises(pkg.MLQError) as e:
        pkg.linear(tw, xd, workspace=ws[: need - 1])
    assert e.value.status == -4
    big = torch.empty(need + 256, dtype=torch.uint8, device=cuda)
    with pytest.raises(pkg.MLQError) as e:
        pkg.linear(tw, xd, workspace=big[16:])  # large enough, misaligned
    assert e.value.status == -1
    assert pkg.workspace_bytes(tw, 1) == 0  # decode GEMV needs none


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("split", [1, 2, 3, 5, 8])
def test_gemm_every_split(pkg, oracle, cuda, qtype, split):
    """Split-K prefill GEMM: every K range count (uneven ranges when the
    groups do not divide, ranges of one group, splits capped at the group
    count), partial slices summed in order; checked against the oracle and
    against the unsplit kernel."""
    torch = _torch()
    _print_case(test="gemm_split", qtype=qtype, split=split)
    try:
        for m, n, k in [(65, 48, 1000), (130, 300, 2100), (200, 17, 640),
                        (129, 40, 4096), (96, 33, 300)]:
            blocks = make_blocks(qtype, n, k, seed=n + k + m)
            x = make_x(m, k, seed=k + 7)
            tw = pkg.upload(qtype, blocks, n, k, device=cuda)
            xd = _dev(x, cuda)
            pkg.set_gemm_split(1)
            ws = torch.empty(pkg.workspace_bytes(tw, m), dtype=torch.uint8, device=cuda)
            one = pkg.linear(tw, xd, workspace=ws).cpu().numpy()
            pkg.set_gemm_split(split)
            need = pkg.workspace_bytes(tw, m)
            groups = -(-k // 128)
            if min(split, groups) > 1:
                assert need >= m * n * 4 * min(split, groups)
            ws = torch.empty(need, dtype=torch.uint8, device=cuda)
            got = pkg.linear(tw, xd, workspace=ws).cpu().numpy()
            ref = oracle.linear(x, blocks, (n, k), qtype, threads=8)
            # fp16 operands (the prefill GEMM's numerics): the stated bar
            assert tolerance_ok(got, ref, x, k).all(), (m, n, k, error_report(got, ref, x, k))
            atol = 1e-3 * np.linalg.norm(x, axis=1, keepdims=True) * np.sqrt(k / 4096)
            assert np.all(np.abs(got - one) <= 1e-3 * atol), (m, n, k)
            again = pkg.linear(tw, xd, workspace=ws).cpu().numpy()
            assert np.array_equal(got, again)  # fixed summation order
    finally:
        pkg.set_gemm_split(0)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("tiles,splits", [(1, 2), (2, 3), (4, 4), (1, 8), (2, 1)])
def test_skinny_split_k(pkg, oracle, cuda, qtype, tiles, splits):
    """Skinny GEMM (9..64 rows) with its K range split over workgroups whose
    partial slices a reduce pass sums in range order. Ragged shapes (rows
    past m, tile groups past n, k tails, more ranges than 128-k groups);
    the stated bar against the oracle, agreement with the unsplit kernel to
    fp32 summation order, repeat calls and graph replays bit-identical,
    bias and SwiGLU epilogues applied once after the sum."""
    torch = _torch()
    _print_case(test="skinny_split", qtype=qtype, tiles=tiles, splits=splits)
    try:
        for m, n, k in [(9, 40, 200), (33, 48, 1001), (64, 256, 4096),
                        (50, 17, 4000), (16, 8200, 256), (61, 1040, 3000)]:
            blocks = make_blocks(qtype, n, k, seed=5 * n + k + m)
            x = make_x(m, k, seed=k + 13)
            tw = pkg.upload(qtype, blocks, n, k, device=cuda)
            xd = _dev(x, cuda)
            ref = oracle.linear(x, blocks, (n, k), qtype, threads=8)
            atol = 1e-3 * np.linalg.norm(x, axis=1, keepdims=True) * np.sqrt(k / 4096)
            pkg.set_skinny_plan(1, 1)
            one = pkg.linear(tw, xd, workspace=torch.empty(
                pkg.workspace_bytes(tw, m), dtype=torch.uint8, device=cuda)).cpu().numpy()
            pkg.set_skinny_plan(tiles, splits)
            need = pkg.workspace_bytes(tw, m)
            ranges = min(splits, -(-k // 128))
            if ranges > 1:
                assert need >= ranges * m * n * 4
            ws = torch.empty(need, dtype=torch.uint8, device=cuda)
            got = pkg.linear(tw, xd, workspace=ws).cpu().numpy()
            assert tolerance_ok(got, ref, x, k).all(), (m, n, k, error_report(got, ref, x, k))
            assert np.all(np.abs(got - one) <= 1e-3 * atol), (m, n, k)
            again = pkg.linear(tw, xd, workspace=ws).cpu().numpy()
            assert np.array_equal(got, again), (m, n, k)
            bias = torch.from_numpy(make_x(1, n, seed=n + 3)[0]).to(cuda)
            plain = pkg.linear(tw, xd, workspace=ws)
            assert torch.equal(pkg.linear(tw, xd, workspace=ws, bias=bias), plain + bias)
            if n % 16 == 0:
                glu = pkg.linear(tw, xd, workspace=ws, bias=bias,
                                 act=pkg.EPI_SWIGLU).cpu().numpy()
                pb = (plain + bias).cpu().numpy().astype(np.float64)
                rows = np.arange(n // 2)
                want = (_silu64(pb[:, 16 * (rows // 8) + rows % 8])
                        * pb[:, 16 * (rows // 8) + 8 + rows % 8])
                assert np.abs(glu - want).max() <= 1e-5 * (np.abs(want).max() + 1e-30)
        # captured in a graph: every replay (with eager work between them)
        # equals the eager result
        y = torch.empty((m, n), dtype=torch.float32, device=cuda)
        stream = torch.cuda.Stream()
        with torch.cuda.stream(stream):
            pkg.linear(tw, xd, y=y, workspace=ws)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            pkg.linear(tw, xd, y=y, workspace=ws)
        for _ in range(3):
            y.zero_()
            pkg.linear(tw, xd, workspace=ws)  # eager call on the same workspace
            graph.replay()
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy(), got)
    finally:
        pkg.set_skinny_plan(0, 0)


def _silu64(g):
    return g / (1.0 + np.exp(-g))


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("m,n,k", [(1, 48, 128), (1, 300, 1001), (1, 48, 9000),
                                   (4, 64, 512), (16, 8200, 256), (40, 100, 300),
                                   (130, 70, 300), (300, 272, 640), (512, 2048, 256)])
def test_fused_bias_matches_separate_add(pkg, cuda, qtype, m, n, k):
    """The bias added in every kernel's epilogue (GEMV with one and several
    K slices, with the refill ring (q4_1 at K = 9000), skinny, split-K
    reduce, prefill GEMM) equals the kernel output plus the bias, bit for
    bit: the same single fp32 addition."""
    torch = _torch()
    _print_case(test="bias", qtype=qtype, m=m, n=n, k=k)
    blocks = make_blocks(qtype, n, k, seed=m + n + 2 * k)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    x = make_x(m, k, seed=k + 11)
    xd = _dev(x if m > 1 else x[0], cuda)
    bias = torch.from_numpy(make_x(1, n, seed=n)[0]).to(cuda)
    plain = pkg.linear(tw, xd)
    fused = pkg.linear(tw, xd, bias=bias)
    assert torch.equal(fused, plain + bias)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("m,ffn,k", [(1, 48, 128), (1, 520, 1001), (1, 40, 9000), (4, 64, 512),
                                     (16, 4104, 256), (40, 56, 300), (130, 40, 300),
                                     (300, 136, 640), (512, 1024, 256)])
def test_fused_swiglu(pkg, oracle, cuda, qtype, m, ffn, k):
    """gate|up interleaved (upload_glu) with the SwiGLU epilogue: the same
    pre-activations as two separate launches (bit for bit), silu(g) * u in
    fp32 within 1e-5 of the float64 formula on them, and within the stated
    tolerance of the oracle (propagated: |silu'| <= 1.1)."""
    torch = _torch()
    _print_case(test="swiglu", qtype=qtype, m=m, ffn=ffn, k=k)
    gate = make_blocks(qtype, ffn, k, seed=ffn + k)
    up = make_blocks(qtype, ffn, k, seed=ffn + k + 1)
    x = make_x(m, k, seed=k + 5)
    xd = _dev(x if m > 1 else x[0], cuda)
    bg = make_x(1, ffn, seed=ffn + 2)[0]
    bu = make_x(1, ffn, seed=ffn + 3)[0]
    tw = pkg.upload_glu(qtype, gate, up, ffn, k, device=cuda)
    bias = torch.from_numpy(pkg.interleave_rows(bg, bu, ffn)).to(cuda)
    got = np.atleast_2d(pkg.linear(tw, xd, bias=bias, act=pkg.EPI_SWIGLU).cpu().numpy())
    assert got.shape == (m, ffn)
    # pre-activations from separate launches of the same kernels
    tg = pkg.upload(qtype, gate, ffn, k, device=cuda)
    tu = pkg.upload(qtype, up, ffn, k, device=cuda)
    g = np.atleast_2d(pkg.linear(tg, xd).cpu().numpy()).astype(np.float64) + bg
    u = np.atleast_2d(pkg.linear(tu, xd).cpu().numpy()).astype(np.float64) + bu
    ref = _silu64(g) * u
    scale = np.abs(ref).max() + 1e-30
    assert np.abs(got - ref).max() <= 1e-5 * scale, np.abs(got - ref).max() / scale
    # against the oracle
    go = oracle.linear(x, gate, (ffn, k), qtype).astype(np.float64) + bg
    uo = oracle.linear(x, up, (ffn, k), qtype).astype(np.float64) + bu
    ro = _silu64(go) * uo
    atol = 1e-3 * np.linalg.norm(x, axis=1, keepdims=True) * np.sqrt(k / 4096)
    bound = (1.1 * np.abs(uo) + np.abs(_silu64(go))) * atol + 1.1 * atol * atol
    err = np.abs(got - ro)
    assert np.all((err <= bound) | (err <= 2e-3 * np.abs(ro))), err.max()


@pytest.mark.parametrize("m", [9, 16])
def test_swiglu_two_tile_skinny_odd_tiles(pkg, oracle, cuda, m):
    """The fp32-x skinny kernel with two weight tiles per workgroup (the
    default plan for q4_0 at 9..16 rows when it saves a round of workgroups)
    on an odd tile count (8208 rows = 513 tiles: the last workgroup holds one
    tile) with the bias + SwiGLU epilogue: forced two-tile and one-tile plans
    agree with each other and with the oracle."""
    torch = _torch()
    qtype, ffn, k = "q4_0", 4104, 256
    _print_case(test="swiglu_t2", m=m, ffn=ffn, k=k)
    gate = make_blocks(qtype, ffn, k, seed=ffn + 7)
    up = make_blocks(qtype, ffn, k, seed=ffn + 8)
    x = make_x(m, k, seed=k + 9)
    xd = _dev(x, cuda)
    bg = make_x(1, ffn, seed=ffn + 4)[0]
    bu = make_x(1, ffn, seed=ffn + 5)[0]
    tw = pkg.upload_glu(qtype, gate, up, ffn, k, device=cuda)
    bias = torch.from_numpy(pkg.interleave_rows(bg, bu, ffn)).to(cuda)
    outs = {}
    try:
        for tiles in (2, 1):
            pkg.set_skinny_plan(tiles, 0)
            outs[tiles] = pkg.linear(tw, xd, bias=bias, act=pkg.EPI_SWIGLU).cpu().numpy()
    finally:
        pkg.set_skinny_plan(0, 0)
    default = pkg.linear(tw, xd, bias=bias, act=pkg.EPI_SWIGLU).cpu().numpy()
    assert outs[2].shape == (m, ffn)
    assert np.array_equal(outs[2], outs[1])
    assert np.array_equal(default, outs[2])
    go = oracle.linear(x, gate, (ffn, k), qtype).astype(np.float64) + bg
    uo = oracle.linear(x, up, (ffn, k), qtype).astype(np.float64) + bu
    ro = _silu64(go) * uo
    atol = 1e-3 * np.linalg.norm(x, axis=1, keepdims=True) * np.sqrt(k / 4096)
    bound = (1.1 * np.abs(uo) + np.abs(_silu64(go))) * atol + 1.1 * atol * atol
    err = np.abs(outs[2] - ro)
    assert np.all((err <= bound) | (err <= 2e-3 * np.abs(ro))), err.max()


def test_gguf_upload_matches_host_repack(pkg, oracle, cuda, tmp_path):
    """Tensors uploaded straight from a mapped GGUF file (device copy +
    device repack) are the same tiled bytes as the host repack of the same
    blocks, and the Linear on them meets the oracle."""
    from synthetic import gguf_writer as gw
    torch = _torch()
    specs = [("blk.0.attn_q.weight", "q8_0", 40, 96), ("blk.0.ffn_up.weight", "q4_0", 33, 1024),
             ("blk.0.ffn_down.weight", "q4_1", 16, 2080)]
    gtype = {"q8_0": gw.GGML_Q8_0, "q4_0": gw.GGML_Q4_0, "q4_1": gw.GGML_Q4_1}
    blocks = {name: make_blocks(qt, n, k, seed=n + k) for name, qt, n, k in specs}
    path = str(tmp_path / "w.gguf")
    gw.write_gguf(path, [("general.architecture", gw.STRING, "qwen2")],
                  [(name, [k, n], gtype[qt], gw.blocks_bytes(blocks[name]))
                   for name, qt, n, k in specs], alignment=64)
    with pkg.GgufFile(path) as g:
        for name, qt, n, k in specs:
            _print_case(test="gguf_upload", tensor=name)
            tw = g.upload(name, device=cuda)
            ref = pkg.upload(qt, blocks[name], n, k, device=cuda)
            assert (tw.qtype, tw.n, tw.k) == (qt, n, k)
            assert torch.equal(tw.buffer, ref.buffer), name
            x = make_x(3, k, seed=k)
            got = pkg.linear(tw, _dev(x, cuda)).cpu().numpy()
            assert tolerance_ok(got, oracle.linear(x, blocks[name], (n, k), qt), x, k).all()


@pytest.mark.parametrize("m", [1, 3, 16])
def test_concatenated_weights_match_separate(pkg, oracle, cuda, m):
    """q|k|v-style fusion: one tiled weight holding several weights' rows
    (shared input) gives each part's outputs in its row range."""
    k = 640
    parts = [(make_blocks("q4_0", n, k, seed=n), n) for n in (48, 16, 21)]
    tw, off = pkg.upload_concat("q4_0", parts, k, device=cuda)
    x = make_x(m, k, seed=5)
    y = pkg.linear(tw, _dev(x if m > 1 else x[0], cuda)).cpu().numpy()
    y = np.atleast_2d(y)
    for i, (blocks, n) in enumerate(parts):
        ref = oracle.linear(x, blocks, (n, k), "q4_0")
        got = y[:, off[i]:off[i + 1]]
        assert tolerance_ok(got, ref, x, k).all(), (i, error_report(got, ref, x, k))


def test_bias_kernel(pkg, cuda):
    torch = _torch()
    y = torch.arange(12, dtype=torch.float32, device=cuda).reshape(3, 4)
    b = torch.tensor([1.0, -2.0, 0.5, 4.0], device=cuda)
    got = pkg.add_bias(y.clone(), b).cpu().numpy()
    assert np.array_equal(got, np.arange(12, dtype=np.float32).reshape(3, 4) +
                          np.array([1.0, -2.0, 0.5, 4.0], np.float32))


def _probe():
    import importlib
    return importlib.import_module("mini_llama_amd.probe")


def test_read_probe_runs_in_bounds(pkg, cuda):
    """The bench's read probe over whole and ragged sizes (a partial last
    8 KiB chunk, a partial last block of waves): it completes, and on data
    that fold to zero it leaves the sink word untouched."""
    torch = _torch()
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device=cuda)
    sink = torch.full((1,), 7, dtype=torch.int32, device=cuda)
    for nbytes in (16, 8192, 8192 + 48, 3 * 8192 * 4 + 16, 1 << 20):
        print(f"read probe {nbytes} B", flush=True)
        _probe().read(buf, nbytes, sink)
    torch.cuda.synchronize()
    assert int(sink.item()) == 7


def test_read_probe_shared_runs_in_bounds(pkg, cuda):
    """The skinny-floor probe at every accepted shared size, with whole and
    ragged per-wave ranges (a partial last 1 KiB load): it completes, and on
    zero data it leaves the sink word untouched."""
    torch = _torch()
    shared = torch.zeros(256 << 10, dtype=torch.uint8, device=cuda)
    wgs = 12
    own = torch.zeros(wgs * 8 * 8192, dtype=torch.uint8, device=cuda)
    sink = torch.full((1,), 7, dtype=torch.int32, device=cuda)
    for sb in (0, 64 << 10, 128 << 10, 256 << 10):
        for opw in (0, 16, 1024, 4608, 8192):
            if sb == 0 and opw == 0:
                continue
            print(f"shared probe shared={sb} own/wave={opw}", flush=True)
            _probe().read_shared(shared, sb, own, opw, wgs, sink)
    torch.cuda.synchronize()
    assert int(sink.item()) == 7


def test_validation_errors(pkg, cuda):
    torch = _torch()
    blocks = make_blocks("q4_0", 16, 64, seed=1)
    tw = pkg.upload("q4_0", blocks, 16, 64, device=cuda)
    with pytest.raises(ValueError):
        pkg.linear(tw, torch.zeros(32, device=cuda))
    with pytest.raises(pkg.MLQError) as e:
        pkg.linear(tw, torch.zeros((9, 64), device=cuda), path=pkg.PATH_GEMV)
    assert e.value.status == -5
    aos = pkg.upload_aos(blocks[:-1], device=cuda)
    with pytest.raises(pkg.MLQError) as e:
        pkg.linear_aos("q4_0", aos, 16, 64, torch.zeros(64, device=cuda))
    assert e.value.status == -3


# --------------------------------------------------------------------------
# Full benchmark shapes: every output against the oracle
# --------------------------------------------------------------------------
CONFIGS = [("c0", "q8_0", 1, 4096, 4096), ("c1", "q4_0", 1, 18944, 3584),
           ("c2", "q4_1", 1, 4096, 14336), ("c3", "q4_0", 4, 4096, 4096),
           ("c3", "q4_0", 16, 4096, 4096), ("c3", "q4_0", 64, 4096, 4096),
           ("c4", "q8_0", 512, 11008, 4096),
           # the decode sweep's seven shapes: q and o [3584, 3584],
           # k and v [512, 3584], gate and up [18944, 3584] (= c1), down
           # [3584, 18944] (ten groups per wave, the deepest slice held
           # whole in registers), and the fused gate|up weight N = 37888
           ("q/o", "q4_0", 1, 3584, 3584), ("k/v", "q4_0", 1, 512, 3584),
           ("down", "q4_0", 1, 3584, 18944), ("gateup", "q4_0", 1, 37888, 3584)]


@pytest.mark.parametrize("cfg,qtype,m,n,k", CONFIGS)
def test_config_shapes(pkg, oracle, cuda, cfg, qtype, m, n, k):
    """Every output of each BASELINE workload through the benchmarked entry
    point (mlq_linear_epi with the per-device workspace: the fp16 copy and
    the prefill GEMM for c4, the skinny GEMM for M = 16 / 64, the GEMV
    below), compared with the reference CPU Linear (the oracle, all output
    rows and columns, the reference thread partition), as the reference's
    CUDA tests compare every element (tests/test_cuda.cc:679-743)."""
    _print_case(test="config", cfg=cfg, qtype=qtype, m=m, n=n, k=k)
    blocks = make_blocks(qtype, n, k, seed=1000 + n)
    x = make_x(m, k, seed=2000 + m)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    y = pkg.linear(tw, _dev(x if m > 1 else x[0], cuda)).cpu().numpy().reshape(m, n)
    assert np.isfinite(y).all()
    threads = max(1, min(16, os.cpu_count() or 1))
    ref = oracle.linear(x, blocks, (n, k), qtype, threads=threads)
    ok = tolerance_ok(y, ref, x, k)
    bad = np.argwhere(~ok)
    assert ok.all(), (len(bad), bad[:8].tolist(), error_report(y, ref, x, k))


def test_linearity_full_c1(pkg, cuda):
    """Size-independent property at the headline shape: W(ax+by) = aWx + bWy."""
    torch = _torch()
    n, k = 18944, 3584
    blocks = make_blocks("q4_0", n, k, seed=77)
    tw = pkg.upload("q4_0", blocks, n, k, device=cuda)
    x = _dev(make_x(1, k, seed=1)[0], cuda)
    z = _dev(make_x(1, k, seed=2)[0], cuda)
    a, b = 0.5, -2.0  # powers of two keep the combination exact
    y = pkg.linear(tw, a * x + b * z)
    y2 = a * pkg.linear(tw, x) + b * pkg.linear(tw, z)
    scale = torch.linalg.vector_norm(x) * np.sqrt(k / 4096) * 1e-3
    assert torch.max(torch.abs(y - y2)).item() <= 4 * scale.item()


def test_cpp_interface_tests(pkg):
    """The C++ host-interface tests (tests/cpp/test_hip_quant.cc)."""
    import subprocess
    r = subprocess.run([pkg.CPP_TEST_PATH], capture_output=True, text=True,
                       timeout=300)
    print(r.stdout[-4000:])
    print(r.stderr[-4000:])
    assert r.returncode == 0
    assert "(skip" not in r.stdout
