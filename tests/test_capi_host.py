"""CPU: the C ABI library and the C++ host library load and export every
declared symbol; the host-side repack implements the layout documented in
include/mlq.h (checked with an independent numpy decoder of that text);
argument validation returns the documented status codes. No GPU calls.
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT, make_blocks

HEADER = os.path.join(ROOT, "include", "mlq.h")
TYPES = ["q8_0", "q4_0", "q4_1"]


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mlq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_symbols(pkg):
    assert declared_symbols() == sorted(pkg.SIGNATURES)


def test_library_exports_every_declared_symbol(pkg):
    lib = ctypes.CDLL(pkg.LIB_PATH)
    for name in declared_symbols():
        assert hasattr(lib, name), name
    pkg.lib()  # binds signatures for all of them


def test_cpp_host_library_exports_reference_interface(pkg):
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", pkg.HOST_LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    for t in ("Q80", "Q40", "Q41"):
        for suffix in ("Linear", "LinearDeviceWeight", "LinearDeviceInput"):
            assert f"mini_llama::hip{t}{suffix}(" in out, (t, suffix)
    for name in ("uploadLinearWeight", "uploadQ40LinearWeight", "findHipWeight",
                 "HipDeviceBuffer::upload", "hipTensorFromHost",
                 "parseBackendKind", "hipLinearUploaded", "lookupTiledWeight",
                 # cuda_matmul.h / cuda_ops.h / cuda_kv_cache.h / cuda_attention.h twins
                 "hipMatmul(", "hipLinear(", "hipLinearDeviceWeight(", "hipLinearDeviceInput(",
                 "hipRmsNorm(", "hipRmsNormDeviceWeight(", "hipRmsNormDeviceInput(",
                 "hipSilu(", "hipSiluDeviceInput(", "hipElementwiseMul(",
                 "hipElementwiseMulDeviceInput(", "hipElementwiseAdd(",
                 "hipElementwiseAddDeviceInput(", "hipElementwiseAddDeviceWeight(",
                 "hipSoftmax(", "hipEmbeddingLookupDeviceWeight(", "hipRope(",
                 "hipRopeDeviceInput(", "HipKvCache::write(", "HipKvCache::writeDevice(",
                 "HipKvCache::readKeyHead(", "HipKvCache::clear(",
                 "hipAttentionDecode(", "hipAttentionDecodeDeviceInput("):
        assert f"mini_llama::{name}" in out, name


def test_status_strings_and_block_bytes(pkg):
    lib = pkg.lib()
    assert lib.mlq_status_string(0) == b"ok"
    assert lib.mlq_status_string(-3) == b"block count mismatch"
    assert [lib.mlq_block_bytes(t) for t in (1, 2, 3, 0)] == [34, 18, 20, 0]


def test_no_device_reported_cleanly(pkg):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is visible")
    c = ctypes.c_int(5)
    assert pkg.lib().mlq_device_count(ctypes.byref(c)) == -6
    assert c.value == 0


# ---------------------------------------------------------------------------
# layout contract: independent decoder of the text in include/mlq.h
# ---------------------------------------------------------------------------
def decode_tiled(image: np.ndarray, lay, qtype: str, n: int, k: int):
    """Codes [n, nb*32] (int), scales [n, nb], mins [n, nb] from a tiled
    image, following the layout comment of include/mlq.h literally."""
    nb = (k + 31) // 32
    G = (nb + 3) // 4
    nt = (n + 15) // 16
    codes = np.zeros((nt * 16, G * 4 * 32), np.int64)
    q = image[lay.qs_off:]
    for t in range(nt):
        for g in range(G):
            for L in range(64):
                nn, kq = L % 16, L // 16
                row = 16 * t + nn
                if qtype == "q8_0":
                    for h in range(2):
                        chunk = q[(((t * G + g) * 2 + h) * 64 + L) * 16:][:16]
                        for u in range(2):
                            b = 4 * g + 2 * h + u
                            for w in range(2):
                                word = chunk[(2 * u + w) * 4:][:4]
                                for i in range(4):
                                    e = 8 * kq + 4 * w + i
                                    byte = word[i // 2 + 2 * (i % 2)]
                                    codes[row, 32 * b + e] = int(byte) - 128
                else:
                    chunk = q[((t * G + g) * 64 + L) * 16:][:16]
                    for j in range(4):
                        b = 4 * g + j
                        word = int.from_bytes(bytes(chunk[4 * j:4 * j + 4]), "little")
                        for i in range(8):
                            nib = i // 2 + 4 * (i % 2)
                            codes[row, 32 * b + 8 * kq + i] = (word >> (4 * nib)) & 0xF
    d16 = image[lay.d_off:].view(np.uint16)
    m16 = image[lay.m_off:].view(np.uint16) if qtype == "q4_1" else None
    d = np.zeros((nt * 16, G * 4), np.uint16)
    m = np.zeros((nt * 16, G * 4), np.uint16)
    for t in range(nt):
        for g in range(G):
            for nn in range(16):
                for j in range(4):
                    idx = ((t * G + g) * 16 + nn) * 4 + j
                    d[16 * t + nn, 4 * g + j] = d16[idx]
                    if m16 is not None:
                        m[16 * t + nn, 4 * g + j] = m16[idx]
    return codes, d, m


def aos_codes(blocks, qtype, n, nb):
    if qtype == "q8_0":
        return blocks["qs"].astype(np.int64).reshape(n, nb * 32)
    qs = blocks["qs"].reshape(n, nb, 16).astype(np.int64)
    return np.concatenate([qs & 0xF, qs >> 4], axis=2).reshape(n, nb * 32)


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("n,k", [(16, 128), (17, 100), (3, 520), (33, 32)])
def test_host_repack_matches_documented_layout(pkg, qtype, n, k):
    blocks = make_blocks(qtype, n, k, seed=n * 7 + k)
    image, lay = pkg.repack_host(qtype, blocks, n, k)
    assert image.size == lay.bytes and lay.nb == (k + 31) // 32
    codes, d, m = decode_tiled(image, lay, qtype, n, k)
    nb = lay.nb
    assert np.array_equal(codes[:n, :nb * 32], aos_codes(blocks, qtype, n, nb))
    assert np.array_equal(d[:n, :nb], blocks["d"].reshape(n, nb))
    if qtype == "q4_1":
        assert np.array_equal(m[:n, :nb], blocks["m"].reshape(n, nb))
    # padding rows / blocks decode to exactly zero value
    pad_value = {"q8_0": 0, "q4_0": 8, "q4_1": 0}[qtype]
    assert np.all(codes[n:] == pad_value) and np.all(codes[:, nb * 32:] == pad_value)
    assert np.all(d[n:] == 0) and np.all(d[:, nb:] == 0)


def test_layout_sizes(pkg):
    # c1: 18944 x 3584 q4_0 has no padding: quants + scales = GGUF bytes
    lay = pkg.weight_layout("q4_0", 18944, 3584)
    assert lay.d_off == 18944 * 112 * 16
    assert lay.bytes == 18944 * 112 * 18
    lay8 = pkg.weight_layout("q8_0", 11008, 4096)
    assert lay8.bytes == 11008 * 128 * 34
    lay41 = pkg.weight_layout("q4_1", 4096, 14336)
    assert lay41.bytes == 4096 * 448 * 20


def test_host_repack_validation(pkg):
    lib = pkg.lib()
    blocks = make_blocks("q4_0", 4, 64, seed=1)
    raw = blocks.view(np.uint8)
    out = np.zeros(1 << 16, np.uint8)
    ok = lib.mlq_repack_host(2, raw.ctypes.data, 8, 4, 64, out.ctypes.data, out.size)
    assert ok == 0
    assert lib.mlq_repack_host(2, raw.ctypes.data, 7, 4, 64, out.ctypes.data, out.size) == -3
    assert lib.mlq_repack_host(2, raw.ctypes.data, 8, 0, 64, out.ctypes.data, out.size) == -2
    assert lib.mlq_repack_host(9, raw.ctypes.data, 8, 4, 64, out.ctypes.data, out.size) == -1
    assert lib.mlq_repack_host(2, None, 8, 4, 64, out.ctypes.data, out.size) == -1
    assert lib.mlq_repack_host(2, raw.ctypes.data, 8, 4, 64, out.ctypes.data, 16) == -4


def test_linear_validation_without_device(pkg):
    """Argument checks run before any device work."""
    lib = pkg.lib()
    w = pkg.weight_layout("q4_0", 16, 64)
    assert lib.mlq_linear(ctypes.byref(w), 1, 1, 1, None) == -1  # base NULL
    w.base = 1
    assert lib.mlq_linear(ctypes.byref(w), None, 1, 1, None) == -1
    assert lib.mlq_linear(ctypes.byref(w), 1, 1, 0, None) == -2
    w.nb = 7  # inconsistent with k
    assert lib.mlq_linear(ctypes.byref(w), 1, 1, 1, None) == -1
    assert lib.mlq_linear_aos(2, 1, 31, 16, 64, 1, 1, 1, 1, 1 << 20, None) == -3
    assert lib.mlq_dequantize(None, 0, 1, 1, None) == -1


def test_epilogue_validation_without_device(pkg):
    """mlq_linear_epi rejects unknown epilogues and SwiGLU on weights whose
    row count is not a whole number of 16-row gate/up tiles."""
    lib = pkg.lib()
    w = pkg.weight_layout("q4_0", 40, 64)
    w.base = 1
    assert lib.mlq_linear_epi(ctypes.byref(w), 1, 1, 1, None, 7, None, 0, None) == -1
    assert lib.mlq_linear_epi(ctypes.byref(w), 1, 1, 1, None, pkg.EPI_SWIGLU, None, 0, None) == -2
    assert lib.mlq_linear_epi(ctypes.byref(w), None, 1, 1, None, 0, None, 0, None) == -1


def test_interleave_rows_permutation(pkg):
    """Rows 16t..16t+7 of the result are gate rows 8t..8t+7 and rows
    16t+8..16t+15 the matching up rows, for any row size."""
    rng = np.random.default_rng(3)
    for rows, row_bytes in [(8, 1), (24, 18 * 3), (64, 4)]:
        gate = rng.integers(0, 256, size=(rows, row_bytes), dtype=np.uint8)
        up = rng.integers(0, 256, size=(rows, row_bytes), dtype=np.uint8)
        out = pkg.interleave_rows(gate, up, rows).reshape(2 * rows, row_bytes)
        for t in range(rows // 8):
            assert np.array_equal(out[16 * t:16 * t + 8], gate[8 * t:8 * t + 8])
            assert np.array_equal(out[16 * t + 8:16 * t + 16], up[8 * t:8 * t + 8])
    lib = pkg.lib()
    buf = np.zeros(64, dtype=np.uint8)
    assert lib.mlq_interleave_rows(buf.ctypes.data, buf.ctypes.data, 12, 1,
                                   buf.ctypes.data) == -2
    assert lib.mlq_interleave_rows(None, buf.ctypes.data, 8, 1, buf.ctypes.data) == -1


def test_cpp_binary_runs_host_checks(pkg):
    """The C++ suite on a host without a GPU: device tests skip, backend
    parsing/validation runs."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("covered by the gpu run")
    r = subprocess.run([pkg.CPP_TEST_PATH], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "backend_hip_parses" in r.stdout


def test_fixture_file_is_regenerable():
    """tests/golden/reference_vectors.json is exactly what its script writes."""
    import json
    import sys
    path = os.path.join(ROOT, "tests", "golden", "reference_vectors.json")
    committed = json.load(open(path))
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import make_fixtures
    assert committed["fp16_rounding"] == make_fixtures.tie_vectors()
    assert committed["reference_tests"] == json.loads(
        json.dumps(make_fixtures.reference_test_vectors()))
