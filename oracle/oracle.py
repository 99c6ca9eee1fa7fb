"""CPU ORACLE bindings — test infrastructure only.

numpy front end (ctypes) for the C restatement in ``quant_ref.c`` of the
reference's CPU quantized Linear (src/quant.cc:32-650, src/threadpool.cc:26-57).
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, and only as the checker / the timed CPU baseline.
The product library never imports it.

Blocks are numpy structured arrays whose dtypes are byte-identical to the
reference's packed structs (include/mini_llama/quantized_tensor.h:36-72).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# GGUF-compatible block dtypes: 34 / 18 / 20 bytes, no padding.
BLOCK_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", (32,))])
BLOCK_Q4_0 = np.dtype([("d", "<u2"), ("qs", "u1", (16,))])
BLOCK_Q4_1 = np.dtype([("d", "<u2"), ("m", "<u2"), ("qs", "u1", (16,))])
BLOCK_DTYPES = {"q8_0": BLOCK_Q8_0, "q4_0": BLOCK_Q4_0, "q4_1": BLOCK_Q4_1}
QK = 32

REF_OK, REF_ERR_SHAPE, REF_ERR_BLOCKS = 0, -1, -2

_LIBS: dict[str, ctypes.CDLL] = {}


def build() -> None:
    """Compile both oracle flavours (scalar and AVX2) in place."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def _lib(flavor: str = "scalar") -> ctypes.CDLL:
    if flavor in _LIBS:
        return _LIBS[flavor]
    name = {"scalar": "liboracle.so", "avx2": "liboracle_avx2.so"}[flavor]
    path = os.path.join(HERE, name)
    if not os.path.exists(path):
        build()
    lib = ctypes.CDLL(path)
    P, I, Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    lib.ref_build_flavor.restype = I
    lib.ref_f32_to_fp16.argtypes = [ctypes.c_float]
    lib.ref_f32_to_fp16.restype = ctypes.c_uint16
    lib.ref_fp16_to_f32.argtypes = [ctypes.c_uint16]
    lib.ref_fp16_to_f32.restype = ctypes.c_float
    lib.ref_f32_to_fp16_array.argtypes = [P, P, Z]
    lib.ref_fp16_to_f32_array.argtypes = [P, P, Z]
    for t in ("q8_0", "q4_0"):
        fn = getattr(lib, f"ref_quantize_{t}")
        fn.argtypes = [P, I, I, P]
        fn.restype = Z
    for t in ("q8_0", "q4_0", "q4_1"):
        fn = getattr(lib, f"ref_dequantize_{t}")
        fn.argtypes = [P, Z, I, I, P]
        fn.restype = I
        fn = getattr(lib, f"ref_linear_{t}")
        fn.argtypes = [P, I, I, P, Z, I, I, P, I]
        fn.restype = I
    _LIBS[flavor] = lib
    return lib


def flavor_available(flavor: str) -> bool:
    """AVX2 flavour needs an AVX2+FMA host."""
    if flavor == "scalar":
        return True
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return " avx2" in flags and " fma" in flags
    except OSError:
        return False


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def f32_to_fp16(values) -> np.ndarray:
    """quant.cc:32-70 on every element (uint16 bit patterns)."""
    src = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(src.shape, dtype=np.uint16)
    _lib().ref_f32_to_fp16_array(_ptr(src), _ptr(out), src.size)
    return out


def fp16_to_f32(bits) -> np.ndarray:
    """quant.cc:72-101 on every element."""
    src = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(src.shape, dtype=np.float32)
    _lib().ref_fp16_to_f32_array(_ptr(src), _ptr(out), src.size)
    return out


def _rows(shape) -> tuple[int, int]:
    # quant.cc:135-138 / 196-197: last dim is the row for rank >= 2.
    shape = tuple(int(s) for s in shape)
    total = int(np.prod(shape)) if shape else 0
    row = shape[-1] if len(shape) >= 2 else total
    return (total // row if row else 0), row


def quantize(src, qtype: str) -> np.ndarray:
    """quantizeToQ80 / quantizeToQ40 (quant.cc:130-302)."""
    x = np.ascontiguousarray(src, dtype=np.float32)
    if x.size == 0:
        return np.zeros(0, BLOCK_DTYPES[qtype])
    n_rows, row = _rows(x.shape)
    nb = (row + QK - 1) // QK
    out = np.zeros(n_rows * nb, BLOCK_DTYPES[qtype])
    n = getattr(_lib(), f"ref_quantize_{qtype}")(_ptr(x), n_rows, row, _ptr(out))
    assert n == out.size
    return out


def dequantize(blocks: np.ndarray, shape, qtype: str) -> np.ndarray:
    """dequantizeFromQ80/Q40/Q41 (quant.cc:192-392); raises on bad blocks."""
    blocks = np.ascontiguousarray(blocks, dtype=BLOCK_DTYPES[qtype])
    n_rows, row = _rows(shape)
    out = np.zeros(tuple(shape), np.float32)
    rc = getattr(_lib(), f"ref_dequantize_{qtype}")(
        _ptr(blocks), blocks.size, n_rows, row, _ptr(out))
    if rc != REF_OK:
        raise ValueError(f"dequantize {qtype}: error {rc}")
    return out


def linear(x, blocks: np.ndarray, w_shape, qtype: str, threads: int = 1,
           flavor: str = "scalar") -> np.ndarray:
    """linear(x, QuantizedTensor) -> linearQ80/Q40/Q41 (ops.cc:28-40,
    quant.cc:401-650). x is [K] or [M, K]; the result rank follows x."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    blocks = np.ascontiguousarray(blocks, dtype=BLOCK_DTYPES[qtype])
    if x.ndim not in (1, 2) or len(w_shape) != 2:
        raise ValueError("linear: expected x [K] or [M, K] and 2-D weight")
    rows, k = (1, x.shape[0]) if x.ndim == 1 else x.shape
    n = int(w_shape[0])
    y = np.zeros((rows, n), np.float32)
    rc = getattr(_lib(flavor), f"ref_linear_{qtype}")(
        _ptr(x), rows, k, _ptr(blocks), blocks.size, n, int(w_shape[1]),
        _ptr(y), int(threads))
    if rc != REF_OK:
        raise ValueError(f"linear {qtype}: error {rc}")
    return y[0] if x.ndim == 1 else y


def linear_raw(x: np.ndarray, blocks: np.ndarray, n: int, k_w: int,
               qtype: str, threads: int = 1, flavor: str = "scalar") -> int:
    """Return code of the oracle Linear without raising (validation tests)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = (1, x.shape[0]) if x.ndim == 1 else x.shape
    y = np.zeros((max(rows, 1), max(n, 1)), np.float32)
    return getattr(_lib(flavor), f"ref_linear_{qtype}")(
        _ptr(x), rows, k, _ptr(blocks), blocks.size, n, k_w, _ptr(y),
        int(threads))
