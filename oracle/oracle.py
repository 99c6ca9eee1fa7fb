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


# ---- decode-step operators and the forward pass (forward_ref.c) ----------------
_FWD_READY: set = set()


def _fwd(flavor: str = "scalar") -> ctypes.CDLL:
    lib = _lib(flavor)
    if flavor in _FWD_READY:
        return lib
    P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    lib.ref_rmsnorm.argtypes = [P, P, P, I, F]
    lib.ref_rmsnorm.restype = None
    lib.ref_softmax.argtypes = [P, P, I]
    lib.ref_softmax.restype = I
    lib.ref_silu.argtypes = [P, P, I]
    lib.ref_silu.restype = None
    lib.ref_swiglu.argtypes = [P, P, P, I]
    lib.ref_swiglu.restype = None
    lib.ref_rope.argtypes = [P, P, I, I, I, I, F, I]
    lib.ref_rope.restype = I
    lib.ref_attention.argtypes = [P, P, P, I, I, I, I, I, I, P]
    lib.ref_attention.restype = None
    lib.ref_linear_f32.argtypes = [P, P, P, I, I]
    lib.ref_linear_f32.restype = None
    lib.ref_argmax.argtypes = [P, I]
    lib.ref_argmax.restype = I
    _FWD_READY.add(flavor)
    return lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rmsnorm(x, w, eps: float) -> np.ndarray:
    """rmsNorm (ops.cc:43-72) on one vector."""
    x, w = _f32(x), _f32(w)
    y = np.empty_like(x)
    _fwd().ref_rmsnorm(_ptr(x), _ptr(w), _ptr(y), x.size, eps)
    return y


def softmax(x) -> np.ndarray:
    """softmax (ops.cc:74-109)."""
    x = _f32(x)
    y = np.empty_like(x)
    if _fwd().ref_softmax(_ptr(x), _ptr(y), x.size) != 0:
        raise ValueError("softmax: empty input")
    return y


def silu(x) -> np.ndarray:
    """silu (ops.cc:111-119)."""
    x = _f32(x)
    y = np.empty_like(x)
    _fwd().ref_silu(_ptr(x), _ptr(y), x.size)
    return y


def swiglu(gate, up) -> np.ndarray:
    """swiGlu (ops.cc:137-140)."""
    g, u = _f32(gate), _f32(up)
    if g.shape != u.shape:
        raise ValueError("swiglu: shape mismatch")
    y = np.empty_like(g)
    _fwd().ref_swiglu(_ptr(g), _ptr(u), _ptr(y), g.size)
    return y


def rope(q, k, pos: int, theta: float, rope_type: int = 0):
    """rope (ops.cc:142-228) on copies of q [n_heads, hd] and k [n_kv, hd]."""
    q, k = _f32(q).copy(), _f32(k).copy()
    if q.ndim != 2 or k.ndim != 2 or q.shape[1] != k.shape[1]:
        raise ValueError("rope: expected q [n_heads, hd] and k [n_kv, hd]")
    rc = _fwd().ref_rope(_ptr(q), _ptr(k), q.shape[0], k.shape[0], q.shape[1], int(pos),
                         float(theta), int(rope_type))
    if rc != 0:
        raise ValueError("rope: rejected arguments")
    return q, k


def attention(q, keys, values, layer: int, pos: int) -> np.ndarray:
    """forwardAttention's CPU arithmetic (forward.cc:526-565): q [n_heads, hd]
    against cache rows 0..pos of `layer` (cache [layers, max_seq, n_kv, hd])."""
    q, keys, values = _f32(q), _f32(keys), _f32(values)
    n_layers, max_seq, n_kv, hd = keys.shape
    out = np.empty_like(q)
    _fwd().ref_attention(_ptr(q), _ptr(keys), _ptr(values), int(layer), int(pos),
                         q.shape[0], n_kv, hd, max_seq, _ptr(out))
    return out


def linear_f32(x, w) -> np.ndarray:
    """linearNaive (matmul_dispatch.cc:32-50): x [K] times W [N, K]^T."""
    x, w = _f32(x).reshape(-1), _f32(w)
    y = np.empty(w.shape[0], np.float32)
    _fwd().ref_linear_f32(_ptr(x), _ptr(w), _ptr(y), w.shape[0], w.shape[1])
    return y


def argmax(x) -> int:
    """argMax (ops.cc:230-246)."""
    x = _f32(x).reshape(-1)
    return int(_fwd().ref_argmax(_ptr(x), x.size))


def linear_weight(x, w: dict, threads: int = 1) -> np.ndarray:
    """The Linear dispatch of forwardLinear's CPU branch (ops.cc:28-40) for a
    model-dict weight {"type", "shape", "data"}. `threads` splits the output
    rows like the reference ThreadPool (each output is one thread's
    sequential sum, so the result does not depend on it)."""
    if w["type"] == "f32":
        return linear_f32(x, np.asarray(w["data"], np.float32).reshape(w["shape"]))
    return linear(_f32(x).reshape(-1), w["data"], w["shape"], w["type"], threads=threads)


def new_cache(model: dict):
    """Zeroed K and V caches [layers, max_seq, n_kv, hd] (KvCache)."""
    c = model["config"]
    hd = c.get("head_dim", c["dim"] // c["n_heads"])
    shape = (c["n_layers"], c["max_seq_len"], c["n_kv_heads"], hd)
    return np.zeros(shape, np.float32), np.zeros(shape, np.float32)


def forward_token(model: dict, cache, token: int, pos: int, threads: int = 1) -> np.ndarray:
    """forwardToken's CPU branch (forward.cc:763-797): embedding, every
    forwardLayer (:642-730) and computelogits (:747-761). `cache` is the
    (keys, values) pair from new_cache, updated at `pos` in place.
    `threads`: the quantized Linears' thread count (same results)."""
    c = model["config"]
    keys, values = cache
    nh, nkv = c["n_heads"], c["n_kv_heads"]
    hd = c.get("head_dim", c["dim"] // nh)
    eps = c["rms_norm_eps"]
    if not (0 <= token < c["vocab_size"]) or not (0 <= pos < c["max_seq_len"]):
        raise ValueError("forward_token: token or position out of range")
    x = _f32(model["token_embedding"][token])
    for li, lw in enumerate(model["layers"]):
        h = rmsnorm(x, lw["attention_norm"], eps)
        parts = []
        for wname, bname in (("wq", "bq"), ("wk", "bk"), ("wv", "bv")):
            y = linear_weight(h, lw[wname], threads)
            b = lw.get(bname)
            if b is not None and np.size(b):
                y = (y + _f32(b)).astype(np.float32)  # addOptionalBias (:402-416)
            parts.append(y)
        q, k = rope(parts[0].reshape(nh, hd), parts[1].reshape(nkv, hd), pos,
                    c["rope_theta"], c.get("rope_type", 0))
        keys[li, pos] = k
        values[li, pos] = parts[2].reshape(nkv, hd)
        att = attention(q, keys, values, li, pos)
        proj = linear_weight(att.reshape(-1), lw["wo"], threads)
        x = (x + proj).astype(np.float32)  # forwardAdd (:312-330)
        h = rmsnorm(x, lw["ffn_norm"], eps)
        ff = linear_weight(swiglu(linear_weight(h, lw["w_gate"], threads),
                                  linear_weight(h, lw["w_up"], threads)), lw["w_down"], threads)
        x = (x + ff).astype(np.float32)
    return linear_weight(rmsnorm(x, model["final_norm"], eps), model["lm_head"], threads)
