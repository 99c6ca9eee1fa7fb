"""mini-llama HIP backend for MI355X: Python front end of the C ABI (libmlq).

ctypes bindings for ``include/mlq.h``. PyTorch is used only for device
memory and streams. There is no CPU fallback: every compute entry point runs
the HIP kernels in ``libmlq.so`` and raises if the library is missing.

The directory name contains a hyphen, so load it with ``load_package()`` from
the repository root helpers (tests/conftest.py, bench.py, __graft_entry__.py),
which registers it as ``mini_llama_amd``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmlq.so")
HOST_LIB_PATH = os.path.join(HERE, "libmini_llama_hip.so")
CPP_TEST_PATH = os.path.join(HERE, "test_hip_quant")

# enum mlq_type (numeric values follow the reference QuantType order)
F32, Q8_0, Q4_0, Q4_1 = 0, 1, 2, 3
TYPES = {"q8_0": Q8_0, "q4_0": Q4_0, "q4_1": Q4_1}
LINEAR_TYPES = {"f32": F32, **TYPES}
BLOCK_BYTES = {"q8_0": 34, "q4_0": 18, "q4_1": 20}
ROPE_NORMAL, ROPE_NEOX = 0, 1
# enum mlq_path
PATH_AUTO, PATH_GEMV, PATH_MFMA = 0, 1, 2
EPI_NONE, EPI_SWIGLU = 0, 1
GEMV_MAX_ROWS = 8

STATUS = {
    0: "ok", -1: "invalid argument", -2: "shape mismatch",
    -3: "block count mismatch", -4: "buffer too small",
    -5: "unsupported shape", -6: "no HIP device", -7: "malformed GGUF file",
    -8: "shape needs more than the fixed no-alloc scratch",
    -100: "HIP runtime error",
}


class MLQError(RuntimeError):
    def __init__(self, status: int, what: str, hip_error: int = 0):
        msg = f"{what}: {STATUS.get(status, 'unknown')} ({status})"
        if status == -100:
            msg += f", hipError_t {hip_error}"
        super().__init__(msg)
        self.status = status
        self.hip_error = hip_error


class MlqWeight(ctypes.Structure):
    """struct mlq_weight (include/mlq.h)."""
    _fields_ = [
        ("base", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("n", ctypes.c_int32),
        ("k", ctypes.c_int32),
        ("nb", ctypes.c_int32),
        ("qs_off", ctypes.c_uint64),
        ("d_off", ctypes.c_uint64),
        ("m_off", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
    ]


class MlqGgufTensor(ctypes.Structure):
    """mlq_gguf_tensor (include/mlq.h)."""
    _fields_ = [
        ("name", ctypes.c_char_p),
        ("ggml_type", ctypes.c_uint32),
        ("n_dims", ctypes.c_uint32),
        ("dims", ctypes.c_uint64 * 8),
        ("offset", ctypes.c_uint64),
        ("bytes", ctypes.c_uint64),
    ]


class MlqKvCache(ctypes.Structure):
    """struct mlq_kv_cache (include/mlq.h)."""
    _fields_ = [("keys", ctypes.c_void_p), ("values", ctypes.c_void_p),
                ("n_layers", ctypes.c_int32), ("max_seq_len", ctypes.c_int32),
                ("n_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32)]


class MlqLayer(ctypes.Structure):
    """struct mlq_layer (include/mlq.h)."""
    _fields_ = [("attn_norm", ctypes.c_void_p),
                ("wq", MlqWeight), ("wk", MlqWeight), ("wv", MlqWeight),
                ("bq", ctypes.c_void_p), ("bk", ctypes.c_void_p), ("bv", ctypes.c_void_p),
                ("wo", MlqWeight), ("ffn_norm", ctypes.c_void_p),
                ("w_gate", MlqWeight), ("w_up", MlqWeight), ("w_down", MlqWeight)]


class MlqModel(ctypes.Structure):
    """struct mlq_model (include/mlq.h)."""
    _fields_ = [("vocab_size", ctypes.c_int32), ("dim", ctypes.c_int32),
                ("hidden_dim", ctypes.c_int32), ("n_layers", ctypes.c_int32),
                ("n_heads", ctypes.c_int32), ("n_kv_heads", ctypes.c_int32),
                ("head_dim", ctypes.c_int32), ("max_seq_len", ctypes.c_int32),
                ("rope_theta", ctypes.c_float), ("rms_norm_eps", ctypes.c_float),
                ("rope_type", ctypes.c_int32),
                ("token_embedding", ctypes.c_void_p), ("final_norm", ctypes.c_void_p),
                ("lm_head", MlqWeight), ("layers", ctypes.POINTER(MlqLayer))]


# Every symbol declared in include/mlq.h, with its ctypes signature.
_P, _I, _Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
_WP = ctypes.POINTER(MlqWeight)
_I64, _F = ctypes.c_int64, ctypes.c_float
_KVP = ctypes.POINTER(MlqKvCache)
_MP = ctypes.POINTER(MlqModel)
SIGNATURES = {
    "mlq_status_string": ([_I], ctypes.c_char_p),
    "mlq_last_hip_error": ([], _I),
    "mlq_device_count": ([ctypes.POINTER(_I)], _I),
    "mlq_block_bytes": ([_I], _Z),
    "mlq_weight_layout": ([_I, _I, _I, _WP], _I),
    "mlq_repack_host": ([_I, _P, _Z, _I, _I, _P, _Z], _I),
    "mlq_repack_device": ([_I, _P, _Z, _I, _I, _P, _Z, _P], _I),
    "mlq_dequantize": ([_WP, _I, _I, _P, _P], _I),
    "mlq_quantize_act_q8_0": ([_P, _I, _I, _P, _Z, _P], _I),
    "mlq_linear": ([_WP, _P, _P, _I, _P], _I),
    "mlq_linear_q8act_workspace": ([_WP, _I, ctypes.POINTER(_Z)], _I),
    "mlq_linear_q8act": ([_WP, _P, _P, _I, _P, _Z, _P], _I),
    "mlq_linear_aos": ([_I, _P, _Z, _I, _I, _P, _P, _I, _P, _Z, _P], _I),
    "mlq_linear_aos_workspace": ([_I, _I, _I, _I, _P], _I),
    "mlq_linear_path": ([_WP, _P, _P, _I, _I, _P], _I),
    "mlq_linear_workspace": ([_WP, _I, ctypes.POINTER(_Z)], _I),
    "mlq_linear_ws": ([_WP, _P, _P, _I, _P, _Z, _P], _I),
    "mlq_linear_epi": ([_WP, _P, _P, _I, _P, _I, _P, _Z, _P], _I),
    "mlq_linear_epi_noalloc": ([_WP, _P, _P, _I, _P, _I, _P], _I),
    "mlq_interleave_rows": ([_P, _P, _I, _Z, _P], _I),
    "mlq_gguf_open": ([ctypes.c_char_p, ctypes.POINTER(_P)], _I),
    "mlq_gguf_last_error": ([], ctypes.c_char_p),
    "mlq_gguf_close": ([_P], None),
    "mlq_gguf_tensor_count": ([_P, ctypes.POINTER(ctypes.c_int64)], _I),
    "mlq_gguf_data_offset": ([_P, ctypes.POINTER(ctypes.c_uint64),
                              ctypes.POINTER(ctypes.c_uint64)], _I),
    "mlq_gguf_tensor_info": ([_P, ctypes.c_int64, ctypes.POINTER(MlqGgufTensor)], _I),
    "mlq_gguf_find": ([_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)], _I),
    "mlq_gguf_data": ([_P, ctypes.c_int64], _P),
    "mlq_gguf_upload": ([_P, ctypes.c_int64, _P, _Z, _WP, _P], _I),
    "mlq_add_bias": ([_P, _P, _I, _I, _P], _I),
    "mlq_set_gemv_split": ([_I], _I),
    "mlq_set_gemm_split": ([_I], _I),
    "mlq_set_skinny_plan": ([_I, _I], _I),
    "mlq_rmsnorm": ([_P, _P, _P, _I, _I, _F, _P], _I),
    "mlq_add": ([_P, _P, _P, _I64, _P], _I),
    "mlq_mul": ([_P, _P, _P, _I64, _P], _I),
    "mlq_silu": ([_P, _P, _I64, _P], _I),
    "mlq_swiglu": ([_P, _P, _P, _I64, _P], _I),
    "mlq_softmax": ([_P, _P, _I64, _P], _I),
    "mlq_embedding": ([_P, _I, _I, _I, _P, _P], _I),
    "mlq_rope": ([_P, _P, _I, _I, _I, _I, _F, _I, _P], _I),
    "mlq_kv_cache_bytes": ([_I, _I, _I, _I, ctypes.POINTER(_Z)], _I),
    "mlq_kv_write": ([_KVP, _I, _I, _P, _P, _P], _I),
    "mlq_attention_workspace": ([_KVP, _I, ctypes.POINTER(_Z)], _I),
    "mlq_attention_decode": ([_KVP, _I, _I, _P, _I, _P, _P, _Z, _P], _I),
    "mlq_argmax": ([_P, _I64, _P, _P], _I),
    "mlq_decode_workspace": ([_MP, ctypes.POINTER(_Z)], _I),
    "mlq_decode_token": ([_MP, _KVP, _I, _I, _P, _P, _P, _P, _Z, _P], _I),
    "mlq_prefill_workspace": ([_MP, _I, ctypes.POINTER(_Z)], _I),
    "mlq_prefill": ([_MP, _KVP, _P, _I, _I, _P, _P, _Z, _P], _I),
    "mlq_argmax_workspace": ([_I64, ctypes.POINTER(_Z)], _I),
    "mlq_greedy_next": ([_P, _I, _P, _P, _P, _Z, _P], _I),
}

_LIB = None


def build(quiet: bool = True) -> None:
    """Compile libmlq.so, libmini_llama_hip.so and the C++ test binary for
    gfx950 in place (always recompiles what changed)."""
    cmd = ["make", "-C", HERE, "-j8"]
    subprocess.run(cmd, check=True,
                   stdout=subprocess.DEVNULL if quiet else None)


def lib() -> ctypes.CDLL:
    """The loaded C ABI library. Raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it first (python -c "
                "'import __graft_entry__ as g; g.build()'). There is no CPU "
                "fallback for the HIP path.")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = handle
    return _LIB


def _check(status: int, what: str) -> None:
    if status != 0:
        raise MLQError(status, what, lib().mlq_last_hip_error())


def device_count() -> int:
    c = ctypes.c_int(0)
    lib().mlq_device_count(ctypes.byref(c))
    return c.value


def weight_layout(qtype: str, n: int, k: int) -> MlqWeight:
    w = MlqWeight()
    _check(lib().mlq_weight_layout(LINEAR_TYPES[qtype], n, k, ctypes.byref(w)),
           "mlq_weight_layout")
    return w


def repack_host(qtype: str, blocks: np.ndarray, n: int, k: int):
    """GGUF AoS blocks (numpy structured or raw bytes) -> (tiled image as a
    uint8 numpy array, MlqWeight layout with base unset)."""
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    bb = BLOCK_BYTES[qtype]
    if raw.size % bb:
        raise ValueError("block buffer is not a whole number of blocks")
    w = weight_layout(qtype, n, k)
    out = np.empty(w.bytes, np.uint8)
    _check(lib().mlq_repack_host(TYPES[qtype], raw.ctypes.data, raw.size // bb,
                                 n, k, out.ctypes.data, out.size),
           "mlq_repack_host")
    return out, w


def _stream(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


class TiledWeight:
    """A weight repacked into the tiled layout, resident in device memory
    (the analogue of HipUploadedWeight)."""

    def __init__(self, qtype: str, n: int, k: int, buffer, layout: MlqWeight):
        self.qtype, self.n, self.k = qtype, n, k
        self.buffer = buffer  # torch uint8 device tensor owning the memory
        self.layout = layout
        self.layout.base = buffer.data_ptr()

    @property
    def nbytes(self) -> int:
        return int(self.layout.bytes)

    @property
    def gguf_bytes(self) -> int:
        """Size of the same weight as GGUF blocks (the algorithmic bytes)."""
        if self.qtype == "f32":
            return 4 * self.n * self.k
        return self.n * ((self.k + 31) // 32) * BLOCK_BYTES[self.qtype]


def upload(qtype: str, blocks: np.ndarray, n: int, k: int,
           device: str = "cuda") -> TiledWeight:
    """Host repack + one host-to-device copy (the upload path)."""
    import torch
    image, layout = repack_host(qtype, blocks, n, k)
    buf = torch.from_numpy(image).to(device)
    return TiledWeight(qtype, n, k, buf, layout)


def upload_f32(w: np.ndarray, device: str = "cuda") -> TiledWeight:
    """An fp32 [n, k] Linear weight as is (type MLQ_F32: the mlq_linear
    family runs the fp32 GEMV on it)."""
    import torch
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    layout = weight_layout("f32", n, k)
    buf = torch.from_numpy(w.view(np.uint8).reshape(-1).copy()).to(device)
    return TiledWeight("f32", n, k, buf, layout)


def upload_concat(qtype: str, parts, k: int, device: str = "cuda"):
    """Several weights that share one input (q|k|v, gate|up) as one tiled
    weight: their rows are concatenated, so one launch computes all of them.
    `parts` is a list of (blocks, n). Returns (TiledWeight, row offsets);
    output rows [off[i], off[i+1]) belong to part i."""
    blocks = np.concatenate([np.ascontiguousarray(b).view(np.uint8).reshape(-1)
                             for b, _ in parts])
    ns = [int(n) for _, n in parts]
    offsets = np.concatenate([[0], np.cumsum(ns)]).tolist()
    return upload(qtype, blocks, offsets[-1], k, device=device), offsets


def interleave_rows(gate: np.ndarray, up: np.ndarray, rows: int) -> np.ndarray:
    """Rows of gate and up interleaved per 16-row tile (8 gate rows, then
    the matching 8 up rows) by mlq_interleave_rows; any row format (GGUF
    block rows, fp32 bias entries)."""
    g = np.ascontiguousarray(gate).view(np.uint8).reshape(-1)
    u = np.ascontiguousarray(up).view(np.uint8).reshape(-1)
    if g.size != u.size or g.size % rows:
        raise ValueError("gate and up must hold `rows` rows of equal size")
    out = np.empty(2 * g.size, dtype=np.uint8)
    _check(lib().mlq_interleave_rows(g.ctypes.data, u.ctypes.data, rows,
                                     g.size // rows, out.ctypes.data),
           "mlq_interleave_rows")
    return out.view(np.asarray(gate).dtype)


def upload_glu(qtype: str, gate_blocks, up_blocks, ffn: int, k: int,
               device: str = "cuda") -> TiledWeight:
    """Gate and up projections [ffn, k] as one tiled weight of 2*ffn rows
    for act=EPI_SWIGLU (ffn % 8 == 0): one launch reads x once and writes
    silu(gate) * up."""
    return upload(qtype, interleave_rows(gate_blocks, up_blocks, ffn),
                  2 * ffn, k, device=device)


GGML_TYPES = {0: "f32", 1: "f16", 2: "q4_0", 3: "q4_1", 8: "q8_0"}


class GgufFile:
    """A GGUF v3 file, memory-mapped and validated by mlq_gguf_open.

    `tensors` lists every tensor (name, GGML type, dims in GGUF order —
    dims[0] innermost —, absolute data offset, bytes); `data(name)` returns
    a copy of its bytes; `upload(name)` makes a TiledWeight of a 2-D
    q8_0 / q4_0 / q4_1 tensor straight from the mapping (device copy +
    device repack, no host block vector)."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        st = lib().mlq_gguf_open(os.fsencode(path), ctypes.byref(h))
        if st != 0:
            raise MLQError(st, "mlq_gguf_open: " +
                           lib().mlq_gguf_last_error().decode(errors="replace"), 0)
        self._h = h
        count = ctypes.c_int64()
        _check(lib().mlq_gguf_tensor_count(h, ctypes.byref(count)), "mlq_gguf_tensor_count")
        off, align = ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib().mlq_gguf_data_offset(h, ctypes.byref(off), ctypes.byref(align)),
               "mlq_gguf_data_offset")
        self.data_offset, self.alignment = off.value, align.value
        self.tensors = []
        for i in range(count.value):
            t = MlqGgufTensor()
            _check(lib().mlq_gguf_tensor_info(h, i, ctypes.byref(t)), "mlq_gguf_tensor_info")
            self.tensors.append({"name": t.name.decode(), "type": t.ggml_type,
                                 "dims": [int(t.dims[d]) for d in range(t.n_dims)],
                                 "offset": int(t.offset), "bytes": int(t.bytes)})
        self._index = {t["name"]: i for i, t in enumerate(self.tensors)}

    def close(self):
        if self._h:
            lib().mlq_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def data(self, name: str) -> np.ndarray:
        i = self._index[name]
        n = self.tensors[i]["bytes"]
        ptr = lib().mlq_gguf_data(self._h, i)
        if not ptr:
            return np.empty(0, dtype=np.uint8)
        return np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint8)),
                                     shape=(n,)).copy()

    def upload(self, name: str, device: str = "cuda", stream=None) -> "TiledWeight":
        import torch
        i = self._index[name]
        t = self.tensors[i]
        if t["type"] not in (2, 3, 8) or len(t["dims"]) != 2:
            raise ValueError(f"{name}: not a 2-D q8_0/q4_0/q4_1 tensor")
        qtype = GGML_TYPES[t["type"]]
        k, n = t["dims"]
        layout = weight_layout(qtype, n, k)
        buf = torch.empty(int(layout.bytes), dtype=torch.uint8, device=device)
        aos = torch.empty(t["bytes"], dtype=torch.uint8, device=device)
        layout.base = buf.data_ptr()
        _check(lib().mlq_gguf_upload(self._h, i, aos.data_ptr(), aos.numel(),
                                     ctypes.byref(layout), _stream(stream)),
               "mlq_gguf_upload")
        torch.cuda.current_stream().synchronize() if stream is None else stream.synchronize()
        return TiledWeight(qtype, n, k, buf, layout)


def upload_aos(blocks: np.ndarray, device: str = "cuda"):
    """Raw GGUF blocks to device memory unchanged (what the reference uploads)."""
    import torch
    raw = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
    return torch.from_numpy(raw.copy()).to(device)


def repack_device(qtype: str, aos_dev, n: int, k: int, stream=None) -> TiledWeight:
    """Repack GGUF blocks already in device memory with the device kernel."""
    import torch
    layout = weight_layout(qtype, n, k)
    buf = torch.empty(int(layout.bytes), dtype=torch.uint8, device=aos_dev.device)
    bb = BLOCK_BYTES[qtype]
    _check(lib().mlq_repack_device(TYPES[qtype], aos_dev.data_ptr(),
                                   aos_dev.numel() // bb, n, k, buf.data_ptr(),
                                   buf.numel(), _stream(stream)),
           "mlq_repack_device")
    return TiledWeight(qtype, n, k, buf, layout)


def dequantize(w: TiledWeight, row0: int = 0, rows: int | None = None,
               stream=None):
    """fp32 [rows, k] dequantized values (exact d*q / d*(q-8) / d*q+m)."""
    import torch
    rows = w.n - row0 if rows is None else rows
    out = torch.empty((rows, w.k), dtype=torch.float32, device=w.buffer.device)
    _check(lib().mlq_dequantize(ctypes.byref(w.layout), row0, rows,
                                out.data_ptr(), _stream(stream)),
           "mlq_dequantize")
    return out


def quantize_act_q8_0(x, stream=None):
    """q8_0 blocks (uint8 [rows * ceil(k/32) * 34], GGUF AoS) of fp32 device
    activations x [k] or [rows, k], as quantizeToQ80 (src/quant.cc:130-190)."""
    import torch
    if x.dtype != torch.float32 or not x.is_cuda:
        raise ValueError("quantize_act_q8_0: x must be a float32 device tensor")
    x = x.contiguous()
    k = x.shape[-1]
    rows = x.numel() // k if x.dim() >= 2 else 1
    out = torch.empty(rows * ((k + 31) // 32) * 34, dtype=torch.uint8, device=x.device)
    _check(lib().mlq_quantize_act_q8_0(x.data_ptr(), rows, k, out.data_ptr(), out.numel(),
                                       _stream(stream)),
           "mlq_quantize_act_q8_0")
    return out


def workspace_bytes(w: TiledWeight, m: int) -> int:
    """Device workspace mlq_linear_ws needs for m activation rows."""
    nbytes = ctypes.c_size_t(0)
    _check(lib().mlq_linear_workspace(ctypes.byref(w.layout), m,
                                      ctypes.byref(nbytes)),
           "mlq_linear_workspace")
    return nbytes.value


_WORKSPACES: dict = {}


def _workspace(device, nbytes: int):
    """Grow-only per-device workspace for `linear` (calls on one device share
    it, so they must be ordered on one stream; pass `workspace=` otherwise)."""
    import torch
    key = torch.device(device).index or 0
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = buf
    return buf


def linear(w: TiledWeight, x, y=None, path: int = PATH_AUTO, stream=None,
           workspace="auto", bias=None, act: int = EPI_NONE):
    """y[m, n] = x[m, k] @ W^T on the device (x fp32 contiguous, 1-D or 2-D).

    path AUTO with a workspace (the default "auto" takes the per-device one)
    runs mlq_linear_epi: optional fused bias (fp32 device tensor [n]) and
    act=EPI_SWIGLU for a weight made by upload_glu (y then has n/2
    columns). workspace=None, or a forced path, runs mlq_linear_path (no
    epilogue; the prefill GEMM then reads fp32 x directly)."""
    import torch
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("x must be a contiguous float32 device tensor")
    m = 1 if x.dim() == 1 else x.shape[0]
    kx = x.shape[-1]
    if kx != w.k:
        raise ValueError(f"in_features mismatch: x has {kx}, weight has {w.k}")
    fused = bias is not None or act != EPI_NONE
    if fused and (path != PATH_AUTO or workspace is None):
        raise ValueError("bias / act need the default path with a workspace")
    if bias is not None and (bias.dtype != torch.float32 or bias.numel() != w.n):
        raise ValueError(f"bias must be float32 with {w.n} elements")
    ny = w.n // 2 if act == EPI_SWIGLU else w.n
    if y is None:
        shape = (ny,) if x.dim() == 1 else (m, ny)
        y = torch.empty(shape, dtype=torch.float32, device=x.device)
    if path == PATH_AUTO and workspace is not None:
        need = workspace_bytes(w, m)
        ws = workspace
        if isinstance(workspace, str):
            ws = _workspace(x.device, need) if need else None
        ws_ptr = ws.data_ptr() if ws is not None else None
        ws_len = ws.numel() * ws.element_size() if ws is not None else 0
        _check(lib().mlq_linear_epi(ctypes.byref(w.layout), x.data_ptr(),
                                    y.data_ptr(), m,
                                    bias.data_ptr() if bias is not None else None,
                                    act, ws_ptr, ws_len, _stream(stream)),
               "mlq_linear_epi")
        return y
    _check(lib().mlq_linear_path(ctypes.byref(w.layout), x.data_ptr(),
                                 y.data_ptr(), m, path, _stream(stream)),
           "mlq_linear")
    return y


def workspace_bytes_q8act(w: TiledWeight, m: int) -> int:
    """Device workspace mlq_linear_q8act needs for m activation rows."""
    nbytes = ctypes.c_size_t(0)
    _check(lib().mlq_linear_q8act_workspace(ctypes.byref(w.layout), m, ctypes.byref(nbytes)),
           "mlq_linear_q8act_workspace")
    return nbytes.value


def linear_q8act(w: TiledWeight, x, y=None, stream=None, workspace=None):
    """mlq_linear_q8act: the int8-MFMA variant for q8_0 weights (x quantized
    to q8_0 blocks first, then an int8 contraction with per-block scales).
    workspace: a uint8 device tensor of at least workspace_bytes_q8act bytes,
    or None for the per-device grow-only one."""
    import torch
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("x must be a contiguous float32 device tensor")
    m = 1 if x.dim() == 1 else x.shape[0]
    if x.shape[-1] != w.k:
        raise ValueError(f"in_features mismatch: x has {x.shape[-1]}, weight has {w.k}")
    need = workspace_bytes_q8act(w, m)
    ws = workspace if workspace is not None else _workspace(x.device, need)
    if y is None:
        y = torch.empty((w.n,) if x.dim() == 1 else (m, w.n), dtype=torch.float32,
                        device=x.device)
    _check(lib().mlq_linear_q8act(ctypes.byref(w.layout), x.data_ptr(), y.data_ptr(), m,
                                  ws.data_ptr(), ws.numel() * ws.element_size(),
                                  _stream(stream)),
           "mlq_linear_q8act")
    return y


def linear_noalloc(w: TiledWeight, x, y=None, bias=None, act: int = EPI_NONE,
                   stream=None):
    """mlq_linear_epi_noalloc: linear() with the library's fixed per-GPU
    scratch instead of a workspace (no allocation inside the call)."""
    import torch
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("x must be a contiguous float32 device tensor")
    m = 1 if x.dim() == 1 else x.shape[0]
    if x.shape[-1] != w.k:
        raise ValueError(f"in_features mismatch: x has {x.shape[-1]}, weight has {w.k}")
    ny = w.n // 2 if act == EPI_SWIGLU else w.n
    if y is None:
        shape = (ny,) if x.dim() == 1 else (m, ny)
        y = torch.empty(shape, dtype=torch.float32, device=x.device)
    _check(lib().mlq_linear_epi_noalloc(ctypes.byref(w.layout), x.data_ptr(), y.data_ptr(), m,
                                        bias.data_ptr() if bias is not None else None,
                                        act, _stream(stream)),
           "mlq_linear_epi_noalloc")
    return y


def aos_workspace_bytes(qtype: str, n: int, k: int, m: int) -> int:
    """mlq_linear_aos_workspace: 0 when the direct AoS GEMV takes the shape."""
    nbytes = ctypes.c_size_t(0)
    _check(lib().mlq_linear_aos_workspace(TYPES[qtype], n, k, m, ctypes.byref(nbytes)),
           "mlq_linear_aos_workspace")
    return nbytes.value


def linear_aos(qtype: str, aos_dev, n: int, k: int, x, workspace=None,
               stream=None):
    """Linear on raw GGUF blocks in device memory: up to 8 rows read the
    blocks as they are, otherwise they are repacked into a workspace."""
    import torch
    m = 1 if x.dim() == 1 else x.shape[0]
    need = aos_workspace_bytes(qtype, n, k, m)
    if workspace is None and need:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    y = torch.empty((n,) if x.dim() == 1 else (m, n), dtype=torch.float32,
                    device=x.device)
    bb = BLOCK_BYTES[qtype]
    _check(lib().mlq_linear_aos(TYPES[qtype], aos_dev.data_ptr(),
                                aos_dev.numel() // bb, n, k, x.data_ptr(),
                                y.data_ptr(), m,
                                workspace.data_ptr() if workspace is not None else None,
                                workspace.numel() if workspace is not None else 0,
                                _stream(stream)),
           "mlq_linear_aos")
    return y


def set_gemv_split(split: int = 0) -> None:
    """Override the GEMV K split (waves per tile; 0 = automatic)."""
    _check(lib().mlq_set_gemv_split(split), "mlq_set_gemv_split")


def set_gemm_split(split: int = 0) -> None:
    """Override the prefill GEMM split-K (workgroups per output tile, each a
    K range; 0 = planner). Workspaces sized before the change may be too
    small afterwards: `linear` with workspace="auto" re-queries the size."""
    _check(lib().mlq_set_gemm_split(split), "mlq_set_gemm_split")


def set_skinny_plan(tiles: int = 0, splits: int = 0) -> None:
    """Override the skinny GEMM's weight tiles per workgroup (1, 2, 4) and K
    ranges per tile group (1..8); 0 = planner. The workspace size may change
    with it."""
    _check(lib().mlq_set_skinny_plan(tiles, splits), "mlq_set_skinny_plan")


def add_bias(y, bias, stream=None):
    m = 1 if y.dim() == 1 else y.shape[0]
    _check(lib().mlq_add_bias(y.data_ptr(), bias.data_ptr(), m, y.shape[-1],
                              _stream(stream)), "mlq_add_bias")
    return y
