"""Bench-only read probes (libmlq_probe.so, built beside libmlq.so): the
single-launch HBM read ceiling and the skinny GEMM's load pattern without
its arithmetic. Measurement aids for bench.py and the probe tests; not part
of the product library or its C ABI."""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(HERE), "libmlq_probe.so")

_P, _I, _Z = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
SIGNATURES = {
    "mlq_probe_read": ([_P, _Z, _P, _P], _I),
    "mlq_probe_read_shared": ([_P, _Z, _P, _Z, _Z, _I, _P, _P], _I),
}
_LIB = None


class ProbeError(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it first (make -C mini-llama_amd)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = handle
    return _LIB


def _stream(stream=None) -> int:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _check(status: int, what: str) -> None:
    if status != 0:
        raise ProbeError(f"{what}: status {status}")


def read(buf, nbytes: int, sink, stream=None) -> None:
    """One streaming read of the first nbytes of a device tensor."""
    _check(lib().mlq_probe_read(buf.data_ptr(), nbytes, sink.data_ptr(), _stream(stream)),
           "mlq_probe_read")


def read_shared(shared, shared_bytes: int, own, own_per_wave: int, workgroups: int,
                sink, stream=None) -> None:
    """The skinny GEMM's loads without its math; `own` is a device tensor of
    at least workgroups * 8 * own_per_wave bytes."""
    own_bytes = own.numel() * own.element_size()
    _check(lib().mlq_probe_read_shared(shared.data_ptr(), shared_bytes, own.data_ptr(),
                                       own_bytes, own_per_wave, workgroups, sink.data_ptr(),
                                       _stream(stream)),
           "mlq_probe_read_shared")
