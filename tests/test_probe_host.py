"""The bench-only read probes (libmlq_probe.so, mini-llama_amd/probe): they
load, and their entry points reject bad arguments before any device work.
They are measurement aids outside the product C ABI (include/mlq.h)."""
import ctypes
import importlib

import pytest


@pytest.fixture(scope="module")
def probe(pkg):
    return importlib.import_module("mini_llama_amd.probe")


def test_probe_library_is_separate(pkg, probe):
    """libmlq.so no longer exports the probes; libmlq_probe.so does."""
    lib = ctypes.CDLL(pkg.LIB_PATH)
    for name in ("mlq_read_probe", "mlq_read_probe_shared", "mlq_probe_read",
                 "mlq_probe_read_shared"):
        assert not hasattr(lib, name), name
    plib = probe.lib()
    for name in probe.SIGNATURES:
        assert hasattr(plib, name), name


def test_read_probe_validation_without_device(probe):
    """mlq_probe_read checks its arguments before any device work: NULL
    pointers, sizes that are zero or not a multiple of 16, misaligned
    pointers."""
    lib = probe.lib()
    assert lib.mlq_probe_read(None, 64, 256, None) == -1
    assert lib.mlq_probe_read(256, 64, None, None) == -1
    assert lib.mlq_probe_read(256, 0, 256, None) == -2
    assert lib.mlq_probe_read(256, 40, 256, None) == -2
    assert lib.mlq_probe_read(264, 64, 256, None) == -2


def test_read_probe_shared_validation_without_device(probe):
    """mlq_probe_read_shared accepts 0/64/128/256 KiB shared regions and at
    most 8 KiB per wave, 16-byte aligned, and only when `own` holds
    workgroups * 8 * own_per_wave bytes, before touching a device."""
    lib = probe.lib()
    own = 256 * 8 * 4608
    ok = (256, 128 << 10, 512, own, 4608, 256, 1024, None)
    assert lib.mlq_probe_read_shared(None, *ok[1:]) == -1
    assert lib.mlq_probe_read_shared(*ok[:2], None, *ok[3:]) == -1
    assert lib.mlq_probe_read_shared(*ok[:6], None, None) == -1
    for sb in (100, 96 << 10, 512 << 10):
        assert lib.mlq_probe_read_shared(256, sb, 512, own, 4608, 256, 1024, None) == -2
    assert lib.mlq_probe_read_shared(256, 0, 512, own, 0, 256, 1024, None) == -2
    assert lib.mlq_probe_read_shared(256, 0, 512, 1 << 30, 8 * 1024 + 16, 256, 1024, None) == -2
    assert lib.mlq_probe_read_shared(256, 0, 512, own, 40 + 1, 256, 1024, None) == -2
    assert lib.mlq_probe_read_shared(256, 0, 512, own, 4608, 0, 1024, None) == -2
    assert lib.mlq_probe_read_shared(264, 64 << 10, 512, own, 4608, 1, 1024, None) == -2
    # the per-wave ranges of 256 workgroups x 8 waves need 256 * 8 * 4608
    # bytes of `own`: one byte less is rejected
    assert lib.mlq_probe_read_shared(256, 0, 512, own - 1, 4608, 256, 1024, None) == -2
