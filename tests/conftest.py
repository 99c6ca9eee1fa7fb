"""Shared pytest setup: the `gpu` marker, package/oracle loaders, seeded
synthetic inputs and the parity tolerance.

Tolerance (from the north-star statement): an output passes when
|y - y_ref| <= 1e-3 * ||x_row|| * sqrt(K) / sqrt(4096)  OR  <= 2e-3 * |y_ref|
(allclose-style: absolute OR relative). Tests that mirror the reference's
own CUDA tests additionally use its absolute 1e-4 / 1e-5 bounds.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__ as graft  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


@pytest.fixture(scope="session")
def oracle():
    return graft.load_oracle()


@pytest.fixture(scope="session")
def pkg():
    return graft.load_package()


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible HIP device")
    return torch.device("cuda:0")


def make_blocks(qtype: str, n: int, k: int, seed: int) -> np.ndarray:
    """Seeded synthetic GGUF blocks (tests/synthetic/synth.py distributions)."""
    graft.load_package()
    from synthetic import synth
    return synth.make_blocks(qtype, n, k, seed)


def make_x(m: int, k: int, seed: int) -> np.ndarray:
    graft.load_package()
    from synthetic import synth
    return synth.make_x(m, k, seed)


def tolerance_ok(y, ref, x2d, k):
    """Boolean mask of outputs inside the stated tolerance."""
    y = np.atleast_2d(y)
    ref = np.atleast_2d(ref)
    x2d = np.atleast_2d(x2d)
    # (the norm in float64: rows near the fp32 limit must not make it inf)
    atol = 1e-3 * np.linalg.norm(x2d.astype(np.float64), axis=1, keepdims=True) * np.sqrt(k / 4096)
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    return (err <= atol) | (err <= 2e-3 * np.abs(ref))


def error_report(y, ref, x2d, k):
    y = np.atleast_2d(y).astype(np.float64)
    ref = np.atleast_2d(ref).astype(np.float64)
    x2d = np.atleast_2d(x2d)
    atol = 1e-3 * np.linalg.norm(x2d.astype(np.float64), axis=1, keepdims=True) * np.sqrt(k / 4096)
    err = np.abs(y - ref)
    rel = err / np.maximum(np.abs(ref), 1e-30)
    return {"max_abs_over_atol": float((err / atol).max()),
            "max_rel": float(rel.max()), "max_abs": float(err.max())}
