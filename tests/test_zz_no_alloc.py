"""GPU: mlq_linear_epi_noalloc (fixed per-GPU scratch, no allocation) gives
the same outputs as mlq_linear_epi with a caller workspace, through the C
ABI, on two calls in a row (the second smaller, so it runs on scratch the
first one left behind), for the skinny and the prefill GEMM paths (the
ones with scratch), with and without the fused epilogues; shapes beyond the
scratch are rejected with MLQ_ERR_SCRATCH_LIMIT before any launch."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import make_blocks, make_x

pytestmark = pytest.mark.gpu

# (qtype, n, k, m_first, m_second): the first call's shape needs more
# scratch than the second's; m > 64 takes the prefill GEMM (split K for the
# few-tile shapes), 9..64 the skinny GEMM, <= 8 the GEMV (no scratch).
CASES = [
    ("q4_0", 4096, 4096, 64, 16),
    ("q8_0", 4096, 4096, 512, 96),
    ("q4_1", 1024, 14336, 300, 40),
    ("q4_0", 3584, 18944, 128, 3),
]


def _dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


@pytest.mark.parametrize("qtype,n,k,m1,m2", CASES)
def test_noalloc_matches_workspace_entry_point(pkg, cuda, qtype, n, k, m1, m2):
    blocks = make_blocks(qtype, n, k, seed=n + k)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    bias = _dev(np.random.default_rng(5).standard_normal(n).astype(np.float32), cuda)
    for m in (m1, m2):
        print(f"noalloc {qtype} n={n} k={k} m={m}", flush=True)
        xd = _dev(make_x(m, k, seed=m), cuda)
        for b, act in ((None, pkg.EPI_NONE), (bias, pkg.EPI_NONE)):
            ws = torch.empty(max(pkg.workspace_bytes(tw, m), 256), dtype=torch.uint8,
                             device=cuda)
            want = pkg.linear(tw, xd, workspace=ws, bias=b, act=act)
            got = pkg.linear_noalloc(tw, xd, bias=b, act=act)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (qtype, n, k, m, b is not None)


def test_noalloc_swiglu_matches(pkg, cuda):
    n, k = 2048, 4096
    gate = make_blocks("q4_0", n // 2, k, seed=1)
    up = make_blocks("q4_0", n // 2, k, seed=2)
    tw = pkg.upload_glu("q4_0", gate, up, n // 2, k, device=cuda)
    for m in (200, 20):
        xd = _dev(make_x(m, k, seed=m), cuda)
        ws = torch.empty(max(pkg.workspace_bytes(tw, m), 256), dtype=torch.uint8, device=cuda)
        want = pkg.linear(tw, xd, workspace=ws, act=pkg.EPI_SWIGLU)
        got = pkg.linear_noalloc(tw, xd, act=pkg.EPI_SWIGLU)
        torch.cuda.synchronize()
        assert torch.equal(got, want), m


def test_noalloc_rejects_shapes_beyond_scratch(pkg, cuda):
    # fp16 copy of x alone: 8192 x 8192 x 2 B = 128 MiB > 64 MiB
    n, k, m = 256, 8192, 8192
    lay = pkg.weight_layout("q4_0", n, k)
    buf = torch.zeros(lay.bytes, dtype=torch.uint8, device=cuda)
    lay.base = buf.data_ptr()
    need = ctypes.c_size_t(0)
    assert pkg.lib().mlq_linear_workspace(ctypes.byref(lay), m, ctypes.byref(need)) == 0
    assert need.value > (64 << 20)
    x = torch.zeros((m, k), dtype=torch.float32, device=cuda)
    y = torch.empty((m, n), dtype=torch.float32, device=cuda)
    rc = pkg.lib().mlq_linear_epi_noalloc(ctypes.byref(lay), x.data_ptr(), y.data_ptr(), m,
                                          None, pkg.EPI_NONE, None)
    assert rc == -8
    assert pkg.lib().mlq_status_string(rc) == b"shape needs more than the fixed no-alloc scratch"
