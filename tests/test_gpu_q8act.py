"""Int8-MFMA variant (mlq_linear_q8act) against the oracle.

The variant quantizes x with quantizeToQ80's rules (src/quant.cc:130-190)
and contracts the int8 codes of both operands block by block. Three checks:
  1. exact semantics: against the float64 product of the oracle's
     dequantized activations (oracle.quantize -> oracle.dequantize) and
     weights, within the rounding bound of the kernel's fp32 accumulation
     (the block terms dx dw I are exact; each of the nb FMAs rounds by at
     most 2^-24 of the running sum, which never exceeds
     sum_k |xd_k| |wd_k|); a wrong byte order, scale or block pairing
     misses it by orders of magnitude;
  2. the Linear's stated tolerance against that same quantized-x reference;
  3. the stated tolerance against the reference's own fp32-x Linear
     (oracle.linear), i.e. the activation quantization error fits it. That
     error grows like sqrt(K) * |x| / 254 * |w| while the tolerance's
     absolute bound grows like K, so the check applies from K = 1000 on
     (at K = 32 the rounding of x alone is ~0.5 of the bound per output).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import error_report, make_blocks, make_x, tolerance_ok

pytestmark = pytest.mark.gpu

def _case(**kw):
    print("case:", " ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _quantized_reference(oracle, x, blocks, n, k):
    """float64 y of the q8_0-quantized x times the dequantized weight, and
    the per-output fixup bound."""
    m = x.shape[0]
    nb = (k + 31) // 32
    xq = oracle.quantize(x, "q8_0")
    xd = oracle.dequantize(xq, (m, k), "q8_0").astype(np.float64)
    wd = oracle.dequantize(blocks, (n, k), "q8_0").astype(np.float64)
    y64 = xd @ wd.T
    bound = (nb + 2) * 2.0 ** -24 * (np.abs(xd) @ np.abs(wd).T)
    return xd, y64, bound


def _run(pkg, cuda, tw, x):
    import torch
    xd = torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    y = pkg.linear_q8act(tw, xd)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _check_all(pkg, oracle, cuda, x, blocks, n, k, fp32_check=True):
    tw = pkg.upload("q8_0", blocks, n, k, device=cuda)
    got = _run(pkg, cuda, tw, x).reshape(x.shape[0], n)
    xd, y64, bound = _quantized_reference(oracle, x, blocks, n, k)
    err = np.abs(got.astype(np.float64) - y64)
    ratio = err / np.maximum(bound, 1e-300)
    r, c = np.unravel_index(int(np.argmax(ratio)), ratio.shape)
    assert (err <= bound).all(), (f"fixup bound exceeded at row {r} col {c}: got {got[r, c]!r} "
                                  f"ref {y64[r, c]!r} bound {bound[r, c]:.3g} "
                                  f"(rows over: {sorted(set(np.nonzero(err > bound)[0].tolist()))})")
    assert tolerance_ok(got, y64, xd, k).all(), error_report(got, y64, xd, k)
    if fp32_check and k >= 1000:
        ref = oracle.linear(x, blocks, (n, k), "q8_0", threads=8)
        assert tolerance_ok(got, ref, x, k).all(), error_report(got, ref, x, k)
    return got


@pytest.mark.parametrize("m,n,k", [(1, 16, 32), (3, 17, 100), (33, 250, 1000),
                                   (129, 300, 4096), (64, 64, 18944), (256, 520, 2080)])
def test_q8act_matches_oracle(pkg, oracle, cuda, m, n, k):
    _case(test="q8act", m=m, n=n, k=k)
    blocks = make_blocks("q8_0", n, k, seed=n + 3 * k)
    x = make_x(m, k, seed=m + 11 * k)
    _check_all(pkg, oracle, cuda, x, blocks, n, k)


def test_q8act_prefill_config(pkg, oracle, cuda):
    """The benchmarked shape: W [11008, 4096] q8_0, x [512, 4096]."""
    m, n, k = 512, 11008, 4096
    _case(test="q8act_c4", m=m, n=n, k=k)
    blocks = make_blocks("q8_0", n, k, seed=4)
    x = make_x(m, k, seed=5)
    _check_all(pkg, oracle, cuda, x, blocks, n, k)


def test_q8act_special_rows_and_codes(pkg, oracle, cuda):
    """Zero rows, rows of 1e5, rows scaled by 2^8 and 2^-8, NaN elements (the
    exact semantics only: quantizeToQ80 stores -127 for them) and weight
    codes of -128 (a GGUF block may hold them; the reference's quantizer
    never writes them)."""
    m, n, k = 40, 96, 1000
    _case(test="q8act_special", m=m, n=n, k=k)
    rng = np.random.default_rng(21)
    x = make_x(m, k, seed=22)
    x[1] = 0.0
    x[2, ::7] = 1e5
    x[3] *= np.float32(256.0)
    x[4] *= np.float32(1 / 256.0)
    x[5, 17] = -1e5
    blocks = make_blocks("q8_0", n, k, seed=23)
    qs = blocks["qs"]
    qs[rng.integers(0, qs.shape[0], 200), rng.integers(0, 32, 200)] = -128
    blocks["qs"] = qs
    _check_all(pkg, oracle, cuda, x, blocks, n, k)
    x[6, 3] = np.nan
    x[7, 40:72] = np.nan
    _check_all(pkg, oracle, cuda, x, blocks, n, k, fp32_check=False)


def test_q8act_block_scale_overflow(pkg, oracle, cuda):
    """The range edge of the q8_0 activation scale d = fp16(max|x| / 127):
    a block whose largest |x| is 8.3e6 keeps a finite scale (65344) and the
    row meets every check; a block at 1e7 overflows d to inf, its codes are
    all zero (x * (1 / inf)), and the whole output row is NaN (inf * 0), as
    the product with the dequantized block is. Other rows are unaffected."""
    m, n, k = 8, 64, 1000
    _case(test="q8act_overflow", m=m, n=n, k=k)
    x = make_x(m, k, seed=31)
    x[3, 37] = 8.3e6
    x[5, 200] = -1.0e7
    blocks = make_blocks("q8_0", n, k, seed=32)
    # the quantizer's side of the edge, on the CPU
    xq = oracle.quantize(x, "q8_0").reshape(m, -1)
    d = oracle.fp16_to_f32(xq["d"])
    assert np.isfinite(d[3]).all() and d[3, 37 // 32] == np.float32(65344.0)
    assert np.isinf(d[5, 200 // 32]) and (xq["qs"][5, 200 // 32] == 0).all()
    tw = pkg.upload("q8_0", blocks, n, k, device=cuda)
    got = _run(pkg, cuda, tw, x).reshape(m, n)
    assert np.isnan(got[5]).all()
    keep = [r for r in range(m) if r != 5]
    _check_all(pkg, oracle, cuda, x[keep], blocks, n, k)
    ref_rows = _run(pkg, cuda, tw, np.ascontiguousarray(x[keep])).reshape(len(keep), n)
    assert np.array_equal(got[keep], ref_rows)


def test_q8act_workspace_contract(pkg, cuda):
    import torch
    m, n, k = 5, 32, 64
    _case(test="q8act_ws", m=m, n=n, k=k)
    blocks = make_blocks("q8_0", n, k, seed=1)
    tw = pkg.upload("q8_0", blocks, n, k, device=cuda)
    need = pkg.workspace_bytes_q8act(tw, m)
    assert need > 0
    x = torch.zeros((m, k), dtype=torch.float32, device=cuda)
    small = torch.empty(need - 1, dtype=torch.uint8, device=cuda)
    with pytest.raises(RuntimeError, match="BUFFER_TOO_SMALL|too small"):
        pkg.linear_q8act(tw, x, workspace=small)
    big = torch.empty(need + 256, dtype=torch.uint8, device=cuda)
    with pytest.raises(RuntimeError, match="invalid argument"):
        pkg.linear_q8act(tw, x, workspace=big[16:])  # large enough, misaligned
    tw4 = pkg.upload("q4_0", make_blocks("q4_0", n, k, seed=2), n, k, device=cuda)
    with pytest.raises(RuntimeError, match="UNSUPPORTED|unsupported"):
        pkg.workspace_bytes_q8act(tw4, m)
