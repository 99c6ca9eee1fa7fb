"""GPU: the quantized Linear accepts any finite fp32 activation, as the
reference's fp32 CPU loop does (src/quant.cc:459-469): every kernel path
carries a row's activations scaled by a power of two chosen from the
row's largest magnitude (integer digits in the one-row GEMV, fp16 hi/lo
pairs in the several-row GEMV, one fp16 rounding in the skinny and prefill
GEMMs), and scales the fp32 results back.

Checked at the BASELINE shapes (c0-c4) on every path: the decode GEMV (one
and several activation rows), the skinny GEMM with and without split K, the
prefill GEMM from the fp16 copy with and without split K, and the GEMM
reading fp32 x directly (no workspace):
  - scaling x by a power of two scales y exactly (the row exponent moves,
    nothing else: a size-independent property, checked on every output):
    y(x * 2^k) = y(x) * 2^k for k in {-24, -16, -8, 8} on the GEMMs, whose
    fp16 copy is always scaled, and on the one-row GEMV at c0-c2, whose
    integer digits always take the slice's exponent; the several-row GEMV
    keeps scale 1 for rows whose largest |x| lies in [2^-10, 2^15), so
    there the relation is checked between scalings outside that window
    (2^-24 vs 2^-16, 2^20 vs 2^28);
  - the scaled results and rows holding +-1e5 meet the oracle within the
    stated tolerance (|dy| <= 1e-3 ||x_row|| sqrt(K / 4096) or 2e-3 |y_ref|);
  - no output is NaN or inf (before, |x| >= 65520 turned whole rows NaN)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import error_report, make_blocks, make_x, tolerance_ok

pytestmark = pytest.mark.gpu

SCALES = [-24, -16, -8, 8]

# (name, qtype, m, n, k, path, gemm_split, skinny_splits)
CASES = [
    ("c0 gemv", "q8_0", 1, 4096, 4096, "auto", 0, 0),
    ("c1 gemv", "q4_0", 1, 18944, 3584, "auto", 0, 0),
    ("c2 gemv", "q4_1", 1, 4096, 14336, "auto", 0, 0),
    ("c3 gemv m4", "q4_0", 4, 4096, 4096, "auto", 0, 0),
    ("c3 skinny m16", "q4_0", 16, 4096, 4096, "auto", 0, 0),
    ("c3 skinny m64", "q4_0", 64, 4096, 4096, "auto", 0, 0),
    ("c3 skinny split", "q4_0", 16, 4096, 4096, "auto", 0, 4),
    ("skinny q4_1 split", "q4_1", 40, 1024, 14336, "auto", 0, 3),
    ("skinny q8_0", "q8_0", 33, 2048, 4096, "auto", 0, 0),
    ("c4 gemm", "q8_0", 512, 11008, 4096, "auto", 0, 0),
    ("c4 gemm split", "q8_0", 512, 11008, 4096, "auto", 3, 0),
    ("gemm q4_1", "q4_1", 200, 1024, 2080, "auto", 0, 0),
    ("c4 gemm fp32 x", "q8_0", 512, 11008, 4096, "mfma", 0, 0),
    ("gemm fp32 x ragged k", "q4_0", 70, 520, 1001, "mfma", 0, 0),
]
REF_ROWS = 6  # rows checked against the oracle when m is large


def _dev(a, cuda):
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _run(pkg, tw, xd, path):
    if path == "mfma":
        return pkg.linear(tw, xd, path=pkg.PATH_MFMA, workspace=None).cpu().numpy()
    return pkg.linear(tw, xd).cpu().numpy()


def _rows(m):
    return np.arange(m) if m <= 16 else np.unique(np.linspace(0, m - 1, REF_ROWS).astype(int))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_any_finite_activation_range(pkg, oracle, cuda, case):
    name, qtype, m, n, k, path, gsplit, ssplits = case
    print(f"range {name}: {qtype} m={m} n={n} k={k} path={path}", flush=True)
    blocks = make_blocks(qtype, n, k, seed=n + 3 * k + m)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    base = make_x(m, k, seed=k + m)
    rows = _rows(m)
    pkg.set_gemm_split(gsplit)
    pkg.set_skinny_plan(0, ssplits)
    try:
        def at(e):
            x = (base * np.float32(2.0 ** e)).astype(np.float32)
            return x, np.atleast_2d(_run(pkg, tw, _dev(x if m > 1 else x[0], cuda), path))

        def exact(ya, yb, e):  # ya == yb * 2^e, bit for bit
            want = (yb.astype(np.float64) * 2.0 ** e).astype(np.float32)
            assert np.array_equal(ya, want), (name, e, np.abs(ya - want).max())

        _, y0 = at(0)
        assert np.isfinite(y0).all()
        ys = {}
        for e in SCALES + [20, 28]:
            x, y = at(e)
            ys[e] = y
            ref = oracle.linear(x[rows], blocks, (n, k), qtype, threads=8)
            ok = tolerance_ok(y[rows], ref, x[rows], k)
            assert ok.all(), (name, e, error_report(y[rows], ref, x[rows], k))
        if path == "auto" and m <= pkg.GEMV_MAX_ROWS:  # the decode GEMV
            exact(ys[-24], ys[-16], -8)
            exact(ys[28], ys[20], 8)
            if m == 1:  # integer digits: the exponent follows every scaling
                for e in SCALES:
                    exact(ys[e], y0, e)
        else:
            for e in SCALES:
                exact(ys[e], y0, e)
        # rows holding +-1e5 among N(0,1) values (fp16 overflows at 65520)
        x = base.copy()
        rng = np.random.default_rng(k)
        for r in range(m):
            idx = rng.choice(k, size=3, replace=False)
            x[r, idx] = np.array([1e5, -1e5, 7e4], np.float32)
        y = np.atleast_2d(_run(pkg, tw, _dev(x if m > 1 else x[0], cuda), path))
        assert np.isfinite(y).all(), name
        ref = oracle.linear(x[rows], blocks, (n, k), qtype, threads=8)
        assert tolerance_ok(y[rows], ref, x[rows], k).all(), (name, error_report(y[rows], ref, x[rows], k))
        # a row spanning the fp32 range: tiny values beside a huge one
        x = base.copy()
        x[0] *= np.float32(1e-30)
        x[0, 5] = np.float32(3e37)
        y = np.atleast_2d(_run(pkg, tw, _dev(x if m > 1 else x[0], cuda), path))
        ref = oracle.linear(x[:1], blocks, (n, k), qtype, threads=8)
        assert np.isfinite(y[0]).all()
        assert tolerance_ok(y[:1], ref, x[:1], k).all(), (name, error_report(y[:1], ref, x[:1], k))
    finally:
        pkg.set_gemm_split(0)
        pkg.set_skinny_plan(0, 0)


@pytest.mark.parametrize("qtype", ["q8_0", "q4_0", "q4_1"])
def test_rmsnorm_folded_gemv_range(pkg, oracle, cuda, qtype):
    """The decode step's GEMV with the input RMSNorm folded in: norm weights
    of 1e5 (normalised activations past the fp16 range) and of 1e-7."""
    import mini_llama_amd.decode as dec
    from synthetic import synth
    cfg = dict(vocab_size=96, dim=256, hidden_dim=512, n_layers=1, n_heads=4, n_kv_heads=2,
               max_seq_len=16)
    for scale in (1e5, 1e-7):
        print(f"range rmsnorm-gemv {qtype} norm x{scale}", flush=True)
        model = synth.synthetic_model(cfg, qtype, seed=11)
        for lw in model["layers"]:
            lw["attention_norm"] = (np.asarray(lw["attention_norm"]) * scale).astype(np.float32)
            lw["ffn_norm"] = (np.asarray(lw["ffn_norm"]) * scale).astype(np.float32)
        dm = dec.DecodeModel(model)
        cache = oracle.new_cache(model)
        for pos, t in enumerate([3, 17, 40]):
            ref = oracle.forward_token(model, cache, t, pos)
            got = dm.forward_token(t, pos).cpu().numpy()
            assert np.isfinite(got).all(), (scale, pos)
            err = np.abs(got - ref).max()
            assert err <= 1e-4 * np.abs(ref).max() + 1e-6, (scale, pos, err)


@pytest.mark.parametrize("qtype", ["q8_0", "q4_0", "q4_1"])
def test_one_row_gemv_tiny_and_non_finite(pkg, oracle, cuda, qtype):
    """One-row GEMV (integer-digit staging) at the ends of the fp32 range:
    a row whose largest |x| lies below 2^-104 (its slice exponent would
    exceed 126, so the values gain 2^64 first) scales exactly against the
    same row at 2^-100 and meets the oracle; a NaN or an inf anywhere in
    the row makes every output non-finite (the reference's fp32 loop
    propagates them the same way), and a finite row after it is unharmed."""
    n, k = 300, 4096
    print(f"range one-row {qtype}", flush=True)
    blocks = make_blocks(qtype, n, k, seed=k + 7)
    tw = pkg.upload(qtype, blocks, n, k, device=cuda)
    base = make_x(1, k, seed=k + 8)[0]

    def run(x):
        return pkg.linear(tw, _dev(x.astype(np.float32), cuda)).cpu().numpy()

    x_tiny = (base * np.float32(2.0 ** -120)).astype(np.float32)
    x_mid = (base * np.float32(2.0 ** -100)).astype(np.float32)
    y_tiny, y_mid = run(x_tiny), run(x_mid)
    want = (y_mid.astype(np.float64) * 2.0 ** -20).astype(np.float32)
    assert np.array_equal(y_tiny, want), np.abs(y_tiny - want).max()
    ref = oracle.linear(x_tiny[None], blocks, (n, k), qtype, threads=8)
    assert tolerance_ok(y_tiny[None], ref, x_tiny[None], k).all(), \
        error_report(y_tiny[None], ref, x_tiny[None], k)
    for bad in (np.nan, np.inf, -np.inf):
        x = base.copy()
        x[1234] = bad
        y = run(x)
        assert not np.isfinite(y).any(), (bad, np.isfinite(y).sum())
    y = run(base)
    ref = oracle.linear(base[None], blocks, (n, k), qtype, threads=8)
    assert np.isfinite(y).all() and tolerance_ok(y[None], ref, base[None], k).all()
