"""GPU: the decode-step operators and the whole decode step through the C ABI
against the CPU oracle (oracle/forward_ref.c, oracle.forward_token).

Tolerances, per operator (float arithmetic whose order differs from the
oracle's):
  rmsnorm      rtol 1e-5 (+1e-6 abs): sum of squares in a different order,
               then the same x*w/scale (the reference's own CUDA test: 2e-4)
  add, mul     bit-exact; silu / swiglu rtol 2e-6 (expf vs double quotient)
  embedding, kv write  bit-exact
  rope         1e-5 + (angle rounding) 2.4e-7 * pos * max|x|: theta^(-2i/hd)
               comes from the device powf, whose last bit may differ from
               glibc's; the float angle pos*freq magnifies that ulp by pos
  attention    rtol 1e-4, atol 1e-5 (the reference's CUDA tests use 1e-4 /
               1e-5): chunked online softmax vs a single pass
  F32 linear   |dy| <= 1e-5 * sum_k |w x| + 1e-6: fp32 sums in another order
  argmax       exact index
  decode step  logits within 1e-4 * max|logits| (+1e-6) of the oracle, and
               the reference's own bound 5e-3 (tests/test_cuda.cc:1226) on the
               tiny model; KV cache rows within the same bounds; greedy tokens
               identical.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _dev(a, cuda):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _ok(pkg, status, what):
    pkg._check(status, what)


def _s(pkg):
    return pkg._stream()


def _sync():
    import torch
    torch.cuda.synchronize()


# ---- rmsnorm / elementwise / embedding ------------------------------------------
@pytest.mark.parametrize("rows,dim", [(1, 8), (1, 33), (3, 64), (1, 3584), (2, 5000), (1, 8192)])
def test_rmsnorm(pkg, oracle, cuda, rows, dim):
    rng = np.random.default_rng(dim)
    x = (rng.standard_normal((rows, dim)) * 3).astype(np.float32)
    w = rng.standard_normal(dim).astype(np.float32)
    xd, wd = _dev(x, cuda), _dev(w, cuda)
    yd = _dev(np.zeros_like(x), cuda)
    _ok(pkg, pkg.lib().mlq_rmsnorm(xd.data_ptr(), wd.data_ptr(), yd.data_ptr(), rows, dim,
                                   1e-5, _s(pkg)), "mlq_rmsnorm")
    y = yd.cpu().numpy()
    for r in range(rows):
        np.testing.assert_allclose(y[r], oracle.rmsnorm(x[r], w, 1e-5), rtol=1e-5, atol=1e-6)


def test_elementwise(pkg, oracle, cuda):
    rng = np.random.default_rng(4)
    for n in (1, 17, 1000, 18944, 300001):
        a = (rng.standard_normal(n) * 4).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        ad, bd = _dev(a, cuda), _dev(b, cuda)
        yd = _dev(np.zeros(n, np.float32), cuda)
        lib = pkg.lib()
        _ok(pkg, lib.mlq_add(ad.data_ptr(), bd.data_ptr(), yd.data_ptr(), n, _s(pkg)), "add")
        assert np.array_equal(yd.cpu().numpy(), a + b)
        _ok(pkg, lib.mlq_mul(ad.data_ptr(), bd.data_ptr(), yd.data_ptr(), n, _s(pkg)), "mul")
        assert np.array_equal(yd.cpu().numpy(), a * b)
        _ok(pkg, lib.mlq_silu(ad.data_ptr(), yd.data_ptr(), n, _s(pkg)), "silu")
        np.testing.assert_allclose(yd.cpu().numpy(), oracle.silu(a), rtol=2e-6, atol=1e-30)
        _ok(pkg, lib.mlq_swiglu(ad.data_ptr(), bd.data_ptr(), yd.data_ptr(), n, _s(pkg)), "swiglu")
        np.testing.assert_allclose(yd.cpu().numpy(), oracle.swiglu(a, b), rtol=2e-6, atol=1e-30)


def test_silu_reference_values(pkg, cuda):
    # tests/test_cuda.cc:329-338 / test_ops.cc:243-277 known answers
    xd = _dev(np.array([0.0, 1.0, 2.0], np.float32), cuda)
    yd = _dev(np.zeros(3, np.float32), cuda)
    _ok(pkg, pkg.lib().mlq_silu(xd.data_ptr(), yd.data_ptr(), 3, _s(pkg)), "silu")
    np.testing.assert_allclose(yd.cpu().numpy(), [0.0, 0.7310586, 1.7615942], atol=1e-5)


def test_embedding(pkg, cuda):
    rng = np.random.default_rng(5)
    table = rng.standard_normal((300, 96)).astype(np.float32)
    td = _dev(table, cuda)
    yd = _dev(np.zeros(96, np.float32), cuda)
    for tok in (0, 2, 299):
        _ok(pkg, pkg.lib().mlq_embedding(td.data_ptr(), 300, 96, tok, yd.data_ptr(), _s(pkg)),
            "mlq_embedding")
        assert np.array_equal(yd.cpu().numpy(), table[tok])
    assert pkg.lib().mlq_embedding(td.data_ptr(), 300, 96, 300, yd.data_ptr(), _s(pkg)) == -1


# ---- rope ---------------------------------------------------------------------------
@pytest.mark.parametrize("rope_type", [0, 1])
@pytest.mark.parametrize("n_heads,n_kv,hd,pos,theta", [
    (4, 2, 8, 3, 1e4),            # tests/test_cuda.cc:486-513
    (28, 4, 128, 0, 1e6), (28, 4, 128, 1, 1e6), (28, 4, 128, 4095, 1e6),
    (32, 8, 128, 32767, 5e5), (12, 2, 64, 200, 1e4), (2, 1, 2, 7, 1e4)])
def test_rope(pkg, oracle, cuda, rope_type, n_heads, n_kv, hd, pos, theta):
    rng = np.random.default_rng(pos + hd)
    q = rng.standard_normal((n_heads, hd)).astype(np.float32)
    k = rng.standard_normal((n_kv, hd)).astype(np.float32)
    qd, kd = _dev(q, cuda), _dev(k, cuda)
    _ok(pkg, pkg.lib().mlq_rope(qd.data_ptr(), kd.data_ptr(), n_heads, n_kv, hd, pos,
                                theta, rope_type, _s(pkg)), "mlq_rope")
    qr, kr = oracle.rope(q, k, pos, theta, rope_type)
    tol = 1e-5 + 2.4e-7 * pos * max(np.abs(q).max(), np.abs(k).max())
    np.testing.assert_allclose(qd.cpu().numpy(), qr, atol=tol, rtol=0)
    np.testing.assert_allclose(kd.cpu().numpy(), kr, atol=tol, rtol=0)
    if pos == 0:
        assert np.array_equal(qd.cpu().numpy(), q)


# ---- KV cache + attention ----------------------------------------------------------------
class Cache:
    def __init__(self, pkg, cuda, n_layers, max_seq, n_kv, hd, keys=None, values=None):
        import torch
        shape = (n_layers, max_seq, n_kv, hd)
        self.keys = _dev(keys, cuda) if keys is not None else torch.zeros(shape, device=cuda)
        self.values = _dev(values, cuda) if values is not None else torch.zeros(shape, device=cuda)
        self.c = pkg.MlqKvCache(self.keys.data_ptr(), self.values.data_ptr(), n_layers, max_seq,
                                n_kv, hd)
        self.pkg = pkg

    def attention(self, q, layer, pos, n_heads, cuda):
        import torch
        lib = self.pkg.lib()
        nbytes = ctypes.c_size_t()
        _ok(self.pkg, lib.mlq_attention_workspace(ctypes.byref(self.c), n_heads,
                                                  ctypes.byref(nbytes)), "workspace")
        ws = torch.empty(nbytes.value, dtype=torch.uint8, device=cuda)
        qd = _dev(np.asarray(q, np.float32), cuda)
        out = torch.empty((n_heads, self.c.head_dim), device=cuda)
        _ok(self.pkg, lib.mlq_attention_decode(ctypes.byref(self.c), layer, pos, qd.data_ptr(),
                                               n_heads, out.data_ptr(), ws.data_ptr(),
                                               ws.numel(), _s(self.pkg)), "attention")
        return out.cpu().numpy()


def _fill_linear(shape, scale, bias):
    """fillLinear of the reference's tests: value i * scale + bias."""
    return (np.arange(np.prod(shape), dtype=np.float32) * np.float32(scale)
            + np.float32(bias)).reshape(shape).astype(np.float32)


def test_kv_write_roundtrip(pkg, cuda):
    # tests/test_cuda.cc:814-858: one row written, the rest untouched
    cache = Cache(pkg, cuda, 2, 4, 2, 3)
    k = _fill_linear((2, 3), 0.5, 1.0)
    v = _fill_linear((2, 3), -0.25, 2.0)
    kd, vd = _dev(k, cuda), _dev(v, cuda)
    _ok(pkg, pkg.lib().mlq_kv_write(ctypes.byref(cache.c), 1, 2, kd.data_ptr(), vd.data_ptr(),
                                    _s(pkg)), "kv_write")
    keys, values = cache.keys.cpu().numpy(), cache.values.cpu().numpy()
    assert np.array_equal(keys[1, 2], k) and np.array_equal(values[1, 2], v)
    keys[1, 2] = 0
    values[1, 2] = 0
    assert not keys.any() and not values.any()
    assert pkg.lib().mlq_kv_write(ctypes.byref(cache.c), 2, 0, kd.data_ptr(), vd.data_ptr(),
                                  _s(pkg)) == -2
    assert pkg.lib().mlq_kv_write(ctypes.byref(cache.c), 0, 4, kd.data_ptr(), vd.data_ptr(),
                                  _s(pkg)) == -2


def test_attention_reference_cases(pkg, oracle, cuda):
    """The reference's CUDA attention tests (tests/test_cuda.cc:962-1141)."""
    n_heads, n_kv, hd = 4, 2, 4
    # matches reference at pos 3 (:962-997)
    keys = np.zeros((1, 8, n_kv, hd), np.float32)
    values = np.zeros_like(keys)
    for p in range(4):
        i = np.arange(n_kv * hd, dtype=np.float32)
        keys[0, p] = (0.1 * (p + 1) + 0.03 * i - 0.2).reshape(n_kv, hd)
        values[0, p] = (-0.05 * p + 0.07 * i + 0.4).reshape(n_kv, hd)
    q = _fill_linear((n_heads, hd), 0.15, -0.3)
    out = Cache(pkg, cuda, 1, 8, n_kv, hd, keys, values).attention(q, 0, 3, n_heads, cuda)
    np.testing.assert_allclose(out, oracle.attention(q, keys, values, 0, 3), atol=1e-4)
    # pos 0 returns V (:999-1029)
    keys = np.zeros((1, 4, n_kv, hd), np.float32)
    values = np.zeros_like(keys)
    keys[0, 0] = _fill_linear((n_kv, hd), 0.2, -1.0)
    values[0, 0] = _fill_linear((n_kv, hd), 0.5, 10.0)
    q = _fill_linear((n_heads, hd), 0.3, 0.25)
    out = Cache(pkg, cuda, 1, 4, n_kv, hd, keys, values).attention(q, 0, 0, n_heads, cuda)
    np.testing.assert_allclose(out, values[0, 0][[0, 0, 1, 1]], atol=1e-5)
    # GQA mapping with zero keys (:1031-1064)
    keys = np.zeros((1, 4, n_kv, hd), np.float32)
    values = np.zeros_like(keys)
    values[0, :3, 0], values[0, :3, 1] = 1.0, 2.0
    q = _fill_linear((n_heads, hd), 0.1, 0.0)
    out = Cache(pkg, cuda, 1, 4, n_kv, hd, keys, values).attention(q, 0, 2, n_heads, cuda)
    np.testing.assert_allclose(out, [[1] * 4, [1] * 4, [2] * 4, [2] * 4], atol=1e-5)
    # layer 1, pos 5 of a two-layer cache (:1105-1141)
    keys = np.zeros((2, 8, n_kv, hd), np.float32)
    values = np.zeros_like(keys)
    i = np.arange(n_kv * hd, dtype=np.float32)
    for layer in range(2):
        for p in range(6):
            keys[layer, p] = (0.02 * i + 0.11 * layer + 0.05 * p - 0.6).reshape(n_kv, hd)
            values[layer, p] = (-0.03 * i + 0.07 * layer - 0.04 * p + 0.8).reshape(n_kv, hd)
    q = _fill_linear((n_heads, hd), -0.09, 0.35)
    out = Cache(pkg, cuda, 2, 8, n_kv, hd, keys, values).attention(q, 1, 5, n_heads, cuda)
    np.testing.assert_allclose(out, oracle.attention(q, keys, values, 1, 5), atol=1e-4)


@pytest.mark.parametrize("n_heads,n_kv,hd,max_seq,pos", [
    (28, 4, 128, 64, 0), (28, 4, 128, 256, 63), (28, 4, 128, 256, 64), (28, 4, 128, 256, 65),
    (28, 4, 128, 4096, 4095), (32, 8, 128, 8192, 5000), (8, 8, 64, 512, 300),
    (16, 1, 256, 600, 599), (16, 16, 80, 100, 99), (4, 2, 8, 128, 127), (6, 3, 4, 40, 33),
    (32, 2, 100, 300, 150), (64, 4, 64, 200, 129),
    # seven query heads per kv head (padded to eight in the kernels)
    (14, 2, 64, 300, 200), (7, 1, 256, 200, 150), (21, 3, 96, 100, 60),
    # more than 128 chunk partials per head: the combine's online max/sum
    # runs over several chunks per lane, and its weighted sum over more than
    # one 32-chunk batch
    (8, 2, 128, 9100, 9000), (6, 3, 96, 4600, 4500)])
def test_attention_matches_oracle(pkg, oracle, cuda, n_heads, n_kv, hd, max_seq, pos):
    rng = np.random.default_rng(pos * 7 + hd)
    keys = rng.standard_normal((2, max_seq, n_kv, hd)).astype(np.float32)
    values = rng.standard_normal((2, max_seq, n_kv, hd)).astype(np.float32)
    q = (rng.standard_normal((n_heads, hd)) * 0.5).astype(np.float32)
    out = Cache(pkg, cuda, 2, max_seq, n_kv, hd, keys, values).attention(q, 1, pos, n_heads, cuda)
    np.testing.assert_allclose(out, oracle.attention(q, keys, values, 1, pos), rtol=1e-4,
                               atol=1e-5)


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_attention_unaligned_buffers(pkg, oracle, cuda, hd):
    """Caches and q that are not 16-byte aligned take the LDS-staged kernel
    (the register kernel loads float4): same results."""
    import torch
    n_heads, n_kv, max_seq, pos = 8, 2, 100, 77
    rng = np.random.default_rng(hd)
    keys = rng.standard_normal((1, max_seq, n_kv, hd)).astype(np.float32)
    values = rng.standard_normal((1, max_seq, n_kv, hd)).astype(np.float32)
    q = (rng.standard_normal((n_heads, hd)) * 0.5).astype(np.float32)
    kbuf = torch.zeros(keys.size + 1, device=cuda)
    vbuf = torch.zeros(values.size + 1, device=cuda)
    kbuf[1:] = torch.from_numpy(keys.reshape(-1)).to(cuda)
    vbuf[1:] = torch.from_numpy(values.reshape(-1)).to(cuda)
    c = pkg.MlqKvCache(kbuf[1:].data_ptr(), vbuf[1:].data_ptr(), 1, max_seq, n_kv, hd)
    lib = pkg.lib()
    nbytes = ctypes.c_size_t()
    _ok(pkg, lib.mlq_attention_workspace(ctypes.byref(c), n_heads, ctypes.byref(nbytes)), "ws")
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=cuda)
    qbuf = torch.zeros(q.size + 1, device=cuda)
    qbuf[1:] = torch.from_numpy(q.reshape(-1)).to(cuda)
    out = torch.empty((n_heads, hd), device=cuda)
    _ok(pkg, lib.mlq_attention_decode(ctypes.byref(c), 0, pos, qbuf[1:].data_ptr(), n_heads,
                                      out.data_ptr(), ws.data_ptr(), ws.numel(), _s(pkg)),
        "attention")
    np.testing.assert_allclose(out.cpu().numpy(), oracle.attention(q, keys, values, 0, pos),
                               rtol=1e-4, atol=1e-5)


def test_attention_validation(pkg, cuda):
    # tests/test_cuda.cc:1143-1184: shape, layer, position, divisibility checks
    cache = Cache(pkg, cuda, 1, 8, 2, 4)
    lib = pkg.lib()
    q = _dev(np.zeros((4, 4), np.float32), cuda)
    out = _dev(np.zeros((4, 4), np.float32), cuda)
    ws = _dev(np.zeros(1 << 16, np.uint8), cuda)

    def call(layer, pos, n_heads, ws_bytes=1 << 16):
        return lib.mlq_attention_decode(ctypes.byref(cache.c), layer, pos, q.data_ptr(), n_heads,
                                        out.data_ptr(), ws.data_ptr(), ws_bytes, _s(pkg))
    assert call(1, 0, 4) == -2
    assert call(0, 8, 4) == -2
    assert call(0, -1, 4) == -2
    assert call(0, 0, 3) == -2
    assert call(0, 0, 0) == -2
    assert call(0, 0, 4, ws_bytes=8) == -4
    assert call(0, 7, 4) == 0


# ---- F32 linear -------------------------------------------------------------------------
@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (1, 100, 37), (3, 48, 64), (9, 33, 128),
                                   (20, 64, 256), (1, 1, 1), (2, 152, 3584)])
def test_linear_f32(pkg, oracle, cuda, m, n, k):
    rng = np.random.default_rng(n + k)
    w = rng.standard_normal((n, k)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    tw = pkg.upload_f32(w, device=cuda)
    xd, bd = _dev(x, cuda), _dev(bias, cuda)
    bound = 1e-5 * (np.abs(x) @ np.abs(w).T) + 1e-6
    y = pkg.linear(tw, xd).cpu().numpy()
    ref = np.stack([oracle.linear_f32(x[r], w) for r in range(m)])
    assert np.all(np.abs(y - ref) <= bound)
    yb = pkg.linear(tw, xd, bias=bd).cpu().numpy()
    assert np.all(np.abs(yb - (ref + bias)) <= bound + 1e-6 * np.abs(bias))


def test_linear_f32_swiglu(pkg, oracle, cuda):
    rng = np.random.default_rng(8)
    hid, k, m = 48, 96, 3
    gate = rng.standard_normal((hid, k)).astype(np.float32)
    up = rng.standard_normal((hid, k)).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    inter = pkg.interleave_rows(gate, up, hid).reshape(2 * hid, k)
    tw = pkg.upload_f32(inter, device=cuda)
    y = pkg.linear(tw, _dev(x, cuda), act=pkg.EPI_SWIGLU).cpu().numpy()
    for r in range(m):
        ref = oracle.swiglu(oracle.linear_f32(x[r], gate), oracle.linear_f32(x[r], up))
        np.testing.assert_allclose(y[r], ref, rtol=1e-4, atol=1e-4)


# ---- argmax ------------------------------------------------------------------------------
def test_argmax(pkg, oracle, cuda):
    import torch
    lib = pkg.lib()
    out = torch.zeros(1, dtype=torch.int32, device=cuda)
    rng = np.random.default_rng(9)
    cases = [np.array([1, 5, 3, 5, 2], np.float32),  # tests/test_ops.cc:320-331
             rng.standard_normal(152064).astype(np.float32),
             np.array([np.nan, 3, 4], np.float32), np.array([1, np.nan, 0.5], np.float32),
             np.array([-np.inf, -np.inf, np.nan], np.float32),
             np.full(5000, np.nan, np.float32), np.full(70000, -np.inf, np.float32),
             np.array([0, np.inf, np.inf], np.float32)]
    tie = np.zeros(100000, np.float32)
    tie[[77777, 1234, 99999]] = 3.0
    cases.append(tie)
    for x in cases:
        xd = _dev(x, cuda)
        _ok(pkg, lib.mlq_argmax(xd.data_ptr(), x.size, out.data_ptr(), _s(pkg)), "argmax")
        assert int(out.item()) == oracle.argmax(x)


# ---- the decode step ----------------------------------------------------------------------
def _tiny(pkg):
    import mini_llama_amd.decode as dec
    return dec.load_manifest_model(os.path.join(GOLDEN, "tiny", "model.json"),
                                   os.path.join(GOLDEN, "tiny", "model.bin"))


def _run_both(pkg, oracle, model, tokens, fuse=True):
    import mini_llama_amd.decode as dec
    dm = dec.DecodeModel(model, fuse=fuse)
    cache = oracle.new_cache(model)
    worst = 0.0
    for pos, t in enumerate(tokens):
        ref = oracle.forward_token(model, cache, t, pos)
        got = dm.forward_token(t, pos).cpu().numpy()
        scale = np.abs(ref).max()
        err = np.abs(got - ref).max()
        worst = max(worst, err / max(scale, 1e-30))
        assert err <= 1e-4 * scale + 1e-6, (pos, err, scale)
    keys, values = dm.keys.cpu().numpy(), dm.values.cpu().numpy()
    n = len(tokens)
    # K/V rows of later layers carry the float differences of every layer
    # before them: bound them relative to the rows' scale (1e-5 of max|.|),
    # and rotated keys also by the RoPE angle term of the rope tolerance
    # above (2.4e-7 * pos * max|k|)
    kmax = np.abs(cache[0][:, :n]).max()
    vmax = np.abs(cache[1][:, :n]).max()
    for p in range(n):
        np.testing.assert_allclose(keys[:, p], cache[0][:, p], rtol=1e-4,
                                   atol=1e-5 * kmax + 2.4e-7 * p * kmax, err_msg=f"pos {p}")
    np.testing.assert_allclose(values[:, :n], cache[1][:, :n], rtol=1e-4, atol=1e-5 * vmax)
    assert not keys[:, n:].any() and not values[:, n:].any()
    return dm, worst


def test_tiny_model_matches_oracle(pkg, oracle, cuda):
    """tests/test_cuda.cc:1188-1266 on the reference's tiny model: logits per
    prefill step within 5e-3 (and far tighter), KV cache rows agree."""
    model = _tiny(pkg)
    tokens = [1] + list(b"hello")
    dm, worst = _run_both(pkg, oracle, model, tokens)
    assert dm.fused_qkv == [True, True] and dm.fused_glu == [False, False]  # hidden 86
    print(f"tiny model: worst logits error / max|logit| = {worst:.2e}")


def test_tiny_model_greedy_generation(pkg, oracle, cuda):
    """tests/test_cuda.cc:1268-1330: prompt "hi" + 4 greedy steps; the
    graph-driven loop, the eager loop and the oracle pick the same tokens."""
    import mini_llama_amd.decode as dec
    model = _tiny(pkg)
    prompt = [1] + list(b"hi")
    cache = oracle.new_cache(model)
    for pos, t in enumerate(prompt):
        logits = oracle.forward_token(model, cache, t, pos)
    want = []
    nxt = oracle.argmax(logits)
    for step in range(5):
        want.append(nxt)
        logits = oracle.forward_token(model, cache, nxt, len(prompt) + step)
        nxt = oracle.argmax(logits)
    dm = dec.DecodeModel(model)
    assert dm.generate_greedy(prompt, 5, graph=True) == want
    dm.reset()
    assert dm.generate_greedy(prompt, 5, graph=False) == want


@pytest.mark.parametrize("qtype,kw,fuse", [
    ("q4_0", {}, True), ("q4_0", {}, False), ("q8_0", {"bias": True}, True),
    ("q4_1", {"cfg": {"rope_type": 1}}, True), ("f32", {"bias": True}, True),
    ("q8_0", {"cfg": {"n_kv_heads": 4, "hidden_dim": 100}}, True),
    ("q4_0", {"cfg": {"n_heads": 8, "n_kv_heads": 1, "dim": 256, "hidden_dim": 512,
                      "max_seq_len": 200}, "lm_head_type": "f32"}, True),
    # head dims the attention kernel fuses RoPE and the cache write into
    # (64 / 128 / 256), both pairings, across workgroup chunks
    ("q4_0", {"cfg": {"dim": 512, "n_heads": 8, "n_kv_heads": 2, "hidden_dim": 512,
                      "max_seq_len": 160}, "tokens": 150}, True),
    ("q8_0", {"cfg": {"dim": 512, "n_heads": 4, "n_kv_heads": 1, "rope_type": 1,
                      "max_seq_len": 160}, "bias": True, "tokens": 100}, True),
    ("q4_1", {"cfg": {"dim": 512, "n_heads": 2, "n_kv_heads": 2, "rope_type": 1}}, True),
    ("q4_0", {"cfg": {"dim": 1024, "n_heads": 16, "n_kv_heads": 2, "hidden_dim": 256,
                      "rope_type": 1, "max_seq_len": 80}}, True),
    # dim not a multiple of 16: the last 16-row tile of the o / down
    # projections (producers of the next RMSNorm input) is partial
    ("q4_0", {"cfg": {"dim": 136, "n_heads": 4, "n_kv_heads": 2, "hidden_dim": 200}}, True),
    ("q8_0", {"cfg": {"dim": 200, "n_heads": 2, "n_kv_heads": 1, "hidden_dim": 96},
              "bias": True}, False)])
def test_synthetic_models_match_oracle(pkg, oracle, cuda, qtype, kw, fuse):
    from synthetic import synth
    cfg = dict(vocab_size=160, dim=128, hidden_dim=256, n_layers=3, n_heads=4, n_kv_heads=2,
               max_seq_len=96)
    kw = dict(kw)
    cfg.update(kw.pop("cfg", {}))
    n_tokens = kw.pop("tokens", 70)  # crosses a chunk boundary
    model = synth.synthetic_model(cfg, qtype, seed=11, **kw)
    rng = np.random.default_rng(3)
    tokens = rng.integers(0, cfg["vocab_size"], n_tokens).tolist()
    _, worst = _run_both(pkg, oracle, model, tokens, fuse=fuse)
    print(f"{qtype} {kw} fuse={fuse}: worst logits error / max|logit| = {worst:.2e}")


def _to_host(x):
    if isinstance(x, dict):
        return {k: _to_host(v) for k, v in x.items()}
    if isinstance(x, list):
        return [_to_host(v) for v in x]
    if hasattr(x, "is_cuda"):
        return x.cpu().numpy()
    return x


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0", "q4_1", "f32"])
def test_device_built_model_matches_oracle(pkg, oracle, cuda, qtype):
    """A model generated on the device (device repack, device q|k|v
    concatenation and gate|up interleave) against the oracle on the same
    bytes brought to the host."""
    import mini_llama_amd.decode as dec
    from synthetic import synth
    cfg = dict(vocab_size=128, dim=128, hidden_dim=192, n_layers=2, n_heads=8, n_kv_heads=2,
               max_seq_len=32, rope_type=1)
    dmodel = synth.synthetic_model_device(cfg, qtype, seed=4, bias=True)
    host = _to_host(dmodel)
    for lw in host["layers"] + [host]:
        for name in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down", "lm_head"):
            w = lw.get(name)
            if w is not None and qtype != "f32":
                w["data"] = w["data"].view(oracle.BLOCK_DTYPES[qtype])
    dm = dec.DecodeModel(dmodel)
    assert all(dm.fused_qkv) and all(dm.fused_glu)
    cache = oracle.new_cache(host)
    for pos, t in enumerate([5, 77, 1, 127, 64]):
        ref = oracle.forward_token(host, cache, t, pos)
        got = dm.forward_token(t, pos).cpu().numpy()
        assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max() + 1e-6, pos


def test_qwen2_7b_layer_at_full_size(pkg, oracle, cuda):
    """One Qwen2-7B-shaped layer (dim 3584, FFN 18944, 28 heads / 4 kv heads,
    head_dim 128, q|k|v biases) in q4_0 at BASELINE's decode shapes, stepped
    over a few positions against the oracle."""
    from synthetic import synth
    cfg = dict(vocab_size=512, dim=3584, hidden_dim=18944, n_layers=1, n_heads=28,
               n_kv_heads=4, max_seq_len=64, rope_theta=1e6, rms_norm_eps=1e-6, rope_type=1)
    model = synth.synthetic_model(cfg, "q4_0", seed=5, bias=True)
    _run_both(pkg, oracle, model, [5, 100, 7, 300])


@pytest.mark.parametrize("dim,n_heads,rope_type", [(128, 4, 0), (512, 4, 1)])
def test_graph_replay_matches_eager_steps(pkg, cuda, dim, n_heads, rope_type):
    """The captured step (device token and position) replayed repeatedly
    gives bitwise the logits of eager steps, with eager work in between
    (head_dim 32: separate RoPE; 128: RoPE fused into attention)."""
    import mini_llama_amd.decode as dec
    from synthetic import synth
    import torch
    cfg = dict(vocab_size=200, dim=dim, hidden_dim=256, n_layers=2, n_heads=n_heads,
               n_kv_heads=2, max_seq_len=80, rope_type=rope_type)
    model = synth.synthetic_model(cfg, "q4_0", seed=2)
    eager = dec.DecodeModel(model)
    graphed = dec.DecodeModel(model)
    prompt = [3, 9, 27]
    for i, t in enumerate(prompt):
        eager.forward_token(t, i)
        graphed.forward_token(t, i)
    graphed.pos_dev.fill_(len(prompt))
    graphed.token_dev.fill_(81)
    g = graphed.greedy_graph()
    tok = 81
    for step in range(6):
        want = eager.forward_token(tok, len(prompt) + step).clone()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(graphed.logits, want), step
        tok = eager.argmax()
        assert int(graphed.token_dev.item()) == tok
        assert int(graphed.pos_dev.item()) == len(prompt) + step + 1


def test_device_position_out_of_range_gives_nan(pkg, cuda):
    """A device-side token or position outside the model yields NaN logits
    (no host check can see it), never an out-of-range access."""
    import mini_llama_amd.decode as dec
    from synthetic import synth
    cfg = dict(vocab_size=64, dim=64, hidden_dim=128, n_layers=1, n_heads=2, n_kv_heads=1,
               max_seq_len=8)
    dm = dec.DecodeModel(synth.synthetic_model(cfg, "q8_0", seed=1))
    for token, pos in ((3, 8), (3, 1 << 30), (3, -5)):
        dm.token_dev.fill_(token)
        dm.pos_dev.fill_(pos)
        dm.step_device()
        assert np.isnan(dm.logits.cpu().numpy()).all(), (token, pos)
    # no cache row was written for a position outside the cache
    assert not dm.keys.cpu().numpy().any() and not dm.values.cpu().numpy().any()
    for token in (64, -1):
        dm.token_dev.fill_(token)
        dm.pos_dev.fill_(2)
        dm.step_device()
        assert np.isnan(dm.logits.cpu().numpy()).all(), token


@pytest.mark.parametrize("qtype", ["q8_0", "q4_0"])
def test_device_position_past_model_in_larger_cache_gives_nan(pkg, cuda, qtype):
    """A cache with more positions than the model (the API allows it): a
    device position at or past the model's max_seq_len gives NaN logits and
    writes no cache row (forwardToken rejects pos >= max_seq_len,
    src/forward.cc:42), though the cache could hold the row."""
    import mini_llama_amd.decode as dec
    from synthetic import synth
    # head_dim 128 (register attention kernel, fused RoPE) and 48 (LDS kernel)
    for dim, n_heads in ((256, 2), (96, 2)):
        cfg = dict(vocab_size=64, dim=dim, hidden_dim=128, n_layers=2, n_heads=n_heads,
                   n_kv_heads=1, max_seq_len=70)
        dm = dec.DecodeModel(synth.synthetic_model(cfg, qtype, seed=3), cache_len=300)
        for pos in (70, 71, 127, 128, 200, 299):
            dm.token_dev.fill_(5)
            dm.pos_dev.fill_(pos)
            dm.step_device()
            assert np.isnan(dm.logits.cpu().numpy()).all(), (dim, pos)
        assert not dm.keys.cpu().numpy().any() and not dm.values.cpu().numpy().any()
        # the last position inside the model still works and writes its row
        dm.pos_dev.fill_(69)
        dm.step_device()
        assert np.isfinite(dm.logits.cpu().numpy()).all()
        assert dm.keys[:, 69].abs().sum().item() > 0 and not dm.keys[:, 70:].any().item()


def test_decode_host_validation(pkg, cuda):
    import mini_llama_amd.decode as dec
    model = _tiny(pkg)
    dm = dec.DecodeModel(model)
    lib = pkg.lib()
    ws = dm.workspace

    def call(token, pos, ws_bytes=None):
        return lib.mlq_decode_token(ctypes.byref(dm._model), ctypes.byref(dm._cache), token, pos,
                                    None, None, dm.logits.data_ptr(), ws.data_ptr(),
                                    ws.numel() if ws_bytes is None else ws_bytes, _s(pkg))
    assert call(128, 0) == -1       # tests/test_forward.cc:105-123
    assert call(-1, 0) == -1
    assert call(1, 128) == -1       # :125-141
    assert call(1, 0, ws_bytes=64) == -4
    assert call(1, 0) == 0


# ---- batched prefill ------------------------------------------------------------------------
PREFILL_CASES = [
    # (qtype, model kwargs, fuse, start, n)
    ("q4_0", {"cfg": {"dim": 512, "n_heads": 4, "n_kv_heads": 2, "rope_type": 1}}, True, 0, 130),
    ("q8_0", {"cfg": {"dim": 512, "n_heads": 8, "n_kv_heads": 2}, "bias": True}, True, 7, 64),
    ("q4_1", {"cfg": {"dim": 256, "n_heads": 4, "n_kv_heads": 4}}, False, 3, 65),
    ("f32", {"cfg": {"dim": 128, "n_heads": 4, "n_kv_heads": 2}, "bias": True}, True, 0, 5),
    ("q4_0", {"cfg": {"dim": 128, "n_heads": 4, "n_kv_heads": 1, "hidden_dim": 100}}, True, 2, 1),
    ("q4_0", {"cfg": {"dim": 512, "n_heads": 2, "n_kv_heads": 1, "rope_type": 1}}, True, 0, 9),
    # prefill GEMM rows with a hidden size off the 128-column grid (the
    # fp16 SwiGLU output's padding) and biases
    ("q8_0", {"cfg": {"dim": 256, "n_heads": 4, "n_kv_heads": 2, "hidden_dim": 200},
              "bias": True}, True, 5, 100),
    # F32 weights with more than 64 rows (no prefill GEMM: the unfused path)
    # and q4_1 fused with biases through the prefill GEMM
    ("f32", {"cfg": {"dim": 128, "n_heads": 4, "n_kv_heads": 2}, "bias": True}, True, 2, 70),
    ("q4_1", {"cfg": {"dim": 256, "n_heads": 8, "n_kv_heads": 2}, "bias": True}, True, 0, 129),
    # 512-token prompts with GQA groups that are not powers of two (the MFMA
    # prefill attention pads them to 4 / 8 heads, padding heads masked) at
    # head_dim 64, 128 and 256
    ("q4_0", {"cfg": {"dim": 384, "n_heads": 6, "n_kv_heads": 2, "max_seq_len": 600,
                      "rope_type": 1}}, True, 0, 512),
    ("q8_0", {"cfg": {"dim": 1280, "n_heads": 10, "n_kv_heads": 2, "max_seq_len": 600},
              "bias": True}, True, 3, 512),
    ("q4_0", {"cfg": {"dim": 1792, "n_heads": 7, "n_kv_heads": 1, "max_seq_len": 600,
                      "rope_type": 1}}, True, 0, 512),
    ("q4_1", {"cfg": {"dim": 896, "n_heads": 7, "n_kv_heads": 1, "max_seq_len": 600}}, True,
     1, 512),
]


@pytest.mark.parametrize("qtype,kw,fuse,start,n", PREFILL_CASES)
def test_prefill_matches_sequential_oracle(pkg, oracle, cuda, qtype, kw, fuse, start, n):
    """mlq_prefill of n tokens after `start` decode steps against the
    oracle's forwardBatch (one forward_token per token): the last logits,
    every K/V row, and decode steps after it. Tolerance: n > 8 runs the
    skinny / prefill GEMMs on fp16-rounded activations (about 1e-4 of the
    scale per Linear, here through two layers and the residuals): 2e-3 of
    max|logit|; n <= 8 keeps the decode GEMV's fp32-class 1e-4."""
    import mini_llama_amd.decode as dec
    from synthetic import synth
    kw = dict(kw)
    cfg = dict(vocab_size=160, dim=128, hidden_dim=256, n_layers=2, n_heads=4, n_kv_heads=2,
               max_seq_len=160)
    cfg.update(kw.pop("cfg", {}))
    model = synth.synthetic_model(cfg, qtype, seed=21, **kw)
    rng = np.random.default_rng(n + start)
    tokens = rng.integers(0, cfg["vocab_size"], start + n + 3).tolist()
    dm = dec.DecodeModel(model, fuse=fuse)
    cache = oracle.new_cache(model)
    for p in range(start):
        oracle.forward_token(model, cache, tokens[p], p)
        dm.forward_token(tokens[p], p)
    for p in range(start, start + n):
        ref = oracle.forward_token(model, cache, tokens[p], p)
    got = dm.prefill(tokens[start:start + n], start).cpu().numpy()
    rel = 2e-3 if n > 8 and qtype != "f32" else 1e-4
    scale = np.abs(ref).max()
    err = np.abs(got - ref).max()
    print(f"prefill {qtype} n={n} start={start}: logits error / max = {err / scale:.2e}")
    assert err <= rel * scale + 1e-6
    keys, values = dm.keys.cpu().numpy(), dm.values.cpu().numpy()
    end = start + n
    for arr, want in ((keys, cache[0]), (values, cache[1])):
        amax = np.abs(want[:, :end]).max()
        assert np.abs(arr[:, :end] - want[:, :end]).max() <= rel * 10 * amax + 2.4e-7 * end * amax
        assert not arr[:, end:].any()
    # decode continues from the prefilled cache
    for p in range(end, end + 3):
        ref = oracle.forward_token(model, cache, tokens[p], p)
        got = dm.forward_token(tokens[p], p).cpu().numpy()
        assert np.abs(got - ref).max() <= rel * np.abs(ref).max() + 1e-6, p


@pytest.mark.parametrize("qtype", ["q4_0", "q8_0"])
def test_prefill_qwen2_7b_layer_at_full_size(pkg, oracle, cuda, qtype):
    """One Qwen2-7B-shaped layer (dim 3584, FFN 18944, 28 heads / 4 kv
    heads: GQA group 7, head_dim 128, q|k|v biases, NeoX RoPE) prefilled over
    512 tokens, the benchmarked prefill workload, against the oracle run
    token by token: last logits, every K/V row, and one decode step after.
    q8_0 at this size takes the large-grid prefill GEMM variant (two
    workgroups per CU)."""
    import os
    import mini_llama_amd.decode as dec
    from synthetic import synth
    cfg = dict(vocab_size=256, dim=3584, hidden_dim=18944, n_layers=1, n_heads=28,
               n_kv_heads=4, max_seq_len=520, rope_theta=1e6, rms_norm_eps=1e-6, rope_type=1)
    model = synth.synthetic_model(cfg, qtype, seed=9, bias=True)
    threads = max(1, min(16, os.cpu_count() or 1))
    n = 512
    tokens = np.random.default_rng(4).integers(0, cfg["vocab_size"], n + 1).tolist()
    print(f"prefill full-size {qtype}: oracle over {n} tokens ({threads} threads)", flush=True)
    cache = oracle.new_cache(model)
    for p in range(n):
        ref = oracle.forward_token(model, cache, tokens[p], p, threads=threads)
    dm = dec.DecodeModel(model)
    got = dm.prefill(tokens[:n], 0).cpu().numpy()
    scale = np.abs(ref).max()
    err = np.abs(got - ref).max()
    print(f"prefill full-size {qtype}: logits error / max = {err / scale:.2e}", flush=True)
    assert err <= 2e-3 * scale + 1e-6
    keys, values = dm.keys.cpu().numpy(), dm.values.cpu().numpy()
    for arr, want in ((keys, cache[0]), (values, cache[1])):
        amax = np.abs(want[:, :n]).max()
        assert np.abs(arr[:, :n] - want[:, :n]).max() <= 2e-2 * amax + 2.4e-7 * n * amax
    ref = oracle.forward_token(model, cache, tokens[n], n, threads=threads)
    got = dm.forward_token(tokens[n], n).cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-3 * np.abs(ref).max() + 1e-6


def test_prefill_tiny_model_greedy(pkg, oracle, cuda):
    """The reference's tiny model (F32 weights): greedy generation with the
    prompt prefilled in one batch picks the oracle's tokens."""
    import mini_llama_amd.decode as dec
    model = _tiny(pkg)
    prompt = [1] + list(b"hello world")
    cache = oracle.new_cache(model)
    for p, t in enumerate(prompt):
        logits = oracle.forward_token(model, cache, t, p)
    want, nxt = [], oracle.argmax(logits)
    for step in range(4):
        want.append(nxt)
        logits = oracle.forward_token(model, cache, nxt, len(prompt) + step)
        nxt = oracle.argmax(logits)
    dm = dec.DecodeModel(model)
    assert dm.generate_greedy(prompt, 4, prefill=True) == want


def test_prefill_host_validation(pkg, cuda):
    import mini_llama_amd.decode as dec
    dm = dec.DecodeModel(_tiny(pkg))
    lib = pkg.lib()
    nbytes = ctypes.c_size_t()
    assert lib.mlq_prefill_workspace(ctypes.byref(dm._model), 0, ctypes.byref(nbytes)) == -2
    _ok(pkg, lib.mlq_prefill_workspace(ctypes.byref(dm._model), 4, ctypes.byref(nbytes)), "ws")
    import torch
    ws = torch.empty(nbytes.value, dtype=torch.uint8, device=cuda)

    def call(toks, start, ws_bytes=None):
        t = np.asarray(toks, np.int32)
        return lib.mlq_prefill(ctypes.byref(dm._model), ctypes.byref(dm._cache), t.ctypes.data,
                               t.size, start, dm.logits.data_ptr(), ws.data_ptr(),
                               ws.numel() if ws_bytes is None else ws_bytes, _s(pkg))
    assert call([1, 2, 128, 3], 0) == -1
    assert call([1, 2, 3, -1], 0) == -1
    assert call([1, 2, 3, 4], 125) == -1      # 125 + 4 > max_seq_len 128
    assert call([1, 2, 3, 4], -1) == -1
    assert call([1, 2, 3, 4], 0, ws_bytes=100) == -4
    assert call([1, 2, 3, 4], 124) == 0
