"""CPU: pins the oracle's decode-step operators (oracle/forward_ref.c) and its
forward composition before they are trusted as the checker of the HIP
decode path. Each check is either a known answer from the reference's own
tests, a library routine, a closed form, or an independent float64
formulation, chosen so that a plausible slip (dropped term, swapped pairing,
wrong sign, wrong head mapping, rope after the cache write, a missing
residual) fails.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import scipy.special

import __graft_entry__ as graft

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# ---- rmsNorm ------------------------------------------------------------------
def test_rmsnorm_reference_known_answers(oracle):
    # tests/test_ops.cc:144-176
    np.testing.assert_allclose(oracle.rmsnorm(np.ones(4), np.ones(4), 1e-5), 1.0, atol=1e-4)
    y = oracle.rmsnorm([2, 0, 0, 0], np.ones(4), 1e-5)
    assert abs(y[0] - 2.0) <= 1e-4 and abs(y[1]) <= 1e-4
    np.testing.assert_allclose(oracle.rmsnorm(np.ones(4), np.full(4, 2.0), 1e-5), 2.0, atol=1e-4)


def test_rmsnorm_closed_form_and_scale_invariance(oracle):
    rng = np.random.default_rng(0)
    for dim in (1, 7, 32, 3584):
        c = np.float32(rng.uniform(0.5, 3.0))
        w = rng.standard_normal(dim).astype(np.float32)
        y = oracle.rmsnorm(np.full(dim, c), w, 1e-5)
        exact = c * w.astype(np.float64) / np.sqrt(float(c) ** 2 + 1e-5)
        # the float sum of dim equal squares carries up to dim/2 ulp of error
        np.testing.assert_allclose(y, exact, rtol=1e-6 + dim * 3e-8, atol=0)
        # eps = 0: scaling x by 2^e scales the float sum of squares and its
        # square root exactly, so y is unchanged bit for bit
        x = rng.standard_normal(dim).astype(np.float32)
        assert np.array_equal(oracle.rmsnorm(x, w, 0.0), oracle.rmsnorm(x * np.float32(8), w, 0.0))
        # float64 brute force with a rounding bound
        ref = x * w.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5)
        np.testing.assert_allclose(oracle.rmsnorm(x, w, 1e-5), ref, rtol=dim * 1.2e-7 + 1e-6,
                                   atol=1e-7)


# ---- softmax / silu / swiglu / argmax ------------------------------------------
def test_softmax_known_answers_and_library(oracle):
    # tests/test_ops.cc:190-212
    np.testing.assert_allclose(oracle.softmax([1, 2, 3]), [0.09003057, 0.24472847, 0.66524096],
                               atol=1e-5)
    np.testing.assert_allclose(oracle.softmax([5, 5, 5]), 1 / 3, atol=1e-5)
    rng = np.random.default_rng(1)
    for n in (1, 2, 65, 1000):
        x = (rng.standard_normal(n) * 6).astype(np.float32)
        np.testing.assert_allclose(oracle.softmax(x), scipy.special.softmax(x.astype(np.float64)),
                                   rtol=2e-6 * np.log2(n + 1) + 1e-6, atol=1e-9)
    with pytest.raises(ValueError):
        oracle.softmax([])


def test_silu_swiglu_known_answers_and_closed_form(oracle):
    # tests/test_ops.cc:243-277
    assert abs(oracle.silu([0.0])[0]) <= 1e-5
    assert abs(oracle.silu([1.0])[0] - 0.7310586) <= 1e-5
    y = oracle.swiglu([0, 1, 2], [1, 2, 3])
    np.testing.assert_allclose(y, [0.0, 0.7310586 * 2, 1.7615942 * 3], atol=1e-4)
    x = np.linspace(-30, 30, 2001).astype(np.float32)
    exact = x.astype(np.float64) * scipy.special.expit(x.astype(np.float64))
    np.testing.assert_allclose(oracle.silu(x), exact, rtol=2e-7, atol=1e-30)
    u = np.linspace(-2, 2, 2001).astype(np.float32)
    np.testing.assert_allclose(oracle.swiglu(x, u), exact * u, rtol=4e-7, atol=1e-30)


def test_argmax_rules(oracle):
    assert oracle.argmax([1, 5, 3, 5, 2]) == 1  # tests/test_ops.cc:320-331
    rng = np.random.default_rng(2)
    for n in (1, 10, 152064):
        x = rng.standard_normal(n).astype(np.float32)
        assert oracle.argmax(x) == int(np.argmax(x))
    assert oracle.argmax([np.nan, 3.0, 4.0]) == 0          # x[0] NaN is never replaced
    assert oracle.argmax([1.0, np.nan, 0.5]) == 0          # NaN never wins
    assert oracle.argmax([-np.inf, -np.inf, np.nan]) == 0
    assert oracle.argmax([0.0, np.inf, np.inf]) == 1


# ---- rope -------------------------------------------------------------------------
def _rope_complex(x, pos, theta, rope_type):
    """The rotation as a complex product in float64: pair i of a head (2i,
    2i+1) or (i, i + hd/2) times exp(1j * pos * theta^(-2i/hd))."""
    x = x.astype(np.float64)
    n, hd = x.shape
    half = hd // 2
    i = np.arange(half)
    ang = pos * theta ** (-(2.0 * i) / hd)
    if rope_type == 0:
        z = (x[:, 0::2] + 1j * x[:, 1::2]) * np.exp(1j * ang)
        out = np.empty_like(x)
        out[:, 0::2], out[:, 1::2] = z.real, z.imag
    else:
        z = (x[:, :half] + 1j * x[:, half:]) * np.exp(1j * ang)
        out = np.concatenate([z.real, z.imag], axis=1)
    return out


@pytest.mark.parametrize("rope_type", [0, 1])
@pytest.mark.parametrize("hd,pos", [(8, 3), (64, 17), (128, 1000), (2, 5)])
def test_rope_against_complex_rotation(oracle, rope_type, hd, pos):
    rng = np.random.default_rng(hd + pos)
    q = rng.standard_normal((4, hd)).astype(np.float32)
    k = rng.standard_normal((2, hd)).astype(np.float32)
    qr, kr = oracle.rope(q, k, pos, 10000.0, rope_type)
    # angle pos * freq is formed in float: its rounding (|angle| * 2^-24)
    # bounds the difference to the exact rotation
    tol = 4e-7 * (1 + pos) * np.abs(q).max() + 2e-6
    np.testing.assert_allclose(qr, _rope_complex(q, pos, 10000.0, rope_type), atol=tol, rtol=0)
    np.testing.assert_allclose(kr, _rope_complex(k, pos, 10000.0, rope_type), atol=tol, rtol=0)
    q0, _ = oracle.rope(q, k, 0, 10000.0, rope_type)
    assert np.array_equal(q0, q)


def test_rope_rejections(oracle):
    q = np.zeros((2, 4), np.float32)
    for args in ((-1, 10000.0, 0), (0, 0.0, 0), (0, np.inf, 0)):
        with pytest.raises(ValueError):
            oracle.rope(q, q, *args)
    with pytest.raises(ValueError):
        oracle.rope(np.zeros((2, 3), np.float32), np.zeros((2, 3), np.float32), 0, 1e4, 0)


# ---- attention --------------------------------------------------------------------
def _attention_f64(q, keys, values, layer, pos):
    """softmax(Q K^T / sqrt(d)) V in float64 matrix form, kv head h // group."""
    n_heads, hd = q.shape
    n_kv = keys.shape[2]
    g = n_heads // n_kv
    k = np.repeat(keys[layer, :pos + 1].astype(np.float64), g, axis=1)    # [t, heads, d]
    v = np.repeat(values[layer, :pos + 1].astype(np.float64), g, axis=1)
    s = np.einsum("hd,thd->ht", q.astype(np.float64), k) / np.sqrt(hd)
    p = scipy.special.softmax(s, axis=1)
    return np.einsum("ht,thd->hd", p, v)


def test_attention_reference_closed_forms(oracle):
    # pos 0 returns V of the mapped kv head (tests/test_cuda.cc:999-1029)
    keys = np.zeros((1, 4, 2, 4), np.float32)
    values = np.zeros_like(keys)
    keys[0, 0] = np.arange(8).reshape(2, 4) * 0.2 - 1.0
    values[0, 0] = np.arange(8).reshape(2, 4) * 0.5 + 10.0
    q = (np.arange(16).reshape(4, 4) * 0.3 + 0.25).astype(np.float32)
    out = oracle.attention(q, keys, values, 0, 0)
    np.testing.assert_allclose(out, values[0, 0][[0, 0, 1, 1]], atol=1e-5)
    # zero keys: uniform weights, V[kv0] = 1, V[kv1] = 2 (:1031-1064)
    keys[:] = 0
    values[0, :3, 0], values[0, :3, 1] = 1.0, 2.0
    out = oracle.attention(q, keys, values, 0, 2)
    np.testing.assert_allclose(out, np.array([[1.0] * 4, [1.0] * 4, [2.0] * 4, [2.0] * 4]),
                               atol=1e-5)


@pytest.mark.parametrize("n_heads,n_kv,hd,pos", [(4, 2, 4, 3), (28, 4, 128, 70), (8, 8, 64, 200),
                                                 (16, 2, 100, 31)])
def test_attention_against_matrix_form(oracle, n_heads, n_kv, hd, pos):
    rng = np.random.default_rng(pos)
    keys = rng.standard_normal((2, pos + 3, n_kv, hd)).astype(np.float32)
    values = rng.standard_normal((2, pos + 3, n_kv, hd)).astype(np.float32)
    q = rng.standard_normal((n_heads, hd)).astype(np.float32)
    out = oracle.attention(q, keys, values, 1, pos)
    np.testing.assert_allclose(out, _attention_f64(q, keys, values, 1, pos), atol=2e-5, rtol=1e-4)
    # one-hot: a key aligned with a large q picks its value row
    keys[1, :, :, 0] = 0
    keys[1, pos // 2, :, 0] = 1.0
    q[:] = 0
    q[:, 0] = 400.0
    out = oracle.attention(q, keys, values, 1, pos)
    g = n_heads // n_kv
    np.testing.assert_allclose(out, values[1, pos // 2][np.arange(n_heads) // g], atol=1e-4)


# ---- F32 linear -------------------------------------------------------------------
def test_linear_f32_exact_and_brute_force(oracle):
    rng = np.random.default_rng(3)
    # small integers: every partial sum is exact in fp32
    x = rng.integers(-8, 9, 300).astype(np.float32)
    w = rng.integers(-8, 9, (50, 300)).astype(np.float32)
    assert np.array_equal(oracle.linear_f32(x, w), (w.astype(np.int64) @ x.astype(np.int64)))
    x = rng.standard_normal(4096).astype(np.float32)
    w = rng.standard_normal((64, 4096)).astype(np.float32)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    bound = 4096 * 6e-8 * (np.abs(w) @ np.abs(x))
    assert np.all(np.abs(oracle.linear_f32(x, w) - ref) <= bound)


# ---- the forward composition --------------------------------------------------------
def _dense(w):
    graft.load_oracle()
    o = graft.load_oracle()
    if w["type"] == "f32":
        return np.asarray(w["data"], np.float64).reshape(w["shape"])
    return o.dequantize(w["data"], w["shape"], w["type"]).astype(np.float64)


def _causal_forward_f64(model, tokens):
    """Float64 full-sequence decoder: logits at every position of `tokens`
    with causal attention over all of them at once (no cache), the
    textbook pre-norm Llama / Qwen2 block."""
    c = model["config"]
    nh, nkv = c["n_heads"], c["n_kv_heads"]
    hd = c.get("head_dim", c["dim"] // nh)
    eps = c["rms_norm_eps"]
    T = len(tokens)

    def norm(x, w):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w

    x = model["token_embedding"][tokens].astype(np.float64)
    for lw in model["layers"]:
        h = norm(x, lw["attention_norm"])
        q = h @ _dense(lw["wq"]).T + np.asarray(lw.get("bq", 0.0), np.float64)
        k = h @ _dense(lw["wk"]).T + np.asarray(lw.get("bk", 0.0), np.float64)
        v = h @ _dense(lw["wv"]).T + np.asarray(lw.get("bv", 0.0), np.float64)
        q = np.stack([_rope_complex(q[t].reshape(nh, hd), t, c["rope_theta"], c.get("rope_type", 0))
                      for t in range(T)])
        k = np.stack([_rope_complex(k[t].reshape(nkv, hd), t, c["rope_theta"], c.get("rope_type", 0))
                      for t in range(T)])
        v = v.reshape(T, nkv, hd)
        g = nh // nkv
        kk, vv = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
        s = np.einsum("thd,uhd->htu", q, kk) / np.sqrt(hd)
        s = s + np.triu(np.full((T, T), -np.inf), 1)[None]
        att = np.einsum("htu,uhd->thd", scipy.special.softmax(s, axis=2), vv).reshape(T, nh * hd)
        x = x + att @ _dense(lw["wo"]).T
        h = norm(x, lw["ffn_norm"])
        gate, up = h @ _dense(lw["w_gate"]).T, h @ _dense(lw["w_up"]).T
        x = x + (gate * scipy.special.expit(gate) * up) @ _dense(lw["w_down"]).T
    return norm(x, model["final_norm"]) @ _dense(model["lm_head"]).T


def _synthetic(pkg, qtype, **kw):
    from synthetic import synth
    cfg = dict(vocab_size=96, dim=64, hidden_dim=96, n_layers=2, n_heads=4, n_kv_heads=2,
               max_seq_len=16)
    cfg.update(kw.pop("cfg", {}))
    return synth.synthetic_model(cfg, qtype, seed=kw.pop("seed", 7), **kw)


@pytest.mark.parametrize("qtype,kw", [("f32", {}), ("q8_0", {"bias": True}),
                                      ("q4_0", {"cfg": {"rope_type": 1}}),
                                      ("q4_1", {"cfg": {"n_kv_heads": 4}})])
def test_forward_matches_float64_causal_decoder(oracle, pkg, qtype, kw):
    model = _synthetic(pkg, qtype, **kw)
    tokens = [3, 17, 95, 0, 42, 42, 7]
    ref = _causal_forward_f64(model, tokens)
    cache = oracle.new_cache(model)
    for pos, t in enumerate(tokens):
        logits = oracle.forward_token(model, cache, t, pos)
        scale = np.abs(ref[pos]).max()
        assert np.abs(logits - ref[pos]).max() <= 2e-5 * scale + 1e-6, (qtype, pos)


def test_forward_tiny_model(oracle, pkg):
    """The reference's tiny test model (models/tiny, a fixture the
    reference's own tests load): the oracle's incremental decode equals the
    float64 causal decoder on the reference's "hello" prompt."""
    import mini_llama_amd.decode as dec
    model = dec.load_manifest_model(os.path.join(GOLDEN, "tiny", "model.json"),
                                    os.path.join(GOLDEN, "tiny", "model.bin"))
    assert model["config"]["head_dim"] == 8 and len(model["layers"]) == 2
    tokens = [1] + list(b"hello")  # AsciiTokenizer::encode: BOS + bytes
    ref = _causal_forward_f64(model, tokens)
    cache = oracle.new_cache(model)
    for pos, t in enumerate(tokens):
        logits = oracle.forward_token(model, cache, t, pos)
        assert np.abs(logits - ref[pos]).max() <= 1e-5
    with pytest.raises(ValueError):
        oracle.forward_token(model, cache, 128, 0)
    with pytest.raises(ValueError):
        oracle.forward_token(model, cache, 1, 128)
