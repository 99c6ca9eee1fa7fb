"""CPU: argument checks of the decode-step C ABI (no device work: every case
returns before a launch), the F32 weight layout, the manifest loader on the
reference's tiny model fixture and the synthetic model builder."""
from __future__ import annotations

import ctypes
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FAKE = 1 << 20  # a non-null pointer that no check dereferences


def test_f32_weight_layout(pkg):
    w = pkg.weight_layout("f32", 100, 37)
    assert (w.type, w.n, w.k, w.bytes, w.qs_off, w.d_off) == (0, 100, 37, 100 * 37 * 4, 0, 0)
    lib = pkg.lib()
    w.base = FAKE
    w.bytes = 10
    assert lib.mlq_linear(ctypes.byref(w), FAKE, FAKE, 1, None) == -1
    w.bytes = 100 * 37 * 4
    assert lib.mlq_linear_path(ctypes.byref(w), FAKE, FAKE, 1, pkg.PATH_MFMA, None) == -5
    nbytes = ctypes.c_size_t(7)
    assert lib.mlq_linear_workspace(ctypes.byref(w), 5, ctypes.byref(nbytes)) == 0
    assert nbytes.value == 0
    assert lib.mlq_dequantize(ctypes.byref(w), 0, 1, FAKE, None) == -1


def test_operator_validation(pkg):
    lib = pkg.lib()
    assert lib.mlq_rmsnorm(None, FAKE, FAKE, 1, 8, 1e-5, None) == -1
    assert lib.mlq_rmsnorm(FAKE, FAKE, FAKE, 0, 8, 1e-5, None) == -2
    assert lib.mlq_rmsnorm(FAKE, FAKE, FAKE, 1, 8, 0.0, None) == -1   # src/cuda_ops.cu:99-101
    assert lib.mlq_rmsnorm(FAKE, FAKE, FAKE, 1, 8, float("nan"), None) == -1
    assert lib.mlq_add(FAKE, None, FAKE, 4, None) == -1
    assert lib.mlq_silu(FAKE, FAKE, 0, None) == -2
    assert lib.mlq_embedding(FAKE, 10, 4, 10, FAKE, None) == -1
    assert lib.mlq_embedding(FAKE, 10, 4, -1, FAKE, None) == -1
    # rope: the checks of rope / cudaRopeDeviceInput (src/ops.cc:187-218)
    assert lib.mlq_rope(FAKE, FAKE, 4, 2, 7, 0, 1e4, 0, None) == -2
    assert lib.mlq_rope(FAKE, FAKE, 4, 2, 8, -1, 1e4, 0, None) == -1
    assert lib.mlq_rope(FAKE, FAKE, 4, 2, 8, 0, 0.0, 0, None) == -1
    assert lib.mlq_rope(FAKE, FAKE, 4, 2, 8, 0, float("inf"), 0, None) == -1
    assert lib.mlq_rope(FAKE, FAKE, 4, 2, 8, 0, 1e4, 2, None) == -1
    assert lib.mlq_argmax(FAKE, 0, FAKE, None) == -2
    assert lib.mlq_greedy_next(FAKE, 10, None, FAKE, FAKE, 1 << 20, None) == -1
    assert lib.mlq_greedy_next(FAKE, 10, FAKE, FAKE, FAKE, 8, None) == -4
    assert lib.mlq_greedy_next(FAKE, 10, FAKE, FAKE, FAKE + 4, 1 << 20, None) == -1


def test_cache_and_attention_validation(pkg):
    lib = pkg.lib()
    nbytes = ctypes.c_size_t()
    assert lib.mlq_kv_cache_bytes(28, 4096, 4, 128, ctypes.byref(nbytes)) == 0
    assert nbytes.value == 28 * 4096 * 4 * 128 * 4
    c = pkg.MlqKvCache(FAKE, FAKE, 2, 64, 4, 128)
    assert lib.mlq_attention_workspace(ctypes.byref(c), 28, ctypes.byref(nbytes)) == 0
    # m, l and hd partials per (query head, chunk): a chunk is the positions
    # one register-kernel workgroup covers (four waves of 64 lanes x 16 fp32
    # values / head_dim: 64 / 32 / 16 at head_dim 64 / 128 / 256), at most
    # the LDS kernel's 32
    assert nbytes.value == 28 * 2 * (2 + 128) * 4
    for hd, chunk in ((64, 32), (128, 32), (256, 16), (80, 32), (8, 32)):
        ch = pkg.MlqKvCache(FAKE, FAKE, 2, 64, 4, hd)
        assert lib.mlq_attention_workspace(ctypes.byref(ch), 8, ctypes.byref(nbytes)) == 0
        assert nbytes.value == 8 * (64 // chunk) * (2 + hd) * 4
    assert lib.mlq_attention_workspace(ctypes.byref(c), 30, ctypes.byref(nbytes)) == -2
    assert lib.mlq_attention_workspace(ctypes.byref(c), 4 * 17, ctypes.byref(nbytes)) == -5
    big = pkg.MlqKvCache(FAKE, FAKE, 1, 8, 1, 512)
    assert lib.mlq_attention_workspace(ctypes.byref(big), 1, ctypes.byref(nbytes)) == -5
    call = lib.mlq_attention_decode
    assert call(ctypes.byref(c), 2, 0, FAKE, 28, FAKE, FAKE, 1 << 20, None) == -2
    assert call(ctypes.byref(c), 0, 64, FAKE, 28, FAKE, FAKE, 1 << 20, None) == -2
    assert call(ctypes.byref(c), 0, 0, FAKE, 28, FAKE, FAKE, 16, None) == -4
    assert call(ctypes.byref(c), 0, 0, FAKE, 28, FAKE, None, 1 << 20, None) == -1
    assert lib.mlq_kv_write(ctypes.byref(c), 0, 64, FAKE, FAKE, None) == -2
    empty = pkg.MlqKvCache(None, FAKE, 2, 64, 4, 128)
    assert lib.mlq_kv_write(ctypes.byref(empty), 0, 0, FAKE, FAKE, None) == -1


def _fake_model(pkg, cfg, qtype="q4_0", fuse_qkv=True, fuse_glu=True):
    """An mlq_model whose weight pointers are fake (only shapes are read)."""
    n_layers = cfg["n_layers"]
    hd = cfg["head_dim"]
    qd, kvd, dim, hid = cfg["n_heads"] * hd, cfg["n_kv_heads"] * hd, cfg["dim"], cfg["hidden_dim"]

    def w(n, k):
        lay = pkg.weight_layout(qtype, n, k)
        lay.base = FAKE
        return lay
    layers = (pkg.MlqLayer * n_layers)()
    for i in range(n_layers):
        lw = layers[i]
        lw.attn_norm = lw.ffn_norm = FAKE
        if fuse_qkv:
            lw.wq = w(qd + 2 * kvd, dim)
        else:
            lw.wq, lw.wk, lw.wv = w(qd, dim), w(kvd, dim), w(kvd, dim)
        lw.wo = w(dim, qd)
        if fuse_glu:
            lw.w_gate = w(2 * hid, dim)
        else:
            lw.w_gate, lw.w_up = w(hid, dim), w(hid, dim)
        lw.w_down = w(dim, hid)
    m = pkg.MlqModel()
    for key in ("vocab_size", "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
                "head_dim", "max_seq_len"):
        setattr(m, key, cfg[key])
    m.rope_theta, m.rms_norm_eps, m.rope_type = 1e6, 1e-6, 1
    m.token_embedding = m.final_norm = FAKE
    m.lm_head = w(cfg["vocab_size"], dim)
    m.layers = layers
    return m, layers


QWEN2_7B = dict(vocab_size=152064, dim=3584, hidden_dim=18944, n_layers=28, n_heads=28,
                n_kv_heads=4, head_dim=128, max_seq_len=4096)


def test_decode_workspace_plan(pkg):
    lib = pkg.lib()
    nbytes = ctypes.c_size_t()
    for fq, fg in ((True, True), (False, False)):
        m, _ = _fake_model(pkg, QWEN2_7B, fuse_qkv=fq, fuse_glu=fg)
        assert lib.mlq_decode_workspace(ctypes.byref(m), ctypes.byref(nbytes)) == 0
        # activations (a few hundred KiB) + attention partials for 4096 positions
        attn = 28 * (4096 // 32) * (2 + 128) * 4
        assert attn <= nbytes.value <= attn + (1 << 20)
    m, layers = _fake_model(pkg, QWEN2_7B)
    layers[3].wo.n = 3583
    assert lib.mlq_decode_workspace(ctypes.byref(m), ctypes.byref(nbytes)) == -2
    m, layers = _fake_model(pkg, QWEN2_7B)
    layers[0].wo.base = None
    assert lib.mlq_decode_workspace(ctypes.byref(m), ctypes.byref(nbytes)) == -1
    m, _ = _fake_model(pkg, QWEN2_7B)
    m.rms_norm_eps = 0.0
    assert lib.mlq_decode_workspace(ctypes.byref(m), ctypes.byref(nbytes)) == -1
    m, _ = _fake_model(pkg, dict(QWEN2_7B, hidden_dim=18940, n_layers=1))
    assert lib.mlq_decode_workspace(ctypes.byref(m), ctypes.byref(nbytes)) == -2  # fused GLU
    m, _ = _fake_model(pkg, dict(QWEN2_7B, n_kv_heads=5, n_layers=1))
    assert lib.mlq_decode_workspace(ctypes.byref(m), ctypes.byref(nbytes)) == -2


def test_decode_token_host_checks(pkg):
    lib = pkg.lib()
    m, _ = _fake_model(pkg, dict(QWEN2_7B, n_layers=2))
    nbytes = ctypes.c_size_t()
    assert lib.mlq_decode_workspace(ctypes.byref(m), ctypes.byref(nbytes)) == 0
    c = pkg.MlqKvCache(FAKE, FAKE, 2, 4096, 4, 128)
    ws = 1 << 24  # 256-aligned fake address

    def call(token, pos, cache=c, ws_ptr=ws, ws_bytes=nbytes.value):
        return lib.mlq_decode_token(ctypes.byref(m), ctypes.byref(cache), token, pos, None, None,
                                    FAKE, ws_ptr, ws_bytes, None)
    assert call(152064, 0) == -1   # validateForwardInputs (src/forward.cc:33-45)
    assert call(0, 4096) == -1
    assert call(0, 0, ws_bytes=nbytes.value - 1) == -4
    assert call(0, 0, ws_ptr=ws + 4) == -1
    assert call(0, 0, cache=pkg.MlqKvCache(FAKE, FAKE, 3, 4096, 4, 128)) == -2
    assert call(0, 0, cache=pkg.MlqKvCache(FAKE, FAKE, 2, 100, 4, 128)) == -2


def test_manifest_loader_reads_the_tiny_model(pkg):
    import mini_llama_amd.decode as dec
    m = dec.load_manifest_model(os.path.join(GOLDEN, "tiny", "model.json"),
                                os.path.join(GOLDEN, "tiny", "model.bin"))
    c = m["config"]
    assert (c["vocab_size"], c["dim"], c["hidden_dim"], c["n_layers"], c["head_dim"]) == \
        (128, 32, 86, 2, 8)
    assert m["token_embedding"].shape == (128, 32)
    assert m["layers"][1]["w_down"]["shape"] == (32, 86)
    # 21 tensors, all of them read (tests/test_cuda.cc:1203-1205 counts 21 uploads)
    names = ("attention_norm", "ffn_norm", "wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down")
    assert 3 + sum(len([k for k in lw if k in names]) for lw in m["layers"]) == 21
    raw = np.fromfile(os.path.join(GOLDEN, "tiny", "model.bin"), dtype=np.float32)
    assert np.array_equal(m["token_embedding"].reshape(-1), raw[:128 * 32])


def test_synthetic_model_weight_scale(pkg, oracle):
    from synthetic import synth
    cfg = dict(vocab_size=64, dim=256, hidden_dim=512, n_layers=1, n_heads=4, n_kv_heads=2,
               max_seq_len=8)
    for qtype in ("q8_0", "q4_0", "q4_1", "f32"):
        m = synth.synthetic_model(cfg, qtype, seed=3)
        w = m["layers"][0]["w_gate"]
        dense = (w["data"] if qtype == "f32" else
                 oracle.dequantize(w["data"], w["shape"], qtype))
        rms = float(np.sqrt(np.mean(dense.astype(np.float64) ** 2)))
        assert 0.6 / 16 < rms < 1.5 / 16, (qtype, rms)   # 1/sqrt(256)
        assert abs(float(dense.mean())) < 0.2 / 16
