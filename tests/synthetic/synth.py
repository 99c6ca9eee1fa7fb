"""Seeded synthetic workloads with the value distributions of the benchmark
configurations (numpy only; fp16 fields via numpy's IEEE binary16 rounding).

  q8_0: q ~ U{-127..127}, d = |N(0, 0.02)| / 127        (value = q*d)
  q4_0: nibbles ~ U{0..15}, d = |N(0, 0.02)| / 8         (value = (q-8)*d)
  q4_1: nibbles ~ U{0..15}, d = |N(0, 0.02)| / 15,
        m ~ N(0, 0.01)                                   (value = q*d + m)
  activations: fp32 ~ N(0, 1)
Blocks are GGUF AoS structured arrays (34 / 18 / 20 bytes each).
"""
from __future__ import annotations

import numpy as np

BLOCK_DTYPES = {
    "q8_0": np.dtype([("d", "<u2"), ("qs", "i1", (32,))]),
    "q4_0": np.dtype([("d", "<u2"), ("qs", "u1", (16,))]),
    "q4_1": np.dtype([("d", "<u2"), ("m", "<u2"), ("qs", "u1", (16,))]),
}


def f16_bits(values) -> np.ndarray:
    return np.asarray(values, np.float32).astype(np.float16).view(np.uint16)


def make_blocks(qtype: str, n: int, k: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    count = n * ((k + 31) // 32)
    out = np.empty(count, BLOCK_DTYPES[qtype])
    if qtype == "q8_0":
        out["qs"] = rng.integers(-127, 128, (count, 32), dtype=np.int8)
        out["d"] = f16_bits(np.abs(rng.normal(0.0, 0.02, count)) / 127.0)
    elif qtype == "q4_0":
        out["qs"] = rng.integers(0, 256, (count, 16), dtype=np.uint8)
        out["d"] = f16_bits(np.abs(rng.normal(0.0, 0.02, count)) / 8.0)
    elif qtype == "q4_1":
        out["qs"] = rng.integers(0, 256, (count, 16), dtype=np.uint8)
        out["d"] = f16_bits(np.abs(rng.normal(0.0, 0.02, count)) / 15.0)
        out["m"] = f16_bits(rng.normal(0.0, 0.01, count))
    else:
        raise ValueError(qtype)
    return out


def make_x(m: int, k: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((m, k), dtype=np.float32)


# ---- synthetic decoder models ---------------------------------------------------
# Element RMS of each code distribution (q8_0: U{-127..127}; q4_0: nibble - 8;
# q4_1: nibble - 7.5 with m = -7.5 d): the scale d is drawn as |N(0, s)| with
# s = rms / code_rms so a weight row has the requested element RMS.
_CODE_RMS = {"q8_0": float(np.sqrt(127 * 128 / 3)), "q4_0": float(np.sqrt(21.5)),
             "q4_1": float(np.sqrt(21.25))}


def make_blocks_scaled(qtype: str, n: int, k: int, seed: int, rms: float) -> np.ndarray:
    """GGUF blocks whose dequantized elements have RMS ~ rms (zero mean)."""
    rng = np.random.default_rng(seed)
    count = n * ((k + 31) // 32)
    out = np.empty(count, BLOCK_DTYPES[qtype])
    d = np.abs(rng.normal(0.0, rms / _CODE_RMS[qtype], count))
    if qtype == "q8_0":
        out["qs"] = rng.integers(-127, 128, (count, 32), dtype=np.int8)
    else:
        out["qs"] = rng.integers(0, 256, (count, 16), dtype=np.uint8)
    if qtype == "q4_1":
        out["m"] = f16_bits(-7.5 * d)
    out["d"] = f16_bits(d)
    return out


def _linear(qtype: str, n: int, k: int, seed: int) -> dict:
    rms = 1.0 / np.sqrt(k)
    if qtype == "f32":
        rng = np.random.default_rng(seed)
        return {"type": "f32", "shape": (n, k),
                "data": (rng.standard_normal((n, k)) * rms).astype(np.float32)}
    return {"type": qtype, "shape": (n, k), "data": make_blocks_scaled(qtype, n, k, seed, rms)}


def synthetic_model(config: dict, qtype: str = "q4_0", seed: int = 0,
                    bias: bool = False, lm_head_type: str | None = None) -> dict:
    """A random decoder in the model-dict format of mini_llama_amd.decode:
    every projection of type `qtype` with element RMS 1/sqrt(in_features),
    norm weights 1 + N(0, 0.1), embedding N(0, 1), optional q/k/v biases
    N(0, 0.1) (Qwen2 style). `config` holds the ModelConfig fields."""
    c = dict(config)
    c.setdefault("head_dim", c["dim"] // c["n_heads"])
    c.setdefault("rope_theta", 10000.0)
    c.setdefault("rms_norm_eps", 1e-5)
    c.setdefault("rope_type", 0)
    rng = np.random.default_rng(seed)
    dim, hid, hd = c["dim"], c["hidden_dim"], c["head_dim"]
    qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd

    def norm():
        return (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32)

    layers = []
    for li in range(c["n_layers"]):
        s = seed * 1000 + li * 16
        layer = {"attention_norm": norm(),
                 "wq": _linear(qtype, qd, dim, s + 1), "wk": _linear(qtype, kvd, dim, s + 2),
                 "wv": _linear(qtype, kvd, dim, s + 3), "wo": _linear(qtype, dim, qd, s + 4),
                 "ffn_norm": norm(),
                 "w_gate": _linear(qtype, hid, dim, s + 5), "w_up": _linear(qtype, hid, dim, s + 6),
                 "w_down": _linear(qtype, dim, hid, s + 7)}
        if bias:
            for name, n in (("bq", qd), ("bk", kvd), ("bv", kvd)):
                layer[name] = (0.1 * rng.standard_normal(n)).astype(np.float32)
        layers.append(layer)
    return {"config": c,
            "token_embedding": rng.standard_normal((c["vocab_size"], dim)).astype(np.float32),
            "final_norm": norm(),
            "lm_head": _linear(lm_head_type or qtype, c["vocab_size"], dim, seed * 1000 + 999),
            "layers": layers}


def device_blocks(torch, gen, qtype: str, n: int, k: int, rms: float, device):
    """GGUF block bytes made on the device (same distributions as
    make_blocks_scaled), [n * ceil(k/32) * block bytes] uint8."""
    count = n * ((k + 31) // 32)
    d = (torch.randn(count, generator=gen, device=device) * (rms / _CODE_RMS[qtype])).abs()
    d16 = d.half()
    parts = [d16.view(torch.uint8).reshape(count, 2)]
    if qtype == "q4_1":
        parts.append((-7.5 * d16.float()).half().view(torch.uint8).reshape(count, 2))
    if qtype == "q8_0":
        qs = torch.randint(-127, 128, (count, 32), generator=gen, device=device,
                           dtype=torch.int16).to(torch.int8).view(torch.uint8)
    else:
        qs = torch.randint(0, 256, (count, 16), generator=gen, device=device,
                           dtype=torch.int16).to(torch.uint8)
    parts.append(qs)
    return torch.cat(parts, dim=1).reshape(-1)


def synthetic_model_device(config: dict, qtype: str = "q4_0", seed: int = 0,
                           bias: bool = False, device: str = "cuda") -> dict:
    """synthetic_model with every array generated on the device (torch),
    for models too large to build on the host quickly (a 7B decoder is
    ~4 GB of q4_0 blocks plus a 2 GB fp32 embedding table)."""
    import torch
    c = dict(config)
    c.setdefault("head_dim", c["dim"] // c["n_heads"])
    c.setdefault("rope_theta", 10000.0)
    c.setdefault("rms_norm_eps", 1e-5)
    c.setdefault("rope_type", 0)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    dim, hid, hd = c["dim"], c["hidden_dim"], c["head_dim"]
    qd, kvd = c["n_heads"] * hd, c["n_kv_heads"] * hd

    def lin(n, k):
        rms = 1.0 / float(np.sqrt(k))
        if qtype == "f32":
            return {"type": "f32", "shape": (n, k),
                    "data": torch.randn(n, k, generator=gen, device=device) * rms}
        return {"type": qtype, "shape": (n, k),
                "data": device_blocks(torch, gen, qtype, n, k, rms, device)}

    def norm():
        return 1.0 + 0.1 * torch.randn(dim, generator=gen, device=device)

    layers = []
    for _ in range(c["n_layers"]):
        layer = {"attention_norm": norm(), "wq": lin(qd, dim), "wk": lin(kvd, dim),
                 "wv": lin(kvd, dim), "wo": lin(dim, qd), "ffn_norm": norm(),
                 "w_gate": lin(hid, dim), "w_up": lin(hid, dim), "w_down": lin(dim, hid)}
        if bias:
            for name, n in (("bq", qd), ("bk", kvd), ("bv", kvd)):
                layer[name] = 0.1 * torch.randn(n, generator=gen, device=device)
        layers.append(layer)
    return {"config": c,
            "token_embedding": torch.randn(c["vocab_size"], dim, generator=gen, device=device),
            "final_norm": norm(), "lm_head": lin(c["vocab_size"], dim), "layers": layers}
