"""The decode step on the device: the Python host mirror of the reference's
forwardToken device branch (src/forward.cc:763-784), its weight upload
(uploadModelWeightsToCuda, src/model.cc:151-199) and CudaKvCache.

A model is a plain dict (the same format the CPU oracle reads):
  {"config": {vocab_size, dim, hidden_dim, n_layers, n_heads, n_kv_heads,
              head_dim, max_seq_len, rope_theta, rms_norm_eps, rope_type},
   "token_embedding": fp32 [vocab, dim], "final_norm": fp32 [dim],
   "lm_head": W,
   "layers": [{"attention_norm", "wq", "wk", "wv", "bq"?, "bk"?, "bv"?, "wo",
               "ffn_norm", "w_gate", "w_up", "w_down"}, ...]}
with every projection W = {"type": "f32" | "q8_0" | "q4_0" | "q4_1",
"shape": (n, k), "data": fp32 [n, k] or GGUF blocks}. Arrays may be numpy
(uploaded; quantized blocks repacked on the host) or torch device tensors
(quantized blocks as raw bytes, repacked by the device kernel).

DecodeModel uploads it once. Where the types allow it, q|k|v become one
concatenated weight (one GEMV with the concatenated bias fused) and
gate|up one interleaved weight whose GEMV applies SwiGLU on the way out; the
residual adds ride on the o and down projections' bias epilogue. Every step
is one mlq_decode_token call (about nine launches per layer), and
greedy_graph() captures step + greedy sampling as one HIP graph that reads
the token and position from device memory, so generation replays it with no
host round trip. There is no CPU fallback: without libmlq.so nothing runs.
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np

from . import (MlqKvCache, MlqLayer, MlqModel, MlqWeight, TiledWeight, _check, _stream,
               interleave_rows, lib, repack_device, upload, upload_concat, upload_f32,
               upload_glu, weight_layout)

CONFIG_KEYS = ("vocab_size", "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
               "head_dim", "max_seq_len")


def _on_device(a) -> bool:
    return hasattr(a, "is_cuda") and a.is_cuda


def _device_linear(qtype: str, data, n: int, k: int) -> TiledWeight:
    """A weight whose data already lives on the device: fp32 [n, k] used as
    is, GGUF blocks (uint8 bytes) repacked by the device kernel."""
    import torch
    raw = data.contiguous().view(-1).view(torch.uint8)
    if qtype == "f32":
        return TiledWeight("f32", n, k, raw, weight_layout("f32", n, k))
    return repack_device(qtype, raw, n, k)


def _upload_linear(w: dict, device) -> TiledWeight:
    n, k = w["shape"]
    if _on_device(w["data"]):
        return _device_linear(w["type"], w["data"], n, k)
    if w["type"] == "f32":
        return upload_f32(np.asarray(w["data"], np.float32).reshape(n, k), device=device)
    return upload(w["type"], w["data"], n, k, device=device)


def _upload_rows(ws: list, device) -> TiledWeight:
    """Row concatenation of weights of one type sharing in_features (GGUF
    block rows or fp32 rows concatenate as bytes)."""
    k = ws[0]["shape"][1]
    n = sum(w["shape"][0] for w in ws)
    if _on_device(ws[0]["data"]):
        import torch
        cat = torch.cat([w["data"].contiguous().view(torch.uint8).reshape(-1) for w in ws])
        return _device_linear(ws[0]["type"], cat, n, k)
    if ws[0]["type"] == "f32":
        return upload_f32(np.concatenate([np.asarray(w["data"], np.float32).reshape(w["shape"])
                                          for w in ws]), device=device)
    tw, _ = upload_concat(ws[0]["type"], [(w["data"], w["shape"][0]) for w in ws], k,
                          device=device)
    return tw


def _upload_gate_up(gate: dict, up: dict, device) -> TiledWeight:
    hid, k = gate["shape"]
    if _on_device(gate["data"]):
        # rows 16t..16t+7 = gate rows 8t..8t+7, 16t+8..16t+15 = up rows (as
        # mlq_interleave_rows), done on the device's row bytes
        import torch
        g = gate["data"].contiguous().view(torch.uint8).reshape(hid // 8, 8, -1)
        u = up["data"].contiguous().view(torch.uint8).reshape(hid // 8, 8, -1)
        return _device_linear(gate["type"], torch.stack([g, u], dim=1).reshape(-1), 2 * hid, k)
    if gate["type"] == "f32":
        g = np.asarray(gate["data"], np.float32).reshape(hid, k)
        u = np.asarray(up["data"], np.float32).reshape(hid, k)
        return upload_f32(interleave_rows(g, u, hid).reshape(2 * hid, k), device=device)
    return upload_glu(gate["type"], gate["data"], up["data"], hid, k, device=device)


class DecodeModel:
    """A model resident on one device with its KV cache and workspace."""

    def __init__(self, model: dict, device: str = "cuda", fuse: bool = True,
                 cache_len: int | None = None):
        """cache_len: KV-cache capacity in positions (default and minimum:
        the model's max_seq_len)."""
        import torch
        c = dict(model["config"])
        c.setdefault("head_dim", c["dim"] // c["n_heads"])
        c.setdefault("rope_type", 0)
        self.config = c
        self.device = torch.device(device)
        self._keep = []  # device tensors and weights referenced by the structs

        def dev(a) -> int:
            if _on_device(a):
                t = a.to(self.device, torch.float32).contiguous()
            else:
                t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(self.device)
            self._keep.append(t)
            return t.data_ptr()

        def weight(tw: TiledWeight) -> MlqWeight:
            self._keep.append(tw)
            return tw.layout

        n_layers = c["n_layers"]
        hd = c["head_dim"]
        self.fused_qkv, self.fused_glu = [], []
        self._layers = (MlqLayer * n_layers)()
        for i, lw in enumerate(model["layers"]):
            L = self._layers[i]
            L.attn_norm = dev(lw["attention_norm"])
            L.ffn_norm = dev(lw["ffn_norm"])
            qkv = [lw["wq"], lw["wk"], lw["wv"]]
            fuse_qkv = fuse and len({w["type"] for w in qkv}) == 1
            biases = [lw.get(b) for b in ("bq", "bk", "bv")]
            biases = [b.cpu().numpy() if _on_device(b) else b for b in biases]
            if fuse_qkv:
                L.wq = weight(_upload_rows(qkv, self.device))
                if any(b is not None and np.size(b) for b in biases):
                    sizes = [w["shape"][0] for w in qkv]
                    L.bq = dev(np.concatenate([
                        np.asarray(b, np.float32) if b is not None and np.size(b)
                        else np.zeros(n, np.float32) for b, n in zip(biases, sizes)]))
            else:
                L.wq, L.wk, L.wv = (weight(_upload_linear(w, self.device)) for w in qkv)
                for name, b in zip(("bq", "bk", "bv"), biases):
                    if b is not None and np.size(b):
                        setattr(L, name, dev(b))
            self.fused_qkv.append(fuse_qkv)
            L.wo = weight(_upload_linear(lw["wo"], self.device))
            gate, up = lw["w_gate"], lw["w_up"]
            fuse_glu = (fuse and gate["type"] == up["type"] and gate["shape"][0] % 8 == 0)
            if fuse_glu:
                L.w_gate = weight(_upload_gate_up(gate, up, self.device))
            else:
                L.w_gate = weight(_upload_linear(gate, self.device))
                L.w_up = weight(_upload_linear(up, self.device))
            self.fused_glu.append(fuse_glu)
            L.w_down = weight(_upload_linear(lw["w_down"], self.device))

        m = MlqModel()
        for key in CONFIG_KEYS:
            setattr(m, key, int(c[key]))
        m.rope_theta = float(c["rope_theta"])
        m.rms_norm_eps = float(c["rms_norm_eps"])
        m.rope_type = int(c["rope_type"])
        m.token_embedding = dev(model["token_embedding"])
        m.final_norm = dev(model["final_norm"])
        m.lm_head = weight(_upload_linear(model["lm_head"], self.device))
        m.layers = self._layers
        self._model = m

        nbytes = ctypes.c_size_t()
        _check(lib().mlq_decode_workspace(ctypes.byref(m), ctypes.byref(nbytes)),
               "mlq_decode_workspace")
        self.workspace = torch.empty(nbytes.value, dtype=torch.uint8, device=self.device)
        cap = max(int(cache_len or 0), c["max_seq_len"])
        shape = (n_layers, cap, c["n_kv_heads"], hd)
        self.keys = torch.zeros(shape, dtype=torch.float32, device=self.device)
        self.values = torch.zeros(shape, dtype=torch.float32, device=self.device)
        self._cache = MlqKvCache(self.keys.data_ptr(), self.values.data_ptr(), n_layers,
                                 cap, c["n_kv_heads"], hd)
        self.logits = torch.empty(c["vocab_size"], dtype=torch.float32, device=self.device)
        self.token_dev = torch.zeros(1, dtype=torch.int32, device=self.device)
        self.pos_dev = torch.zeros(1, dtype=torch.int32, device=self.device)
        _check(lib().mlq_argmax_workspace(c["vocab_size"], ctypes.byref(nbytes)),
               "mlq_argmax_workspace")
        self.argmax_ws = torch.empty(nbytes.value, dtype=torch.uint8, device=self.device)
        self._prefill_ws = None

    @property
    def weight_bytes(self) -> int:
        """Bytes of every Linear weight as stored in its source format (GGUF
        blocks or fp32): the bytes one decode step must stream."""
        return sum(k.gguf_bytes for k in self._keep if isinstance(k, TiledWeight))

    def reset(self) -> None:
        """Clear the KV cache (CudaKvCache::clear)."""
        self.keys.zero_()
        self.values.zero_()

    def forward_token(self, token: int, pos: int, stream=None):
        """logits [vocab] for `token` at position `pos` (forwardToken). The
        returned tensor is overwritten by the next step."""
        ws = self.workspace
        _check(lib().mlq_decode_token(ctypes.byref(self._model), ctypes.byref(self._cache),
                                      int(token), int(pos), None, None,
                                      self.logits.data_ptr(), ws.data_ptr(), ws.numel(),
                                      _stream(stream)),
               "mlq_decode_token")
        return self.logits

    def prefill(self, tokens, start_pos: int = 0, stream=None):
        """logits [vocab] of the last of `tokens` after running all of them
        at positions start_pos.. at once (forwardBatch with [n, K] Linears);
        their K/V rows land in the cache. Overwritten by the next step."""
        import torch
        toks = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(-1))
        nbytes = ctypes.c_size_t()
        _check(lib().mlq_prefill_workspace(ctypes.byref(self._model), toks.size,
                                           ctypes.byref(nbytes)), "mlq_prefill_workspace")
        if self._prefill_ws is None or self._prefill_ws.numel() < nbytes.value:
            self._prefill_ws = torch.empty(nbytes.value, dtype=torch.uint8, device=self.device)
        ws = self._prefill_ws
        _check(lib().mlq_prefill(ctypes.byref(self._model), ctypes.byref(self._cache),
                                 toks.ctypes.data, toks.size, int(start_pos),
                                 self.logits.data_ptr(), ws.data_ptr(), ws.numel(),
                                 _stream(stream)),
               "mlq_prefill")
        return self.logits

    def step_device(self, stream=None) -> None:
        """One decode step for the token and position held in token_dev /
        pos_dev, then token_dev = argmax(logits) and pos_dev += 1."""
        ws = self.workspace
        s = _stream(stream)
        _check(lib().mlq_decode_token(ctypes.byref(self._model), ctypes.byref(self._cache),
                                      0, 0, self.token_dev.data_ptr(), self.pos_dev.data_ptr(),
                                      self.logits.data_ptr(), ws.data_ptr(), ws.numel(), s),
               "mlq_decode_token")
        self._greedy(s)

    def _greedy(self, s) -> None:
        _check(lib().mlq_greedy_next(self.logits.data_ptr(), self.config["vocab_size"],
                                     self.token_dev.data_ptr(), self.pos_dev.data_ptr(),
                                     self.argmax_ws.data_ptr(), self.argmax_ws.numel(), s),
               "mlq_greedy_next")

    def greedy_graph(self):
        """A torch.cuda.CUDAGraph of step_device (captured on a side stream)."""
        import torch
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            self.step_device(stream=s)
        torch.cuda.current_stream(self.device).wait_stream(s)
        return g

    def argmax(self, stream=None) -> int:
        """Greedy choice over the current logits (argMax) on the device."""
        import torch
        out = torch.empty(1, dtype=torch.int32, device=self.device)
        _check(lib().mlq_argmax(self.logits.data_ptr(), self.logits.numel(), out.data_ptr(),
                                _stream(stream)), "mlq_argmax")
        return int(out.item())

    def generate_greedy(self, prompt, n_new: int, graph: bool = True,
                        prefill: bool = False) -> list:
        """The reference's greedy loop (tests/test_forward.cc:53-84): each
        prompt token at its position (or all of them at once with
        prefill=True), then n_new sampled tokens, each fed back at the next
        position. Returns the n_new new tokens."""
        import torch
        prompt = [int(t) for t in prompt]
        if not prompt or len(prompt) + n_new > self.config["max_seq_len"]:
            raise ValueError("prompt empty or longer than the cache")
        if prefill:
            self.prefill(prompt, 0)
        else:
            for i, t in enumerate(prompt):
                self.forward_token(t, i)
        self.pos_dev.fill_(len(prompt) - 1)
        self._greedy(_stream(None))
        history = torch.empty(n_new, dtype=torch.int32, device=self.device)
        history[0:1].copy_(self.token_dev)
        g = self.greedy_graph() if graph and n_new > 1 else None
        for i in range(1, n_new):
            if g is not None:
                g.replay()
            else:
                self.step_device()
            history[i:i + 1].copy_(self.token_dev)
        return history.cpu().tolist()


def load_manifest_model(json_path: str, bin_path: str) -> dict:
    """A model in the reference's manifest format (model.json + raw fp32
    model.bin; loadModel, src/loader.cc:805-1000): config fields as
    parseConfig reads them (head_dim = dim / n_heads, NORMAL rope), tensors
    by name at their byte offsets, every projection fp32."""
    with open(json_path, "r", encoding="utf-8") as f:
        manifest = json.load(f)
    c = {key: int(manifest["config"][key]) for key in
         ("vocab_size", "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
          "max_seq_len")}
    c["rope_theta"] = float(manifest["config"]["rope_theta"])
    c["rms_norm_eps"] = float(manifest["config"]["rms_norm_eps"])
    c["head_dim"] = c["dim"] // c["n_heads"]
    c["rope_type"] = 0
    size = os.path.getsize(bin_path)
    raw = np.memmap(bin_path, dtype=np.uint8, mode="r", shape=(size,))
    tensors = {}
    for t in manifest["tensors"]:
        if t.get("dtype", "float32") != "float32":
            raise ValueError(f"{t['name']}: only float32 tensors are supported")
        off, nbytes = int(t["offset"]), int(t["byte_size"])
        if off + nbytes > size or nbytes != 4 * int(np.prod(t["shape"])):
            raise ValueError(f"{t['name']}: bad offset or size")
        tensors[t["name"]] = np.array(raw[off:off + nbytes]).view(np.float32).reshape(t["shape"])

    def lin(name):
        a = tensors[name]
        return {"type": "f32", "shape": tuple(a.shape), "data": a}

    layers = []
    for i in range(c["n_layers"]):
        p = f"layers.{i}."
        layer = {"attention_norm": tensors[p + "attention_norm"],
                 "ffn_norm": tensors[p + "ffn_norm"]}
        for name in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            layer[name] = lin(p + name)
        for name in ("bq", "bk", "bv"):
            if p + name in tensors:
                layer[name] = tensors[p + name]
        layers.append(layer)
    return {"config": c, "token_embedding": tensors["token_embedding"],
            "final_norm": tensors["final_norm"], "lm_head": lin("lm_head"),
            "layers": layers}
