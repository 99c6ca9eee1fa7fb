#!/usr/bin/env python3
"""Benchmark of the MI355X block-quantized Linear path (one JSON line).

Headline (`value`): q4_0 decode GEMV at the Qwen2-7B FFN-up shape
(W [18944, 3584], M = 1) in algorithmic HBM GB/s:
bytes = N*ceil(K/32)*18 + 4*M*K + 4*M*N per call. A step is one call on one
activation vector. Weights rotate over >= 512 MB of distinct device copies so
every call streams its weight from HBM (MI355X has a 256 MB Infinity Cache).
The timed launches are captured in one HIP graph and bracketed by HIP events
on the stream they run on.

Also reported in the same line: the q8_0 prefill GEMM (configs[4], M=512,
W [11008, 4096]) in TFLOP/s against the dense fp16 MFMA peak; `configs`
holds the other BASELINE configurations (configs[0], [2] and [3] at M = 4,
16, 64 for q4_0, 16 and 64 for q8_0 / q4_1) in GB/s and fraction of 8 TB/s,
and configs[4]'s 196-GEMV decode sweep (28 Qwen2-7B layers x q,k,v,o,gate,
up,down at M = 1) launched separately, fused (q|k|v, gate|up) and fused
with the bias / SwiGLU epilogues; `roofline.read_ceiling` is one plain
streaming read of the headline's weight bytes (mlq_probe_read in the
bench-only libmlq_probe.so), the
single-launch ceiling the headline is compared against.
`decode_step` reports whole-model decode: a Qwen2-7B-shaped q4_0
model stepped token by token through mlq_decode_token, captured with its
greedy sampling as one HIP graph, in tokens/s and algorithmic GB/s (weights
+ KV cache rows read per token), and its 512-token prefill; `prefill_q8_0`
is the same prefill on a q8_0 model. `prefill_int8` is configs[4] through
the int8-MFMA variant (activation quantize pass + int8 GEMM, both timed;
`vs_fp16` > 1 would mean it beats the fp16 GEMM). `prefill.mfma_ceiling` is a dense fp16 / bf16 GEMM
of the same shape through torch.matmul (hipBLASLt) on the same box, the
ceiling the quantized GEMM is compared against. `cpu_baseline` is the
reference CPU path (the oracle restatement) on the host cores, one thread
per physical core up to the job's 16-thread CPU share, with lscpu's
figures; `cpu_baseline_builds` times every BASELINE workload (configs[0]
to [4] and the decode sweep) in the scalar and the AVX2 build beside this
run's GPU time. `configs.llc_hot` repeats c0-c3 on one weight copy
(Infinity-Cache resident: labelled LLC-hot, not HBM). `--all` adds the
GGUF upload rate.

Profiling modes (one kernel family per run, for rocprofv3 counter passes):
`--mode headline` launches only the headline GEMV (eagerly with `--eager`),
`--mode copy` runs a plain device-to-device copy of 256 MiB, the known-size
reference that scales the FETCH_SIZE / WRITE_SIZE counters to bytes;
`--mode case --case qtype,m,n,k` launches one Linear shape (the skinny and
prefill GEMM counter summaries in profiles/ come from it), `--mode
read-ceiling` times the read probe at every BASELINE weight size and
`--mode sweep` the three 196-GEMV sweeps alone, `--mode skinny-floor` the
load-only floors of the skinny GEMM's access pattern (mlq_probe_read_shared),
`--mode int8-ab` the fp16 prefill GEMM against the int8 variant on three
prefill shapes. `configs.c1_aos` /
`c0_aos` time mlq_linear_aos on raw GGUF blocks (the direct AoS GEMV).
`roofline.traffic` is read from profiles/hbm_traffic_gemv_q4_0_c1.md (the
summary of those counter runs) when it is present, else null.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
# seeded synthetic weights, activations and models (shared with the tests)
sys.path.insert(1, os.path.join(ROOT, "tests"))
import __graft_entry__ as graft  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
MFMA_I8_PEAK_TOPS = 5000.0
ROTATE_BYTES = 512 << 20
COPY_BYTES = 256 << 20
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic_gemv_q4_0_c1.md")

GGUF_BLOCK = {"q8_0": 34, "q4_0": 18, "q4_1": 20}


def alg_bytes(qtype, m, n, k):
    return n * ((k + 31) // 32) * GGUF_BLOCK[qtype] + 4 * m * k + 4 * m * n


def alg_flops(m, n, k):
    return 2 * m * n * k


class Case:
    """One shape: rotated weight copies, fixed activations, output buffer."""

    def __init__(self, pkg, torch, qtype, m, n, k, seed, rotate=True):
        from synthetic import synth
        self.pkg, self.torch = pkg, torch
        self.qtype, self.m, self.n, self.k = qtype, m, n, k
        blocks = synth.make_blocks(qtype, n, k, seed)
        base = pkg.upload(qtype, blocks, n, k, device="cuda")
        copies = max(1, -(-ROTATE_BYTES // base.nbytes)) if rotate else 1
        self.weights = [base]
        for _ in range(copies - 1):
            buf = base.buffer.clone()
            self.weights.append(pkg.TiledWeight(qtype, n, k, buf,
                                                pkg.weight_layout(qtype, n, k)))
        x = synth.make_x(m, k, seed + 1)
        self.x = torch.from_numpy(x if m > 1 else x[0]).to("cuda")
        self.y = torch.empty((m, n) if m > 1 else (n,), dtype=torch.float32,
                             device="cuda")

    def launch(self, i):
        self.pkg.linear(self.weights[i % len(self.weights)], self.x, self.y)


def time_graph(torch, launch, steps, warmup):
    """Capture `steps` launches in a HIP graph; return seconds for one replay
    bracketed by events on the capturing stream (after `warmup` eager and
    one warm replay)."""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(max(warmup, 1)):
            launch(i)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            launch(i)
    graph.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3


def time_eager(torch, launch, steps, warmup):
    """Plain back-to-back launches on one stream (what counter passes see)."""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(max(warmup, 1)):
            launch(i)
        stream.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(steps):
            launch(i)
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3


def read_traffic():
    """HBM bytes per launch of the headline kernel, from the committed
    counter summary (a line `traffic_bytes_per_launch: N`), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1].strip()))
    except OSError:
        return None
    return None


def probe_lib():
    """The bench-only read probes (mini-llama_amd/probe, libmlq_probe.so)."""
    import importlib
    graft.load_package()
    return importlib.import_module("mini_llama_amd.probe")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def bench_case(pkg, torch, qtype, m, n, k, steps, warmup, seed, eager=False, rotate=True):
    log(f"{qtype} m={m} n={n} k={k}: setup{'' if rotate else ' (one weight copy)'}")
    c = Case(pkg, torch, qtype, m, n, k, seed, rotate=rotate)
    sec = (time_eager if eager else time_graph)(torch, c.launch, steps, warmup)
    per = sec / steps
    out = {"qtype": qtype, "m": m, "n": n, "k": k, "copies": len(c.weights),
           "us_per_call": per * 1e6,
           "gbs": alg_bytes(qtype, m, n, k) / per / 1e9,
           "tflops": alg_flops(m, n, k) / per / 1e12}
    assert torch.isfinite(c.y).all().item()
    log(f"{qtype} m={m} n={n} k={k}: {out['us_per_call']:.2f} us/call, "
        f"{out['gbs']:.0f} GB/s, {out['tflops']:.1f} TFLOP/s")
    del c
    torch.cuda.empty_cache()
    return out


def bench_dense_ceiling(torch, m, n, k, steps, warmup):
    """A dense GEMM of the prefill shape on the same box: torch.matmul of
    x [m, k] and W [n, k]^T (hipBLASLt), fp16 and bf16 operands, fp32
    accumulate, W rotated over >= 512 MB of copies like the quantized case.
    It has no weight decode to do, so it bounds what the matrix cores give
    this shape through the vendor library."""
    out = {}
    for name, dt in (("fp16", torch.float16), ("bf16", torch.bfloat16)):
        g = torch.Generator(device="cuda")
        g.manual_seed(11)
        x = torch.randn(m, k, device="cuda", generator=g).to(dt)
        copies = max(1, -(-ROTATE_BYTES // (n * k * 2)))
        ws = [torch.randn(n, k, device="cuda", generator=g).to(dt) for _ in range(copies)]
        y = torch.empty(m, n, device="cuda", dtype=dt)

        def launch(i):
            torch.matmul(x, ws[i % copies].t(), out=y)
        per = time_graph(torch, launch, steps, warmup) / steps
        out[name] = {"us_per_call": round(per * 1e6, 2),
                     "tflops": round(alg_flops(m, n, k) / per / 1e12, 1),
                     "copies": copies}
        log(f"dense {name} {m}x{n}x{k}: {per * 1e6:.2f} us")
        del x, ws, y
        torch.cuda.empty_cache()
    return out


def bench_int8(pkg, torch, m, n, k, steps, warmup, seed, eager=False):
    """The int8-MFMA variant (mlq_linear_q8act: q8_0 activation quantize pass
    + int8 GEMM, both inside the timed region) on q8_0 weights."""
    log(f"int8 q8_0 m={m} n={n} k={k}: setup")
    c = Case(pkg, torch, "q8_0", m, n, k, seed)
    ws = torch.empty(pkg.workspace_bytes_q8act(c.weights[0], m), dtype=torch.uint8,
                     device="cuda")

    def launch(i):
        pkg.linear_q8act(c.weights[i % len(c.weights)], c.x, c.y, workspace=ws)
    per = (time_eager if eager else time_graph)(torch, launch, steps, warmup) / steps
    out = {"qtype": "q8_0", "m": m, "n": n, "k": k, "us_per_call": per * 1e6,
           "tops": alg_flops(m, n, k) / per / 1e12}
    assert torch.isfinite(c.y).all().item()
    log(f"int8 q8_0 m={m} n={n} k={k}: {out['us_per_call']:.2f} us/call, "
        f"{out['tops']:.1f} TOPS")
    del c
    torch.cuda.empty_cache()
    return out


SWEEP_SHAPES = [("q", 3584, 3584), ("k", 512, 3584), ("v", 512, 3584),
                ("o", 3584, 3584), ("gate", 18944, 3584), ("up", 18944, 3584),
                ("down", 3584, 18944)]


def bench_sweep(pkg, torch, steps, warmup, mode):
    """28 layers x {q,k,v,o,gate,up,down} q4_0 GEMVs (hidden 3584, FFN 18944,
    GQA kv 512), M = 1, one fixed x per input size, one graph = one decode
    step's Linear work (3.67 GB of weights, far past the 256 MB Infinity
    Cache). mode "separate" launches the 196 GEMVs one by one; "fused"
    repacks q|k|v and gate|up as concatenated weights (each pair/triple
    shares its input), so a layer is 4 launches instead of 7; "epilogue"
    also adds the q|k|v bias in the kernel (Qwen2 has one) and interleaves
    gate|up for the SwiGLU epilogue, which writes silu(gate) * up (18944
    floats instead of 2 x 18944) — no separate bias, SiLU or multiply
    launch. The weight bytes and flops are the same in every mode. Blocks are
    generated on the device and repacked there (mlq_repack_device)."""
    from synthetic import synth
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5000)
    xs = {kk: torch.from_numpy(synth.make_x(1, kk, 900 + kk)[0]).to("cuda")
          for kk in (3584, 18944)}
    bb = GGUF_BLOCK["q4_0"]
    log(f"sweep ({mode}): building 28 layers on the device")
    calls = []
    for layer in range(28):
        blk = {name: (synth.device_blocks(torch, gen, "q4_0", n, k, 1.0 / np.sqrt(k), "cuda"),
                      n, k) for name, n, k in SWEEP_SHAPES}
        if mode == "separate":
            groups = [[name] for name, _, _ in SWEEP_SHAPES]
        else:
            groups = [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]]
        for g in groups:
            k = blk[g[0]][2]
            row = ((k + 31) // 32) * bb
            bias, act = None, pkg.EPI_NONE
            if len(g) == 1:
                aos, n = blk[g[0]][0], blk[g[0]][1]
            elif mode == "epilogue" and g[0] == "gate":
                ffn = blk["gate"][1]
                # 16-row tiles of 8 gate rows then the matching 8 up rows
                aos = torch.stack([blk["gate"][0].view(ffn // 8, 8 * row),
                                   blk["up"][0].view(ffn // 8, 8 * row)], dim=1).reshape(-1)
                n, act = 2 * ffn, pkg.EPI_SWIGLU
            else:
                aos = torch.cat([blk[nm][0] for nm in g])
                n = sum(blk[nm][1] for nm in g)
                if mode == "epilogue":
                    bias = torch.from_numpy(synth.make_x(1, n, 77 + layer)[0]).to("cuda")
            w = pkg.repack_device("q4_0", aos, n, k)
            del aos
            ny = n // 2 if act == pkg.EPI_SWIGLU else n
            y = torch.empty(ny, dtype=torch.float32, device="cuda")
            calls.append((w, xs[k], y, bias, act))
        del blk
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    def step(_):
        for w, x, y, bias, act in calls:
            pkg.linear(w, x, y, bias=bias, act=act)

    steps = max(1, steps)
    sec = time_graph(torch, step, steps, warmup) / steps
    for _, _, y, _, _ in calls:
        assert torch.isfinite(y).all().item()
    total = sum(alg_bytes("q4_0", 1, n, k) for _ in range(28) for _, n, k in SWEEP_SHAPES)
    flops = sum(alg_flops(1, n, k) for _ in range(28) for _, n, k in SWEEP_SHAPES)
    launches = len(calls)
    del calls
    torch.cuda.empty_cache()
    log(f"sweep ({mode}): {sec * 1e6:.1f} us/step, {total / sec / 1e9:.0f} GB/s")
    return {"gemvs": 196, "launches": launches, "us_per_step": sec * 1e6,
            "gbs": total / sec / 1e9, "bytes": total, "tflops": flops / sec / 1e12}


def bench_aos(pkg, torch, qtype, m, n, k, steps, warmup, seed):
    """mlq_linear_aos on raw GGUF blocks (the reference's device-weight
    meaning), rotated over >= 512 MB of copies: the direct AoS GEMV (m <= 8,
    no workspace) or the repack + tiled kernels."""
    import ctypes
    from synthetic import synth
    blocks = synth.make_blocks(qtype, n, k, seed)
    raw = pkg.upload_aos(blocks, device="cuda")
    copies = max(1, -(-ROTATE_BYTES // raw.numel()))
    bufs = [raw] + [raw.clone() for _ in range(copies - 1)]
    x = torch.from_numpy(synth.make_x(m, k, seed + 1)).to("cuda")
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    need = pkg.aos_workspace_bytes(qtype, n, k, m)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    lib, t, bb = pkg.lib(), pkg.TYPES[qtype], pkg.BLOCK_BYTES[qtype]

    def launch(i):
        b = bufs[i % len(bufs)]
        rc = lib.mlq_linear_aos(t, b.data_ptr(), b.numel() // bb, n, k, x.data_ptr(),
                                y.data_ptr(), m, ws.data_ptr() if need else None, need,
                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, rc
    sec = time_graph(torch, launch, steps, warmup) / steps
    assert torch.isfinite(y).all().item()
    out = {"qtype": qtype, "m": m, "n": n, "k": k, "copies": len(bufs),
           "path": "direct AoS GEMV" if need == 0 else "repack + tiled",
           "us_per_call": round(sec * 1e6, 3),
           "gbs": round(alg_bytes(qtype, m, n, k) / sec / 1e9, 1)}
    out["frac_hbm"] = round(out["gbs"] / HBM_PEAK_GBS, 4)
    log(f"aos {qtype} m={m} n={n} k={k}: {out['us_per_call']} us ({out['path']})")
    del bufs, raw
    torch.cuda.empty_cache()
    return out


READ_SIZES = [("c0 q8_0 4096x4096", "q8_0", 4096, 4096),
              ("c1 q4_0 18944x3584", "q4_0", 18944, 3584),
              ("c2 q4_1 4096x14336", "q4_1", 4096, 14336),
              ("c3 q4_0 4096x4096", "q4_0", 4096, 4096),
              ("c4 q8_0 11008x4096", "q8_0", 11008, 4096),
              ("q|k|v q4_0 4608x3584", "q4_0", 4608, 3584),
              ("gate|up q4_0 37888x3584", "q4_0", 37888, 3584)]


def bench_read_ceiling(pkg, torch, steps, warmup, sizes=None):
    """HBM read ceiling of ONE launch per size: mlq_probe_read (a streaming
    dwordx4 read, nothing else) over the tiled bytes of each BASELINE
    weight, plus 256 MiB and 1 GiB for the asymptote. Launches rotate over
    distinct regions of a pool of >= 512 MB + size (no Infinity-Cache reuse)
    and are timed as one HIP graph like the Linear cases."""
    sizes = READ_SIZES if sizes is None else sizes
    items = [(name, int(pkg.weight_layout(qt, n, k).bytes)) for name, qt, n, k in sizes]
    items += [("256 MiB", 256 << 20), ("1 GiB", 1 << 30)]
    probe = probe_lib()
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = {}
    for name, nbytes in items:
        nbytes = nbytes // 16 * 16
        stride = -(-nbytes // 4096) * 4096
        slots = max(2, -(-ROTATE_BYTES // stride) + 1)
        pool = torch.empty(slots * stride, dtype=torch.uint8, device="cuda")
        pool.fill_(0)  # first touch outside the timed region
        views = [pool[i * stride:i * stride + nbytes] for i in range(slots)]

        def launch(i):
            probe.read(views[i % slots], nbytes, sink)
        n_steps = max(10, min(steps, int(4e10 // nbytes)))
        sec = time_graph(torch, launch, n_steps, warmup) / n_steps
        out[name] = {"bytes": nbytes, "us": round(sec * 1e6, 3),
                     "gbs": round(nbytes / sec / 1e9, 1),
                     "frac_hbm": round(nbytes / sec / 1e9 / HBM_PEAK_GBS, 4),
                     "copies": slots}
        log(f"read ceiling {name}: {nbytes} B, {sec * 1e6:.2f} us, {nbytes / sec / 1e9:.0f} GB/s")
        del views, pool
        torch.cuda.empty_cache()
    assert int(sink.item()) == 0
    return out


SKINNY_FLOOR_CASES = [  # (name, shared bytes per workgroup, own bytes per wave)
    ("weights 36 KiB/WG", 0, 4608),
    ("x 128 KiB/WG", 128 << 10, 0),
    ("x 256 KiB/WG", 256 << 10, 0),
    ("weights + x fp16 M=16 (128 KiB)", 128 << 10, 4608),
    ("weights + x fp32 M=16 (256 KiB)", 256 << 10, 4608),
    ("weights + x fp16 M=4..8 (64 KiB)", 64 << 10, 4608),
]


def bench_skinny_floor(pkg, torch, steps, warmup):
    """Load-only floors of the skinny GEMM's pattern at q4_0 W[4096, 4096]
    (configs[3]): mlq_probe_read_shared with 256 workgroups of 8 waves, each
    workgroup streaming its 36 KiB weight tile from HBM (rotated over a
    >= 512 MB pool) and/or reading the same x region (resident in L2 / the
    Infinity Cache after the first launch). Timed as one HIP graph."""
    wgs = 256
    probe = probe_lib()
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    shared = torch.ones(256 << 10, dtype=torch.uint8, device="cuda")
    out = {}
    for name, sb, opw in SKINNY_FLOOR_CASES:
        per = max(opw, 16) * 8 * wgs
        stride = -(-per // 4096) * 4096
        slots = max(2, -(-ROTATE_BYTES // stride) + 1)
        pool = torch.zeros(slots * stride, dtype=torch.uint8, device="cuda")
        views = [pool[i * stride:i * stride + per] for i in range(slots)]

        def launch(i):
            probe.read_shared(shared, sb, views[i % slots], opw, wgs, sink)
        sec = time_graph(torch, launch, steps, warmup) / steps
        out[name] = {"shared_bytes": sb, "own_bytes_per_wave": opw,
                     "us": round(sec * 1e6, 3)}
        log(f"skinny floor {name}: {sec * 1e6:.2f} us")
        del views, pool
        torch.cuda.empty_cache()
    assert int(sink.item()) == 0
    return out


def bench_gguf_load(pkg, torch, layers=4):
    """Weight load from a GGUF file: `layers` Qwen2-7B layers (q4_0, 7
    Linear tensors each, ~131 MB per layer) written to a temporary file,
    then loaded twice — the reference's way (each tensor read into a host
    buffer, src/gguf.cc:621-662, then one host-to-device copy of the AoS
    blocks, src/cuda_weight_upload.cc; its AoS vector build is left out, in
    its favour) and through GgufFile.upload (mapped file, device copy,
    device repack to the tiled layout). GB/s of GGUF bytes, page cache warm
    for both."""
    import tempfile
    from synthetic import synth
    from synthetic import gguf_writer as gw
    tensors = []
    for layer in range(layers):
        for i, (name, n, k) in enumerate(SWEEP_SHAPES):
            blocks = synth.make_blocks("q4_0", n, k, 7000 + 10 * layer + i)
            tensors.append((f"blk.{layer}.{name}.weight", [k, n], gw.GGML_Q4_0,
                            gw.blocks_bytes(blocks)))
    total = sum(len(t[3]) for t in tensors)
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "model.gguf")
        gw.write_gguf(path, [("general.architecture", gw.STRING, "qwen2")], tensors)
        del tensors
        with pkg.GgufFile(path) as g:
            infos = list(g.tensors)
            for t in infos:  # warm the page cache
                g.data(t["name"])
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ws = [g.upload(t["name"], device="cuda") for t in infos]
            torch.cuda.synchronize()
            ours = time.perf_counter() - t0
        del ws
        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        held = []
        with open(path, "rb") as f:
            for t in infos:
                f.seek(t["offset"])
                raw = np.frombuffer(f.read(t["bytes"]), dtype=np.uint8)
                held.append(torch.from_numpy(raw.copy()).to("cuda"))
        torch.cuda.synchronize()
        ref = time.perf_counter() - t0
        del held
        torch.cuda.empty_cache()
    return {"bytes": total, "tensors": len(infos), "gguf_upload_gbs": total / ours / 1e9,
            "reference_style_gbs": total / ref / 1e9, "gguf_upload_s": ours,
            "reference_style_s": ref}


QWEN2_7B = dict(vocab_size=152064, dim=3584, hidden_dim=18944, n_layers=28, n_heads=28,
                n_kv_heads=4, max_seq_len=4096, rope_theta=1e6, rms_norm_eps=1e-6,
                rope_type=1)


def decode_bytes(dm, pos):
    """Algorithmic HBM bytes of one decode step at position `pos`: every
    Linear weight once (GGUF bytes), the KV rows 0..pos of every layer read
    and one row written, the embedding row and the logits."""
    c = dm.config
    row = c["n_kv_heads"] * c["head_dim"] * 4
    kv = c["n_layers"] * (2 * (pos + 1) * row + 2 * row)
    return dm.weight_bytes + kv + 4 * c["dim"] + 4 * c["vocab_size"]


def bench_decode(pkg, torch, steps, warmup, context=1024, qtype="q4_0", prefill_tokens=512):
    """Whole decode steps of a Qwen2-7B-shaped q4_0 model (28 layers, q|k|v
    biases, NeoX rope, random weights) at positions context..context+steps-1:
    eager mlq_decode_token calls, then one HIP graph of step + greedy
    sampling replayed per token. Tokens/s and algorithmic GB/s."""
    import mini_llama_amd.decode as dec
    from synthetic import synth
    log(f"decode: building a {QWEN2_7B['n_layers']}-layer {qtype} model on the device")
    model = synth.synthetic_model_device(QWEN2_7B, qtype, seed=7, bias=True)
    dm = dec.DecodeModel(model)
    del model
    torch.cuda.synchronize()
    n_eager = max(5, min(steps, 50))
    for i in range(max(warmup, 1)):
        dm.forward_token(1, context + i)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(n_eager):
        dm.forward_token(1 + i, context + i)
    end.record()
    torch.cuda.synchronize()
    eager_ms = start.elapsed_time(end) / n_eager
    log("decode: capturing the step graph")
    dm.token_dev.fill_(1)
    dm.pos_dev.fill_(context)
    g = dm.greedy_graph()
    for _ in range(max(warmup, 1)):
        g.replay()
    dm.pos_dev.fill_(context)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        g.replay()
    end.record()
    torch.cuda.synchronize()
    graph_ms = start.elapsed_time(end) / steps
    end_pos = int(dm.pos_dev.item())
    assert end_pos == context + steps, end_pos
    assert np.isfinite(dm.logits.cpu().numpy()).all()
    nbytes = decode_bytes(dm, context + steps // 2)
    gbs = nbytes / (graph_ms * 1e-3) / 1e9
    out = {"workload": f"Qwen2-7B-shaped {qtype} decode step (28 layers, dim 3584, FFN 18944, "
                       "28/4 heads, head_dim 128, vocab 152064, q|k|v bias), "
                       f"positions {context}..{context + steps - 1}",
           "tokens_per_s": 1e3 / graph_ms, "ms_per_token": graph_ms,
           "ms_per_token_eager": eager_ms, "bytes_per_token": nbytes,
           "weight_bytes": dm.weight_bytes, "gbs": gbs, "steps": steps,
           "roofline_tokens_per_s": HBM_PEAK_GBS * 1e9 / nbytes,
           "frac_hbm": gbs / HBM_PEAK_GBS}
    if prefill_tokens:
        out["prefill"] = bench_prefill(dm, torch, prefill_tokens, max(2, steps // 25))
    return out


def bench_prefill(dm, torch, n, reps):
    """mlq_prefill of an n-token prompt at position 0 (every Linear on
    [n, K]), repeated; tokens/s and the Linear FLOP rate (2 * n * the
    parameters of every layer's projections, lm_head for the last row)."""
    c = dm.config
    rng = np.random.default_rng(3)
    toks = rng.integers(0, c["vocab_size"], n).tolist()
    log(f"prefill: {n} tokens x {reps}")
    dm.prefill(toks, 0)
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dm.prefill(toks, 0)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    hd, dim, hid = c["head_dim"], c["dim"], c["hidden_dim"]
    layer = dim * (c["n_heads"] + 2 * c["n_kv_heads"]) * hd + c["n_heads"] * hd * dim + 3 * dim * hid
    flops = 2.0 * n * layer * c["n_layers"] + 2.0 * c["vocab_size"] * dim
    return {"tokens": n, "ms": ms, "tokens_per_s": n / (ms * 1e-3),
            "linear_tflops": flops / (ms * 1e-3) / 1e12, "reps": reps}


def bench_prefill_model(pkg, torch, qtype, n, reps):
    """mlq_prefill of an n-token prompt on a Qwen2-7B-shaped model of
    another block type (the decode-step model is q4_0)."""
    import mini_llama_amd.decode as dec
    from synthetic import synth
    log(f"prefill: building a {QWEN2_7B['n_layers']}-layer {qtype} model on the device")
    model = synth.synthetic_model_device(QWEN2_7B, qtype, seed=9, bias=True)
    dm = dec.DecodeModel(model)
    del model
    out = bench_prefill(dm, torch, n, reps)
    out["workload"] = (f"Qwen2-7B-shaped {qtype} prefill of {n} tokens at position 0 "
                       "(every Linear on [n, K], attention, lm_head on the last row)")
    del dm
    return {kk: (round(v, 4) if isinstance(v, float) else v) for kk, v in out.items()}


CPU_SHARE = 16  # host threads one GPU's job may use on the GPU boxes


def host_cpu():
    """lscpu's view of the host: model, sockets, physical cores, threads,
    plus the CPUs this process may run on (its affinity mask)."""
    info = {}
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            info[key.strip()] = val.strip()
    except Exception:  # lscpu absent: affinity only
        pass

    def num(key):
        try:
            return int(info.get(key, ""))
        except ValueError:
            return None
    sockets, per_socket, per_core = num("Socket(s)"), num("Core(s) per socket"), num("Thread(s) per core")
    physical = sockets * per_socket if sockets and per_socket else None
    return {"model": info.get("Model name"), "sockets": sockets, "cores_per_socket": per_socket,
            "threads_per_core": per_core, "physical_cores": physical,
            "logical_cpus": num("CPU(s)"), "affinity_cpus": len(os.sched_getaffinity(0))}


def cpu_threads(cpu):
    """Threads for the CPU leg: one per physical core the process may use
    (the reference's default is hardware_concurrency, src/threadpool.cc:13-20),
    capped at the job's CPU share on the GPU boxes."""
    cores = cpu["physical_cores"] or cpu["affinity_cpus"]
    return max(1, min(cores, cpu["affinity_cpus"], CPU_SHARE))


def cpu_baseline(qtype, n, k, budget_s=10.0, flavor="scalar", threads=None):
    """The reference CPU path (oracle restatement of linearQ40 / linearQ80
    with the reference thread partition), timed on this host's cores; flavor
    "avx2" is the build with the reference's AVX2 q8_0 loop (quant.cc:505-628;
    q4_0 / q4_1 have no SIMD path there, quant.cc:637-650)."""
    oracle = graft.load_oracle()
    graft.load_package()
    from synthetic import synth
    if threads is None:
        threads = cpu_threads(host_cpu())
    blocks = synth.make_blocks(qtype, n, k, 1)
    x = synth.make_x(1, k, 2)[0]
    oracle.linear(x, blocks, (n, k), qtype, threads=threads, flavor=flavor)  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.linear(x, blocks, (n, k), qtype, threads=threads, flavor=flavor)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 1000:
            break
    per = el / reps
    build = "scalar -O2" if flavor == "scalar" else "-O2 -mavx2 -mfma"
    return {"value": alg_bytes(qtype, 1, n, k) / per / 1e9, "unit": "GB/s",
            "cores": threads, "kind": "port",
            "sample": f"{reps} full {qtype} GEMV calls W[{n},{k}] M=1 "
                      f"({per * 1e3:.2f} ms/call, {threads} threads, "
                      f"{build} build of oracle/quant_ref.c)"}


def cpu_time(oracle, qtype, blocks, x, n, k, budget_s, flavor, threads):
    """Seconds per call of the oracle Linear (the reference CPU path) on x
    ([k] or [m, k]), repeated until `budget_s` or 1000 calls; a single warm
    call longer than the budget is the sample itself."""
    t0 = time.perf_counter()
    oracle.linear(x, blocks, (n, k), qtype, threads=threads, flavor=flavor)
    first = time.perf_counter() - t0
    if first >= budget_s:
        return first, 1
    reps, t0 = 0, time.perf_counter()
    while True:
        oracle.linear(x, blocks, (n, k), qtype, threads=threads, flavor=flavor)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 1000:
            return el / reps, reps


# every BASELINE workload: (config, key of its GPU result, qtype, m, n, k)
CPU_WORKLOADS = [("configs[0]", "c0", "q8_0", 1, 4096, 4096),
                 ("configs[1]", "headline", "q4_0", 1, 18944, 3584),
                 ("configs[2]", "c2", "q4_1", 1, 4096, 14336),
                 ("configs[3] M=4", "c3_m4", "q4_0", 4, 4096, 4096),
                 ("configs[3] M=16", "c3_m16", "q4_0", 16, 4096, 4096),
                 ("configs[3] M=64", "c3_m64", "q4_0", 64, 4096, 4096),
                 ("configs[4] prefill", "prefill", "q8_0", 512, 11008, 4096)]


def cpu_all_configs(result, threads, budget_s):
    """The reference CPU path on every BASELINE workload, built both ways
    (-O2 and -O2 -mavx2 -mfma, CMakeLists.txt:16-25, 192; only q8_0 has an
    AVX2 loop, quant.cc:505-628, q4_0 / q4_1 run the scalar loop in both
    builds), at `threads` threads, next to the GPU time of the same run.
    The decode sweep is timed as one Qwen2-7B layer's seven GEMVs, x 28."""
    oracle = graft.load_oracle()
    graft.load_package()
    from synthetic import synth
    gpu_us = {"headline": result["ms_per_step"] * 1e3,
              "prefill": result["prefill"]["us_per_call"]}
    for key, v in result["configs"].items():
        if "us_per_call" in v:
            gpu_us[key] = v["us_per_call"]
    rows = []
    flavors = [f for f in ("scalar", "avx2") if oracle.flavor_available(f)]
    for tag, key, qt, m, n, k in CPU_WORKLOADS:
        blocks = synth.make_blocks(qt, n, k, 3000)
        x = synth.make_x(m, k, 3001)
        x = x[0] if m == 1 else x
        for flavor in flavors:
            log(f"cpu {tag} {flavor}")
            per, reps = cpu_time(oracle, qt, blocks, x, n, k, budget_s, flavor, threads)
            row = {"config": tag, "build": flavor, "qtype": qt, "m": m, "n": n, "k": k,
                   "us_per_call": round(per * 1e6, 1), "cores": threads,
                   "sample": f"{reps} call(s) of x[{m},{k}] . W[{n},{k}]^T"}
            if m >= 256:
                row["value"], row["unit"] = round(alg_flops(m, n, k) / per / 1e9, 2), "GFLOP/s"
            else:
                row["value"], row["unit"] = round(alg_bytes(qt, m, n, k) / per / 1e9, 3), "GB/s"
            if key in gpu_us:
                row["gpu_us_per_call"] = round(gpu_us[key], 2)
                row["gpu_speedup"] = round(per * 1e6 / gpu_us[key], 1)
            rows.append(row)
    # one decode-step layer: q, k, v, o, gate, up, down (x 28 layers)
    layer = [(n, k, synth.make_blocks("q4_0", n, k, 6000 + i),
              synth.make_x(1, k, 6100 + i)[0]) for i, (_, n, k) in enumerate(SWEEP_SHAPES)]
    for flavor in flavors:
        log(f"cpu sweep {flavor}")
        reps, t0 = 0, time.perf_counter()
        while True:
            for n, k, blocks, x in layer:
                oracle.linear(x, blocks, (n, k), "q4_0", threads=threads, flavor=flavor)
            reps += 1
            if time.perf_counter() - t0 >= budget_s:
                break
        per = (time.perf_counter() - t0) / reps * 28
        row = {"config": "configs[4] decode sweep (196 GEMVs)", "build": flavor, "qtype": "q4_0",
               "us_per_call": round(per * 1e6, 1), "cores": threads,
               "value": round(sum(alg_bytes("q4_0", 1, n, k) for _, n, k in SWEEP_SHAPES) * 28
                              / per / 1e9, 3), "unit": "GB/s",
               "sample": f"{reps} pass(es) over one layer's 7 GEMVs, x 28 layers"}
        sw = result["configs"].get("sweep", {})
        if "us_per_step" in sw:
            row["gpu_us_per_call"] = sw["us_per_step"]
            row["gpu_speedup"] = round(per * 1e6 / sw["us_per_step"], 1)
        rows.append(row)
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--all", action="store_true",
                    help="also run the GGUF upload timing and the extra bench shapes")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU leg")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--mode", choices=["full", "headline", "copy", "decode", "case",
                                       "read-ceiling", "sweep", "skinny-floor",
                                       "int8-ab"],
                    default="full", help="headline/copy/decode/case: profiling runs")
    ap.add_argument("--case", default="q4_0,16,4096,4096",
                    help="--mode case: qtype,m,n,k of the one shape to launch")
    ap.add_argument("--context", type=int, default=1024,
                    help="first position of the timed decode steps")
    ap.add_argument("--eager", action="store_true",
                    help="launch eagerly instead of replaying a HIP graph")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (no multi-GPU path); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    pkg = graft.load_package()
    pkg.lib()
    assert torch.cuda.is_available(), "bench.py needs a HIP device"

    if args.mode == "copy":
        src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        src.fill_(1)
        torch.cuda.synchronize()
        sec = time_eager(torch, lambda i: dst.copy_(src), args.steps, args.warmup)
        print(json.dumps({"mode": "copy", "bytes_read": COPY_BYTES,
                          "bytes_written": COPY_BYTES,
                          "us_per_copy": sec / args.steps * 1e6}), flush=True)
        return
    if args.mode == "decode":
        r = bench_decode(pkg, torch, min(args.steps, 200), args.warmup, args.context)
        print(json.dumps({"mode": "decode", **r}), flush=True)
        return
    if args.mode == "read-ceiling":
        r = bench_read_ceiling(pkg, torch, args.steps, args.warmup)
        print(json.dumps({"mode": "read-ceiling", "sizes": r}), flush=True)
        return
    if args.mode == "skinny-floor":
        r = bench_skinny_floor(pkg, torch, args.steps, args.warmup)
        print(json.dumps({"mode": "skinny-floor", "cases": r}), flush=True)
        return
    if args.mode == "sweep":
        r = {mode: bench_sweep(pkg, torch, max(1, args.steps // 100), 1, mode)
             for mode in ("separate", "fused", "epilogue")}
        print(json.dumps({"mode": "sweep", **r}), flush=True)
        return
    if args.mode == "int8-ab":
        # fp16 GEMM (default prefill path) against the int8 variant, same box
        rows = []
        for (m, n, k) in ((512, 11008, 4096), (1024, 11008, 4096), (2048, 4096, 4096)):
            f16 = bench_case(pkg, torch, "q8_0", m, n, k, min(args.steps, 200),
                             min(args.warmup, 5), seed=4000, eager=args.eager)
            i8 = bench_int8(pkg, torch, m, n, k, min(args.steps, 200), min(args.warmup, 5),
                            seed=4000, eager=args.eager)
            rows.append({"m": m, "n": n, "k": k, "fp16_us": round(f16["us_per_call"], 2),
                         "int8_us": round(i8["us_per_call"], 2),
                         "fp16_tflops": round(f16["tflops"], 1),
                         "int8_tops": round(i8["tops"], 1)})
        print(json.dumps({"mode": "int8-ab", "cases": rows}), flush=True)
        return
    if args.mode == "case":
        qt, m, n, k = args.case.split(",")
        r = bench_case(pkg, torch, qt, int(m), int(n), int(k), args.steps, args.warmup,
                       seed=100, eager=args.eager)
        print(json.dumps({"mode": "case", **r}), flush=True)
        return
    head = bench_case(pkg, torch, "q4_0", 1, 18944, 3584, args.steps,
                      args.warmup, seed=1000, eager=args.eager)
    if args.mode == "headline":
        print(json.dumps({"mode": "headline", **head}), flush=True)
        return
    # every other BASELINE config (GEMV / skinny shapes), a few seconds each,
    # measured right after the headline, before the GEMM-heavy workloads:
    # taken after the prefill and decode runs the same GEMVs read slower for
    # a while (one box: c2 9.07 vs 8.48 us, c0 5.10 vs 4.97)
    extra = {}
    for name, qt, m, n, k in [("c0", "q8_0", 1, 4096, 4096),
                              ("c2", "q4_1", 1, 4096, 14336),
                              ("c3_m4", "q4_0", 4, 4096, 4096),
                              ("c3_m16", "q4_0", 16, 4096, 4096),
                              ("c3_m64", "q4_0", 64, 4096, 4096),
                              ("c3_m16_q8_0", "q8_0", 16, 4096, 4096),
                              ("c3_m64_q8_0", "q8_0", 64, 4096, 4096),
                              ("c3_m16_q4_1", "q4_1", 16, 4096, 4096),
                              ("c3_m64_q4_1", "q4_1", 64, 4096, 4096)]:
        r = bench_case(pkg, torch, qt, m, n, k, args.steps, args.warmup, 100)
        extra[name] = {kk: (round(v, 3) if isinstance(v, float) else v)
                       for kk, v in r.items()}
        extra[name]["frac_hbm"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
    pre_steps = max(10, min(200, args.steps // 5))
    prefill = bench_case(pkg, torch, "q8_0", 512, 11008, 4096, pre_steps,
                         min(args.warmup, 5), seed=4000)
    result = {
        "metric": "q-GEMV achieved HBM GB/s (% of 8 TB/s); prefill q8_0 GEMM "
                  "TOPS (% MFMA)",
        "value": round(head["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["us_per_call"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights x fp32 activations (23-bit integer activations as fp16 digits, exact MFMA sums, fp32 accumulate)",
        "data": "synthetic (seeded; BASELINE.json distributions)",
        "config": {"workload": "configs[1]: q4_0 GEMV W[18944,3584] M=1 "
                               "(Qwen2-7B FFN-up), weights rotated over "
                               f"{head['copies']} HBM copies",
                   "m": 1, "n": 18944, "k": 3584, "qtype": "q4_0"},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic()},
        "prefill": {"workload": "configs[4]: q8_0 GEMM W[11008,4096] x "
                                "X[512,4096] fp32",
                    "us_per_call": round(prefill["us_per_call"], 2),
                    "tflops": round(prefill["tflops"], 1),
                    "peak_tflops": MFMA_F16_PEAK_TFLOPS,
                    "frac": round(prefill["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
                    "dtype": "fp16 MFMA, fp32 accumulate"},
    }
    dense = bench_dense_ceiling(torch, 512, 11008, 4096, pre_steps, min(args.warmup, 5))
    result["prefill"]["mfma_ceiling"] = {
        "what": "dense fp16 / bf16 GEMM of the same shape through torch.matmul (hipBLASLt), "
                "no weight decode, weights rotated like the quantized case",
        **dense,
        "ours_vs_fp16": round(dense["fp16"]["us_per_call"] / prefill["us_per_call"], 3)}
    pre8 = bench_int8(pkg, torch, 512, 11008, 4096, pre_steps, min(args.warmup, 5), seed=4000)
    result["prefill_int8"] = {
        "workload": "configs[4] int8 variant: X quantized to q8_0 (quantizeToQ80 rules) "
                    "+ int8 MFMA GEMM with per-block fp32 fixup, both timed",
        "us_per_call": round(pre8["us_per_call"], 2), "tops": round(pre8["tops"], 1),
        "peak_tops": MFMA_I8_PEAK_TOPS, "frac": round(pre8["tops"] / MFMA_I8_PEAK_TOPS, 4),
        "vs_fp16": round(prefill["us_per_call"] / pre8["us_per_call"], 3),
        "dtype": "int8 MFMA, int32 per block, fp32 fixup"}
    try:
        dec = bench_decode(pkg, torch, min(args.steps, 200), min(args.warmup, 5), args.context)
        result["decode_step"] = {kk: (round(v, 4) if isinstance(v, float) else v)
                                 for kk, v in dec.items()}
    except Exception as e:  # reported, never fatal to the headline line
        result["decode_step"] = {"error": f"{type(e).__name__}: {e}"}
    torch.cuda.empty_cache()
    try:
        result["prefill_q8_0"] = bench_prefill_model(pkg, torch, "q8_0", 512,
                                                     max(2, min(args.steps, 200) // 25))
    except Exception as e:  # reported, never fatal to the headline line
        result["prefill_q8_0"] = {"error": f"{type(e).__name__}: {e}"}
    torch.cuda.empty_cache()
    # "LLC-hot": one weight copy, resident in the 256 MB Infinity Cache after
    # the warm-up launches; not an HBM figure
    hot = {}
    for name, qt, m, n, k in [("c0", "q8_0", 1, 4096, 4096), ("c1", "q4_0", 1, 18944, 3584),
                              ("c2", "q4_1", 1, 4096, 14336), ("c3_m4", "q4_0", 4, 4096, 4096),
                              ("c3_m16", "q4_0", 16, 4096, 4096),
                              ("c3_m64", "q4_0", 64, 4096, 4096)]:
        r = bench_case(pkg, torch, qt, m, n, k, args.steps, args.warmup, 100, rotate=False)
        hot[name] = {"us_per_call": round(r["us_per_call"], 3), "gbs": round(r["gbs"], 1)}
    extra["llc_hot"] = {"what": "single weight copy re-read every call (Infinity-Cache "
                                "resident): LLC-hot, not HBM bandwidth", **hot}
    # raw GGUF block pointers (mlq_linear_aos, the reference's device-weight
    # meaning) at configs[1] and configs[0]
    extra["c1_aos"] = bench_aos(pkg, torch, "q4_0", 1, 18944, 3584, args.steps,
                                args.warmup, 1000)
    extra["c0_aos"] = bench_aos(pkg, torch, "q8_0", 1, 4096, 4096, args.steps,
                                args.warmup, 100)
    # configs[4]'s decode sweep: 196 GEMVs of one Qwen2-7B decode step
    for mode, key in (("separate", "sweep"), ("fused", "sweep_fused"),
                      ("epilogue", "sweep_epilogue")):
        sw = bench_sweep(pkg, torch, max(1, args.steps // 100), 1, mode)
        sw["frac_hbm"] = round(sw["gbs"] / HBM_PEAK_GBS, 4)
        extra[key] = {kk: (round(v, 3) if isinstance(v, float) else v)
                      for kk, v in sw.items()}
    # the one-launch read ceiling at the headline's weight bytes
    rc = bench_read_ceiling(pkg, torch, args.steps, args.warmup, sizes=READ_SIZES[1:2])
    result["roofline"]["read_ceiling"] = {
        "gbs": rc[READ_SIZES[1][0]]["gbs"], "bytes": rc[READ_SIZES[1][0]]["bytes"],
        "asymptote_gbs_1gib": rc["1 GiB"]["gbs"],
        "frac_of_ceiling": round(head["gbs"] / rc[READ_SIZES[1][0]]["gbs"], 4),
        "probe": "mlq_probe_read (libmlq_probe.so): streaming dwordx4 read of the same bytes, one launch"}
    result["configs"] = extra
    if args.all:
        gl = bench_gguf_load(pkg, torch)
        extra["gguf_load"] = {kk: (round(v, 3) if isinstance(v, float) else v)
                              for kk, v in gl.items()}
        result["configs"] = extra
    if not args.no_cpu:
        log("cpu baseline")
        cpu = host_cpu()
        threads = cpu_threads(cpu)
        result["cpu_baseline"] = cpu_baseline("q4_0", 18944, 3584, args.cpu_budget,
                                              threads=threads)
        result["cpu_baseline"]["value"] = round(result["cpu_baseline"]["value"], 3)
        result["cpu_baseline"]["lscpu"] = cpu
        result["cpu_baseline"]["threads_rule"] = (
            f"one per physical core, capped at the job's {CPU_SHARE}-thread CPU share")
        # the same build at 1 thread and half the threads: how the rate scales
        curve = {}
        for t in sorted({1, max(1, threads // 2)} - {threads}):
            v = cpu_baseline("q4_0", 18944, 3584, min(3.0, args.cpu_budget), threads=t)
            curve[str(t)] = round(v["value"], 3)
        curve[str(threads)] = result["cpu_baseline"]["value"]
        result["cpu_baseline"]["gbs_by_threads"] = curve
        # every BASELINE workload with and without the reference's AVX2
        # build, beside this run's GPU times
        result["cpu_baseline_builds"] = cpu_all_configs(result, threads,
                                                         min(1.0, args.cpu_budget))
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
