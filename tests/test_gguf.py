"""CPU: the GGUF v3 reader (mlq_gguf_*) against files written by
tests/synthetic/gguf_writer.py — tensor infos, data offsets and bytes exactly as
written, and the reference reader's acceptance rules (src/gguf.cc:398-573):
each malformed variant is rejected with MLQ_ERR_FORMAT, each accepted
alignment spelling accepted. No GPU calls.
"""
from __future__ import annotations

import numpy as np
import pytest

import __graft_entry__ as graft
from conftest import make_blocks

graft.load_package()
from synthetic import gguf_writer as gw  # noqa: E402

FORMAT = -7  # MLQ_ERR_FORMAT


def _tensors():
    rng = np.random.default_rng(5)
    q8 = make_blocks("q8_0", 48, 96, seed=1)
    q4 = make_blocks("q4_0", 16, 64, seed=2)
    q41 = make_blocks("q4_1", 32, 160, seed=3)
    f32 = rng.standard_normal(3584).astype(np.float32)
    f16 = rng.standard_normal((4, 7)).astype(np.float16)
    return [("blk.0.ffn_up.weight", [96, 48], gw.GGML_Q8_0, gw.blocks_bytes(q8)),
            ("blk.0.attn_q.weight", [64, 16], gw.GGML_Q4_0, gw.blocks_bytes(q4)),
            ("blk.0.ffn_down.weight", [160, 32], gw.GGML_Q4_1, gw.blocks_bytes(q41)),
            ("output_norm.weight", [3584], gw.GGML_F32, f32.tobytes()),
            ("odd.f16", [7, 4], gw.GGML_F16, f16.tobytes()),
            ("unknown.type", [5, 3], 30, b"")]


METADATA = [("general.architecture", gw.STRING, "qwen2"),
            ("qwen2.block_count", gw.U32, 28),
            ("qwen2.rope.freq_base", gw.F32, 1000000.0),
            ("x.u8", gw.U8, 7), ("x.i8", gw.I8, -7), ("x.u16", gw.U16, 700),
            ("x.i16", gw.I16, -700), ("x.i32", gw.I32, -70000), ("x.bool", gw.BOOL, True),
            ("x.u64", gw.U64, 2 ** 40), ("x.i64", gw.I64, -(2 ** 40)), ("x.f64", gw.F64, 0.25),
            ("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["a", "bb", "<|im_start|>"])),
            ("tokenizer.ggml.token_type", gw.ARRAY, (gw.I32, [1, 2, 3])),
            ("x.nested", gw.ARRAY, (gw.ARRAY, [(gw.U8, [1, 2]), (gw.U8, [3])]))]


@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_reader_returns_what_was_written(pkg, tmp_path, alignment):
    path = str(tmp_path / "m.gguf")
    tensors = _tensors()
    offsets = gw.write_gguf(path, METADATA, tensors, alignment=alignment)
    with pkg.GgufFile(path) as g:
        assert g.alignment == (alignment or 32)
        assert g.data_offset % g.alignment == 0
        assert [t["name"] for t in g.tensors] == [t[0] for t in tensors]
        for info, (name, dims, gtype, raw) in zip(g.tensors, tensors):
            assert info["dims"] == dims and info["type"] == gtype, name
            if gtype == 30:
                assert info["bytes"] == 0  # unsized type: listed, no data
                continue
            assert info["offset"] == offsets[name] and info["bytes"] == len(raw)
            assert g.data(name).tobytes() == raw, name


def _rejects(pkg, path):
    with pytest.raises(pkg.MLQError) as e:
        pkg.GgufFile(path)
    assert e.value.status == FORMAT
    return str(e.value)


def test_reader_rejects_what_the_reference_rejects(pkg, tmp_path):
    t = _tensors()
    p = str(tmp_path / "bad.gguf")
    cases = {
        "magic": dict(magic=b"GGUX"),
        "version 2": dict(version=2),
        "truncated data": dict(truncate=5),
        "tensor count beyond the file": dict(tensor_count=6),
    }
    for label, kw in cases.items():
        # t[:5]: the file ends with the last sized tensor's data
        gw.write_gguf(p, METADATA, t[:5], **kw)
        _rejects(pkg, p)
    bad_tensors = {
        "duplicate name": t[:2] + [t[1]],
        "zero dim": [("z", [0, 16], gw.GGML_F32, b"")],
        "nine dims": [("n", [1] * 9, gw.GGML_F32, b"\0" * 4)],
        "q4_0 numel not a multiple of 32": [("q", [48, 1], gw.GGML_Q4_0, b"\0" * 36)],
    }
    for label, tens in bad_tensors.items():
        gw.write_gguf(p, [], tens)
        _rejects(pkg, p)
    gw.write_gguf(p, METADATA + [METADATA[0]], t)  # duplicate key
    assert "duplicate metadata key" in _rejects(pkg, p)


@pytest.mark.parametrize("vtype,value,expect", [
    (gw.U32, 64, 64), (gw.U64, 1 << 20, 1 << 20), (gw.I16, 128, 128), (gw.U8, 16, 16),
    (gw.STRING, "256", 256), (gw.STRING, " +512", 512), (gw.F32, 64.0, 64),
    (gw.F64, 64.0000001, 64),  # "%g" prints 64
    (gw.U32, 48, None), (gw.U32, 0, None), (gw.U64, 1 << 21, None), (gw.I32, -32, None),
    (gw.BOOL, True, None), (gw.STRING, "0x40", None), (gw.STRING, "", None),
    (gw.F32, 64.5, None), (gw.F64, 2.0 ** 20, None),  # "1.04858e+06"
    (gw.ARRAY, (gw.U32, [64]), None)])
def test_alignment_spellings(pkg, tmp_path, vtype, value, expect):
    """general.alignment as the reference reads it: the value's printed text
    parsed as an unsigned decimal, then a power of two <= 1 MiB."""
    p = str(tmp_path / "a.gguf")
    raw = gw.blocks_bytes(make_blocks("q8_0", 2, 32, seed=9))
    off = gw.write_gguf(p, [("general.alignment", vtype, value)],
                        [("w", [32, 2], gw.GGML_Q8_0, raw)],
                        layout_alignment=expect or 32)
    if expect is None:
        assert "alignment" in _rejects(pkg, p)
        return
    with pkg.GgufFile(p) as g:
        assert g.alignment == expect
        assert g.tensors[0]["offset"] == off["w"] and g.data("w").tobytes() == raw


def test_upload_argument_checks(pkg, tmp_path):
    p = str(tmp_path / "u.gguf")
    gw.write_gguf(p, METADATA, _tensors())
    lib = pkg.lib()
    with pkg.GgufFile(p) as g:
        w = pkg.weight_layout("q8_0", 48, 96)
        w.base = 1
        i_f32 = [t["name"] for t in g.tensors].index("output_norm.weight")
        assert lib.mlq_gguf_upload(g._h, i_f32, 1, 1 << 20, w, None) == -5
        assert lib.mlq_gguf_upload(g._h, 0, 1, 10, w, None) == -4
        w2 = pkg.weight_layout("q8_0", 47, 96)
        w2.base = 1
        assert lib.mlq_gguf_upload(g._h, 0, 1, 1 << 20, w2, None) == -2
        assert lib.mlq_gguf_upload(g._h, 99, 1, 1 << 20, w, None) == -1
        idx = pkg.ctypes.c_int64()
        assert lib.mlq_gguf_find(g._h, b"blk.0.attn_q.weight", pkg.ctypes.byref(idx)) == 0
        assert idx.value == 1
        assert lib.mlq_gguf_find(g._h, b"nope", pkg.ctypes.byref(idx)) == -2
