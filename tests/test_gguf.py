"""GGUF container parsing / writing and expert-slab addressing (host only).

The format facts checked here are the GGUF specification's (header, value
types, tensor table, alignment) and the reference's expert addressing
(crates/engine/src/lib.rs:541-593, 3963-3973; crates/stream/src/lib.rs:14-48);
files are written by this package's writer or assembled by hand with struct.
"""
import struct

import numpy as np
import pytest

from pulsar_amd import formats as fm
from pulsar_amd import gguf as G

TT = G.TensorType


def _kv(key, ty, payload):
    k = key.encode()
    return struct.pack("<Q", len(k)) + k + struct.pack("<I", ty) + payload


def test_row_bytes_table():
    # closed forms: ceil(n / block) * bytes
    assert G.type_row_bytes(TT.Q4_K, 4096) == 16 * 144
    assert G.type_row_bytes(TT.Q6_K, 4096) == 16 * 210
    assert G.type_row_bytes(TT.Q2_K, 1536) == 6 * 84
    assert G.type_row_bytes(TT.IQ2_XXS, 4096) == 16 * 66
    assert G.type_row_bytes(TT.MXFP4, 2880) == 90 * 17
    assert G.type_row_bytes(TT.Q8_0, 704) == 22 * 34
    assert G.type_row_bytes(TT.Q4_K, 300) == 2 * 144  # partial super-block rounds up
    assert G.type_row_bytes(TT.F32, 7) == 28 and G.type_row_bytes(TT.BF16, 7) == 14
    assert G.type_row_bytes(999, 256) is None
    # the kernels' own table agrees for every format they run
    for ty, q in G.QUANT_OF_TYPE.items():
        for n in (256, 512, 2880 if q == fm.QUANT_MXFP4 else 4096):
            assert G.type_row_bytes(ty, n) == fm.row_bytes(q, n)


def test_parse_every_value_type():
    kvs = [
        _kv("a.u8", 0, struct.pack("<B", 200)), _kv("a.i8", 1, struct.pack("<b", -5)),
        _kv("a.u16", 2, struct.pack("<H", 60000)), _kv("a.i16", 3, struct.pack("<h", -30000)),
        _kv("a.u32", 4, struct.pack("<I", 4000000000)), _kv("a.i32", 5, struct.pack("<i", -7)),
        _kv("a.f32", 6, struct.pack("<f", 1.5)), _kv("a.bool", 7, struct.pack("<?", True)),
        _kv("a.str", 8, struct.pack("<Q", 3) + b"abc"),
        _kv("a.arr", 9, struct.pack("<IQ", 8, 2) + struct.pack("<Q", 1) + b"x" + struct.pack("<Q", 2) + b"yz"),
        _kv("a.nested", 9, struct.pack("<IQ", 9, 1) + struct.pack("<IQ", 4, 2) + struct.pack("<II", 1, 2)),
        _kv("a.u64", 10, struct.pack("<Q", 1 << 40)), _kv("a.i64", 11, struct.pack("<q", -(1 << 40))),
        _kv("a.f64", 12, struct.pack("<d", 0.25)),
    ]
    head = struct.pack("<IIQQ", G.GGUF_MAGIC, 3, 0, len(kvs)) + b"".join(kvs)
    g = G.Gguf.parse(head)
    m = g.metadata
    assert (m["a.u8"], m["a.i8"], m["a.u16"], m["a.i16"]) == (200, -5, 60000, -30000)
    assert (m["a.u32"], m["a.i32"], m["a.f32"], m["a.bool"]) == (4000000000, -7, 1.5, True)
    assert m["a.str"] == "abc" and m["a.arr"] == ["x", "yz"] and m["a.nested"] == [[1, 2]]
    assert (m["a.u64"], m["a.i64"], m["a.f64"]) == (1 << 40, -(1 << 40), 0.25)
    assert g.version == 3 and g.tensors == [] and g.alignment == 32
    assert g.data_offset == -(-len(head) // 32) * 32


@pytest.mark.parametrize("head,msg", [
    (struct.pack("<IIQQ", 0x12345678, 3, 0, 0), "not a GGUF"),
    (struct.pack("<IIQQ", G.GGUF_MAGIC, 1, 0, 0), "version"),
    (struct.pack("<IIQQ", G.GGUF_MAGIC, 4, 0, 0), "version"),
    (struct.pack("<IIQ", G.GGUF_MAGIC, 3, 0), "truncated"),
    (struct.pack("<IIQQ", G.GGUF_MAGIC, 3, 0, 1) + _kv("k", 13, b""), "value type"),
    (struct.pack("<IIQQ", G.GGUF_MAGIC, 3, 0, 1) + _kv("k", 8, struct.pack("<Q", 2) + b"\xff\xfe"), "utf-8"),
    (struct.pack("<IIQQ", G.GGUF_MAGIC, 3, 1 << 21, 0), "tensor count"),
    (struct.pack("<IIQQ", G.GGUF_MAGIC, 3, 0, 1) + _kv("k", 8, struct.pack("<Q", 100) + b"ab"), "truncated"),
])
def test_parse_errors(head, msg):
    with pytest.raises(G.GgufError, match=msg):
        G.Gguf.parse(head)


def _rand(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8).tobytes()


def test_write_parse_round_trip(tmp_path):
    p = tmp_path / "t.gguf"
    md = {"general.architecture": "qwen3moe", "qwen3moe.expert_count": 4, "general.name": "tiny",
          "qwen3moe.rope_freq_base": 1e6, "tokenizer.ggml.tokens": ["a", "b", "c"], "big": 1 << 40, "neg": -3}
    E, ff, hid = 4, 256, 512
    tensors = [
        ("blk.0.ffn_gate_exps.weight", (hid, ff, E), TT.Q4_K, _rand(E * ff * 2 * 144, 1)),
        ("blk.0.ffn_up_exps.weight", (hid, ff, E), TT.Q4_K, _rand(E * ff * 2 * 144, 2)),
        ("blk.0.ffn_down_exps.weight", (ff, hid, E), TT.Q6_K, _rand(E * hid * 210, 3)),
        ("blk.0.ffn_gate_inp.weight", (hid, E), TT.F32, _rand(hid * E * 4, 4)),
        ("output_norm.weight", (7,), TT.F32, _rand(28, 5)),  # odd size: the next offset is re-aligned
    ]
    offs = G.write_gguf(p, md, tensors, alignment=64)
    raw = p.read_bytes()
    g = G.Gguf.open(p)
    assert g.alignment == 64 and g.data_offset % 64 == 0 and g.metadata["general.alignment"] == 64
    for k, v in md.items():
        assert g.metadata[k] == (pytest.approx(v) if isinstance(v, float) else v)
    assert [t.name for t in g.tensors] == [t[0] for t in tensors]
    for (name, dims, ty, data), t in zip(tensors, g.tensors):
        assert t.dims == tuple(dims) and t.ty == ty and t.offset % 64 == 0
        a = g.data_offset + t.offset
        assert a == offs[name] and raw[a:a + t.byte_size()] == data
    assert g.arch_meta("expert_count") == 4 and g.architecture() == "qwen3moe"
    # unconsumed: what no lookup asked for
    g.tensor("blk.0.ffn_gate_inp.weight")
    assert "blk.0.ffn_gate_inp.weight" not in g.unconsumed() and "output_norm.weight" in g.unconsumed()
    # a head that stops right after the tensor table still parses
    assert G.Gguf.parse(raw[:g.data_offset]).tensors[2].offset == g.tensors[2].offset


def test_layer_experts_and_reads(tmp_path):
    p = tmp_path / "m.gguf"
    E, ff, hid = 3, 320, 576
    md = {"general.architecture": "gpt-oss", "gpt-oss.expert_count": E}
    mx = lambda rows, cols, s: _rand(E * rows * (cols // 32) * 17, s)  # noqa: E731
    tensors = [
        ("blk.0.ffn_gate_exps.weight", (hid, ff, E), TT.MXFP4, mx(ff, hid, 1)),
        ("blk.0.ffn_up_exps.weight", (hid, ff, E), TT.MXFP4, mx(ff, hid, 2)),
        ("blk.0.ffn_down_exps.weight", (ff, hid, E), TT.MXFP4, mx(hid, ff, 3)),
        ("blk.0.ffn_gate_exps.bias", (ff, E), TT.F32, _rand(E * ff * 4, 4)),
        ("blk.0.ffn_up_exps.bias", (ff, E), TT.F32, _rand(E * ff * 4, 5)),
        ("blk.0.ffn_down_exps.bias", (hid, E), TT.F32, _rand(E * hid * 4, 6)),
        # layer 1: fused gate_up (gemma4-style), Q2_K down
        ("blk.1.ffn_gate_up_exps.weight", (512, 2 * 256, E), TT.Q4_K, _rand(E * 512 * 2 * 144, 7)),
        ("blk.1.ffn_down_exps.weight", (256, 512, E), TT.Q2_K, _rand(E * 512 * 84, 8)),
    ]
    offs = G.write_gguf(p, md, tensors)
    g = G.Gguf.open(p)
    lx = G.layer_experts(g, 0)
    assert lx.fused_up_off == 0 and lx.n_ff == ff
    assert lx.gate.quant == fm.QUANT_MXFP4 and lx.gate.row_bytes == fm.row_bytes(fm.QUANT_MXFP4, hid)
    assert lx.gate.expert_bytes == ff * lx.gate.row_bytes and lx.down.rows == hid
    assert lx.gate.abs_offset == offs["blk.0.ffn_gate_exps.weight"]
    assert lx.gate.slab(2) == (lx.gate.abs_offset + 2 * lx.gate.expert_bytes, lx.gate.expert_bytes)
    assert [b.name for b in lx.biases] == [f"blk.0.ffn_{x}_exps.bias" for x in ("gate", "up", "down")]
    with pytest.raises(IndexError):
        lx.gate.slab(E)
    l1 = G.layer_experts(g, 1)
    assert l1.up is l1.gate and l1.n_ff == 256 and l1.fused_up_off == 256 * 2 * 144
    assert l1.down.quant == fm.QUANT_Q2_K and l1.biases == (None, None, None)
    # the read plan: every *_exps.weight slab in file order
    reads = G.expert_reads(g, p.stat().st_size)
    exps = [t for t in tensors if t[0].endswith("_exps.weight")]
    assert len(reads) == len(exps) * E
    for j, (name, dims, ty, data) in enumerate(exps):
        eb = len(data) // E
        assert reads[j * E:(j + 1) * E] == [(offs[name] + e * eb, eb) for e in range(E)]
    assert G.plan_to_string(reads[:2]) == f"{reads[0][0]} {reads[0][1]}\n{reads[1][0]} {reads[1][1]}\n"
    with pytest.raises(G.GgufError, match="beyond eof"):
        G.expert_reads(g, p.stat().st_size - 1)
    with pytest.raises(G.GgufError, match="no routed expert"):
        G.layer_experts(g, 2)


def test_expert_errors(tmp_path):
    p = tmp_path / "bad.gguf"
    md = {"general.architecture": "x", "x.expert_count": 2}
    G.write_gguf(p, md, [("blk.0.ffn_gate_exps.weight", (256, 4, 2), TT.Q5_0, _rand(2 * 4 * 176, 1)),
                         ("blk.0.ffn_up_exps.weight", (256, 4, 3), TT.Q4_K, _rand(3 * 4 * 144, 2))])
    g = G.Gguf.open(p)
    with pytest.raises(G.GgufError, match="unsupported expert type"):
        G.ExpertTensor.of(g, g.tensors[0], 2)
    with pytest.raises(G.GgufError, match="dims"):
        G.ExpertTensor.of(g, g.tensors[1], 2)
    with pytest.raises(G.GgufError, match="expert_count"):
        G.layer_experts(G.Gguf(3, {}, [], 32, 0), 0)
    with pytest.raises(G.GgufError, match="data bytes"):
        G.write_gguf(tmp_path / "x.gguf", {}, [("t", (256,), TT.Q4_K, b"\0" * 10)])
