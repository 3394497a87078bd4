"""GGUF container and expert-slab addressing for the expert kernels.

What a loader needs so that checkpoint weights drive the kernels as they
sit in the file:

* the GGUF header, metadata and tensor table (crates/gguf/src/lib.rs:
  parse 268-330, value types 460-497, alignment / data offset 317-322),
  read from the head of the file only (tensor data is never touched while
  parsing), plus a writer for the same layout (tests, synthetic files);
* tensor types and their block layouts (crates/gguf/src/lib.rs:45-180) and
  row bytes `ceil(n / block) * block_bytes`;
* routed-expert tensors `blk.<l>.ffn_{gate,up,down}_exps.weight`
  [n_expert][rows][row_bytes] as uniform per-expert slabs: expert e at
  `data_offset + tensor.offset + e * expert_bytes`
  (crates/engine/src/lib.rs:541-593, crates/stream/src/lib.rs:14-48), with
  a fused `ffn_gate_up_exps` tensor serving gate and up (up rows start
  `row_bytes * n_ff` bytes into the slab, crates/engine/src/lib.rs:3963-3973)
  and `SLAB_SLACK` bytes after every device slab
  (crates/engine/src/lib.rs:595-600);
* the device upload of one layer's banks as a `kernels.ExpertBank`.

The table of type ids and block layouts is the GGUF format's, so it matches
the reference's; the code is this package's own.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass, field
from enum import IntEnum
from pathlib import Path

from . import formats as fm

GGUF_MAGIC = 0x46554747  # "GGUF" little-endian
DEFAULT_ALIGNMENT = 32
SLAB_SLACK = 256  # bytes after every device expert slab


class GgufError(ValueError):
    """Malformed or unsupported GGUF content (the reference's gguf::Error)."""


class TensorType(IntEnum):
    """GGML storage type ids (crates/gguf/src/lib.rs:83-110)."""
    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q2_K = 10
    Q3_K = 11
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    Q8_K = 15
    IQ2_XXS = 16
    IQ2_XS = 17
    IQ3_XXS = 18
    IQ1_S = 19
    IQ4_NL = 20
    IQ3_S = 21
    IQ2_S = 22
    IQ4_XS = 23
    I32 = 26
    BF16 = 30
    MXFP4 = 39
    NVFP4 = 40


# (values per block, bytes per block), crates/gguf/src/lib.rs:145-173
BLOCK_LAYOUT = {
    TensorType.F32: (1, 4), TensorType.I32: (1, 4),
    TensorType.F16: (1, 2), TensorType.BF16: (1, 2),
    TensorType.Q4_0: (32, 18), TensorType.Q5_0: (32, 22), TensorType.Q5_1: (32, 24), TensorType.Q8_0: (32, 34),
    TensorType.Q2_K: (256, 84), TensorType.Q3_K: (256, 110), TensorType.Q4_K: (256, 144),
    TensorType.Q5_K: (256, 176), TensorType.Q6_K: (256, 210), TensorType.Q8_K: (256, 292),
    TensorType.IQ2_XXS: (256, 66), TensorType.IQ2_XS: (256, 74), TensorType.IQ2_S: (256, 82),
    TensorType.IQ1_S: (256, 50), TensorType.IQ3_XXS: (256, 98), TensorType.IQ3_S: (256, 110),
    TensorType.IQ4_XS: (256, 136), TensorType.IQ4_NL: (32, 18),
    TensorType.MXFP4: (32, 17), TensorType.NVFP4: (64, 36),
}

# file type -> kernel quant code (crates/engine/src/lib.rs:551-573: every
# expert format the reference dispatches)
QUANT_OF_TYPE = {
    TensorType.IQ2_XXS: fm.QUANT_IQ2_XXS,
    TensorType.Q2_K: fm.QUANT_Q2_K,
    TensorType.Q4_K: fm.QUANT_Q4_K,
    TensorType.Q5_K: fm.QUANT_Q5_K,
    TensorType.Q6_K: fm.QUANT_Q6_K,
    TensorType.Q3_K: fm.QUANT_Q3_K,
    TensorType.IQ2_XS: fm.QUANT_IQ2_XS,
    TensorType.IQ3_XXS: fm.QUANT_IQ3_XXS,
    TensorType.Q4_0: fm.QUANT_Q4_0,
    TensorType.Q5_1: fm.QUANT_Q5_1,
    TensorType.Q8_0: fm.QUANT_Q8_0,
    TensorType.IQ4_XS: fm.QUANT_IQ4_XS,
    TensorType.IQ4_NL: fm.QUANT_IQ4_NL,
    TensorType.IQ3_S: fm.QUANT_IQ3_S,
    TensorType.IQ2_S: fm.QUANT_IQ2_S,
    TensorType.IQ1_S: fm.QUANT_IQ1_S,
    TensorType.MXFP4: fm.QUANT_MXFP4,
    TensorType.NVFP4: fm.QUANT_NVFP4,
}


def type_from_id(ty: int):
    """TensorType for a known id, else the raw int (the reference's Other)."""
    try:
        return TensorType(ty)
    except ValueError:
        return int(ty)


def type_row_bytes(ty, n: int) -> int | None:
    """Bytes of a row of n values of type ty; None when the layout is unknown."""
    lay = BLOCK_LAYOUT.get(ty)
    if lay is None:
        return None
    bs, bb = lay
    return -(-n // bs) * bb


# metadata value types (crates/gguf/src/lib.rs:460-497)
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}
T_STRING, T_ARRAY = 8, 9


@dataclass
class TensorInfo:
    name: str
    dims: tuple  # GGUF order, fastest-varying first
    ty: object  # TensorType or raw id
    offset: int  # relative to the data section

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    def byte_size(self) -> int | None:
        """Total bytes (row = dims[0]), None for an unknown type."""
        if not self.dims:
            return None
        rb = type_row_bytes(self.ty, self.dims[0])
        if rb is None:
            return None
        rows = 1
        for d in self.dims[1:]:
            rows *= d
        return rb * max(rows, 1)


class _Cursor:
    def __init__(self, buf):
        self.buf, self.at = buf, 0

    def take(self, n: int):
        end = self.at + n
        if n < 0 or end > len(self.buf):
            raise GgufError(f"truncated at byte {self.at}: need {n}, have {len(self.buf) - self.at}")
        s = self.buf[self.at:end]
        self.at = end
        return s

    def unpack(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.unpack("<Q")
        at = self.at
        raw = bytes(self.take(n))
        try:
            return raw.decode("utf-8")
        except UnicodeDecodeError:
            raise GgufError(f"invalid utf-8 in string at byte {at}") from None

    def value(self, ty: int, depth: int = 0):
        if ty in _SCALAR:
            v = self.unpack(_SCALAR[ty])
            return bool(v) if ty == 7 else v
        if ty == T_STRING:
            return self.string()
        if ty == T_ARRAY:
            if depth > 2:
                raise GgufError(f"unknown metadata value type {ty}")
            ety = self.unpack("<I")
            count = self.unpack("<Q")
            if count > 1 << 26:
                raise GgufError(f"implausible array element count {count}")
            return [self.value(ety, depth + 1) for _ in range(count)]
        raise GgufError(f"unknown metadata value type {ty}")


@dataclass
class Gguf:
    version: int
    metadata: dict
    tensors: list
    alignment: int
    data_offset: int  # absolute file offset of the tensor data section
    _consumed: set = field(default_factory=set, repr=False)

    @staticmethod
    def parse(head) -> "Gguf":
        """Header + metadata + tensor table from the head of a GGUF file
        (crates/gguf/src/lib.rs:268-330); `head` need not hold tensor data."""
        c = _Cursor(memoryview(head))
        magic = c.unpack("<I")
        if magic != GGUF_MAGIC:
            raise GgufError(f"not a GGUF file (magic {magic:#010x})")
        version = c.unpack("<I")
        if version not in (2, 3):
            raise GgufError(f"unsupported GGUF version {version}")
        n_tensors, n_kv = c.unpack("<Q"), c.unpack("<Q")
        if n_tensors > 1 << 20:
            raise GgufError(f"implausible tensor count {n_tensors}")
        if n_kv > 1 << 20:
            raise GgufError(f"implausible metadata kv count {n_kv}")
        metadata = {}
        for _ in range(n_kv):
            key = c.string()
            metadata[key] = c.value(c.unpack("<I"))
        tensors = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.unpack("<I")
            if nd > 8:
                raise GgufError(f"implausible tensor dim count {nd}")
            dims = tuple(c.unpack("<Q") for _ in range(nd))
            ty = type_from_id(c.unpack("<I"))
            tensors.append(TensorInfo(name, dims, ty, c.unpack("<Q")))
        align = metadata.get("general.alignment")
        if not (isinstance(align, int) and not isinstance(align, bool) and align > 0 and align & (align - 1) == 0):
            align = DEFAULT_ALIGNMENT
        data_offset = -(-c.at // align) * align
        return Gguf(version, metadata, tensors, align, data_offset)

    @staticmethod
    def open(path, head_bytes: int = 32 << 20) -> "Gguf":
        """Parse a file's header from (at most) its first head_bytes bytes."""
        with open(path, "rb") as f:
            return Gguf.parse(f.read(head_bytes))

    def architecture(self):
        a = self.metadata.get("general.architecture")
        return a if isinstance(a, str) else None

    def arch_meta(self, suffix: str):
        a = self.architecture()
        return None if a is None else self.metadata.get(f"{a}.{suffix}")

    def tensor(self, name: str):
        """Tensor by name (marks it consumed), None if absent."""
        for t in self.tensors:
            if t.name == name:
                self._consumed.add(name)
                return t
        return None

    def unconsumed(self) -> list:
        """Names of tensors nothing looked up, in file order
        (crates/gguf/src/lib.rs:360-389)."""
        return [t.name for t in self.tensors if t.name not in self._consumed]


def _value_bytes(v) -> tuple:
    """(type id, encoded value) for a Python metadata value."""
    if isinstance(v, bool):
        return 7, struct.pack("<?", v)
    if isinstance(v, int):
        if 0 <= v < 1 << 32:
            return 4, struct.pack("<I", v)
        if -(1 << 31) <= v < 0:
            return 5, struct.pack("<i", v)
        return (10, struct.pack("<Q", v)) if v >= 0 else (11, struct.pack("<q", v))
    if isinstance(v, float):
        return 6, struct.pack("<f", v)
    if isinstance(v, str):
        b = v.encode("utf-8")
        return T_STRING, struct.pack("<Q", len(b)) + b
    if isinstance(v, (list, tuple)):
        if not v:
            return T_ARRAY, struct.pack("<IQ", 4, 0)
        enc = [_value_bytes(x) for x in v]
        ety = enc[0][0]
        if any(e[0] != ety for e in enc):
            raise GgufError("mixed-type metadata array")
        return T_ARRAY, struct.pack("<IQ", ety, len(v)) + b"".join(e[1] for e in enc)
    raise GgufError(f"unsupported metadata value {type(v).__name__}")


def write_gguf(path, metadata: dict, tensors, alignment: int = DEFAULT_ALIGNMENT, version: int = 3) -> dict:
    """Write a GGUF file. tensors: (name, dims, type, data bytes) with data of
    exactly the layout's byte size; offsets are aligned to `alignment`.
    Returns {name: absolute data offset}."""
    md = dict(metadata)
    if alignment != DEFAULT_ALIGNMENT:
        md["general.alignment"] = alignment
    head = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(md)))
    for k, v in md.items():
        kb = k.encode("utf-8")
        ty, vb = _value_bytes(v)
        head += struct.pack("<Q", len(kb)) + kb + struct.pack("<I", ty) + vb
    offs, off = [], 0
    for name, dims, ty, data in tensors:
        size = TensorInfo(name, tuple(dims), ty, 0).byte_size()
        if size is None or len(data) != size:
            raise GgufError(f"{name}: {len(data)} data bytes for a {size}-byte tensor")
        offs.append(off)
        off = -(-(off + size) // alignment) * alignment
    for (name, dims, ty, _), o in zip(tensors, offs):
        nb = name.encode("utf-8")
        head += struct.pack("<Q", len(nb)) + nb + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", int(ty), o)
    data_offset = -(-len(head) // alignment) * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_offset - len(head)))
        pos = 0
        for (_, _, _, data), o in zip(tensors, offs):
            f.write(b"\0" * (o - pos))
            f.write(bytes(data))
            pos = o + len(data)
    return {t[0]: data_offset + o for t, o in zip(tensors, offs)}


@dataclass(frozen=True)
class ExpertTensor:
    """One routed-expert tensor as uniform per-expert slabs
    (crates/engine/src/lib.rs:541-593)."""
    name: str
    abs_offset: int  # file offset of expert 0
    expert_bytes: int  # one expert's slab
    row_bytes: int
    rows: int  # rows per expert
    n_expert: int
    quant: int  # kernel quant code

    @staticmethod
    def of(g: Gguf, t: TensorInfo, n_expert: int) -> "ExpertTensor":
        quant = QUANT_OF_TYPE.get(t.ty)
        if quant is None:
            raise GgufError(f"{t.name}: unsupported expert type {t.ty!r}")
        if len(t.dims) != 3 or t.dims[2] != n_expert:
            raise GgufError(f"{t.name}: unexpected exps dims {t.dims}")
        rb = type_row_bytes(t.ty, t.dims[0])
        return ExpertTensor(t.name, g.data_offset + t.offset, rb * t.dims[1], rb, t.dims[1], n_expert, quant)

    def slab(self, e: int) -> tuple:
        """(file offset, length) of expert e's slab."""
        if not 0 <= e < self.n_expert:
            raise IndexError(f"expert {e} of {self.n_expert}")
        return self.abs_offset + e * self.expert_bytes, self.expert_bytes


@dataclass(frozen=True)
class LayerExperts:
    gate: ExpertTensor
    up: ExpertTensor  # the gate tensor itself when fused
    down: ExpertTensor
    fused_up_off: int  # bytes from a gate row block to its up rows (0 = separate tensors)
    n_ff: int
    biases: tuple  # TensorInfo or None for gate / up / down (f32 [n_expert][dim])


def layer_experts(g: Gguf, layer: int) -> LayerExperts:
    """The routed-expert tensors of one layer. A fused ffn_gate_up_exps
    tensor holds, per expert, n_ff gate rows then n_ff up rows
    (crates/engine/src/lib.rs:3963-3973)."""
    n_expert = g.arch_meta("expert_count")
    if not isinstance(n_expert, int):
        raise GgufError("missing expert_count")
    name = lambda s: f"blk.{layer}.{s}"  # noqa: E731
    fused = g.tensor(name("ffn_gate_up_exps.weight"))
    if fused is not None:
        gate = ExpertTensor.of(g, fused, n_expert)
        if gate.rows % 2:
            raise GgufError(f"{fused.name}: odd fused row count {gate.rows}")
        n_ff = gate.rows // 2
        up, up_off = gate, gate.row_bytes * n_ff
    else:
        tg, tu = g.tensor(name("ffn_gate_exps.weight")), g.tensor(name("ffn_up_exps.weight"))
        if tg is None or tu is None:
            raise GgufError(f"layer {layer}: no routed expert tensors")
        gate, up, up_off = ExpertTensor.of(g, tg, n_expert), ExpertTensor.of(g, tu, n_expert), 0
        n_ff = gate.rows
    td = g.tensor(name("ffn_down_exps.weight"))
    if td is None:
        raise GgufError(f"layer {layer}: no ffn_down_exps")
    down = ExpertTensor.of(g, td, n_expert)
    biases = tuple(g.tensor(name(f"ffn_{p}_exps.bias")) for p in ("gate", "up", "down"))
    return LayerExperts(gate, up, down, up_off, n_ff, biases)


def expert_reads(g: Gguf, model_len: int) -> list:
    """Every routed-expert slab of the file as (offset, length), tensor by
    tensor in file order (crates/stream/src/lib.rs:14-48)."""
    n_expert = g.arch_meta("expert_count")
    if not isinstance(n_expert, int):
        raise GgufError("missing expert_count")
    out = []
    for t in g.tensors:
        if not t.name.endswith("_exps.weight"):
            continue
        if len(t.dims) != 3 or t.dims[2] != n_expert:
            raise GgufError(f"{t.name}: unexpected exps dims {t.dims}")
        rb = type_row_bytes(t.ty, t.dims[0])
        if rb is None:
            raise GgufError(f"{t.name}: unmodeled type {t.ty!r}")
        eb = rb * t.dims[1]
        base = g.data_offset + t.offset
        for e in range(n_expert):
            if base + (e + 1) * eb > model_len:
                raise GgufError(f"{t.name}: expert {e} beyond eof")
            out.append((base + e * eb, eb))
    if not out:
        raise GgufError("no *_exps.weight tensors found")
    return out


def plan_to_string(reads) -> str:
    """The streaming plan format: "offset len" per line."""
    return "".join(f"{o} {n}\n" for o, n in reads)


def upload_layer(path, g: Gguf, layer: int, device="cuda"):
    """Copy one layer's expert tensors from the file to the device, each as
    one slab [n_expert][rows][row_bytes] followed by SLAB_SLACK zero bytes,
    and describe them for the kernels. Returns (LayerExperts, ExpertBank,
    keep-alive device buffers)."""
    import numpy as np
    import torch

    from . import kernels as K

    lx = layer_experts(g, layer)
    with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        def dev_slab(t: ExpertTensor):
            n = t.expert_bytes * t.n_expert
            if t.abs_offset + n > len(mm):
                raise GgufError(f"{t.name}: beyond eof")
            host = np.frombuffer(mm, dtype=np.uint8, count=n, offset=t.abs_offset)
            buf = torch.zeros(n + SLAB_SLACK, dtype=torch.uint8, device=device)
            buf[:n].copy_(torch.from_numpy(host.copy()))
            return buf

        def dev_bias(ti):
            if ti is None:
                return None
            if ti.ty != TensorType.F32:
                raise GgufError(f"{ti.name}: bias type {ti.ty!r} (f32 expected)")
            n = ti.byte_size()
            host = np.frombuffer(mm, dtype=np.float32, count=n // 4, offset=g.data_offset + ti.offset)
            return torch.from_numpy(host.copy()).to(device)

        gate = dev_slab(lx.gate)
        up = gate if lx.fused_up_off else dev_slab(lx.up)
        down = dev_slab(lx.down)
        gb, ub, db = (dev_bias(b) for b in lx.biases)
    bank = K.ExpertBank(gate.data_ptr(), up.data_ptr() + lx.fused_up_off, down.data_ptr(),
                        gb.data_ptr() if gb is not None else None, ub.data_ptr() if ub is not None else None,
                        db.data_ptr() if db is not None else None,
                        lx.gate.expert_bytes, lx.up.expert_bytes, lx.down.expert_bytes,
                        lx.n_ff if gb is not None else 0, lx.n_ff if ub is not None else 0,
                        lx.down.rows if db is not None else 0)
    return lx, bank, (gate, up, down, gb, ub, db)
