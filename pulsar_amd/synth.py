"""Seeded synthetic weights and activations for the benchmark configurations.

Byte layouts are the reference's (crates/gguf/src/lib.rs:145-180); the value
distributions are the ones the benchmark configurations state:
  Q4_K   : f16 d, dmin ~ U[1e-3, 1e-2]; scales[12], qs[128] uniform bytes
  Q6_K   : ql, qh uniform bytes; int8 scales ~ U{-32..31}; f16 d ~ U[1e-3, 1e-2]
  Q2_K   : scale/min nibbles and 2-bit qs uniform; f16 d, dmin ~ U[1e-3, 1e-2]
  IQ2_XXS: grid indices, sign bits and 4-bit scales uniform; f16 d ~ U[1e-3, 1e-2]
  MXFP4  : E2M1 codes uniform; E8M0 exponent ~ U{118..126}
  other formats (parity tests): uniform bytes with every f16 scale
           ~ U[1e-3, 1e-2] (Q5_1's min with a random sign), NVFP4 UE4M3
           scales with exponent field 4..10
  activations ~ N(0, 1) fp32; biases ~ N(0, 0.02)
Everything derives from numpy's PCG64 seeded per tensor, so a (seed, name)
pair always yields the same bytes.
"""
from __future__ import annotations

import zlib
from dataclasses import dataclass

import numpy as np

from .formats import (
    BLOCK_LAYOUT,
    QUANT_IQ1_S,
    QUANT_IQ2_S,
    QUANT_IQ2_XS,
    QUANT_IQ2_XXS,
    QUANT_IQ3_S,
    QUANT_IQ3_XXS,
    QUANT_IQ4_NL,
    QUANT_IQ4_XS,
    QUANT_MXFP4,
    QUANT_NVFP4,
    QUANT_Q2_K,
    QUANT_Q3_K,
    QUANT_Q4_0,
    QUANT_Q4_K,
    QUANT_Q5_1,
    QUANT_Q5_K,
    QUANT_Q6_K,
    QUANT_Q8_0,
    row_bytes,
)


def rng_for(seed: int, name: str) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64([seed, zlib.crc32(name.encode())]))


def _f16_uniform(rng: np.random.Generator, shape, lo=1e-3, hi=1e-2) -> np.ndarray:
    return rng.uniform(lo, hi, size=shape).astype(np.float32).astype(np.float16).view(np.uint16)


def _put_u16(blocks: np.ndarray, off: int, vals: np.ndarray) -> None:
    blocks[..., off] = (vals & 0xFF).astype(np.uint8)
    blocks[..., off + 1] = (vals >> 8).astype(np.uint8)


def quant_matrix(quant: int, rows: int, cols: int, rng: np.random.Generator) -> np.ndarray:
    """uint8 array [rows, row_bytes(quant, cols)] of seeded random blocks."""
    rb = row_bytes(quant, cols)
    if quant == QUANT_MXFP4:
        nblk = rb // 17
        raw = np.frombuffer(rng.bytes(rows * rb), dtype=np.uint8).reshape(rows, nblk, 17).copy()
        raw[..., 0] = rng.integers(118, 127, size=(rows, nblk), dtype=np.uint8)
        return raw.reshape(rows, rb)
    bb = BLOCK_LAYOUT[quant][1]
    nb = rb // bb
    raw = np.frombuffer(rng.bytes(rows * rb), dtype=np.uint8).reshape(rows, nb, bb).copy()
    # every other format: f16 scales uniform in [1e-3, 1e-2] at these offsets
    # of each block (Q5_1's min with a random sign), NVFP4's UE4M3 scales with
    # exponent fields 4..10; the remaining bytes stay uniform random
    d_offs = {QUANT_Q5_K: (0, 2), QUANT_Q3_K: (108,), QUANT_IQ2_XS: (0,), QUANT_IQ3_XXS: (0,), QUANT_IQ4_XS: (0,),
              QUANT_IQ3_S: (0,), QUANT_IQ2_S: (0,), QUANT_IQ1_S: (0,), QUANT_Q8_0: (0,), QUANT_Q4_0: (0,),
              QUANT_IQ4_NL: (0,), QUANT_Q5_1: (0,)}
    if quant in d_offs:
        for off in d_offs[quant]:
            _put_u16(raw, off, _f16_uniform(rng, (rows, nb)))
        if quant == QUANT_Q5_1:
            m = _f16_uniform(rng, (rows, nb)) | (rng.integers(0, 2, (rows, nb)).astype(np.uint16) << 15)
            _put_u16(raw, 2, m)
        return raw.reshape(rows, rb)
    if quant == QUANT_NVFP4:
        ex = rng.integers(4, 11, size=(rows, nb, 4), dtype=np.uint8)
        raw[..., 0:4] = (ex << 3) | rng.integers(0, 8, size=(rows, nb, 4), dtype=np.uint8)
        return raw.reshape(rows, rb)
    if quant == QUANT_Q4_K:
        _put_u16(raw, 0, _f16_uniform(rng, (rows, nb)))
        _put_u16(raw, 2, _f16_uniform(rng, (rows, nb)))
    elif quant == QUANT_Q6_K:
        raw[..., 192:208] = rng.integers(-32, 32, size=(rows, nb, 16), dtype=np.int8).view(np.uint8)
        _put_u16(raw, 208, _f16_uniform(rng, (rows, nb)))
    elif quant == QUANT_Q2_K:
        _put_u16(raw, 80, _f16_uniform(rng, (rows, nb)))
        _put_u16(raw, 82, _f16_uniform(rng, (rows, nb)))
    elif quant == QUANT_IQ2_XXS:
        _put_u16(raw, 0, _f16_uniform(rng, (rows, nb)))
    return raw.reshape(rows, rb)


def activations(n_tok: int, n: int, rng: np.random.Generator) -> np.ndarray:
    return rng.standard_normal(size=(n_tok, n), dtype=np.float32)


@dataclass(frozen=True)
class MoESpec:
    """One routed-MoE layer configuration."""

    name: str
    hidden: int
    n_expert: int
    ffn: int
    k_used: int
    n_tok: int
    gate_quant: int
    down_quant: int
    act_op: int = 0
    shared: bool = False  # one always-on shared expert of the same shape
    biases: bool = False  # per-expert fp32 biases and a router bias

    @property
    def gate_row_bytes(self) -> int:
        return row_bytes(self.gate_quant, self.hidden)

    @property
    def down_row_bytes(self) -> int:
        return row_bytes(self.down_quant, self.ffn)

    @property
    def expert_bytes(self) -> int:
        return 2 * self.ffn * self.gate_row_bytes + self.hidden * self.down_row_bytes

    @property
    def n_slots(self) -> int:
        return self.k_used + (1 if self.shared else 0)


# Benchmark configurations 3-5 (configs 1-2 are dense matvecs).
C3 = MoESpec("c3_moe_decode_q4k_q6k", 2048, 256, 512, 8, 1, QUANT_Q4_K, QUANT_Q6_K, shared=True)
C4_Q2K = MoESpec("c4_moe_chunk16_q2k", 4096, 128, 1536, 8, 16, QUANT_Q2_K, QUANT_Q2_K)
C4_IQ2 = MoESpec("c4_moe_chunk16_iq2xxs", 4096, 128, 1536, 8, 16, QUANT_IQ2_XXS, QUANT_IQ2_XXS)
C5_B1 = MoESpec("c5_moe_mxfp4_b1", 2880, 32, 2880, 4, 1, QUANT_MXFP4, QUANT_MXFP4, act_op=2, biases=True)
C5_B64 = MoESpec("c5_moe_mxfp4_b64", 2880, 32, 2880, 4, 64, QUANT_MXFP4, QUANT_MXFP4, act_op=2, biases=True)


@dataclass
class MoEBank:
    """Host copy of one layer's weights: expert banks [E][rows][row_bytes]
    (the GGUF *_exps tensor layout), optional shared expert, router."""

    spec: MoESpec
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray
    router_w: np.ndarray  # fp32 [n_expert, hidden]
    router_b: np.ndarray | None
    gate_b: np.ndarray | None  # fp32 [E, ffn]
    up_b: np.ndarray | None
    down_b: np.ndarray | None  # fp32 [E, hidden]
    sh_gate: np.ndarray | None = None
    sh_up: np.ndarray | None = None
    sh_down: np.ndarray | None = None


def moe_bank(spec: MoESpec, seed: int, n_expert: int | None = None) -> MoEBank:
    """Seeded weights for `spec` (optionally only the first n_expert experts)."""
    E = spec.n_expert if n_expert is None else n_expert
    g = quant_matrix(spec.gate_quant, E * spec.ffn, spec.hidden, rng_for(seed, "gate"))
    u = quant_matrix(spec.gate_quant, E * spec.ffn, spec.hidden, rng_for(seed, "up"))
    d = quant_matrix(spec.down_quant, E * spec.hidden, spec.ffn, rng_for(seed, "down"))
    rw = (rng_for(seed, "router").standard_normal((spec.n_expert, spec.hidden)) /
          np.sqrt(spec.hidden)).astype(np.float32)
    bank = MoEBank(spec, g.reshape(E, spec.ffn, -1), u.reshape(E, spec.ffn, -1),
                   d.reshape(E, spec.hidden, -1), rw, None, None, None, None)
    if spec.biases:
        bank.router_b = (rng_for(seed, "router_b").standard_normal(spec.n_expert) * 0.02).astype(np.float32)
        bank.gate_b = (rng_for(seed, "gate_b").standard_normal((E, spec.ffn)) * 0.02).astype(np.float32)
        bank.up_b = (rng_for(seed, "up_b").standard_normal((E, spec.ffn)) * 0.02).astype(np.float32)
        bank.down_b = (rng_for(seed, "down_b").standard_normal((E, spec.hidden)) * 0.02).astype(np.float32)
    if spec.shared:
        bank.sh_gate = quant_matrix(spec.gate_quant, spec.ffn, spec.hidden, rng_for(seed, "sh_gate"))
        bank.sh_up = quant_matrix(spec.gate_quant, spec.ffn, spec.hidden, rng_for(seed, "sh_up"))
        bank.sh_down = quant_matrix(spec.down_quant, spec.hidden, spec.ffn, rng_for(seed, "sh_down"))
    return bank


def csr_by_expert(selected: np.ndarray, n_used: int):
    """Host CSR of (token, slot) pairs grouped by expert id in order of first
    appearance (crates/engine/src/lib.rs:8357-8392): returns (expert ids,
    starts[n_group+1], pairs packing token << 4 | slot)."""
    order: dict[int, list[int]] = {}
    flat = selected.reshape(-1)
    for si, e in enumerate(flat):
        e = int(e)
        if e < 0:
            continue
        order.setdefault(e, []).append(((si // n_used) << 4) | (si % n_used))
    ids = np.array(list(order.keys()), dtype=np.int64)
    starts = np.zeros(len(ids) + 1, dtype=np.uint32)
    pairs = []
    for i, e in enumerate(ids):
        pairs.extend(order[int(e)])
        starts[i + 1] = len(pairs)
    return ids, starts, np.array(pairs, dtype=np.uint32)
