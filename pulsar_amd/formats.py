"""Quant codes and block layouts of the expert formats on the hot path.

Codes: crates/kernels/src/lib.rs:55-73. Layouts: crates/gguf/src/lib.rs:145-180
(block size in values, bytes per block); a row of n values takes
ceil(n / block) * block_bytes bytes (crates/gguf/src/lib.rs:175-180).
"""
from __future__ import annotations

QUANT_Q2_K = 0
QUANT_IQ2_XXS = 1
QUANT_Q4_K = 2
QUANT_Q6_K = 4
QUANT_MXFP4 = 12
QUANT_A4_OK = 0x8000_0000

ACT_SILU = 0
ACT_SWIGLU_OAI = 2

QK_K = 256
Q8_K_BLOCK_BYTES = 292  # f32 d, i8 qs[256], i16 bsums[16]
EXPERT_PTRS_BYTES = 48  # six pointers

# (values per block, bytes per block)
BLOCK_LAYOUT = {
    QUANT_Q2_K: (256, 84),
    QUANT_IQ2_XXS: (256, 66),
    QUANT_Q4_K: (256, 144),
    QUANT_Q6_K: (256, 210),
    QUANT_MXFP4: (32, 17),
}

NAMES = {
    QUANT_Q2_K: "Q2_K",
    QUANT_IQ2_XXS: "IQ2_XXS",
    QUANT_Q4_K: "Q4_K",
    QUANT_Q6_K: "Q6_K",
    QUANT_MXFP4: "MXFP4",
}


def row_bytes(quant: int, n: int) -> int:
    """Bytes one row of n values occupies (GGUF TensorType::row_bytes)."""
    bs, bb = BLOCK_LAYOUT[quant]
    return -(-n // bs) * bb


def q8k_blocks(n: int) -> int:
    """q8_K blocks per activation row of n values (tail zero-padded)."""
    return -(-n // QK_K)
