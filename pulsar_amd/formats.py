"""Quant codes and block layouts of the expert formats on the hot path.

Codes: crates/kernels/src/lib.rs:55-73. Layouts: crates/gguf/src/lib.rs:145-180
(block size in values, bytes per block); a row of n values takes
ceil(n / block) * block_bytes bytes (crates/gguf/src/lib.rs:175-180).
"""
from __future__ import annotations

QUANT_Q2_K = 0
QUANT_IQ2_XXS = 1
QUANT_Q4_K = 2
QUANT_Q5_K = 3
QUANT_Q6_K = 4
QUANT_Q3_K = 5
QUANT_IQ2_XS = 6
QUANT_IQ3_XXS = 7
QUANT_Q4_0 = 8
QUANT_Q5_1 = 9
QUANT_Q8_0 = 10
QUANT_IQ4_XS = 11
QUANT_MXFP4 = 12
QUANT_IQ4_NL = 13
QUANT_IQ3_S = 14
QUANT_IQ2_S = 15
QUANT_IQ1_S = 16
QUANT_NVFP4 = 17
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
    QUANT_Q5_K: (256, 176),
    QUANT_Q6_K: (256, 210),
    QUANT_Q3_K: (256, 110),
    QUANT_IQ2_XS: (256, 74),
    QUANT_IQ3_XXS: (256, 98),
    QUANT_Q4_0: (32, 18),
    QUANT_Q5_1: (32, 24),
    QUANT_Q8_0: (32, 34),
    QUANT_IQ4_XS: (256, 136),
    QUANT_MXFP4: (32, 17),
    QUANT_IQ4_NL: (32, 18),
    QUANT_IQ3_S: (256, 110),
    QUANT_IQ2_S: (256, 82),
    QUANT_IQ1_S: (256, 50),
    QUANT_NVFP4: (64, 36),
}

NAMES = {
    QUANT_Q2_K: "Q2_K",
    QUANT_IQ2_XXS: "IQ2_XXS",
    QUANT_Q4_K: "Q4_K",
    QUANT_Q5_K: "Q5_K",
    QUANT_Q6_K: "Q6_K",
    QUANT_Q3_K: "Q3_K",
    QUANT_IQ2_XS: "IQ2_XS",
    QUANT_IQ3_XXS: "IQ3_XXS",
    QUANT_Q4_0: "Q4_0",
    QUANT_Q5_1: "Q5_1",
    QUANT_Q8_0: "Q8_0",
    QUANT_IQ4_XS: "IQ4_XS",
    QUANT_MXFP4: "MXFP4",
    QUANT_IQ4_NL: "IQ4_NL",
    QUANT_IQ3_S: "IQ3_S",
    QUANT_IQ2_S: "IQ2_S",
    QUANT_IQ1_S: "IQ1_S",
    QUANT_NVFP4: "NVFP4",
}

# formats of the dense pulsar_matmul_kq (pulsar_kernels.cu:5090-5142); every
# format above is an expert format of the MoE entry points
DENSE_QUANTS = (QUANT_Q2_K, QUANT_IQ2_XXS, QUANT_Q4_K, QUANT_Q5_K, QUANT_Q6_K, QUANT_Q3_K, QUANT_IQ4_XS,
                QUANT_IQ4_NL, QUANT_NVFP4)


def row_bytes(quant: int, n: int) -> int:
    """Bytes one row of n values occupies (GGUF TensorType::row_bytes)."""
    bs, bb = BLOCK_LAYOUT[quant]
    return -(-n // bs) * bb


def q8k_blocks(n: int) -> int:
    """q8_K blocks per activation row of n values (tail zero-padded)."""
    return -(-n // QK_K)
