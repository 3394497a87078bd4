"""The oracle against the reference's own CPU-lane test recipes.

crates/quant/src/cpu_dot.rs:819-1097 builds rows from the in-test LCG
(`state*6364136223846793005 + 1442695040888963407`, mapped to
((state >> 33) as f32 / 2^31) - 1), turns every draw into a byte with
`(lcg * 127 + 128) as u8`, caps the f16 scale exponents with `&= 0x3b`,
quantizes an LCG activation row to q8_K and requires the lane dot to be within
rel 1e-4 of an f64 dequant-times-dequant reference. The same seeds and sizes
are replayed here. The reference's IQ2_XXS test encodes its row with a
quantizer that is outside this path (crates/quant/src/iq.rs), so IQ2_XXS uses
the random-byte recipe of its iq2_xs/iq3_xxs siblings instead; Q6_K and MXFP4
have no lane test in the reference and get the same recipe here.
"""
import numpy as np
import pytest

import oracle
from pulsar_amd.formats import QUANT_IQ2_XXS, QUANT_MXFP4, QUANT_Q2_K, QUANT_Q4_K, QUANT_Q6_K, row_bytes


def recipe_row(seed: int, quant: int, n: int):
    nbytes = row_bytes(quant, n)
    draws = oracle.lcg_stream(seed, nbytes + n)
    byte_f = draws[:nbytes] * np.float32(127.0) + np.float32(128.0)
    row = byte_f.astype(np.float32).astype(np.int64).clip(0, 255).astype(np.uint8)
    act = draws[nbytes:].copy()
    return row, act


def mask_scales(row: np.ndarray, quant: int, n: int) -> np.ndarray:
    row = row.copy()
    if quant == QUANT_MXFP4:
        # keep E8M0 exponents in a range whose values stay finite in f32
        for b in range(n // 32):
            row[17 * b] = 100 + row[17 * b] % 40
        return row
    bb = {QUANT_Q2_K: 84, QUANT_Q4_K: 144, QUANT_Q6_K: 210, QUANT_IQ2_XXS: 66}[quant]
    hi_bytes = {QUANT_Q2_K: (81, 83), QUANT_Q4_K: (1, 3), QUANT_Q6_K: (209,), QUANT_IQ2_XXS: (1,)}[quant]
    for b in range(n // 256):
        for o in hi_bytes:
            row[b * bb + o] &= 0x3B
    return row


def f64_reference(quant, row, xq, n):
    deq = oracle.dequant_row(quant, row, n)
    d, qs, _ = oracle.q8k_fields(xq[None])
    act = (d[0][:, None].astype(np.float64) * qs[0].astype(np.float64)).reshape(-1)[:n]
    return float(np.dot(deq, act))


@pytest.mark.parametrize(
    "quant,seed,n",
    [
        (QUANT_Q2_K, 99, 5120),       # q2k_dot_matches_dequant_and_scalar
        (QUANT_Q4_K, 424242, 5120),   # q4k_dot_matches_dequant_and_scalar
        (QUANT_IQ2_XXS, 42, 2048),    # dot_matches_dequant_reference (n, seed)
        (QUANT_IQ2_XXS, 555, 5120),   # iq2_xs recipe, applied to iq2_xxs
        (QUANT_Q6_K, 7331, 5120),
        (QUANT_MXFP4, 777, 5120),
    ],
)
def test_lane_dot_matches_f64_dequant(quant, seed, n):
    row, act = recipe_row(seed, quant, n)
    row = mask_scales(row, quant, n)
    xq = oracle.quantize_q8_k(act)[0]
    got, abs_sum = oracle.vec_dot(quant, row, xq, n)
    ref = f64_reference(quant, row, xq, n)
    rel = abs(got - ref) / max(abs(ref), 1e-6)
    assert rel < 1e-4, (got, ref, rel)
    # the condition-aware bound used for GPU parity is never looser than this
    assert abs(got - ref) <= 1e-5 * abs_sum + 1e-30


def test_lcg_matches_reference_definition():
    # first draws of seed 42, recomputed from the stated recurrence in Python ints
    st = 42
    want = []
    for _ in range(5):
        st = (st * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        want.append(np.float32(np.float32(st >> 33) / np.float32(2.0**31)) - np.float32(1.0))
    assert np.array_equal(oracle.lcg_stream(42, 5), np.array(want, dtype=np.float32))


def test_q8k_quantizer_on_recipe_activation():
    # cpu_dot.rs:26-50 restated in numpy on the recipe's activation row
    _, act = recipe_row(424242, QUANT_Q4_K, 5120)
    xq = oracle.quantize_q8_k(act)[0]
    d, qs, bs = oracle.q8k_fields(xq[None])
    blocks = act.reshape(-1, 256)
    amax = np.abs(blocks).max(axis=1)
    assert np.array_equal(d[0], (amax / np.float32(127.0)).astype(np.float32))
    inv = (np.float32(127.0) / amax).astype(np.float32)
    prod = (blocks * inv[:, None]).astype(np.float32)
    p64 = prod.astype(np.float64)  # exact; +0.5 in f64 cannot round
    q = np.clip(np.sign(p64) * np.floor(np.abs(p64) + 0.5), -127, 127).astype(np.int8)
    assert np.array_equal(qs[0], q)
    assert np.array_equal(bs[0], q.reshape(-1, 16, 16).astype(np.int32).sum(-1).astype(np.int16))
