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
from pulsar_amd import formats as fm
from pulsar_amd.formats import QUANT_IQ2_XXS, QUANT_MXFP4, QUANT_Q2_K, QUANT_Q4_K, QUANT_Q6_K, row_bytes

# f16 scale bytes whose high byte gets `&= 0x3b` (finite, small), per block:
# (block bytes, offsets of the high bytes inside the block)
F16_HI = {
    QUANT_Q2_K: (84, (81, 83)), QUANT_Q4_K: (144, (1, 3)), QUANT_Q6_K: (210, (209,)), QUANT_IQ2_XXS: (66, (1,)),
    fm.QUANT_Q5_K: (176, (1, 3)), fm.QUANT_Q3_K: (110, (109,)), fm.QUANT_IQ2_XS: (74, (1,)),
    fm.QUANT_IQ3_XXS: (98, (1,)), fm.QUANT_IQ4_XS: (136, (1,)), fm.QUANT_IQ3_S: (110, (1,)),
    fm.QUANT_IQ2_S: (82, (1,)), fm.QUANT_IQ1_S: (50, (1,)), fm.QUANT_Q8_0: (34, (1,)), fm.QUANT_Q4_0: (18, (1,)),
    fm.QUANT_IQ4_NL: (18, (1,)), fm.QUANT_Q5_1: (24, (1, 3)), fm.QUANT_NVFP4: (36, ()),
}


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
    bb, hi_bytes = F16_HI[quant]
    for b in range(len(row) // bb):
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
        (fm.QUANT_Q3_K, 7331, 5120),     # q3k_dot_matches_dequant_and_scalar
        (fm.QUANT_IQ2_XS, 555, 5120),    # iq2xs_dot_matches_dequant_and_scalar
        (fm.QUANT_IQ3_XXS, 777, 5120),   # iq3xxs_dot_matches_dequant_and_scalar
        # formats with no lane test in the reference: the same recipe
        (fm.QUANT_Q5_K, 4242, 5120),
        (fm.QUANT_IQ4_XS, 1111, 5120),
        (fm.QUANT_Q8_0, 2222, 5120),
        (fm.QUANT_Q4_0, 3333, 5120),
        (fm.QUANT_Q5_1, 4444, 5120),
        (fm.QUANT_IQ4_NL, 5555, 5120),
        (fm.QUANT_IQ3_S, 6666, 5120),
        (fm.QUANT_IQ2_S, 7777, 5120),
        (fm.QUANT_IQ1_S, 8888, 5120),
        (fm.QUANT_NVFP4, 9999, 5120),
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


# ---- cross-format identities: formats that reduce to one another on
# chosen fields must dequantize to the same values, which pins the bit
# positions each restatement reads (a swapped nibble or misplaced high bit
# in either fails here)

def _f16(x: float) -> bytes:
    return int(oracle.f32_to_f16(x)).to_bytes(2, "little")


def test_q5k_without_high_bits_is_q4k():
    rng = np.random.default_rng(1)
    for _ in range(20):
        q4 = rng.integers(0, 256, 144, dtype=np.uint8)
        q4[1] &= 0x3B
        q4[3] &= 0x3B
        q5 = np.concatenate([q4[:16], np.zeros(32, np.uint8), q4[16:]])
        assert np.array_equal(oracle.dequant_row(fm.QUANT_Q5_K, q5, 256), oracle.dequant_row(QUANT_Q4_K, q4, 256))
        act = rng.standard_normal(256).astype(np.float32)
        xq = oracle.quantize_q8_k(act)[0]
        # same integer sums and the same fp32 epilogue: bit-identical dots
        assert oracle.vec_dot(fm.QUANT_Q5_K, q5, xq, 256)[0] == oracle.vec_dot(QUANT_Q4_K, q4, xq, 256)[0]
        # with every sub-block scale 1 and min 0, bit `bit` of qh[i] adds
        # exactly 16 d to value 32 bit + i and to no other
        q5u = q5.copy()
        q5u[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
        bit, i = int(rng.integers(0, 8)), int(rng.integers(0, 32))
        q5h = q5u.copy()
        q5h[16 + i] |= 1 << bit
        delta = oracle.dequant_row(fm.QUANT_Q5_K, q5h, 256) - oracle.dequant_row(fm.QUANT_Q5_K, q5u, 256)
        assert list(np.flatnonzero(delta)) == [32 * bit + i]
        assert delta[32 * bit + i] == 16 * oracle.f16_to_f32(int(q5[0]) | (int(q5[1]) << 8))


def test_q5_1_without_high_bits_is_q4_0():
    rng = np.random.default_rng(2)
    for _ in range(20):
        d = float(rng.uniform(1e-3, 1e-2))
        qs = rng.integers(0, 256, (8, 16), dtype=np.uint8)
        q40 = b"".join(_f16(d) + qs[k].tobytes() for k in range(8))
        q51 = b"".join(_f16(d) + _f16(-8.0 * oracle.f16_to_f32(int(oracle.f32_to_f16(d)))) + bytes(4) + qs[k].tobytes()
                       for k in range(8))
        a = oracle.dequant_row(fm.QUANT_Q4_0, np.frombuffer(q40, np.uint8), 256)
        b = oracle.dequant_row(fm.QUANT_Q5_1, np.frombuffer(q51, np.uint8), 256)
        assert np.array_equal(a, b)
        # qh bit i lifts value i of the block (low nibbles 0..15, high 16..31) by 16 d
        k, i = int(rng.integers(0, 8)), int(rng.integers(0, 32))
        q51h = bytearray(q51)
        q51h[24 * k + 4 + i // 8] |= 1 << (i % 8)
        c = oracle.dequant_row(fm.QUANT_Q5_1, np.frombuffer(bytes(q51h), np.uint8), 256)
        assert list(np.flatnonzero(c - b)) == [32 * k + i]
        assert np.isclose((c - b)[32 * k + i], 16 * oracle.f16_to_f32(int(oracle.f32_to_f16(d))))


def test_iq4_nl_matches_iq4_xs_at_unit_scales():
    rng = np.random.default_rng(3)
    for _ in range(10):
        d = float(rng.uniform(1e-3, 1e-2))
        qs = rng.integers(0, 256, (8, 16), dtype=np.uint8)
        # ls = 33 for every sub-block: low nibble 1, high two bits 2
        xs = _f16(d) + (0xAAAA).to_bytes(2, "little") + bytes([0x11] * 4) + qs.tobytes()
        nl = b"".join(_f16(d) + qs[k].tobytes() for k in range(8))
        a = oracle.dequant_row(fm.QUANT_IQ4_XS, np.frombuffer(xs, np.uint8), 256)
        b = oracle.dequant_row(fm.QUANT_IQ4_NL, np.frombuffer(nl, np.uint8), 256)
        assert np.array_equal(a, b)
        act = rng.standard_normal(256).astype(np.float32)
        xq = oracle.quantize_q8_k(act)[0]
        ga, sa = oracle.vec_dot(fm.QUANT_IQ4_XS, np.frombuffer(xs, np.uint8), xq, 256)
        gb, _ = oracle.vec_dot(fm.QUANT_IQ4_NL, np.frombuffer(nl, np.uint8), xq, 256)
        assert abs(ga - gb) <= 1e-5 * sa + 1e-30


def test_nvfp4_repacks_mxfp4():
    """An NVFP4 block holding MXFP4's codes (E2M1 both) at a scale both can
    express decodes to the same values: pins NVFP4's nibble order (low =
    value i, high = i + 8 of each 16) against MXFP4's (i, i + 16 of 32) and
    the UE4M3 scale against E8M0."""
    rng = np.random.default_rng(4)
    # 2^(e8 - 127) in UE4M3: normal (exponent field e8 - 120, mantissa 0)
    # for e8 in 121..135, subnormal (mantissa 2^(e8 - 118), field 0) below
    for e8 in (118, 119, 120, 121, 126, 127, 130, 135):
        codes = rng.integers(0, 16, 256, dtype=np.uint8)
        mx = bytearray()
        for k in range(8):
            c = codes[32 * k:32 * k + 32]
            mx += bytes([e8]) + bytes(int(c[i]) | (int(c[16 + i]) << 4) for i in range(16))
        ue = (e8 - 120) << 3 if e8 >= 121 else 1 << (e8 - 118)
        nv = bytearray()
        for k in range(4):
            nv += bytes([ue] * 4)
            for sub in range(4):
                c = codes[64 * k + 16 * sub:64 * k + 16 * sub + 16]
                nv += bytes(int(c[i]) | (int(c[8 + i]) << 4) for i in range(8))
        a = oracle.dequant_row(QUANT_MXFP4, np.frombuffer(bytes(mx), np.uint8), 256)
        b = oracle.dequant_row(fm.QUANT_NVFP4, np.frombuffer(bytes(nv), np.uint8), 256)
        assert np.array_equal(a, b)


@pytest.mark.parametrize("quant", [fm.QUANT_Q3_K, fm.QUANT_IQ2_XS, fm.QUANT_IQ3_XXS, fm.QUANT_IQ4_XS, fm.QUANT_IQ3_S,
                                   fm.QUANT_IQ2_S, fm.QUANT_IQ1_S, fm.QUANT_Q5_K])
def test_exact_integer_sums_match_float_form(quant):
    """The integer super-block sums the kernels use (block_dot's i0, i1)
    reproduce the reference's per-group float accumulation within rounding."""
    row, act = recipe_row(31, quant, 1024)
    row = mask_scales(row, quant, 1024)
    xq = oracle.quantize_q8_k(act)[0]
    bb = fm.BLOCK_LAYOUT[quant][1]
    d, _, _ = oracle.q8k_fields(xq[None])
    for b in range(4):
        f, i0, i1 = oracle.block_dot(quant, row, b, xq[292 * b:292 * (b + 1)])[:3]
        blk = row[b * bb:(b + 1) * bb]
        f16 = lambda o: oracle.f16_to_f32(int(blk[o]) | (int(blk[o + 1]) << 8))  # noqa: E731
        yd = float(d[0][b])
        alt = {
            fm.QUANT_Q3_K: lambda: f16(108) * yd * i0,
            fm.QUANT_IQ2_XS: lambda: 0.125 * f16(0) * yd * i0,
            fm.QUANT_IQ3_XXS: lambda: 0.25 * f16(0) * yd * i0,
            fm.QUANT_IQ4_XS: lambda: f16(0) * yd * i0,
            fm.QUANT_IQ3_S: lambda: f16(0) * yd * i0,
            fm.QUANT_IQ2_S: lambda: 0.125 * f16(0) * yd * i0,
            fm.QUANT_IQ1_S: lambda: f16(0) * yd * (i0 + 0.125 * i1),
            fm.QUANT_Q5_K: lambda: f16(0) * yd * i0 - f16(2) * yd * i1,
        }[quant]()
        assert abs(alt - f) <= 1e-6 * max(abs(f), abs(alt)) + 1e-30, (b, f, alt)
