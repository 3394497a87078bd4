"""Pins for the oracle that do not come from the reference's test recipes:
closed forms, textbook definitions, independent restatements and invariants,
chosen so that a dropped term, a wrong index or sign, or a transposed
operand in oracle/pulsar_oracle.c fails at least one of them.
"""
import math

import numpy as np
import pytest

import oracle
from pulsar_amd import synth
from pulsar_amd.formats import QUANT_IQ2_XXS, QUANT_MXFP4, QUANT_Q2_K, QUANT_Q4_K, QUANT_Q6_K, row_bytes
from tests.conftest import REFERENCE

rng = np.random.default_rng(1234)


# ------------------------------------------------------------------ q8_K --

def q8k_one(x):
    d, qs, bs = oracle.q8k_fields(oracle.quantize_q8_k(np.asarray(x, np.float32)[None]))
    return d[0], qs[0], bs[0]


def test_q8k_round_half_away_from_zero():
    # amax = 127 makes inv = 1 exactly, so q = round(x): ties go away from 0
    x = np.zeros(256, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]
    d, qs, _ = q8k_one(x)
    assert d[0] == np.float32(1.0)
    assert list(qs[0, :9]) == [127, 1, -1, 2, -2, 3, -3, 127, -127]


def test_q8k_extremes_zero_block_and_bounds():
    x = rng.standard_normal(1024).astype(np.float32) * 3
    x[256:512] = 0.0
    x[700] = -50.0  # amax element of block 2 is negative
    d, qs, bs = q8k_one(x)
    assert d[1] == 0 and not qs[1].any() and not bs[1].any()
    assert qs[2, 700 - 512] == -127
    assert np.abs(qs.astype(int)).max() <= 127
    for b in (0, 2, 3):
        blk = x[256 * b:256 * b + 256]
        assert abs(int(qs[b, np.argmax(np.abs(blk))])) == 127
        assert d[b] == np.float32(np.abs(blk).max() / np.float32(127))
    assert np.array_equal(bs, qs.reshape(4, 16, 16).astype(np.int32).sum(-1))


def test_q8k_tail_is_zero_padded():
    # 300 values -> 2 blocks; the tail behaves exactly like explicit zeros
    x = rng.standard_normal(300).astype(np.float32)
    pad = np.zeros(512, np.float32)
    pad[:300] = x
    assert np.array_equal(oracle.quantize_q8_k(x[None]), oracle.quantize_q8_k(pad[None]))


def test_f16_conversions_textbook():
    for h in [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0xC000, 0x2E66]:
        assert oracle.f16_to_f32(h) == float(np.array(h, np.uint16).view(np.float16))
    vals = rng.uniform(-65000, 65000, 2000).astype(np.float32)
    vals = np.concatenate([vals, rng.uniform(-1e-4, 1e-4, 2000).astype(np.float32)])
    for v in vals:
        assert oracle.f32_to_f16(float(v)) == int(np.float16(v).view(np.uint16))


# ------------------------------------------- integer stages, unit scales --

def with_unit_scales(quant, row, d_bits, dmin_bits=0):
    """Rewrites every super-block's f16 d (and dmin) field."""
    row = row.copy()
    if quant == QUANT_MXFP4:
        row.reshape(-1, 17)[:, 0] = 128  # 2^(128-127) = 2: values = doubled E2M1
        return row
    bb, d_off, m_off = {QUANT_Q4_K: (144, 0, 2), QUANT_Q2_K: (84, 80, 82), QUANT_Q6_K: (210, 208, None),
                        QUANT_IQ2_XXS: (66, 0, None)}[quant]
    blk = row.reshape(-1, bb)
    blk[:, d_off] = d_bits & 0xFF
    blk[:, d_off + 1] = d_bits >> 8
    if m_off is not None:
        blk[:, m_off] = dmin_bits & 0xFF
        blk[:, m_off + 1] = dmin_bits >> 8
    return row


@pytest.mark.parametrize("quant", [QUANT_Q4_K, QUANT_Q2_K, QUANT_Q6_K, QUANT_IQ2_XXS, QUANT_MXFP4])
def test_integer_stage_equals_dequant_integers(quant):
    """With scales that make the f64 dequant integral, the exact int32 stage
    of po_block_dot must equal sum(dequant * q8) computed element-wise from
    the format description (po_dequant_row, a separate formulation)."""
    n = 512
    row = synth.quant_matrix(quant, 1, n, synth.rng_for(7, f"int{quant}"))[0]
    xq = oracle.quantize_q8_k(rng.standard_normal(n).astype(np.float32)[None])[0]
    _, qs, _ = oracle.q8k_fields(xq[None])
    q8 = qs[0].reshape(-1).astype(np.int64)
    one, eight = 0x3C00, 0x4800
    if quant in (QUANT_Q4_K, QUANT_Q2_K):
        r_i = with_unit_scales(quant, row, one, 0)
        r_m = with_unit_scales(quant, row, 0, one)
        for b in range(2):
            _, i0, i1, _ = oracle.block_dot(quant, r_i, b, xq[292 * b:292 * (b + 1)])
            want_i = np.dot(oracle.dequant_row(quant, r_i, n)[256 * b:256 * (b + 1)].astype(np.int64),
                            q8[256 * b:256 * (b + 1)])
            want_m = -np.dot(oracle.dequant_row(quant, r_m, n)[256 * b:256 * (b + 1)].astype(np.int64),
                             q8[256 * b:256 * (b + 1)])
            assert (i0, i1) == (want_i, want_m)
    elif quant == QUANT_Q6_K:
        r = with_unit_scales(quant, row, one)
        for b in range(2):
            _, i0, _, _ = oracle.block_dot(quant, r, b, xq[292 * b:292 * (b + 1)])
            want = np.dot(oracle.dequant_row(quant, r, n)[256 * b:256 * (b + 1)].astype(np.int64),
                          q8[256 * b:256 * (b + 1)])
            assert i0 == want
    elif quant == QUANT_IQ2_XXS:
        r = with_unit_scales(quant, row, eight)  # 0.125 * 8 = 1
        for b in range(2):
            _, i0, _, _ = oracle.block_dot(quant, r, b, xq[292 * b:292 * (b + 1)])
            want = np.dot(oracle.dequant_row(quant, r, n)[256 * b:256 * (b + 1)].astype(np.int64),
                          q8[256 * b:256 * (b + 1)])
            assert i0 == want
    else:
        r = with_unit_scales(quant, row, 0)
        deq = oracle.dequant_row(quant, r, n)  # = doubled E2M1 codes (integers)
        for b in range(2):
            _, _, _, sumi = oracle.block_dot(quant, r, b, xq[292 * b:292 * (b + 1)])
            want = [int(np.dot(deq[256 * b + 32 * k:256 * b + 32 * k + 32].astype(np.int64),
                               q8[256 * b + 32 * k:256 * b + 32 * k + 32])) for k in range(8)]
            assert list(sumi) == want


def test_q6k_matches_chunk16_restatement():
    """Q6_K has three reference statements (pulsar_kernels.cu:1830-1861,
    3163-3188, 5920-5948); this restates the chunk16 one (per 16 values c:
    half k = c>>3, cc = c&7, quarter qq = cc>>1, ql offset k*64+(qq&1)*32+(cc&1)*16,
    qh offset k*32+(cc&1)*16, low shift (qq>>1)*4, high shift 2*qq, scale sc[c])
    and compares its exact integer sum with the oracle's."""
    for trial in range(20):
        row = synth.quant_matrix(QUANT_Q6_K, 1, 256, synth.rng_for(trial, "q6"))[0]
        xq = oracle.quantize_q8_k(rng.standard_normal(256).astype(np.float32)[None])[0]
        _, qs, _ = oracle.q8k_fields(xq[None])
        q8 = qs[0, 0].astype(np.int64)
        ql, qh, sc = row[:128].astype(np.int64), row[128:192].astype(np.int64), row[192:208].view(np.int8)
        isum = 0
        for c in range(16):
            k, cc = c >> 3, c & 7
            qq = cc >> 1
            loff = k * 64 + (qq & 1) * 32 + (cc & 1) * 16
            hoff = k * 32 + (cc & 1) * 16
            v = ((ql[loff:loff + 16] >> ((qq >> 1) * 4)) & 15) | (((qh[hoff:hoff + 16] >> (2 * qq)) & 3) << 4)
            isum += int(sc[c]) * int(np.dot(v - 32, q8[16 * c:16 * c + 16]))
        _, i0, _, _ = oracle.block_dot(QUANT_Q6_K, row, 0, xq)
        assert i0 == isum


def test_mxfp4_dequant_is_textbook_ocp():
    # E2M1: sign bit 3, magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6}; E8M0 scale 2^(e-127)
    row = np.zeros(17, np.uint8)
    row[0] = 130
    codes = np.arange(32) % 16
    row[1:17] = (codes[:16] | (codes[16:] << 4)).astype(np.uint8)
    mags = [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    want = [(-1 if c & 8 else 1) * mags[c & 7] * 8.0 for c in codes]
    assert list(oracle.dequant_row(QUANT_MXFP4, row, 32)) == want


def test_iq2xxs_tables():
    """Grid magnitudes are 8/25/43, entries distinct, and equal to both
    vendored reference copies when the reference checkout is present; the
    sign table is i | parity(i) << 7 (crates/quant/src/iq.rs:495-497)."""
    row = np.zeros(66, np.uint8)
    row[0:2] = [0x00, 0x48]  # d = 8 -> 0.125 * d * (2*0+1) = 1
    entries = []
    for idx in range(256):
        aux0 = idx  # group 0, first 8 values use grid entry idx, no signs
        row[2:6] = np.array([aux0], "<u4").view(np.uint8)
        row[6:10] = 0
        v = oracle.dequant_row(QUANT_IQ2_XXS, row, 256)[:8]
        assert set(np.unique(v)) <= {8.0, 25.0, 43.0}
        entries.append(sum(int(m) << (8 * j) for j, m in enumerate(v)))
    assert len(set(entries)) == 256
    # sign bits: 7 stored bits, bit 7 restores even parity
    for s7 in range(128):
        row[2:6] = 0
        row[6:10] = np.array([s7], "<u4").view(np.uint8)
        v = oracle.dequant_row(QUANT_IQ2_XXS, row, 256)[:8]
        bits = [int(x < 0) for x in v]
        assert bits[:7] == [(s7 >> i) & 1 for i in range(7)]
        assert sum(bits) % 2 == 0
    inc = REFERENCE / "crates/kernels/cuda/iq2_tables.inc"
    rs = REFERENCE / "crates/quant/src/cpu_dot_tables.rs"
    if not (inc.exists() and rs.exists()):
        pytest.skip("reference checkout absent: vendored-table comparison skipped")
    import re

    for path, marker in ((inc, "cuda_iq2xxs_grid[256] = {"), (rs, "IQ2XXS_GRID: [u64; 256] = [")):
        body = path.read_text().split(marker, 1)[1].split("}", 1)[0].split("]", 1)[0]
        vals = [int(t, 16) for t in re.findall(r"0x[0-9a-fA-F]+", body)]
        assert vals == entries, path


def test_brute_force_one_superblock_each_format():
    for quant in (QUANT_Q4_K, QUANT_Q2_K, QUANT_Q6_K, QUANT_IQ2_XXS, QUANT_MXFP4):
        for t in range(10):
            row = synth.quant_matrix(quant, 1, 256, synth.rng_for(t, f"bf{quant}"))[0]
            x = rng.standard_normal(256).astype(np.float32)
            xq = oracle.quantize_q8_k(x[None])[0]
            d, qs, _ = oracle.q8k_fields(xq[None])
            ref = float(np.dot(oracle.dequant_row(quant, row, 256), float(d[0, 0]) * qs[0, 0].astype(np.float64)))
            got, abs_sum = oracle.vec_dot(quant, row, xq, 256)
            assert abs(got - ref) <= 1e-5 * max(abs_sum, abs(ref)) + 1e-12, (quant, got, ref)


# ------------------------------------------------------- glu and router --

def test_glu_closed_forms():
    for g, u in rng.uniform(-12, 12, (200, 2)):
        g32, u32 = float(np.float32(g)), float(np.float32(u))
        silu = g32 / (1 + math.exp(-g32)) * u32
        assert abs(oracle.glu(g32, u32, 0) - silu) <= 1e-6 * max(1.0, abs(silu))
        gc, uc = min(g32, 7.0), min(max(u32, -7.0), 7.0)
        oai = gc / (1 + math.exp(-1.702 * gc)) * (uc + 1)
        assert abs(oracle.glu(g32, u32, 2) - oai) <= 1e-6 * max(1.0, abs(oai))


def test_router_softmax_mode_equals_llama_order():
    """mode 1 selects on raw logits and exp-normalises the winners; the
    reference's self-test states it as full softmax -> top-k -> renormalise
    (pulsar_kernels.cu:1093-1143). Same ids, weights within 1e-5."""
    for n_expert, k, n_tok in ((256, 8, 5), (128, 8, 6), (32, 4, 9), (384, 8, 3)):
        logits = (rng.standard_normal((n_tok, n_expert)) * 4).astype(np.float32)
        sel, w = oracle.router_select(logits, np.zeros(n_expert, np.float32), n_expert, k, 1.0, n_tok, 1)
        for t in range(n_tok):
            p = np.exp(logits[t].astype(np.float64) - logits[t].max())
            p /= p.sum()
            top = np.argsort(-p, kind="stable")[:k]
            assert list(sel[t]) == list(top)
            assert np.allclose(w[t], p[top] / p[top].sum(), atol=1e-5, rtol=0)


def _f32_ulps(a, b):
    """Distance in f32 units in the last place (finite values)."""
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, np.int64(-(2 ** 31)) - ia, ia)
    ib = np.where(ib < 0, np.int64(-(2 ** 31)) - ib, ib)
    return np.abs(ia - ib)


def _matmul_f32_closed(w, x):
    """out[t][o] = sum_i w[o][i] x[t][i] (pulsar_kernels.cu:6504-6535) in
    f64 by numpy's own product, rounded once to f32."""
    return (x.astype(np.float64) @ w.astype(np.float64).T).astype(np.float32)


@pytest.mark.parametrize("out_dim,in_dim,n_tok", [(256, 2048, 3), (128, 4096, 2), (32, 2880, 4), (7, 300, 1)])
def test_matmul_f32_equals_f64_closed_form(out_dim, in_dim, n_tok):
    """po_matmul_f32 against an f64 product by another route (numpy's
    blocked matmul), rounded to f32: within 1 ulp (the two f64 sums differ
    only in order, so the f32 roundings can differ at a rounding boundary)."""
    w = (rng.standard_normal((out_dim, in_dim)) / np.sqrt(in_dim)).astype(np.float32)
    x = rng.standard_normal((n_tok, in_dim)).astype(np.float32)
    got = oracle.matmul_f32(w, x, in_dim, out_dim, n_tok)
    want = _matmul_f32_closed(w, x)
    assert _f32_ulps(got, want).max() <= 1
    # an f32 running sum (a plausible mistake) is further than 1 ulp away
    acc = np.zeros((n_tok, out_dim), np.float32)
    for i in range(in_dim):
        acc += x[:, i:i + 1] * w[None, :, i]
    if in_dim >= 2048:
        assert _f32_ulps(acc, want).max() > 1


def test_matmul_f32_closed_form_catches_transpose_and_token_swap():
    """The comparison above fails for a transposed weight operand and for
    swapped tokens, so it pins the operand roles and the output layout."""
    n = 256
    w = rng.standard_normal((n, n)).astype(np.float32)
    x = rng.standard_normal((2, n)).astype(np.float32)
    got = oracle.matmul_f32(w, x, n, n, 2)
    assert _f32_ulps(got, _matmul_f32_closed(w, x)).max() <= 1
    assert _f32_ulps(got, _matmul_f32_closed(np.ascontiguousarray(w.T), x)).max() > 1000
    assert _f32_ulps(got, _matmul_f32_closed(w, x[::-1].copy())).max() > 1000


def test_add_bias_rows_equals_broadcast_add():
    """po_add_bias_rows (pulsar_kernels.cu:3621-3638) is x[r][i] + b[i] in
    f32, bit for bit, and not b[r] or a bias of the wrong length."""
    for rows, dim in ((1, 32), (4, 256), (64, 2880), (3, 7)):
        x = rng.standard_normal((rows, dim)).astype(np.float32)
        b = (rng.standard_normal(dim) * 0.02).astype(np.float32)
        got = oracle.add_bias_rows(x, b, dim, rows)
        assert np.array_equal(got.view(np.uint32), (x + b[None, :]).view(np.uint32))
        if rows > 1 and dim > 1:
            assert not np.array_equal(got, x + np.resize(b, rows)[:, None])


def _mode1_closed(raw, bias, k, scale):
    """Router mode 1 with a selection bias (pulsar_kernels.cu:968-971,
    1036-1046): ids = top-k of f32(raw + bias), higher first, ties to the
    lower index; weights = exp(raw_w - max raw_w) / sum * scale over the
    winners' RAW logits, in f64."""
    score = (raw + bias).astype(np.float32)
    ids = sorted(range(len(raw)), key=lambda e: (-float(score[e]), e))[:k]
    z = raw[ids].astype(np.float64)
    p = np.exp(z - z.max())
    return ids, p / p.sum() * scale


@pytest.mark.parametrize("n_expert,k,seed", [(256, 8, 0), (128, 8, 1), (32, 4, 2), (9, 9, 3)])
def test_router_softmax_mode_with_selection_bias(n_expert, k, seed):
    r = np.random.default_rng(seed)
    n_tok = 5
    raw = (r.permutation(n_expert)[None, :] * 0.05 + r.integers(-3, 4, (n_tok, 1))).astype(np.float32)
    raw[1] = raw[1][::-1]
    # biases large enough to reorder the raw logits, so selection by raw
    # alone and selection by raw + bias differ
    bias = (r.permutation(n_expert) * 0.03 - n_expert * 0.015).astype(np.float32)
    # an exact tie of raw + bias between two experts: the lower index wins
    raw[2, 7 % n_expert] = raw[2, 3]
    bias[7 % n_expert] = bias[3]
    sel, w = oracle.router_select(raw, bias, n_expert, k, 2.5, n_tok, 1)
    for t in range(n_tok):
        ids, want = _mode1_closed(raw[t], bias, k, 2.5)
        assert list(sel[t]) == ids, t
        np.testing.assert_allclose(w[t].astype(np.float64), want, rtol=2e-6, atol=1e-7)
    if k < n_expert:
        # the bias changes the selection here, and weighting by raw + bias
        # instead of raw (a plausible misreading) changes the weights
        by_raw = [sorted(range(n_expert), key=lambda e: (-float(raw[t, e]), e))[:k] for t in range(n_tok)]
        assert any(list(sel[t]) != by_raw[t] for t in range(n_tok))
        ids, want = _mode1_closed(raw[0], bias, k, 2.5)
        z = (raw[0, ids] + bias[ids]).astype(np.float64)
        wrong = np.exp(z - z.max())
        wrong = wrong / wrong.sum() * 2.5
        assert np.abs(wrong - want).max() > 1e-3
        assert np.abs(w[0] - wrong).max() > 1e-3


def test_router_nan_scores_never_win():
    """A NaN score compares neither greater nor equal (pulsar_kernels.cu:
    922-925), so NaN experts are never selected; once the finite experts
    are taken (their scores set to -inf) the lowest-index taken expert wins
    again; a token whose scores are all NaN keeps the start value
    (UINT32_MAX, prob 0) in every slot: id -1 (cu:979-1009; the reference
    kernel's padding lanes, when it has them, would give id n_expert
    instead, an id outside the bank). Mode 0 then divides 0 by the 6.1e-5
    floor, mode 1 softmaxes k zeros to 1/k."""
    n_expert, k = 8, 4
    raw = np.zeros((3, n_expert), np.float32)
    raw[0] = [0.5, np.nan, 0.25, np.nan, 1.0, np.nan, np.nan, np.nan]
    raw[1] = np.nan
    raw[2] = np.arange(n_expert, dtype=np.float32)
    bias = np.zeros(n_expert, np.float32)
    bias[5] = np.nan  # a NaN bias makes that expert's score NaN
    for mode in (0, 1):
        sel, w = oracle.router_select(raw, bias, n_expert, k, 2.0, 3, mode)
        # finite experts 4, 0, 2 by score, then -inf ties: lowest index 0
        assert list(sel[0]) == [4, 0, 2, 0], mode
        assert list(sel[1]) == [-1] * k, mode
        assert list(sel[2]) == [7, 6, 4, 3], mode  # 5 has a NaN bias
        if mode == 0:
            assert (w[1] == 0).all()
        else:
            np.testing.assert_array_equal(w[1], np.full(k, 2.0 / k, np.float32))
        assert np.isfinite(w).all()


def test_router_sigmoid_mode_and_ties():
    n_expert, k = 64, 8
    logits = (rng.standard_normal((3, n_expert)) * 4).astype(np.float32)
    bias = rng.standard_normal(n_expert).astype(np.float32)
    sel, w = oracle.router_select(logits, bias, n_expert, k, 2.5, 3, 0)
    for t in range(3):
        p = 1 / (1 + np.exp(-logits[t].astype(np.float64)))
        top = np.argsort(-(p + bias), kind="stable")[:k]
        assert list(sel[t]) == list(top)
        assert np.allclose(w[t], p[top] / p[top].sum() * 2.5, atol=1e-5, rtol=0)
    tied = np.zeros((1, 16), np.float32)
    sel, _ = oracle.router_select(tied, None, 16, 4, 1.0, 1, 1)
    assert list(sel[0]) == [0, 1, 2, 3]


# ------------------------------------------------------- MoE composition --

def small_layer(quant_g=QUANT_Q4_K, quant_d=QUANT_Q6_K, hidden=512, ffn=256, E=6, n_used=3, n_tok=2):
    g = synth.quant_matrix(quant_g, E * ffn, hidden, synth.rng_for(1, "g")).reshape(E, ffn, -1)
    u = synth.quant_matrix(quant_g, E * ffn, hidden, synth.rng_for(1, "u")).reshape(E, ffn, -1)
    d = synth.quant_matrix(quant_d, E * hidden, ffn, synth.rng_for(1, "d")).reshape(E, hidden, -1)
    sel = rng.integers(0, E, (n_tok, n_used))
    w = rng.uniform(0.1, 1.0, (n_tok, n_used)).astype(np.float32)
    x = rng.standard_normal((n_tok, hidden)).astype(np.float32)
    return g, u, d, sel, w, x


def test_moe_pair_null_slot_weight_linearity_and_down_sum():
    g, u, d, sel, w, x = small_layer()
    E, ffn, grb = g.shape[0], g.shape[1], g.shape[2]
    hidden, drb = d.shape[1], d.shape[2]
    n_tok, n_used = sel.shape
    entries = [(g[e], u[e], d[e]) for e in sel.reshape(-1)]
    entries[1] = (None, None, None)
    ptrs = oracle.host_ptrs(entries)
    xq = oracle.quantize_q8_k(x)
    mid = oracle.moe_pair_swiglu(ptrs, w, xq, hidden, ffn, n_used, n_tok, grb, QUANT_Q4_K, 0)
    assert not mid[1].any()
    mid2 = oracle.moe_pair_swiglu(ptrs, w * 2, xq, hidden, ffn, n_used, n_tok, grb, QUANT_Q4_K, 0)
    assert np.array_equal(mid2, mid * 2)  # scaling by 2 is exact in fp32
    # gate/up rows are the dense matvec of the expert
    e0 = sel[0, 0]
    gd = oracle.matmul_kq(g[e0], xq[0], hidden, ffn, 1, grb, QUANT_Q4_K)[0]
    ud = oracle.matmul_kq(u[e0], xq[0], hidden, ffn, 1, grb, QUANT_Q4_K)[0]
    want = np.array([oracle.glu(float(a), float(b), 0) for a, b in zip(gd, ud)], np.float32) * w[0, 0]
    assert np.array_equal(mid[0], want)
    midq = oracle.quantize_q8_k(mid)
    out = oracle.moe_down(ptrs, midq, ffn, hidden, n_used, n_tok, drb, QUANT_Q6_K)
    for t in range(n_tok):
        acc = np.zeros(hidden, np.float32)
        for s in range(n_used):
            if t * n_used + s == 1:
                continue
            acc += oracle.matmul_kq(d[sel[t, s]], midq[t * n_used + s], ffn, hidden, 1, drb, QUANT_Q6_K)[0]
        assert np.array_equal(out[t], acc)


def test_moe_down_bias_formula():
    n_tok, n_used, hidden = 2, 3, 64
    b = [rng.standard_normal(hidden).astype(np.float32) for _ in range(3)]
    entries = [(None, None, None, None, None, b[i % 3]) for i in range(n_tok * n_used)]
    entries[4] = (None,) * 6
    ptrs = oracle.host_ptrs(entries)
    w = rng.uniform(0.1, 1, (n_tok, n_used)).astype(np.float32)
    base = rng.standard_normal((n_tok, hidden)).astype(np.float32)
    got = oracle.moe_down_bias(base, ptrs, w, hidden, n_used, n_tok)
    for t in range(n_tok):
        acc = np.zeros(hidden, np.float32)
        for s in range(n_used):
            if t * n_used + s != 4:
                acc += w[t, s] * b[(t * n_used + s) % 3]
        assert np.array_equal(got[t], base[t] + acc)


def test_lane_threads_equal_serial_composition():
    g, u, d, sel, w, x = small_layer(hidden=512, ffn=512, E=5, n_used=3, n_tok=3)
    entries = [(g[e], u[e], d[e]) for e in sel.reshape(-1)]
    ptrs = oracle.host_ptrs(entries)
    hidden, ffn = x.shape[1], g.shape[1]
    n_tok, n_used = sel.shape
    xq = oracle.quantize_q8_k(x)
    mid = oracle.moe_pair_swiglu(ptrs, w, xq, hidden, ffn, n_used, n_tok, g.shape[2], QUANT_Q4_K, 0)
    serial = oracle.moe_down(ptrs, oracle.quantize_q8_k(mid), ffn, hidden, n_used, n_tok, d.shape[2], QUANT_Q6_K)
    for threads in (1, 4):
        lane = oracle.lane_moe(ptrs, w, x, hidden, ffn, hidden, n_used, n_tok, g.shape[2], QUANT_Q4_K,
                               d.shape[2], QUANT_Q6_K, 0, threads)
        assert np.array_equal(lane, serial)


def test_error_contract():
    w = np.zeros((4, row_bytes(QUANT_Q4_K, 256)), np.uint8)
    xq = oracle.quantize_q8_k(np.ones((1, 256), np.float32))
    assert oracle.matmul_kq(w, xq, 256, 4, 1, w.shape[1], QUANT_Q4_K) is not None
    assert oracle.matmul_kq(w, xq, 200, 4, 1, w.shape[1], QUANT_Q4_K) is None  # in_dim % 256
    assert oracle.matmul_kq(w, xq, 256, 4, 1, w.shape[1], QUANT_MXFP4) is None  # not a dense format
    assert oracle.matmul_kq(w, xq, 256, 0, 1, w.shape[1], QUANT_Q4_K) is None
    assert oracle.router_select(np.zeros((1, 8), np.float32), None, 8, 9, 1.0, 1, 1) is None
