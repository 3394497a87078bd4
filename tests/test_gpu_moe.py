"""GPU parity of the routed-MoE stages against the oracle.

Stage tolerances (derived from the row-dot tolerance in tests/gpu_util.py):
  pair : |d mid| <= 1e-5 * w * (1.5 (|u|+1) A_g + (|g|+1) A_u) + 4e-7 |mid|,
         A_g, A_u = sum_b |f_b| of the gate/up row dots; the last term covers
         the device expf against the host expf (a few ulp);
  down : fed the oracle's own mid q8_K, |d out| <= 1e-5 * sum_s A_s;
  slot sum, down bias: bit-exact (same operation order on both sides).
"""
import numpy as np
import pytest
import torch

import oracle
from pulsar_amd import formats as fm
from pulsar_amd import kernels as K
from pulsar_amd import synth
from pulsar_amd.formats import (ACT_SILU, ACT_SWIGLU_OAI, QUANT_IQ2_XXS, QUANT_MXFP4, QUANT_Q2_K, QUANT_Q4_K,
                                QUANT_Q6_K, q8k_blocks, row_bytes)
from tests.gpu_util import TOL_REL, down, up, up_f32, zeros_f32

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(2024)


class Layer:
    """A small expert bank on host and device, with routed (token, slot) pointers."""

    def __init__(self, gq, dq, hidden, ffn, E, n_used, n_tok, biases=False, null_slots=(), seed=0):
        self.gq, self.dq, self.hidden, self.ffn, self.E = gq, dq, hidden, ffn, E
        self.n_used, self.n_tok = n_used, n_tok
        self.grb, self.drb = row_bytes(gq, hidden), row_bytes(dq, ffn)
        r = synth.rng_for(seed, f"layer{gq}{dq}{hidden}{ffn}")
        self.g = synth.quant_matrix(gq, E * ffn, hidden, r).reshape(E, ffn, -1)
        self.u = synth.quant_matrix(gq, E * ffn, hidden, r).reshape(E, ffn, -1)
        self.d = synth.quant_matrix(dq, E * hidden, ffn, r).reshape(E, hidden, -1)
        self.gb = self.ub = self.db = None
        if biases:
            self.gb = (r.standard_normal((E, ffn)) * 0.02).astype(np.float32)
            self.ub = (r.standard_normal((E, ffn)) * 0.02).astype(np.float32)
            self.db = (r.standard_normal((E, hidden)) * 0.02).astype(np.float32)
        self.sel = r.integers(0, E, (n_tok, n_used))
        for si in null_slots:
            self.sel.reshape(-1)[si] = -1
        self.w = r.uniform(0.1, 1.0, (n_tok, n_used)).astype(np.float32)
        self.x = r.standard_normal((n_tok, hidden)).astype(np.float32)
        # device copies (+256 B slack after each bank, like the engine's slabs)
        self.dg, self.du, self.dd = (up(np.concatenate([a.reshape(-1), np.zeros(256, np.uint8)]))
                                     for a in (self.g, self.u, self.d))
        self.dbias = [None if b is None else up_f32(b) for b in (self.gb, self.ub, self.db)]

    def host_entries(self, e):
        if e < 0:
            return (None,) * 6
        b = [None if a is None else a[e] for a in (self.gb, self.ub, self.db)]
        return (self.g[e], self.u[e], self.d[e], *b)

    def dev_entries(self, e):
        if e < 0:
            return (0,) * 6
        gb, ub, db = self.dbias
        return (self.dg.data_ptr() + e * self.ffn * self.grb, self.du.data_ptr() + e * self.ffn * self.grb,
                self.dd.data_ptr() + e * self.hidden * self.drb,
                0 if gb is None else gb.data_ptr() + e * self.ffn * 4,
                0 if ub is None else ub.data_ptr() + e * self.ffn * 4,
                0 if db is None else db.data_ptr() + e * self.hidden * 4)

    def ptrs(self):
        flat = self.sel.reshape(-1)
        return (oracle.host_ptrs([self.host_entries(e) for e in flat]),
                up(K.expert_ptrs([self.dev_entries(e) for e in flat])))


def pair_bound(L: Layer, xq, act_op):
    """Per (token*slot, row) tolerance for the pair stage."""
    bound = np.zeros((L.n_tok * L.n_used, L.ffn))
    for t in range(L.n_tok):
        for s in range(L.n_used):
            e = L.sel[t, s]
            if e < 0:
                continue
            for r in range(L.ffn):
                g, ag = oracle.vec_dot(L.gq, L.g[e, r], xq[t], L.hidden)
                u, au = oracle.vec_dot(L.gq, L.u[e, r], xq[t], L.hidden)
                bound[t * L.n_used + s, r] = TOL_REL * L.w[t, s] * (1.5 * (abs(u) + 1) * ag + (abs(g) + 1) * au)
    return bound


def down_bound(L: Layer, midq):
    mb = -(-L.ffn // 256) * 292
    bound = np.zeros((L.n_tok, L.hidden))
    for t in range(L.n_tok):
        for s in range(L.n_used):
            e = L.sel[t, s]
            if e < 0:
                continue
            q = midq[t * L.n_used + s]
            for r in range(L.hidden):
                bound[t, r] += oracle.vec_dot(L.dq, L.d[e, r], q, L.ffn)[1]
    return TOL_REL * bound + 1e-30


def run_pair(L: Layer, act_op, dptrs, xq):
    mid = zeros_f32((L.n_tok * L.n_used, L.ffn))
    K.moe_pair_swiglu(mid, dptrs, up_f32(L.w), up(xq), L.hidden, L.ffn, L.n_used, L.n_tok, L.grb, L.gq, act_op)
    return down(mid)


def check_pair_down(L: Layer, act_op):
    hptrs, dptrs = L.ptrs()
    xq = oracle.quantize_q8_k(L.x)
    got_mid = run_pair(L, act_op, dptrs, xq)
    want_mid = oracle.moe_pair_swiglu(hptrs, L.w, xq, L.hidden, L.ffn, L.n_used, L.n_tok, L.grb, L.gq, act_op)
    bound = pair_bound(L, xq, act_op) + 4e-7 * np.abs(want_mid) + 1e-30
    err = np.abs(got_mid.astype(np.float64) - want_mid)
    assert (err <= bound).all(), f"pair: max err {err.max():.3e} (worst ratio {(err / bound).max():.2f})"
    for si, e in enumerate(L.sel.reshape(-1)):
        if e < 0:
            assert not got_mid[si].any()  # NULL slot writes zeros
    # down on the oracle's own mid q8_K
    midq = oracle.quantize_q8_k(want_mid)
    out = zeros_f32((L.n_tok, L.hidden))
    K.moe_down(out, dptrs, up(midq), L.ffn, L.hidden, L.n_used, L.n_tok, L.drb, L.dq)
    got = down(out)
    want = oracle.moe_down(hptrs, midq, L.ffn, L.hidden, L.n_used, L.n_tok, L.drb, L.dq)
    err = np.abs(got.astype(np.float64) - want)
    bound = down_bound(L, midq)
    assert (err <= bound).all(), f"down: max err {err.max():.3e} (worst ratio {(err / bound).max():.2f})"
    return hptrs, dptrs, xq, want_mid, midq, want


@pytest.mark.parametrize("gq,dq", [(QUANT_Q4_K, QUANT_Q6_K), (QUANT_Q2_K, QUANT_Q2_K),
                                   (QUANT_IQ2_XXS, QUANT_IQ2_XXS), (QUANT_Q6_K, QUANT_Q4_K)])
def test_pair_down_kquants(dev, gq, dq):
    L = Layer(gq, dq, hidden=512, ffn=256, E=8, n_used=4, n_tok=3, null_slots=(6,))
    check_pair_down(L, ACT_SILU)


@pytest.mark.parametrize("hidden,ffn", [(2880, 704), (512, 320)])
def test_pair_down_mxfp4_tails_biases_oai(dev, hidden, ffn):
    L = Layer(QUANT_MXFP4, QUANT_MXFP4, hidden=hidden, ffn=ffn, E=4, n_used=4, n_tok=2, biases=True,
              null_slots=(1,))
    hptrs, dptrs, xq, mid, midq, out = check_pair_down(L, ACT_SWIGLU_OAI)
    # down bias: bit-exact against the oracle
    d_out = up_f32(out)
    K.moe_down_bias(d_out, dptrs, up_f32(L.w), L.hidden, L.n_used, L.n_tok)
    want = oracle.moe_down_bias(out, hptrs, L.w, L.hidden, L.n_used, L.n_tok)
    assert np.array_equal(down(d_out), want)


@pytest.mark.parametrize("gq,dq,hidden,ffn,E,n_used,n_tok", [
    (QUANT_MXFP4, QUANT_MXFP4, 2880, 2880, 6, 4, 1),  # the c5 batch-1 shape
    (QUANT_Q4_K, QUANT_Q6_K, 512, 2048, 10, 8, 5),
])
def test_pair_two_passes_per_wave(dev, gq, dq, hidden, ffn, E, n_used, n_tok):
    """Launches of more than 2048 pair blocks run two row passes per wave
    (the second pass's loads in flight during the first)."""
    mx = gq == QUANT_MXFP4
    L = Layer(gq, dq, hidden=hidden, ffn=ffn, E=E, n_used=n_used, n_tok=n_tok, biases=mx, null_slots=(2,))
    check_pair_down(L, ACT_SWIGLU_OAI if mx else ACT_SILU)


def test_pair_down_decode_shapes(dev):
    """The c3 shape (hidden 2048, FFN 512, 8 routed + 1 shared slot) at a
    reduced expert count."""
    L = Layer(QUANT_Q4_K, QUANT_Q6_K, hidden=2048, ffn=512, E=10, n_used=9, n_tok=1)
    check_pair_down(L, ACT_SILU)


@pytest.mark.parametrize("gq,dq,n_tok", [(QUANT_Q2_K, QUANT_Q2_K, 16), (QUANT_IQ2_XXS, QUANT_IQ2_XXS, 16),
                                          (QUANT_Q2_K, QUANT_Q2_K, 40), (QUANT_IQ2_XXS, QUANT_IQ2_XXS, 40),
                                          (QUANT_Q4_K, QUANT_Q6_K, 16), (QUANT_Q4_K, QUANT_Q6_K, 40),
                                          (QUANT_Q6_K, QUANT_Q4_K, 24), (fm.QUANT_Q5_K, fm.QUANT_Q5_K, 40)])
def test_grouped_mfma_kquants(dev, gq, dq, n_tok):
    """K-quant / IQ2_XXS groups run on the matrix cores: pair and down
    against the oracle (more than 16 pairs per group at n_tok 40: several
    pair tiles), NULL slots, the slot sum in slot order."""
    L = Layer(gq, dq, hidden=1024, ffn=512, E=6, n_used=4, n_tok=n_tok, null_slots=(3, 17))
    hptrs, dptrs, xq, want_mid, midq, want_out = check_pair_down(L, ACT_SILU)
    ids, starts, pairs = synth.csr_by_expert(L.sel, L.n_used)
    gptrs = up(K.expert_ptrs([L.dev_entries(int(e)) for e in ids]))
    mid = zeros_f32((L.n_tok * L.n_used, L.ffn))
    K.moe_pair_swiglu_grouped(mid, gptrs, up(starts), up(pairs), up_f32(L.w), up(xq), L.hidden, L.ffn,
                              L.n_used, len(ids), L.grb, gq, ACT_SILU)
    got_mid = down(mid)
    bound = pair_bound(L, xq, ACT_SILU) + 4e-7 * np.abs(want_mid) + 1e-30
    err = np.abs(got_mid.astype(np.float64) - want_mid)
    assert (err <= bound).all(), f"grouped pair: max err {err.max():.3e} (worst ratio {(err / bound).max():.2f})"
    for si, e in enumerate(L.sel.reshape(-1)):
        if e < 0:
            assert not got_mid[si].any()  # NULL slots are not in any group: rows stay zero
    partial = zeros_f32((L.n_tok * L.n_used, L.hidden))
    K.moe_down_grouped(partial, gptrs, up(starts), up(pairs), up(midq), L.ffn, L.hidden, L.n_used, len(ids),
                       L.drb, dq)
    out = zeros_f32((L.n_tok, L.hidden))
    K.moe_slot_sum(out, partial, L.hidden, L.n_used, L.n_tok)
    err = np.abs(down(out).astype(np.float64) - want_out)
    bound = down_bound(L, midq)
    assert (err <= bound).all(), f"grouped down: max err {err.max():.3e} (worst ratio {(err / bound).max():.2f})"
    # slot sum is the in-order sum of the partials
    p = down(partial).reshape(L.n_tok, L.n_used, L.hidden)
    acc = np.zeros((L.n_tok, L.hidden), np.float32)
    for s in range(L.n_used):
        acc += p[:, s]
    assert np.array_equal(down(out), acc)


@pytest.mark.parametrize("gq", [QUANT_Q2_K, QUANT_IQ2_XXS, QUANT_Q4_K, QUANT_Q6_K, fm.QUANT_Q5_K])
def test_grouped_mfma_pair_row_tail(dev, gq):
    """A pair stage whose row count (200) is not a multiple of the 16-row
    tile, and 3 super-blocks (768) over the 4 waves' ranges."""
    L = Layer(gq, gq, hidden=768, ffn=200, E=5, n_used=3, n_tok=9)
    hptrs, dptrs = L.ptrs()
    xq = oracle.quantize_q8_k(L.x)
    want_mid = oracle.moe_pair_swiglu(hptrs, L.w, xq, L.hidden, L.ffn, L.n_used, L.n_tok, L.grb, L.gq, ACT_SILU)
    ids, starts, pairs = synth.csr_by_expert(L.sel, L.n_used)
    gptrs = up(K.expert_ptrs([L.dev_entries(int(e)) for e in ids]))
    mid = zeros_f32((L.n_tok * L.n_used, L.ffn))
    K.moe_pair_swiglu_grouped(mid, gptrs, up(starts), up(pairs), up_f32(L.w), up(xq), L.hidden, L.ffn,
                              L.n_used, len(ids), L.grb, gq, ACT_SILU)
    bound = pair_bound(L, xq, ACT_SILU) + 4e-7 * np.abs(want_mid) + 1e-30
    err = np.abs(down(mid).astype(np.float64) - want_mid)
    assert (err <= bound).all(), f"grouped pair: max err {err.max():.3e} (worst ratio {(err / bound).max():.2f})"


@pytest.mark.parametrize("n_tok", [3, 40])
def test_grouped_mxfp4_mfma(dev, n_tok):
    """MXFP4 groups run on the matrix cores (more than 16 pairs per group at
    n_tok 40: two pair tiles); tail super-blocks (576 = 2 x 256 + 64, 320 =
    256 + 64), biases, swiglu_oai and NULL slots."""
    L = Layer(QUANT_MXFP4, QUANT_MXFP4, hidden=576, ffn=320, E=6, n_used=4, n_tok=n_tok, biases=True,
              null_slots=(1, 6))
    hptrs, dptrs, xq, want_mid, midq, want_out = check_pair_down(L, ACT_SWIGLU_OAI)
    ids, starts, pairs = synth.csr_by_expert(L.sel, L.n_used)
    gptrs = up(K.expert_ptrs([L.dev_entries(int(e)) for e in ids]))
    mid = zeros_f32((L.n_tok * L.n_used, L.ffn))
    K.moe_pair_swiglu_grouped(mid, gptrs, up(starts), up(pairs), up_f32(L.w), up(xq), L.hidden, L.ffn,
                              L.n_used, len(ids), L.grb, QUANT_MXFP4, ACT_SWIGLU_OAI)
    got_mid = down(mid)
    bound = pair_bound(L, xq, ACT_SWIGLU_OAI) + 4e-7 * np.abs(want_mid) + 1e-30
    err = np.abs(got_mid.astype(np.float64) - want_mid)
    assert (err <= bound).all(), f"grouped mfma pair: max err {err.max():.3e}"
    partial = zeros_f32((L.n_tok * L.n_used, L.hidden))
    K.moe_down_grouped(partial, gptrs, up(starts), up(pairs), up(midq), L.ffn, L.hidden, L.n_used, len(ids),
                       L.drb, QUANT_MXFP4)
    out = zeros_f32((L.n_tok, L.hidden))
    K.moe_slot_sum(out, partial, L.hidden, L.n_used, L.n_tok)
    # the down bias is a separate stage on both paths
    want = oracle.moe_down(hptrs, midq, L.ffn, L.hidden, L.n_used, L.n_tok, L.drb, QUANT_MXFP4)
    err = np.abs(down(out).astype(np.float64) - want)
    assert (err <= down_bound(L, midq)).all(), f"grouped mfma down: max err {err.max():.3e}"


def _random_grouped_cases(n_per_format=3):
    """Seeded random grouped-layer shapes per format: input widths with odd
    and even super-block counts (the staged pair rows' pitch differs), row
    counts off the block size, 1-11 tokens of 1-4 slots over 2-9 experts
    (a slot may repeat its token's expert), NULL slots."""
    r = np.random.default_rng(8191)
    cases = []
    for q in (QUANT_Q2_K, QUANT_IQ2_XXS, QUANT_Q4_K, fm.QUANT_Q5_K, QUANT_Q6_K, QUANT_MXFP4):
        for _ in range(n_per_format):
            if q == QUANT_MXFP4:
                hidden, ffn = 32 * int(r.integers(8, 48)), 32 * int(r.integers(4, 16))
            else:
                hidden, ffn = 256 * int(r.integers(1, 7)), 256 * int(r.integers(1, 3))
            E, n_used, n_tok = int(r.integers(2, 10)), int(r.integers(1, 5)), int(r.integers(1, 12))
            n_null = int(r.integers(0, 3))
            nulls = tuple(int(v) for v in r.choice(n_tok * n_used, size=min(n_null, n_tok * n_used - 1),
                                                    replace=False)) if n_tok * n_used > 1 else ()
            cases.append((q, hidden, ffn, E, n_used, n_tok, nulls, int(r.integers(0, 1 << 30))))
    return cases


@pytest.mark.parametrize("q,hidden,ffn,E,n_used,n_tok,nulls,seed", _random_grouped_cases())
def test_grouped_random_shapes(dev, q, hidden, ffn, E, n_used, n_tok, nulls, seed):
    """Grouped pair and down stages against the oracle on seeded random
    shapes (every grouped format; MXFP4 with biases and swiglu_oai)."""
    mx = q == QUANT_MXFP4
    L = Layer(q, q, hidden=hidden, ffn=ffn, E=E, n_used=n_used, n_tok=n_tok, biases=mx, null_slots=nulls,
              seed=seed)
    _grouped_vs_oracle(L, q)


@pytest.mark.parametrize("q,hidden,ffn", [(QUANT_Q2_K, 512, 768), (QUANT_IQ2_XXS, 768, 512),
                                          (QUANT_Q4_K, 512, 512), (fm.QUANT_Q5_K, 256, 512),
                                          (QUANT_Q6_K, 512, 256), (QUANT_MXFP4, 1280, 416)])
def test_grouped_many_pairs_per_expert(dev, q, hidden, ffn):
    """Groups of 20-39 pairs (two or three pair tiles per weight pass) over
    matrices of several row tiles per wave: each pair tile walks the wave's
    row tiles again from the first. 40 tokens x 2 slots over 3 experts, one
    NULL slot."""
    L = Layer(q, q, hidden=hidden, ffn=ffn, E=3, n_used=2, n_tok=40, biases=q == QUANT_MXFP4, seed=5)
    L.sel[:, 0] = 0
    L.sel[:, 1] = np.where(np.arange(40) % 2 == 0, 1, 2)
    L.sel[7, 1] = -1
    _grouped_vs_oracle(L, q)


@pytest.mark.parametrize("q", [QUANT_Q2_K, QUANT_IQ2_XXS, QUANT_Q4_K, QUANT_MXFP4])
def test_grouped_partial_row_tiles(dev, q):
    """Row counts that end inside a wave's 16-row tile (and inside its
    second row tile where a wave takes two): each row's value depends only
    on its own weights, so the first n rows of a launch over n rows equal,
    bit for bit, those of the launch over the whole matrix. Groups of
    several pair tiles are included (20 tokens x 2 slots over 3 experts)."""
    hidden, ffn = (512, 256)
    L = Layer(q, q, hidden=hidden, ffn=ffn, E=3, n_used=2, n_tok=20, biases=q == QUANT_MXFP4, seed=11)
    L.sel[3, 1] = -1
    act = ACT_SWIGLU_OAI if q == QUANT_MXFP4 else ACT_SILU
    hptrs, dptrs = L.ptrs()
    xq = up(oracle.quantize_q8_k(L.x))
    ids, starts, pairs = synth.csr_by_expert(L.sel, L.n_used)
    gptrs = up(K.expert_ptrs([L.dev_entries(int(e)) for e in ids]))
    starts, pairs, w = up(starts), up(pairs), up_f32(L.w)
    n_pairs = L.n_tok * L.n_used

    def pair(rows):
        # NaN-filled: the CSR stage leaves the NULL slot's row alone in both launches
        mid = torch.full((n_pairs, rows), float("nan"), dtype=torch.float32, device=dev)
        K.moe_pair_swiglu_grouped(mid, gptrs, starts, pairs, w, xq, hidden, rows, L.n_used, len(ids), L.grb, q,
                                  act)
        return down(mid)

    full = pair(ffn)
    for rows in (200, 24, 8, 1):
        assert np.array_equal(pair(rows).view(np.uint32), full[:, :rows].view(np.uint32)), rows
    midq = up(oracle.quantize_q8_k(np.nan_to_num(full)))

    def down_rows(rows):
        part = torch.zeros((n_pairs, rows), dtype=torch.float32, device=dev)
        K.moe_down_grouped(part, gptrs, starts, pairs, midq, ffn, rows, L.n_used, len(ids), L.drb, q)
        return down(part)

    full_d = down_rows(hidden)
    for rows in (200, 40, 8, 1):
        assert np.array_equal(down_rows(rows).view(np.uint32), full_d[:, :rows].view(np.uint32)), rows


def _grouped_vs_oracle(L: Layer, q):
    act = ACT_SWIGLU_OAI if q == QUANT_MXFP4 else ACT_SILU
    hptrs, dptrs = L.ptrs()
    xq = oracle.quantize_q8_k(L.x)
    want_mid = oracle.moe_pair_swiglu(hptrs, L.w, xq, L.hidden, L.ffn, L.n_used, L.n_tok, L.grb, L.gq, act)
    ids, starts, pairs = synth.csr_by_expert(L.sel, L.n_used)
    gptrs = up(K.expert_ptrs([L.dev_entries(int(e)) for e in ids]))
    mid = zeros_f32((L.n_tok * L.n_used, L.ffn))
    K.moe_pair_swiglu_grouped(mid, gptrs, up(starts), up(pairs), up_f32(L.w), up(xq), L.hidden, L.ffn,
                              L.n_used, len(ids), L.grb, q, act)
    got_mid = down(mid)
    bound = pair_bound(L, xq, act) + 4e-7 * np.abs(want_mid) + 1e-30
    err = np.abs(got_mid.astype(np.float64) - want_mid)
    assert (err <= bound).all(), f"grouped pair: max err {err.max():.3e} (worst ratio {(err / bound).max():.2f})"
    for si, e in enumerate(L.sel.reshape(-1)):
        if e < 0:
            assert not got_mid[si].any()
    midq = oracle.quantize_q8_k(want_mid)
    partial = zeros_f32((L.n_tok * L.n_used, L.hidden))
    K.moe_down_grouped(partial, gptrs, up(starts), up(pairs), up(midq), L.ffn, L.hidden, L.n_used, len(ids),
                       L.drb, q)
    out = zeros_f32((L.n_tok, L.hidden))
    K.moe_slot_sum(out, partial, L.hidden, L.n_used, L.n_tok)
    want = oracle.moe_down(hptrs, midq, L.ffn, L.hidden, L.n_used, L.n_tok, L.drb, q)
    err = np.abs(down(out).astype(np.float64) - want)
    bound = down_bound(L, midq)
    assert (err <= bound).all(), f"grouped down: max err {err.max():.3e} (worst ratio {(err / bound).max():.2f})"


def test_grouped_contract(dev):
    buf = up(np.zeros(4096, np.uint8))
    with pytest.raises(K.KernelError):  # in_dim % 256 (pulsar_kernels.cu:3488)
        K.moe_pair_swiglu_grouped(buf, buf, buf, buf, buf, buf, 2880, 64, 4, 1, 1530, QUANT_Q4_K, 0)
    with pytest.raises(K.KernelError):  # MXFP4: whole 32-value blocks
        K.moe_pair_swiglu_grouped(buf, buf, buf, buf, buf, buf, 2870, 64, 4, 1, 1530, QUANT_MXFP4, 0)
    with pytest.raises(K.KernelError):  # n_used > 16 cannot be packed in pairs
        K.moe_pair_swiglu_grouped(buf, buf, buf, buf, buf, buf, 256, 64, 17, 1, 144, QUANT_Q4_K, 0)
    with pytest.raises(K.KernelError):  # mid_dim % 256 for the grouped down
        K.moe_down_grouped(buf, buf, buf, buf, buf, 704, 64, 4, 1, 374, QUANT_Q6_K)
    with pytest.raises(K.KernelError):
        K.moe_pair_swiglu(buf, buf, buf, buf, 256, 64, 4, 1, 144, 99, 0)  # unknown quant
    torch.cuda.synchronize()


# ------------------------------------------------------------------ router --

@pytest.mark.parametrize("n_expert,k,n_tok,mode", [(256, 8, 1, 1), (128, 8, 16, 1), (32, 4, 64, 1),
                                                   (64, 8, 7, 0), (896, 16, 3, 1), (256, 6, 5, 2)])
def test_router_select(dev, n_expert, k, n_tok, mode):
    n_sh = 2 if mode == 2 else 0
    logits = (rng.standard_normal((n_tok, n_expert + n_sh)) * 4).astype(np.float32)
    bias = rng.standard_normal(n_expert).astype(np.float32) if mode != 1 else np.zeros(n_expert, np.float32)
    n_slot = k + n_sh
    sel = torch.zeros((n_tok, n_slot), dtype=torch.int32, device=dev)
    w = zeros_f32((n_tok, n_slot))
    K.router_select(sel, w, up_f32(logits), up_f32(bias), n_expert, k, 1.5, n_tok, mode, n_sh)
    want_sel, want_w = oracle.router_select(logits, bias, n_expert, k, 1.5, n_tok, mode, n_sh)
    assert np.array_equal(down(sel), want_sel)
    assert np.allclose(down(w), want_w, rtol=0, atol=1e-6)


@pytest.mark.parametrize("n_expert,k,n_tok", [(256, 8, 1), (128, 8, 16), (32, 4, 64)])
def test_router_select_softmax_with_selection_bias(dev, n_expert, k, n_tok):
    """Mode 1 selects on raw logit + bias and weights the winners by their
    raw logits (pulsar_kernels.cu:968-971, 1036-1046); the biases are large
    enough to change the selection."""
    logits = (rng.standard_normal((n_tok, n_expert)) * 2).astype(np.float32)
    bias = (rng.standard_normal(n_expert) * 2).astype(np.float32)
    sel = torch.zeros((n_tok, k), dtype=torch.int32, device=dev)
    w = zeros_f32((n_tok, k))
    K.router_select(sel, w, up_f32(logits), up_f32(bias), n_expert, k, 1.5, n_tok, 1, 0)
    want_sel, want_w = oracle.router_select(logits, bias, n_expert, k, 1.5, n_tok, 1, 0)
    raw_sel, _ = oracle.router_select(logits, np.zeros(n_expert, np.float32), n_expert, k, 1.5, n_tok, 1, 0)
    assert not np.array_equal(want_sel, raw_sel)
    assert np.array_equal(down(sel), want_sel)
    assert np.allclose(down(w), want_w, rtol=0, atol=1e-6)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("n_expert", [300, 120, 64])
def test_router_select_ties_inf_nan(dev, mode, n_expert):
    """Tied scores go to the lower index; -inf and NaN logits: NaN never
    wins, and once only -inf remain the lowest index wins again (the
    reference's removed experts are set to -inf, not dropped); a token
    whose logits are all NaN selects -1 with prob 0 in every slot."""
    k, n_tok = 12, 5
    logits = np.full((n_tok, n_expert), 0.5, np.float32)   # all tied
    logits[1, ::7] = -np.inf
    logits[1, 3:5] = 2.0
    logits[2, :] = -np.inf
    logits[2, 10:13] = 1.0                                  # 3 finite, k = 12
    logits[3, ::3] = np.nan
    logits[3, min(100, n_expert - 1)] = 3.0
    logits[4, :] = np.nan
    bias = np.zeros(n_expert, np.float32)
    sel = torch.zeros((n_tok, k), dtype=torch.int32, device=dev)
    w = zeros_f32((n_tok, k))
    K.router_select(sel, w, up_f32(logits), up_f32(bias), n_expert, k, 1.0, n_tok, mode, 0)
    want_sel, want_w = oracle.router_select(logits, bias, n_expert, k, 1.0, n_tok, mode, 0)
    assert np.array_equal(down(sel), want_sel)
    assert (want_sel[4] == -1).all()
    got_w = down(w)
    assert np.array_equal(np.isnan(got_w), np.isnan(want_w))
    ok = ~np.isnan(want_w)
    assert np.allclose(got_w[ok], want_w[ok], rtol=0, atol=1e-6)


@pytest.mark.parametrize("with_bias", [False, True])
def test_router_select_sigmoid_edges(dev, with_bias):
    """Sigmoid scores (mode 0) at the edges of both of its branches: +-0,
    +-inf, NaN, logits that saturate the sigmoid to exactly 1 (ties broken
    by the lower index) and large negative logits whose scores are tiny
    but well separated."""
    n_expert, k, n_tok = 256, 8, 4
    logits = (rng.standard_normal((n_tok, n_expert)) * 3).astype(np.float32)
    logits[0, ::5] = 40.0                                   # sigmoid == 1: a tie run
    logits[0, 1] = -0.0
    logits[0, 2] = 0.0
    logits[1, :] = -np.inf
    logits[1, 20:40] = -(30.0 + np.arange(20, dtype=np.float32))  # exp(x) / (1 + exp(x)) branch
    logits[1, 50] = np.nan
    logits[2, :] = np.nan
    logits[2, 7] = np.inf
    logits[2, 9] = -np.inf
    logits[3, ::2] = -0.0
    logits[3, 1::2] = 0.0
    bias = ((rng.standard_normal(n_expert) * 0.25).astype(np.float32) if with_bias
            else np.zeros(n_expert, np.float32))
    sel = torch.zeros((n_tok, k), dtype=torch.int32, device=dev)
    w = zeros_f32((n_tok, k))
    K.router_select(sel, w, up_f32(logits), up_f32(bias), n_expert, k, 1.0, n_tok, 0, 0)
    want_sel, want_w = oracle.router_select(logits, bias, n_expert, k, 1.0, n_tok, 0, 0)
    assert np.array_equal(down(sel), want_sel)
    got_w = down(w)
    assert np.array_equal(np.isnan(got_w), np.isnan(want_w))
    ok = ~np.isnan(want_w)
    assert np.allclose(got_w[ok], want_w[ok], rtol=0, atol=1e-6)


def test_matmul_f32_and_bias(dev):
    for in_dim, out_dim, n_tok in ((2048, 256, 1), (4096, 128, 16), (2880, 32, 64), (37, 5, 3)):
        wt = (rng.standard_normal((out_dim, in_dim)) / np.sqrt(in_dim)).astype(np.float32)
        x = rng.standard_normal((n_tok, in_dim)).astype(np.float32)
        out = zeros_f32((n_tok, out_dim))
        K.matmul_f32(out, up_f32(wt), up_f32(x), in_dim, out_dim, n_tok)
        want = oracle.matmul_f32(wt, x, in_dim, out_dim, n_tok)
        scale = np.abs(x) @ np.abs(wt).T
        assert (np.abs(down(out) - want) <= 1e-6 * scale + 1e-30).all()
        b = rng.standard_normal(out_dim).astype(np.float32)
        before = down(out)
        K.add_bias_rows(out, up_f32(b), out_dim, n_tok)
        assert np.array_equal(down(out), oracle.add_bias_rows(before, b, out_dim, n_tok))


@pytest.mark.parametrize("out_dim", [8, 12, 16, 24, 32, 40, 64, 100, 128, 136, 256])
def test_gemv_block_order_every_split(dev, out_dim):
    """The router GEMV's blocks are ordered over the 8 XCDs by a row x token-
    group split chosen per shape (none, or 2 / 4 / 8 row bands): every
    (row, token) output must come out once, equal to the oracle's, for token
    counts that give every split and group counts that divide it or not, and
    the fused router's logits bit-identical to matmul_f32's."""
    in_dim = 96
    wt = (rng.standard_normal((out_dim, in_dim)) / np.sqrt(in_dim)).astype(np.float32)
    for n_tok in (1, 2, 5, 8, 16, 17, 32, 33, 64, 128):
        x = rng.standard_normal((n_tok, in_dim)).astype(np.float32)
        out = torch.full((n_tok, out_dim), float("nan"), dtype=torch.float32, device=dev)
        K.matmul_f32(out, up_f32(wt), up_f32(x), in_dim, out_dim, n_tok)
        want = oracle.matmul_f32(wt, x, in_dim, out_dim, n_tok)
        got = down(out)
        scale = np.abs(x) @ np.abs(wt).T
        assert (np.abs(got - want) <= 1e-6 * scale + 1e-30).all(), (out_dim, n_tok)
        logits = torch.full((n_tok, out_dim), float("nan"), dtype=torch.float32, device=dev)
        xq = torch.zeros(n_tok * q8k_blocks(in_dim) * 292, dtype=torch.uint8, device=dev)
        K.router_logits_q8(logits, xq, up_f32(x), up_f32(wt), None, in_dim, out_dim, n_tok)
        assert np.array_equal(down(logits).view(np.uint32), got.view(np.uint32)), (out_dim, n_tok)


# ------------------------------------------------- device routing, graphs --

@pytest.mark.parametrize("E,k,n_tok", [(12, 6, 20), (300, 15, 128), (4, 1, 2)])
def test_route_ptrs_and_group_csr(dev, E, k, n_tok):
    hidden, ffn = 256, 256
    L = Layer(QUANT_Q4_K, QUANT_Q4_K, hidden=hidden, ffn=ffn, E=E, n_used=k, n_tok=n_tok, biases=True)
    sel = rng.integers(0, E, (n_tok, k)).astype(np.int32)
    sel[n_tok // 2, k // 2] = -1  # unrouted
    sel[n_tok - 1, 0] = E + 5  # out of range -> NULL
    rw = rng.uniform(0.1, 1, (n_tok, k)).astype(np.float32)
    gsz, dsz = ffn * L.grb, hidden * L.drb
    bank = K.ExpertBank(L.dg.data_ptr(), L.du.data_ptr(), L.dd.data_ptr(), L.dbias[0].data_ptr(),
                        L.dbias[1].data_ptr(), L.dbias[2].data_ptr(), gsz, gsz, dsz, ffn, ffn, hidden)
    shared = (11 << 20, 12 << 20, 13 << 20)  # opaque addresses: only copied, never dereferenced
    n_slots = k + 1
    ptrs = torch.zeros(n_tok * n_slots * 48, dtype=torch.uint8, device=dev)
    slot_w = zeros_f32((n_tok, n_slots))
    K.moe_route_ptrs(ptrs, slot_w, up(sel), up_f32(rw), bank, E, [shared], n_tok, k)
    got = down(ptrs).view(K.EXPERT_PTRS_DTYPE).reshape(n_tok, n_slots)
    want_w = np.concatenate([rw, np.ones((n_tok, 1), np.float32)], axis=1)
    assert np.array_equal(down(slot_w), want_w)
    for t in range(n_tok):
        for s in range(n_slots):
            if s == k:
                want = shared + (0, 0, 0)
            elif 0 <= sel[t, s] < E:
                want = L.dev_entries(int(sel[t, s]))
            else:
                want = (0,) * 6
            assert tuple(int(v) for v in got[t, s]) == tuple(want), (t, s)
    # CSR by gate pointer, first appearance order, NULL gates skipped
    max_groups = E + 1
    gptrs = torch.zeros(max_groups * 48, dtype=torch.uint8, device=dev)
    starts = torch.zeros(max_groups + 1, dtype=torch.int32, device=dev)
    pairs = torch.zeros(n_tok * n_slots, dtype=torch.int32, device=dev)
    K.moe_group_csr(gptrs, starts, pairs, ptrs, n_tok, n_slots, max_groups)
    ids = np.concatenate([np.where((sel >= 0) & (sel < E), sel, -1), np.full((n_tok, 1), E)], axis=1)
    want_ids, want_starts, want_pairs = synth.csr_by_expert(ids, n_slots)
    g = down(gptrs).view(K.EXPERT_PTRS_DTYPE)
    ng = len(want_ids)
    assert np.array_equal(down(starts)[:ng + 1], want_starts)
    assert (down(starts)[ng:] == want_starts[-1]).all()
    assert np.array_equal(down(pairs)[:len(want_pairs)].astype(np.uint32), want_pairs)
    for gi, e in enumerate(want_ids):
        want = shared + (0, 0, 0) if e == E else L.dev_entries(int(e))
        assert tuple(int(v) for v in g[gi]) == tuple(want)
    assert not g[ng:].view(np.uint64).any()


def test_graph_replays_match_eager(dev):
    """The pair/quantize/down chain captured into a HIP graph on a capture
    stream (pulsar_set_stream) and replayed three times, with eager work in
    between, reproduces the eager result bit for bit every time."""
    L = Layer(QUANT_Q4_K, QUANT_Q6_K, hidden=2048, ffn=512, E=10, n_used=9, n_tok=1)
    _, dptrs = L.ptrs()
    xq = up(oracle.quantize_q8_k(L.x))
    w = up_f32(L.w)
    mid = zeros_f32((L.n_used, L.ffn))
    midq = torch.zeros(L.n_used * 2 * 292, dtype=torch.uint8, device=dev)
    out = zeros_f32((1, L.hidden))

    def chain():
        K.moe_pair_swiglu(mid, dptrs, w, xq, L.hidden, L.ffn, L.n_used, 1, L.grb, L.gq, ACT_SILU)
        K.quantize_q8_k(midq, mid, L.ffn, L.n_used)
        K.moe_down(out, dptrs, midq, L.ffn, L.hidden, L.n_used, 1, L.drb, L.dq)

    chain()
    eager = down(out).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        K.set_stream(torch.cuda.current_stream())
        try:
            chain()
        finally:
            K.set_stream(None)
    for _ in range(3):
        out.zero_()
        mid.fill_(123.0)
        torch.cuda.synchronize()
        g.replay()
        assert np.array_equal(down(out), eager)
        chain()  # eager work between replays
        assert np.array_equal(down(out), eager)


def test_library_selftests(dev):
    """pulsar_moe_selftest / pulsar_router_selftest: the library's own checks
    against its host mirrors (the reference ABI's self-test entry points)."""
    assert K.router_selftest()
    assert K.moe_selftest()


def test_grouped_wide_rows_lane_fallback(dev):
    """Rows too wide for the MFMA kernel's staged activations (14336 values:
    56 q8_K blocks per pair > the 16 KiB tile) run the grouped lane kernels."""
    L = Layer(QUANT_Q4_K, QUANT_Q6_K, hidden=14336, ffn=256, E=3, n_used=2, n_tok=3)
    hptrs, dptrs = L.ptrs()
    xq = oracle.quantize_q8_k(L.x)
    want_mid = oracle.moe_pair_swiglu(hptrs, L.w, xq, L.hidden, L.ffn, L.n_used, L.n_tok, L.grb, L.gq, ACT_SILU)
    ids, starts, pairs = synth.csr_by_expert(L.sel, L.n_used)
    gptrs = up(K.expert_ptrs([L.dev_entries(int(e)) for e in ids]))
    mid = zeros_f32((L.n_tok * L.n_used, L.ffn))
    K.moe_pair_swiglu_grouped(mid, gptrs, up(starts), up(pairs), up_f32(L.w), up(xq), L.hidden, L.ffn,
                              L.n_used, len(ids), L.grb, QUANT_Q4_K, ACT_SILU)
    bound = pair_bound(L, xq, ACT_SILU) + 4e-7 * np.abs(want_mid) + 1e-30
    err = np.abs(down(mid).astype(np.float64) - want_mid)
    assert (err <= bound).all(), f"grouped pair (lane): max err {err.max():.3e}"


NEW_FORMATS = [fm.QUANT_Q5_K, fm.QUANT_Q3_K, fm.QUANT_IQ2_XS, fm.QUANT_IQ3_XXS, fm.QUANT_Q4_0, fm.QUANT_Q5_1,
               fm.QUANT_Q8_0, fm.QUANT_IQ4_XS, fm.QUANT_IQ4_NL, fm.QUANT_IQ3_S, fm.QUANT_IQ2_S, fm.QUANT_IQ1_S,
               fm.QUANT_NVFP4]


@pytest.mark.parametrize("q", NEW_FORMATS, ids=lambda q: fm.NAMES[q])
def test_pair_down_every_format(dev, q):
    """The remaining expert formats (pulsar_kernels.cu:2649-2668) through the
    plain pair / down stages against the oracle; 3 tokens, a NULL slot, 768
    inputs (3 super-blocks) and 512 mid values."""
    L = Layer(q, q, hidden=768, ffn=512, E=6, n_used=4, n_tok=3, null_slots=(5,))
    check_pair_down(L, ACT_SILU)


@pytest.mark.parametrize("q", NEW_FORMATS, ids=lambda q: fm.NAMES[q])
def test_grouped_every_format(dev, q):
    """The same formats through the grouped entry points (Q5_K on the matrix
    cores, the rest on the lane kernels)."""
    L = Layer(q, q, hidden=512, ffn=256, E=5, n_used=4, n_tok=12, null_slots=(7,))
    hptrs, dptrs = L.ptrs()
    xq = oracle.quantize_q8_k(L.x)
    want_mid = oracle.moe_pair_swiglu(hptrs, L.w, xq, L.hidden, L.ffn, L.n_used, L.n_tok, L.grb, q, ACT_SILU)
    ids, starts, pairs = synth.csr_by_expert(L.sel, L.n_used)
    gptrs = up(K.expert_ptrs([L.dev_entries(int(e)) for e in ids]))
    mid = zeros_f32((L.n_tok * L.n_used, L.ffn))
    K.moe_pair_swiglu_grouped(mid, gptrs, up(starts), up(pairs), up_f32(L.w), up(xq), L.hidden, L.ffn,
                              L.n_used, len(ids), L.grb, q, ACT_SILU)
    bound = pair_bound(L, xq, ACT_SILU) + 4e-7 * np.abs(want_mid) + 1e-30
    err = np.abs(down(mid).astype(np.float64) - want_mid)
    assert (err <= bound).all(), f"grouped pair: max err {err.max():.3e}"
    midq = oracle.quantize_q8_k(want_mid)
    partial = zeros_f32((L.n_tok * L.n_used, L.hidden))
    K.moe_down_grouped(partial, gptrs, up(starts), up(pairs), up(midq), L.ffn, L.hidden, L.n_used, len(ids),
                       L.drb, q)
    out = zeros_f32((L.n_tok, L.hidden))
    K.moe_slot_sum(out, partial, L.hidden, L.n_used, L.n_tok)
    want = oracle.moe_down(hptrs, midq, L.ffn, L.hidden, L.n_used, L.n_tok, L.drb, q)
    err = np.abs(down(out).astype(np.float64) - want)
    assert (err <= down_bound(L, midq)).all(), f"grouped down: max err {err.max():.3e}"


@pytest.mark.parametrize("n_used", [1, 8, 9, 16])
def test_slot_sum_batches_exact(dev, n_used):
    """moe_slot_sum loads its slots in batches of 8; the sum stays the
    reference's slot-order float sum from +0 (cu:2791-2806), bit for bit,
    across a batch boundary and a partial last batch."""
    n_tok, out_dim = 3, 1000
    r = np.random.default_rng(n_used)
    p = (r.standard_normal((n_tok, n_used, out_dim)) * 10.0 ** r.integers(-3, 4, (n_tok, n_used, 1))).astype(np.float32)
    want = np.zeros((n_tok, out_dim), np.float32)
    for s in range(n_used):
        want += p[:, s]
    out = zeros_f32((n_tok, out_dim))
    K.moe_slot_sum(out, up_f32(p.reshape(n_tok * n_used, out_dim)), out_dim, n_used, n_tok)
    assert np.array_equal(down(out).view(np.uint32), want.view(np.uint32))
