"""The expert-indexed grouped path (moe_route -> moe_pair_swiglu_experts ->
quantize -> moe_down_experts) against the CSR path it replaces
(moe_route_group -> moe_pair_swiglu_grouped -> quantize ->
moe_down_grouped, itself checked against the oracle in test_gpu_moe.py and
test_gpu_fullsize.py): routing outputs, every mid row and every partial row
bit-identical, unrouted slots written as 0."""
import numpy as np
import pytest
import torch

from pulsar_amd import formats as fm
from pulsar_amd import kernels as K
from pulsar_amd.formats import (ACT_SILU, ACT_SWIGLU_OAI, QUANT_IQ2_XXS, QUANT_MXFP4, QUANT_Q2_K, QUANT_Q4_K,
                                QUANT_Q6_K, q8k_blocks)
from tests.gpu_util import down
from tests.test_gpu_fused import _bank
from tests.test_gpu_moe import Layer

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(4242)


def _logits(E, n_tok, mode):
    lg = rng.standard_normal((n_tok, E)).astype(np.float32)
    lg[0, 1] = lg[0, 2]  # a tie: the lower index wins
    if n_tok > 2:
        lg[2] = np.nan  # mode 1: routes nowhere (NULL slots); mode 0: NaN scores
    if n_tok > 3:
        lg[3] = -np.inf  # every score -inf: expert 0 in every slot (a repeated expert)
    return lg


@pytest.mark.parametrize("E,k,n_tok,n_sh,mode,select_bias",
                         [(128, 8, 16, 0, 1, False), (32, 4, 64, 0, 1, True), (256, 8, 3, 1, 1, False),
                          (300, 6, 40, 2, 0, True), (12, 3, 200, 0, 1, False), (64, 12, 9, 3, 1, False),
                          (1000, 16, 5, 0, 0, True), (20, 5, 70, 0, 1, False)])
def test_route_matches_separate_calls(dev, E, k, n_tok, n_sh, mode, select_bias):
    """moe_route against router_select + moe_route_ptrs: sel, weights,
    pointers and slot weights bit-identical (ties, an all-NaN token, an
    all--inf token, shared slots, a selection bias)."""
    L = Layer(QUANT_Q4_K, QUANT_Q4_K, hidden=256, ffn=256, E=E + n_sh, n_used=k, n_tok=1)
    bank = _bank(L)
    shared = [L.dev_entries(E + i) for i in range(n_sh)]
    n_slots = k + n_sh
    f32 = dict(dtype=torch.float32, device=dev)
    logits = torch.from_numpy(_logits(E, n_tok, mode)).to(dev)
    sb = torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(dev) if select_bias else None

    def bufs():
        return dict(sel=torch.zeros((n_tok, k), dtype=torch.int32, device=dev), rw=torch.zeros((n_tok, k), **f32),
                    ptrs=torch.zeros(n_tok * n_slots * 48, dtype=torch.uint8, device=dev),
                    slot_w=torch.zeros((n_tok, n_slots), **f32))

    a = bufs()
    K.router_select(a["sel"], a["rw"], logits, sb if sb is not None else torch.zeros(E, **f32), E, k, 1.25, n_tok,
                    mode, 0)
    K.moe_route_ptrs(a["ptrs"], a["slot_w"], a["sel"], a["rw"], bank, E, shared, n_tok, k)
    b = bufs()
    active = torch.full((2 + E,), 0xdead, dtype=torch.int32, device=dev)
    K.moe_route(b["sel"], b["rw"], b["ptrs"], b["slot_w"], active, logits, sb, E, k, 1.25, mode, bank, shared, n_tok)
    torch.cuda.synchronize()
    for name in a:
        assert np.array_equal(down(a[name]).view(np.uint8), down(b[name]).view(np.uint8)), name
    # active: distinct selected experts by first appearance, and the NULL slot count
    sel = down(b["sel"]).reshape(-1)
    ids = []
    for e in sel:
        if 0 <= e < E and e not in ids:
            ids.append(int(e))
    act = down(active)
    assert act[0] == len(ids) and act[1] == int(np.count_nonzero((sel < 0) | (sel >= E)))
    assert list(act[2:2 + len(ids)]) == ids


def _edge_logits(E, seed):
    """Rows that stress a top-k's order and ties: ties across the k-th
    place, fewer non-NaN (or non--inf) scores than slots, +-inf, +-0, an
    all-NaN row, an all--inf row, duplicates of the maximum."""
    r = np.random.default_rng(seed)
    rows = []
    rows.append(np.full(E, 0.5))                                     # all equal
    rows.append(r.integers(0, 3, E) / 2.0)                            # three values: ties straddle place k
    x = np.full(E, np.nan); x[r.choice(E, min(3, E), replace=False)] = r.standard_normal(min(3, E))
    rows.append(x)                                                    # three scores, the rest NaN
    x = np.full(E, np.nan); x[r.choice(E, min(5, E), replace=False)] = [-np.inf, 1.0, -np.inf, 2.0, 0.0][:min(5, E)]
    rows.append(x)                                                    # NaN, -inf and a few scores
    x = np.full(E, -np.inf); x[r.choice(E, min(2, E), replace=False)] = [3.0, -1.0][:min(2, E)]
    rows.append(x)                                                    # two scores above -inf
    x = r.standard_normal(E); x[r.choice(E, min(4, E), replace=False)] = np.inf
    rows.append(x)                                                    # several +inf
    rows.append(r.choice([0.0, -0.0, 1e-30, -1e-30], E))              # signed zeros and tiny values
    rows.append(np.full(E, np.nan))                                   # every score NaN
    rows.append(np.full(E, -np.inf))                                  # every score -inf
    x = r.standard_normal(E); x[r.choice(E, min(6, E), replace=False)] = x.max()
    rows.append(x)                                                    # the maximum six times
    x = np.full(E, np.nan); x[E - 1] = 0.25
    rows.append(x)                                                    # one score, at the last index
    rows.append(r.standard_normal(E))
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("E,k,mode,select_bias",
                         [(32, 4, 1, False), (50, 8, 0, True), (100, 8, 1, False), (128, 16, 0, False),
                          (256, 8, 1, True), (256, 1, 0, False), (500, 12, 1, False), (1000, 16, 1, True),
                          (64, 64, 1, False), (256, 64, 0, True)])
def test_route_topk_edges(dev, E, k, mode, select_bias):
    """The routing of moe_route (a token per wave) and of moe_pair_routed
    (the fused decode pair stage) against router_select's round-by-round
    top-k, bit for bit, on rows built to stress the selection order."""
    L = Layer(QUANT_Q4_K, QUANT_Q4_K, hidden=256, ffn=256, E=E, n_used=k, n_tok=1)
    bank = _bank(L)
    f32 = dict(dtype=torch.float32, device=dev)
    lg_h = _edge_logits(E, E * 131 + k)
    n_tok = lg_h.shape[0]
    logits = torch.from_numpy(lg_h).to(dev)
    sb = torch.from_numpy((np.random.default_rng(E).standard_normal(E) * 0.1).astype(np.float32)).to(dev) \
        if select_bias else None

    def bufs():
        return dict(sel=torch.zeros((n_tok, k), dtype=torch.int32, device=dev), rw=torch.zeros((n_tok, k), **f32),
                    ptrs=torch.zeros(n_tok * k * 48, dtype=torch.uint8, device=dev),
                    slot_w=torch.zeros((n_tok, k), **f32))

    a = bufs()
    K.router_select(a["sel"], a["rw"], logits, sb if sb is not None else torch.zeros(E, **f32), E, k, 1.25, n_tok,
                    mode, 0)
    K.moe_route_ptrs(a["ptrs"], a["slot_w"], a["sel"], a["rw"], bank, E, [], n_tok, k)
    outs = []
    if k <= 16:  # moe_route's slot limit
        b = bufs()
        active = torch.zeros((2 + E,), dtype=torch.int32, device=dev)
        K.moe_route(b["sel"], b["rw"], b["ptrs"], b["slot_w"], active, logits, sb, E, k, 1.25, mode, bank, [],
                    n_tok)
        outs.append(("moe_route", b))
    c = bufs()
    xq = torch.zeros(n_tok * q8k_blocks(256) * 292, dtype=torch.uint8, device=dev)
    K.quantize_q8_k(xq, torch.from_numpy(L.x.repeat(n_tok, 0)).to(dev), 256, n_tok)
    mid = torch.zeros((n_tok * k, 256), **f32)
    K.moe_pair_routed(mid, c["ptrs"], c["slot_w"], c["sel"], c["rw"], logits, sb, E, k, 1.25, mode, bank, [], xq,
                      256, 256, n_tok, L.grb, QUANT_Q4_K, ACT_SILU)
    outs.append(("moe_pair_routed", c))
    torch.cuda.synchronize()
    for who, b in outs:
        for name in a:
            assert np.array_equal(down(a[name]).view(np.uint8), down(b[name]).view(np.uint8)), (who, name)


CASES = [
    # gq, dq, hidden, ffn, E, k, n_tok, n_sh, mode, act, biases
    (QUANT_Q2_K, QUANT_Q2_K, 1024, 512, 64, 8, 16, 0, 1, ACT_SILU, False),
    (QUANT_IQ2_XXS, QUANT_IQ2_XXS, 512, 768, 40, 6, 12, 1, 1, ACT_SILU, False),
    (QUANT_Q4_K, QUANT_Q6_K, 512, 256, 96, 8, 20, 1, 1, ACT_SILU, False),
    (fm.QUANT_Q5_K, fm.QUANT_Q5_K, 512, 512, 16, 4, 9, 0, 0, ACT_SILU, False),
    (QUANT_MXFP4, QUANT_MXFP4, 576, 320, 8, 4, 64, 0, 1, ACT_SWIGLU_OAI, True),
    # lane kernels (formats without a matrix-core grouped kernel)
    (fm.QUANT_Q3_K, fm.QUANT_IQ4_XS, 512, 256, 10, 3, 7, 1, 1, ACT_SILU, True),
    (fm.QUANT_Q8_0, fm.QUANT_IQ2_S, 256, 512, 6, 2, 5, 0, 0, ACT_SWIGLU_OAI, False),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"g{c[0]}d{c[1]}h{c[2]}f{c[3]}E{c[4]}k{c[5]}t{c[6]}s{c[7]}")
def test_expert_grouped_stages_match_csr(dev, case):
    gq, dq, hidden, ffn, E, k, n_tok, n_sh, mode, act, biases = case
    L = Layer(gq, dq, hidden=hidden, ffn=ffn, E=E + n_sh, n_used=k, n_tok=1, biases=biases)
    bank = _bank(L)
    shared = [L.dev_entries(E + i) for i in range(n_sh)]
    n_slots = k + n_sh
    f32 = dict(dtype=torch.float32, device=dev)
    u8 = dict(dtype=torch.uint8, device=dev)
    x = torch.from_numpy(rng.standard_normal((n_tok, hidden)).astype(np.float32)).to(dev)
    xq = torch.zeros(n_tok * q8k_blocks(hidden) * 292, **u8)
    K.quantize_q8_k(xq, x, hidden, n_tok)
    logits = torch.from_numpy(_logits(E, n_tok, mode)).to(dev)
    max_groups = min(E + n_sh, n_tok * n_slots)
    nb_mid = q8k_blocks(ffn)

    def bufs(fill):
        return dict(sel=torch.zeros((n_tok, k), dtype=torch.int32, device=dev), rw=torch.zeros((n_tok, k), **f32),
                    ptrs=torch.zeros(n_tok * n_slots * 48, **u8), slot_w=torch.zeros((n_tok, n_slots), **f32),
                    mid=torch.full((n_tok * n_slots, ffn), fill, **f32),
                    midq=torch.zeros(n_tok * n_slots * nb_mid * 292, **u8),
                    partial=torch.full((n_tok * n_slots, hidden), fill, **f32),
                    out=torch.zeros((n_tok, hidden), **f32))

    a = bufs(0.0)  # the CSR path leaves unlisted rows alone: zeroed beforehand
    gptrs = torch.zeros(max_groups * 48, **u8)
    starts = torch.zeros(max_groups + 1, dtype=torch.int32, device=dev)
    pairs = torch.zeros(n_tok * n_slots, dtype=torch.int32, device=dev)
    K.moe_route_group(a["sel"], a["rw"], a["ptrs"], a["slot_w"], gptrs, starts, pairs, logits, None, E, k, 1.0,
                      mode, bank, shared, n_tok, max_groups)
    K.moe_pair_swiglu_grouped(a["mid"], gptrs, starts, pairs, a["slot_w"], xq, hidden, ffn, n_slots, max_groups,
                              L.grb, gq, act)
    K.quantize_q8_k(a["midq"], a["mid"], ffn, n_tok * n_slots)
    K.moe_down_grouped(a["partial"], gptrs, starts, pairs, a["midq"], ffn, hidden, n_slots, max_groups, L.drb, dq)
    K.moe_slot_sum(a["out"], a["partial"], hidden, n_slots, n_tok)

    b = bufs(float("nan"))  # every row must be written
    active = torch.zeros(2 + E, dtype=torch.int32, device=dev)
    K.moe_route(b["sel"], b["rw"], b["ptrs"], b["slot_w"], active, logits, None, E, k, 1.0, mode, bank, shared,
                n_tok)
    K.moe_pair_swiglu_experts(b["mid"], b["sel"], active, b["slot_w"], xq, bank, E, shared, n_tok, k, hidden, ffn,
                              L.grb, gq, act)
    K.quantize_q8_k(b["midq"], b["mid"], ffn, n_tok * n_slots)
    K.moe_down_experts(b["partial"], b["sel"], active, b["midq"], bank, E, shared, n_tok, k, ffn, hidden, L.drb,
                       dq)
    K.moe_slot_sum(b["out"], b["partial"], hidden, n_slots, n_tok)
    torch.cuda.synchronize()
    sel = down(b["sel"])
    if mode == 1 and n_tok > 2:
        assert (sel[2] == -1).all()  # the all-NaN token: NULL slots, whose rows must be 0
    for name in a:
        ga, gb = down(a[name]), down(b[name])
        assert np.array_equal(ga.view(np.uint8), gb.view(np.uint8)), name


def test_experts_contract(dev):
    L = Layer(QUANT_Q4_K, QUANT_Q6_K, hidden=256, ffn=256, E=4, n_used=2, n_tok=1)
    bank = _bank(L)
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    with pytest.raises(K.KernelError):  # more than 16 slots
        K.moe_pair_swiglu_experts(buf, buf, buf, buf, buf, bank, 4, None, 1, 17, 256, 256, L.grb, QUANT_Q4_K, 0)
    with pytest.raises(K.KernelError):  # in_dim not a multiple of 256
        K.moe_pair_swiglu_experts(buf, buf, buf, buf, buf, bank, 4, None, 1, 2, 200, 256, L.grb, QUANT_Q4_K, 0)
    with pytest.raises(K.KernelError):  # mid_dim not a multiple of 256
        K.moe_down_experts(buf, buf, buf, buf, bank, 4, None, 1, 2, 100, 256, L.drb, QUANT_Q6_K)
    with pytest.raises(K.KernelError):  # no active list
        K.moe_down_experts(buf, buf, None, buf, bank, 4, None, 1, 2, 256, 256, L.drb, QUANT_Q6_K)
    with pytest.raises(K.KernelError):  # softmax mode 2 (sink slots) is not routed here
        K.moe_route(buf, buf, buf, buf, buf, buf, None, 4, 2, 1.0, 2, bank, None, 1)
    with pytest.raises(K.KernelError):  # more than 16 slots
        K.moe_route(buf, buf, buf, buf, buf, buf, None, 40, 17, 1.0, 1, bank, None, 1)
    torch.cuda.synchronize()


@pytest.mark.parametrize("dq,ffn", [(QUANT_Q6_K, 2048), (QUANT_IQ2_XXS, 2048), (QUANT_MXFP4, 2880)],
                         ids=["q6k", "iq2xxs", "mxfp4"])
def test_grouped_fma_epilogue_error_bound(dev, dq, ffn):
    """The grouped stages of the single-product formats fold each super-block
    value into the row sum with one fused multiply-add (one rounding, where
    the CPU lane rounds the product, then the sum); the super-blocks are
    added in the lane's order. So every partial row stays within one f32
    rounding of the running magnitude per super-block step of the lane's
    value: |delta| <= n_steps * 2^-23 * sum_b |f_b|, n_steps the row's
    super-blocks (MXFP4: its 32-value blocks too). Checked on every routed
    pair's down row against the oracle's row dots."""
    import oracle

    hidden, E, k, n_tok = 512, 12, 4, 9
    L = Layer(QUANT_Q4_K, dq, hidden=hidden, ffn=ffn, E=E, n_used=k, n_tok=1)
    bank = _bank(L)
    logits = torch.from_numpy(rng.standard_normal((n_tok, E)).astype(np.float32)).to(dev)
    u8 = dict(dtype=torch.uint8, device=dev)
    sel = torch.zeros((n_tok, k), dtype=torch.int32, device=dev)
    rw = torch.zeros((n_tok, k), dtype=torch.float32, device=dev)
    ptrs = torch.zeros(n_tok * k * 48, **u8)
    slot_w = torch.zeros((n_tok, k), dtype=torch.float32, device=dev)
    active = torch.zeros(2 + E, dtype=torch.int32, device=dev)
    K.moe_route(sel, rw, ptrs, slot_w, active, logits, None, E, k, 1.0, 1, bank, None, n_tok)
    mids = (rng.standard_normal((n_tok * k, ffn)) * 0.05).astype(np.float32)
    midq = oracle.quantize_q8_k(mids)
    partial = torch.full((n_tok * k, hidden), float("nan"), dtype=torch.float32, device=dev)
    K.moe_down_experts(partial, sel, active, torch.from_numpy(midq.reshape(-1)).to(dev), bank, E, None, n_tok, k,
                       ffn, hidden, L.drb, dq)
    torch.cuda.synchronize()
    got = down(partial)
    ids = down(sel).reshape(-1)
    n_steps = -(-ffn // 256) + (ffn // 32 if dq == QUANT_MXFP4 else 0)
    worst = 0.0
    for so, e in enumerate(ids):
        want, scale = oracle.rows_dot(L.d[e], L.drb, hidden, midq[so:so + 1], ffn, 1, dq, 4)
        ratio = np.abs(got[so] - want[0]) / np.maximum(scale[0], 1e-30)
        worst = max(worst, float(ratio.max()))
    assert worst <= n_steps * 2.0 ** -23, (worst, n_steps)
