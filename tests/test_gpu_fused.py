"""The fused decode-layer entry points against the separate ones they
replace: every output (logits, q8_K bytes, routing, pointers, mid, out) must
be bit-identical, since the fused kernels run the same arithmetic in the
same order. The separate entry points are checked against the oracle in
test_gpu_moe.py / test_gpu_q8k_matvec.py."""
import numpy as np
import pytest
import torch

from pulsar_amd import formats as fm
from pulsar_amd import kernels as K
from pulsar_amd.formats import (ACT_SILU, ACT_SWIGLU_OAI, QUANT_IQ2_XXS, QUANT_MXFP4, QUANT_Q2_K, QUANT_Q4_K,
                                QUANT_Q6_K, q8k_blocks)
from tests.gpu_util import down, up_f32, zeros_f32
from tests.test_gpu_moe import Layer

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(77)

CASES = [
    # gq, dq, hidden, ffn, E, k, n_tok, n_shared, mode, act, biases, logit_bias, select_bias
    (QUANT_Q4_K, QUANT_Q6_K, 512, 256, 64, 8, 1, 1, 1, ACT_SILU, False, False, False),
    (QUANT_Q4_K, QUANT_Q6_K, 1024, 256, 256, 8, 2, 1, 1, ACT_SILU, False, False, False),
    (QUANT_MXFP4, QUANT_MXFP4, 576, 320, 8, 4, 3, 0, 1, ACT_SWIGLU_OAI, True, True, False),
    (QUANT_Q2_K, QUANT_IQ2_XXS, 512, 512, 40, 6, 2, 0, 0, ACT_SILU, False, False, True),
    (QUANT_IQ2_XXS, QUANT_Q2_K, 256, 768, 300, 5, 4, 2, 1, ACT_SILU, False, True, True),
    # formats beyond the benchmark configurations (LDS grid tables, float partials)
    (fm.QUANT_Q5_K, fm.QUANT_IQ4_XS, 512, 256, 16, 4, 2, 1, 1, ACT_SILU, False, False, False),
    (fm.QUANT_IQ1_S, fm.QUANT_NVFP4, 512, 512, 12, 3, 3, 0, 0, ACT_SILU, False, True, True),
    (fm.QUANT_Q8_0, fm.QUANT_Q3_K, 768, 256, 10, 2, 2, 0, 1, ACT_SWIGLU_OAI, True, False, False),
    (fm.QUANT_IQ3_S, fm.QUANT_IQ2_S, 256, 512, 8, 4, 1, 1, 1, ACT_SILU, False, False, False),
    # two experts per top-k lane (65..128 experts) and exactly one (64)
    (QUANT_Q4_K, QUANT_Q6_K, 256, 256, 100, 8, 2, 0, 1, ACT_SILU, False, False, True),
    (QUANT_MXFP4, QUANT_MXFP4, 320, 256, 128, 4, 3, 1, 1, ACT_SWIGLU_OAI, True, True, False),
    (QUANT_Q2_K, QUANT_Q2_K, 256, 256, 65, 6, 2, 0, 0, ACT_SILU, False, False, True),
    # the c5 batch-1 shape (MXFP4 rows staged through LDS)
    (QUANT_MXFP4, QUANT_MXFP4, 2880, 2880, 6, 4, 1, 0, 1, ACT_SWIGLU_OAI, True, True, False),
]


def _bank(L: Layer):
    gsz, dsz = L.ffn * L.grb, L.hidden * L.drb
    gb, ub, db = (0 if b is None else b.data_ptr() for b in L.dbias)
    return K.ExpertBank(L.dg.data_ptr(), L.du.data_ptr(), L.dd.data_ptr(), gb or None, ub or None, db or None,
                        gsz, gsz, dsz, L.ffn, L.ffn, L.hidden)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"g{c[0]}d{c[1]}h{c[2]}f{c[3]}E{c[4]}k{c[5]}t{c[6]}m{c[8]}")
def test_fused_layer_matches_separate_calls(dev, case):
    gq, dq, hidden, ffn, E, k, n_tok, n_sh, mode, act, biases, logit_bias, select_bias = case
    L = Layer(gq, dq, hidden=hidden, ffn=ffn, E=E + n_sh, n_used=k, n_tok=n_tok, biases=biases)
    # routed experts 0..E-1; shared experts are the last n_sh of the bank
    shared = [L.dev_entries(E + i) for i in range(n_sh)]
    bank = _bank(L)
    n_slots = k + n_sh
    f32 = dict(dtype=torch.float32, device=dev)
    x = torch.from_numpy(rng.standard_normal((n_tok, hidden)).astype(np.float32)).to(dev)
    if n_tok > 1:
        x[-1] = float("nan") if mode == 1 else x[-1]  # an all-NaN token routes nowhere
    wr = torch.from_numpy((rng.standard_normal((E, hidden)) / np.sqrt(hidden)).astype(np.float32)).to(dev)
    lb = torch.from_numpy((rng.standard_normal(E) * 0.3).astype(np.float32)).to(dev) if logit_bias else None
    sb = torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(dev) if select_bias else None
    nb_in, nb_mid = q8k_blocks(hidden), q8k_blocks(ffn)

    def bufs():
        return dict(logits=torch.zeros((n_tok, E), **f32),
                    xq=torch.zeros(n_tok * nb_in * 292, dtype=torch.uint8, device=dev),
                    sel=torch.zeros((n_tok, k), dtype=torch.int32, device=dev),
                    rw=torch.zeros((n_tok, k), **f32),
                    ptrs=torch.zeros(n_tok * n_slots * 48, dtype=torch.uint8, device=dev),
                    slot_w=torch.zeros((n_tok, n_slots), **f32),
                    mid=torch.zeros((n_tok * n_slots, ffn), **f32),
                    midq=torch.zeros(n_tok * n_slots * nb_mid * 292, dtype=torch.uint8, device=dev),
                    out=torch.zeros((n_tok, hidden), **f32))

    a = bufs()  # separate entry points
    K.matmul_f32(a["logits"], wr, x, hidden, E, n_tok)
    if lb is not None:
        K.add_bias_rows(a["logits"], lb, E, n_tok)
    zero = torch.zeros(E, **f32)
    K.router_select(a["sel"], a["rw"], a["logits"], sb if sb is not None else zero, E, k, 1.25, n_tok, mode, 0)
    K.moe_route_ptrs(a["ptrs"], a["slot_w"], a["sel"], a["rw"], bank, E, shared, n_tok, k)
    K.quantize_q8_k(a["xq"], x, hidden, n_tok)
    K.moe_pair_swiglu(a["mid"], a["ptrs"], a["slot_w"], a["xq"], hidden, ffn, n_slots, n_tok, L.grb, gq, act)
    K.quantize_q8_k(a["midq"], a["mid"], ffn, n_tok * n_slots)
    K.moe_down(a["out"], a["ptrs"], a["midq"], ffn, hidden, n_slots, n_tok, L.drb, dq)
    if biases:
        K.moe_down_bias(a["out"], a["ptrs"], a["slot_w"], hidden, n_slots, n_tok)

    b = bufs()  # fused
    K.router_logits_q8(b["logits"], b["xq"], x, wr, lb, hidden, E, n_tok)
    K.moe_pair_routed(b["mid"], b["ptrs"], b["slot_w"], b["sel"], b["rw"], b["logits"], sb, E, k, 1.25, mode,
                      bank, shared, b["xq"], hidden, ffn, n_tok, L.grb, gq, act)
    K.moe_down_f32(b["out"], b["ptrs"], b["slot_w"], b["mid"], ffn, hidden, n_slots, n_tok, L.drb, dq, biases)
    torch.cuda.synchronize()

    for name in ("logits", "xq", "sel", "rw", "ptrs", "slot_w", "mid", "out"):
        ga, gb = down(a[name]), down(b[name])
        assert np.array_equal(ga.view(np.uint8), gb.view(np.uint8)), name
    assert np.isfinite(down(b["out"])[: n_tok - 1]).all()

    # pair_routed + quantize + down_biased (the MXFP4 decode path)
    c = bufs()
    K.router_logits_q8(c["logits"], c["xq"], x, wr, lb, hidden, E, n_tok)
    K.moe_pair_routed(c["mid"], c["ptrs"], c["slot_w"], c["sel"], c["rw"], c["logits"], sb, E, k, 1.25, mode,
                      bank, shared, c["xq"], hidden, ffn, n_tok, L.grb, gq, act)
    K.quantize_q8_k(c["midq"], c["mid"], ffn, n_tok * n_slots)
    K.moe_down_biased(c["out"], c["ptrs"], c["slot_w"], c["midq"], ffn, hidden, n_slots, n_tok, L.drb, dq)
    torch.cuda.synchronize()
    for name in ("logits", "xq", "sel", "rw", "ptrs", "slot_w", "mid", "midq", "out"):
        ga, gc = down(a[name]), down(c[name])
        assert np.array_equal(ga.view(np.uint8), gc.view(np.uint8)), name


def test_fused_error_contract(dev):
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    bank = K.ExpertBank(buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), None, None, None, 0, 0, 0, 0, 0, 0)
    with pytest.raises(K.KernelError):  # softmax mode 2 (sink slots) is not fused
        K.moe_pair_routed(buf, buf, buf, buf, buf, buf, None, 8, 2, 1.0, 2, bank, None, buf, 256, 256, 1, 144,
                          QUANT_Q4_K, ACT_SILU)
    with pytest.raises(K.KernelError):  # more than 64 slots
        K.moe_pair_routed(buf, buf, buf, buf, buf, buf, None, 128, 65, 1.0, 1, bank, None, buf, 256, 256, 1, 144,
                          QUANT_Q4_K, ACT_SILU)
    with pytest.raises(K.KernelError):  # staged mid rows beyond 64 KiB
        K.moe_down_f32(buf, buf, None, buf, 256 * 60, 256, 4, 1, 210 * 60, QUANT_Q6_K, False)
    with pytest.raises(K.KernelError):  # bias without slot weights
        K.moe_down_f32(buf, buf, None, buf, 256, 256, 4, 1, 210, QUANT_Q6_K, True)
    with pytest.raises(K.KernelError):
        K.router_logits_q8(buf, buf, buf, buf, None, 0, 8, 1)
    with pytest.raises(K.KernelError):
        K.moe_down_biased(buf, buf, None, buf, 256, 256, 2, 1, 210, QUANT_Q6_K)
    torch.cuda.synchronize()


@pytest.mark.parametrize("E,k,n_tok,n_sh,mode,select_bias",
                         [(128, 8, 16, 0, 1, False), (32, 4, 64, 0, 1, True), (256, 8, 3, 1, 1, False),
                          (300, 6, 40, 2, 0, True), (12, 3, 200, 0, 1, False), (64, 6, 33, 1, 0, True),
                          (20, 5, 70, 0, 1, False)])
def test_route_group_matches_separate_calls(dev, E, k, n_tok, n_sh, mode, select_bias):
    """router_select + moe_route_ptrs + moe_group_csr against the fused
    launch: every output bit-identical (ties, an all-NaN token, shared
    slots, a selection bias). The expert counts give lane groups of 4, 8,
    16, 32 and 64 lanes per token."""
    hidden = ffn = 256
    L = Layer(QUANT_Q4_K, QUANT_Q4_K, hidden=hidden, ffn=ffn, E=E + n_sh, n_used=k, n_tok=1)
    bank = _bank(L)
    shared = [L.dev_entries(E + i) for i in range(n_sh)]
    n_slots = k + n_sh
    f32 = dict(dtype=torch.float32, device=dev)
    lg = rng.standard_normal((n_tok, E)).astype(np.float32)
    lg[0, 1] = lg[0, 2]  # a tie: the lower index wins
    if n_tok > 2:
        lg[2] = np.nan  # routes nowhere (mode 1) / NaN scores (mode 0)
    logits = torch.from_numpy(lg).to(dev)
    sb = torch.from_numpy((rng.standard_normal(E) * 0.1).astype(np.float32)).to(dev) if select_bias else None
    max_groups = min(E + n_sh, n_tok * n_slots)

    def bufs():
        return dict(sel=torch.zeros((n_tok, k), dtype=torch.int32, device=dev), rw=torch.zeros((n_tok, k), **f32),
                    ptrs=torch.zeros(n_tok * n_slots * 48, dtype=torch.uint8, device=dev),
                    slot_w=torch.zeros((n_tok, n_slots), **f32),
                    gptrs=torch.zeros(max_groups * 48, dtype=torch.uint8, device=dev),
                    starts=torch.zeros(max_groups + 1, dtype=torch.int32, device=dev),
                    pairs=torch.zeros(n_tok * n_slots, dtype=torch.int32, device=dev))

    a = bufs()
    zero = torch.zeros(E, **f32)
    K.router_select(a["sel"], a["rw"], logits, sb if sb is not None else zero, E, k, 1.25, n_tok, mode, 0)
    K.moe_route_ptrs(a["ptrs"], a["slot_w"], a["sel"], a["rw"], bank, E, shared, n_tok, k)
    K.moe_group_csr(a["gptrs"], a["starts"], a["pairs"], a["ptrs"], n_tok, n_slots, max_groups)
    b = bufs()
    K.moe_route_group(b["sel"], b["rw"], b["ptrs"], b["slot_w"], b["gptrs"], b["starts"], b["pairs"], logits, sb,
                      E, k, 1.25, mode, bank, shared, n_tok, max_groups)
    torch.cuda.synchronize()
    for name in a:
        ga, gb = down(a[name]), down(b[name])
        assert np.array_equal(ga.view(np.uint8), gb.view(np.uint8)), name


def test_slot_sum_bias_matches_separate_calls(dev):
    L = Layer(QUANT_Q4_K, QUANT_Q4_K, hidden=512, ffn=256, E=5, n_used=4, n_tok=7, biases=True,
              null_slots=(2, 9))
    hptrs, dptrs = L.ptrs()
    f32 = dict(dtype=torch.float32, device=dev)
    partial = torch.from_numpy(rng.standard_normal((L.n_tok * L.n_used, L.hidden)).astype(np.float32)).to(dev)
    w = up_f32(L.w)
    a = torch.zeros((L.n_tok, L.hidden), **f32)
    K.moe_slot_sum(a, partial, L.hidden, L.n_used, L.n_tok)
    K.moe_down_bias(a, dptrs, w, L.hidden, L.n_used, L.n_tok)
    b = torch.zeros((L.n_tok, L.hidden), **f32)
    K.moe_slot_sum_bias(b, partial, dptrs, w, L.hidden, L.n_used, L.n_tok)
    torch.cuda.synchronize()
    assert np.array_equal(down(a).view(np.uint32), down(b).view(np.uint32))
    with pytest.raises(K.KernelError):
        K.moe_route_group(a, a, a, a, a, a, a, a, None, 8, 17, 1.0, 1, _bank(L), None, 1, 8)  # > 16 slots
