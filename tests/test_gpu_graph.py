"""The launch-stream contract of the reference: every entry point launches on
the calling thread's per-thread default stream (the reference compiles with
--default-stream=per-thread, crates/kernels/build.rs:42-48), so a decode
chain can be recorded by beginning a thread-local capture on that stream
(Graph::capture, crates/kernels/src/lib.rs:755-790) without any call that
names a stream. Each graph is replayed several times, with eager work and
synchronisations in between and its outputs cleared before each replay, and
every replay must equal the eager run bit for bit."""
import numpy as np
import pytest
import torch

from pulsar_amd import kernels as K
from pulsar_amd import runtime
from pulsar_amd.formats import ACT_SILU, QUANT_Q2_K, QUANT_Q4_K, QUANT_Q6_K, q8k_blocks
from tests.gpu_util import down, up_f32
from tests.test_gpu_fused import _bank
from tests.test_gpu_moe import Layer

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(2024)


def _replays_match(graph, outs, want, other_work):
    for rep in range(3):
        for t in outs.values():
            t.zero_()  # a fill kernel on torch's stream, finished before the replay
        torch.cuda.synchronize()
        graph.launch()
        runtime.sync()
        for name, t in outs.items():
            assert np.array_equal(down(t).view(np.uint8), want[name].view(np.uint8)), (rep, name)
        other_work()  # eager launches between replays
        runtime.sync()


def test_reference_chain_captures_on_per_thread_stream(dev):
    """pair -> quantize(mid) -> down, the reference's decode launches
    (crates/engine/src/lib.rs:8472-8498), recorded on the per-thread stream."""
    hidden, ffn, E, n_used, n_tok = 1024, 512, 12, 9, 1
    L = Layer(QUANT_Q4_K, QUANT_Q6_K, hidden=hidden, ffn=ffn, E=E, n_used=n_used, n_tok=n_tok, null_slots=(4,))
    _, dptrs = L.ptrs()
    f32 = dict(dtype=torch.float32, device=dev)
    w = up_f32(L.w)
    x = up_f32(L.x)
    xq = torch.zeros(n_tok * q8k_blocks(hidden) * 292, dtype=torch.uint8, device=dev)
    mid = torch.zeros((n_tok * n_used, ffn), **f32)
    midq = torch.zeros(n_tok * n_used * q8k_blocks(ffn) * 292, dtype=torch.uint8, device=dev)
    out = torch.zeros((n_tok, hidden), **f32)

    def chain():
        K.quantize_q8_k(xq, x, hidden, n_tok)
        K.moe_pair_swiglu(mid, dptrs, w, xq, hidden, ffn, n_used, n_tok, L.grb, QUANT_Q4_K, ACT_SILU)
        K.quantize_q8_k(midq, mid, ffn, n_tok * n_used)
        K.moe_down(out, dptrs, midq, ffn, hidden, n_used, n_tok, L.drb, QUANT_Q6_K)

    chain()
    runtime.sync()
    outs = {"xq": xq, "mid": mid, "midq": midq, "out": out}
    want = {k: down(v).copy() for k, v in outs.items()}
    assert np.abs(want["out"]).max() > 0
    g = runtime.Graph.capture(chain)
    other = torch.zeros_like(out)
    _replays_match(g, outs, want, lambda: K.moe_down(other, dptrs, midq, ffn, hidden, n_used, n_tok, L.drb,
                                                      QUANT_Q6_K))


def test_fused_and_grouped_chains_capture(dev):
    """The fused decode layer (3 launches) and the grouped chunk layer
    (router_logits_q8 -> route_group -> grouped pair -> quantize -> grouped
    down -> slot sum) recorded on the per-thread stream. Every (token, slot)
    of the chunk is routed (finite logits), so the grouped down rewrites the
    whole partial buffer; it is cleared before each replay with the other
    outputs, so a replay that skipped a pair would show."""
    hidden, ffn, E, k = 512, 256, 24, 4
    for n_tok, grouped in ((1, False), (16, True)):
        L = Layer(QUANT_Q2_K, QUANT_Q2_K, hidden=hidden, ffn=ffn, E=E, n_used=k, n_tok=1)
        bank = _bank(L)
        f32 = dict(dtype=torch.float32, device=dev)
        x = up_f32(rng.standard_normal((n_tok, hidden)).astype(np.float32))
        wr = up_f32((rng.standard_normal((E, hidden)) / np.sqrt(hidden)).astype(np.float32))
        nb_in, nb_mid = q8k_blocks(hidden), q8k_blocks(ffn)
        max_groups = min(E, n_tok * k)
        b = dict(logits=torch.zeros((n_tok, E), **f32),
                 xq=torch.zeros(n_tok * nb_in * 292, dtype=torch.uint8, device=dev),
                 sel=torch.zeros((n_tok, k), dtype=torch.int32, device=dev),
                 rw=torch.zeros((n_tok, k), **f32),
                 ptrs=torch.zeros(n_tok * k * 48, dtype=torch.uint8, device=dev),
                 slot_w=torch.zeros((n_tok, k), **f32),
                 mid=torch.zeros((n_tok * k, ffn), **f32),
                 midq=torch.zeros(n_tok * k * nb_mid * 292, dtype=torch.uint8, device=dev),
                 gptrs=torch.zeros(max_groups * 48, dtype=torch.uint8, device=dev),
                 starts=torch.zeros(max_groups + 1, dtype=torch.int32, device=dev),
                 pairs=torch.zeros(n_tok * k, dtype=torch.int32, device=dev),
                 out=torch.zeros((n_tok, hidden), **f32),
                 partial=torch.zeros((n_tok * k, hidden), **f32))
        partial = b["partial"]

        def chain():
            K.router_logits_q8(b["logits"], b["xq"], x, wr, None, hidden, E, n_tok)
            if not grouped:
                K.moe_pair_routed(b["mid"], b["ptrs"], b["slot_w"], b["sel"], b["rw"], b["logits"], None, E, k,
                                  1.0, 1, bank, None, b["xq"], hidden, ffn, n_tok, L.grb, QUANT_Q2_K, ACT_SILU)
                K.moe_down_f32(b["out"], b["ptrs"], b["slot_w"], b["mid"], ffn, hidden, k, n_tok, L.drb,
                               QUANT_Q2_K, False)
                return
            K.moe_route_group(b["sel"], b["rw"], b["ptrs"], b["slot_w"], b["gptrs"], b["starts"], b["pairs"],
                              b["logits"], None, E, k, 1.0, 1, bank, None, n_tok, max_groups)
            K.moe_pair_swiglu_grouped(b["mid"], b["gptrs"], b["starts"], b["pairs"], b["slot_w"], b["xq"],
                                      hidden, ffn, k, max_groups, L.grb, QUANT_Q2_K, ACT_SILU)
            K.quantize_q8_k(b["midq"], b["mid"], ffn, n_tok * k)
            K.moe_down_grouped(partial, b["gptrs"], b["starts"], b["pairs"], b["midq"], ffn, hidden, k,
                               max_groups, L.drb, QUANT_Q2_K)
            K.moe_slot_sum(b["out"], partial, hidden, k, n_tok)

        chain()
        runtime.sync()
        want = {name: down(t).copy() for name, t in b.items()}
        assert np.abs(want["out"]).max() > 0
        g = runtime.Graph.capture(chain)
        other = torch.zeros_like(b["out"])
        _replays_match(g, b, want, lambda: K.router_logits_q8(b["logits"], b["xq"], x, wr, None, hidden, E,
                                                               n_tok) or other.zero_())


def test_expert_chain_replays_follow_new_inputs(dev):
    """The expert-indexed chunk layer (router_logits_q8 -> moe_route ->
    experts gate / up -> quantize -> experts down -> slot sum), captured once
    and replayed on new activations copied into the captured input: the
    routing, the count of touched experts and the groups change from replay
    to replay inside the same graph (its grids are sized for the most
    groups; blocks past the count exit), and each replay must equal an eager
    run of the chain on the same input bit for bit. One input sends every
    token to the same experts (k groups), another spreads them."""
    hidden, ffn, E, k, n_tok = 512, 256, 24, 4, 12
    L = Layer(QUANT_Q2_K, QUANT_Q2_K, hidden=hidden, ffn=ffn, E=E, n_used=k, n_tok=1)
    bank = _bank(L)
    f32 = dict(dtype=torch.float32, device=dev)
    x = torch.zeros((n_tok, hidden), **f32)
    wr = up_f32((rng.standard_normal((E, hidden)) / np.sqrt(hidden)).astype(np.float32))
    nb_in, nb_mid = q8k_blocks(hidden), q8k_blocks(ffn)
    b = dict(logits=torch.zeros((n_tok, E), **f32),
             xq=torch.zeros(n_tok * nb_in * 292, dtype=torch.uint8, device=dev),
             sel=torch.zeros((n_tok, k), dtype=torch.int32, device=dev),
             rw=torch.zeros((n_tok, k), **f32),
             ptrs=torch.zeros(n_tok * k * 48, dtype=torch.uint8, device=dev),
             slot_w=torch.zeros((n_tok, k), **f32),
             active=torch.zeros(2 + E, dtype=torch.int32, device=dev),
             mid=torch.zeros((n_tok * k, ffn), **f32),
             midq=torch.zeros(n_tok * k * nb_mid * 292, dtype=torch.uint8, device=dev),
             partial=torch.zeros((n_tok * k, hidden), **f32),
             out=torch.zeros((n_tok, hidden), **f32))

    def chain():
        K.router_logits_q8(b["logits"], b["xq"], x, wr, None, hidden, E, n_tok)
        K.moe_route(b["sel"], b["rw"], b["ptrs"], b["slot_w"], b["active"], b["logits"], None, E, k, 1.0, 1, bank,
                    None, n_tok)
        K.moe_pair_swiglu_experts(b["mid"], b["sel"], b["active"], b["slot_w"], b["xq"], bank, E, None, n_tok, k,
                                  hidden, ffn, L.grb, QUANT_Q2_K, ACT_SILU)
        K.quantize_q8_k(b["midq"], b["mid"], ffn, n_tok * k)
        K.moe_down_experts(b["partial"], b["sel"], b["active"], b["midq"], bank, E, None, n_tok, k, ffn, hidden,
                           L.drb, QUANT_Q2_K)
        K.moe_slot_sum(b["out"], b["partial"], hidden, k, n_tok)

    x.copy_(up_f32(rng.standard_normal((n_tok, hidden)).astype(np.float32)))
    chain()
    runtime.sync()
    g = runtime.Graph.capture(chain)
    one = rng.standard_normal(hidden).astype(np.float32)
    inputs = [rng.standard_normal((n_tok, hidden)).astype(np.float32),
              np.tile(one, (n_tok, 1)),  # every token on the same k experts
              (rng.standard_normal((n_tok, hidden)) * 3.0).astype(np.float32)]
    counts = []
    for xi in inputs:
        x.copy_(up_f32(xi))
        for t in b.values():
            t.zero_()
        torch.cuda.synchronize()
        g.launch()
        runtime.sync()
        got = {name: down(t).copy() for name, t in b.items()}
        for t in b.values():
            t.zero_()
        torch.cuda.synchronize()
        chain()
        runtime.sync()
        for name, t in b.items():
            assert np.array_equal(got[name].view(np.uint8), down(t).view(np.uint8)), name
        counts.append(int(got["active"][0]))
        assert np.abs(got["out"]).max() > 0
    assert counts[1] == k and counts[0] > k, counts


def test_set_stream_none_restores_per_thread_default(dev):
    """pulsar_set_stream(NULL) routes launches back to the per-thread default
    stream: a capture begun there records them."""
    s = torch.cuda.Stream()
    K.set_stream(s)
    K.set_stream(None)
    n = 512
    x = up_f32(rng.standard_normal((2, n)).astype(np.float32))
    xq = torch.zeros(2 * 2 * 292, dtype=torch.uint8, device=dev)
    g = runtime.Graph.capture(lambda: K.quantize_q8_k(xq, x, n, 2))
    torch.cuda.synchronize()
    g.launch()
    runtime.sync()
    assert down(xq).any()
