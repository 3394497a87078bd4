"""Benchmark of the quantized expert-matvec hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME ...] [--no-cpu]
                    [--pmc-run WORKLOAD]

Prints ONE JSON line. The headline (`value`) is the largest single-GPU
configuration: a routed-MoE chunk layer of 16 tokens,
hidden 4096, 128 Q2_K experts of FFN 1536, top-8 by a softmax router, run
through the expert-indexed grouped path (router_logits_q8 -> moe_route ->
grouped gate/up -> quantize -> grouped down -> slot sum). `value` is that layer's
algorithmic HBM GB/s: the weight bytes of the distinct experts it touches
(each once), the router weights and the activations in and out, divided by
the layer time. A step is one layer; exactly K steps are timed. `roofline`
is the layer's dominant kernel, the grouped gate/up stage
(moe_grouped_mmq_kq_kernel<0, true, ExpertGroups>), timed on its own with HIP events over
max(K, 100) graph-replayed launches on pre-routed chunks (a replay's host
launch call, 25-75 us before its first kernel starts, spread over 100
launches rather than K). Every other configuration is reported
under "results":
  c1  Q4_K 4096x4096 matvec, batch 1
  c2  Q6_K 8192x4096 matvec, batch 1 and 16-token chunk
  c3  routed-MoE decode layer (Q4_K gate/up, Q6_K down, top-8 of 256 + shared)
  c4  the headline, and the same layer with IQ2_XXS experts
  c5  gpt-oss MXFP4 MoE layer (top-4 of 32, biases, swiglu_oai), batch 1 and 64
Inputs are resident in HBM before the timed region; weights rotate over
distinct device copies / layer banks (>= 2.2 GB) and each timed replay of the
result configurations covers at least 2.2 GB of weights whatever --steps is
(it times max(K, enough steps) and reports the time per step), so the 256 MB
Infinity Cache cannot serve them; each layer step routes a different seeded
token batch. Timing: HIP events on the per-thread default stream (the stream
every pulsar_* launch uses) around the steps, eagerly and as HIP-graph
replays captured on that stream (the reference decodes from CUDA graphs,
crates/kernels/src/lib.rs:755-811); the reported figure is the median of
five timed replays, each of the same K steps between synchronizations,
after the graph has been replayed untimed for 50 ms (the first replays after
a pause run 4-8% slower while the GPU's clocks ramp up).

cpu_baseline: the oracle's C restatement of the reference CPU lane
(oracle/pulsar_oracle.c, AVX2 dots bit-identical to the scalar ones, the
Lane's job split) timed on this host's cores on a bounded sample of the
headline workload; a reported baseline, not the target.

--pmc-run WORKLOAD runs only a workload for the `rocprofv3 --pmc` passes
(no timing, no JSON): ten eager steps of c2_chunk16, c3, c4_q2k, c4_iq2xxs,
c5_b64 or c5_b1, twenty launches of c1 ("all" runs each), then five copies
of a 256 MiB device buffer that calibrate FETCH_SIZE / WRITE_SIZE.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "expert matvec HBM GB/s (% of peak); routed-MoE layer µs/token, 1 GPU"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA, TOP/s
ROTATE_BYTES = 2_200_000_000
STAGE_LAUNCHES = 100  # launches per timed replay in the grouped stage timing
HEADLINE = "c4_moe_chunk16_q2k"
ROOF_KERNEL = "pk::moe_grouped_mmq_kq_kernel<0u, true, pk::ExpertGroups>"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", nargs="*", default=None, help="subset of result names")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--pmc-run", default=None,
                    help="only the workload of the rocprofv3 --pmc passes (no timing, no JSON)")
    return ap.parse_args()


class Timer:
    """HIP events on the launch stream (the per-thread default stream every
    pulsar_* launch uses) around n steps, two ways: eager launches from
    Python, and replays of a HIP graph holding the same n steps, captured
    on that stream as the reference's decode graphs are
    (crates/kernels/src/lib.rs:755-811). The graph figure is the median of
    REPLAYS timed replays, each of exactly n steps between synchronizations
    (one replay of a ~3 ms layer chain moved by up to 5% from run to run),
    after untimed replays of the same graph for WARM_S seconds."""

    REPLAYS = 5
    WARM_S = 0.05

    def __init__(self, torch, K):
        from pulsar_amd import runtime

        self.torch, self.K, self.rt = torch, K, runtime

    def run(self, step, steps: int, warmup: int) -> dict:
        rt = self.rt
        for i in range(warmup):
            step(i)
        rt.sync()
        e0, e1 = rt.Event(), rt.Event()
        e0.record()
        for i in range(steps):
            step(warmup + i)
        e1.record()
        e1.synchronize()
        eager = e0.elapsed_ms(e1) / steps
        g = rt.Graph.capture(lambda: [step(warmup + i) for i in range(steps)])
        # untimed replays for WARM_S of GPU work first: after a pause the
        # first replays run 4-8% slower and level off after ~25 ms (the
        # clocks ramping up), which the timed replays should not carry
        t_warm = time.perf_counter()
        while True:
            g.launch()
            rt.sync()
            if time.perf_counter() - t_warm >= self.WARM_S:
                break
        times = []
        for _ in range(self.REPLAYS):
            e0.record()
            g.launch()
            e1.record()
            e1.synchronize()
            times.append(e0.elapsed_ms(e1) / steps)
        del g
        rt.sync()
        return {"ms": float(np.median(times)), "ms_eager": eager, "ms_replays": [round(t, 6) for t in times]}


def dev_copies(torch, host: np.ndarray, min_total: int, slack: int = 256):
    """Distinct device copies of `host` (+slack bytes each) totalling >= min_total."""
    n = max(1, -(-min_total // host.nbytes))
    base = torch.from_numpy(np.ascontiguousarray(host).view(np.uint8).reshape(-1)).cuda()
    buf = torch.empty((n, host.nbytes + slack), dtype=torch.uint8, device="cuda")
    buf.zero_()
    for i in range(n):
        buf[i, : host.nbytes].copy_(base)
    return buf


def covering_steps(steps: int, bytes_per_step: float) -> int:
    """Steps per timed replay: at least `steps`, and enough that the replay
    reads >= ROTATE_BYTES of distinct weights."""
    return max(steps, int(-(-ROTATE_BYTES // max(1.0, bytes_per_step))))


# ----------------------------------------------------------------- matvec --

def bench_matvec(ctx, name, quant, rows, cols, n_tok, steps, warmup):
    torch, K, synth, fm = ctx["torch"], ctx["K"], ctx["synth"], ctx["fm"]
    w = synth.quant_matrix(quant, rows, cols, synth.rng_for(11, name))
    rb = fm.row_bytes(quant, cols)
    copies = dev_copies(torch, w, ROTATE_BYTES)
    x = synth.activations(n_tok, cols, synth.rng_for(12, name))
    xq = torch.zeros(n_tok * fm.q8k_blocks(cols) * 292, dtype=torch.uint8, device="cuda")
    K.quantize_q8_k(xq, torch.from_numpy(x).cuda(), cols, n_tok)
    out = torch.zeros((n_tok, rows), dtype=torch.float32, device="cuda")
    n = copies.shape[0]
    ptrs = [copies[i].data_ptr() for i in range(n)]

    def step(i):
        K.matmul_kq(out, ptrs[i % n], xq, cols, rows, n_tok, rb, quant)

    launches = max(steps, n)  # every copy once per replay
    tm = ctx["timer"].run(step, launches, warmup)
    ms = tm["ms"]
    alg = w.nbytes + xq.numel() + out.numel() * 4
    res = {
        "kernel": ("pk::mmq_gemm_kernel" if (n_tok >= 5 and quant in (fm.QUANT_Q4_K, fm.QUANT_Q6_K))
                   else "pk::matvec_kernel"),
        "alg_bytes": alg,
        "us_per_launch": ms * 1e3,
        "us_per_launch_eager": tm["ms_eager"] * 1e3,
        "GBps": alg / (ms * 1e-3) / 1e9,
        "rotation_copies": n,
        "launches_per_replay": launches,
        "weight_bytes_per_replay": launches * w.nbytes,
    }
    res["pct_of_peak"] = 100 * res["GBps"] / HBM_PEAK_GBS
    if n_tok > 1:
        res["int_ops"] = 2 * rows * cols * n_tok
        # int8 MFMA roofline: dense 5.0 POP/s on MI355X
        res["TOPS"] = res["int_ops"] / (ms * 1e-3) / 1e12
        res["mfma_frac_time_derived"] = res["TOPS"] / INT8_PEAK_TOPS
    del copies
    return res


# ------------------------------------------------------------- MoE layers --

class DevLayer:
    """`n_banks` device copies of one layer's weights plus its router."""

    def __init__(self, ctx, spec, n_banks):
        torch, synth = ctx["torch"], ctx["synth"]
        bank = synth.moe_bank(spec, seed=21)
        self.spec, self.host = spec, bank
        gsz, dsz = spec.ffn * spec.gate_row_bytes, spec.hidden * spec.down_row_bytes
        self.gsz, self.dsz = gsz, dsz
        self.banks = []
        for _ in range(n_banks):
            b = {"gate": dev_copies(torch, bank.gate, 0), "up": dev_copies(torch, bank.up, 0),
                 "down": dev_copies(torch, bank.down, 0),
                 "router_w": torch.from_numpy(bank.router_w).cuda()}
            for k in ("router_b", "gate_b", "up_b", "down_b"):
                a = getattr(bank, k)
                b[k] = None if a is None else torch.from_numpy(np.ascontiguousarray(a)).cuda()
            if spec.shared:
                b["sh"] = [dev_copies(torch, a, 0) for a in (bank.sh_gate, bank.sh_up, bank.sh_down)]
            self.banks.append(b)

    def bank_desc(self, K, b):
        s = self.spec
        return K.ExpertBank(
            b["gate"].data_ptr(), b["up"].data_ptr(), b["down"].data_ptr(),
            None if b["gate_b"] is None else b["gate_b"].data_ptr(),
            None if b["up_b"] is None else b["up_b"].data_ptr(),
            None if b["down_b"] is None else b["down_b"].data_ptr(),
            self.gsz, self.gsz, self.dsz, s.ffn, s.ffn, s.hidden,
        )


class LayerBufs:
    """Activations and per-step routing buffers of one layer configuration."""

    def __init__(self, ctx, s, n_sel: int, n_x: int):
        torch, fm, synth = ctx["torch"], ctx["fm"], ctx["synth"]
        f32 = dict(dtype=torch.float32, device="cuda")
        u8 = dict(dtype=torch.uint8, device="cuda")
        xs = synth.activations(n_x * s.n_tok, s.hidden, synth.rng_for(31, s.name))
        self.xs = torch.from_numpy(xs).cuda().view(n_x, s.n_tok, s.hidden)
        self.n_x = n_x
        self.n_slots = n_slots = s.n_slots
        self.nb_in, self.nb_mid = fm.q8k_blocks(s.hidden), fm.q8k_blocks(s.ffn)
        self.logits = torch.zeros((s.n_tok, s.n_expert), **f32)
        self.zero_bias = torch.zeros(s.n_expert, **f32)
        self.sel_all = torch.zeros((n_sel, s.n_tok, s.k_used), dtype=torch.int32, device="cuda")
        self.rw = torch.zeros((s.n_tok, s.k_used), **f32)
        self.ptrs = torch.zeros(s.n_tok * n_slots * 48, **u8)
        self.slot_w = torch.zeros((s.n_tok, n_slots), **f32)
        self.xq = torch.zeros(s.n_tok * self.nb_in * 292, **u8)
        self.mid = torch.zeros((s.n_tok * n_slots, s.ffn), **f32)
        self.midq = torch.zeros(s.n_tok * n_slots * self.nb_mid * 292, **u8)
        self.out = torch.zeros((s.n_tok, s.hidden), **f32)
        self.max_groups = min(s.n_expert, s.n_tok * n_slots)
        self.gptrs = torch.zeros(self.max_groups * 48, **u8)
        self.starts = torch.zeros(self.max_groups + 1, dtype=torch.int32, device="cuda")
        self.pairs = torch.zeros(s.n_tok * n_slots, dtype=torch.int32, device="cuda")
        self.partial = torch.zeros((s.n_tok * n_slots, s.hidden), **f32)
        self.active = torch.zeros(2 + s.n_expert, dtype=torch.int32, device="cuda")


def layer_step(ctx, s, L, B, descs, shared, path):
    """One layer per call. path: "plain" (reference entry points with device
    routing), "grouped" (router_logits_q8 + moe_route + the expert-indexed
    grouped stages + moe_slot_sum[_bias]: six launches), "grouped_csr"
    (router_logits_q8 + moe_route_group + the CSR grouped stages, partial
    zeroed by a fill kernel, + moe_slot_sum[_bias]: seven), "grouped_split"
    (the CSR grouped stages behind the reference's separate router, select,
    pointer and CSR entry points: ten or eleven), "fused" (router_logits_q8 +
    moe_pair_routed + moe_down_f32: three launches) or "fused_q"
    (router_logits_q8 + moe_pair_routed + quantize_q8_k + moe_down_biased:
    four; for wide mid rows, where every fused-down block re-quantizing the
    token's whole mid costs more than one quantize launch)."""
    K = ctx["K"]
    n_banks = len(L.banks)
    n_slots = B.n_slots

    def step(i):
        b = L.banks[i % n_banks]
        desc = descs[i % n_banks]
        sh = shared[i % n_banks] if shared else None
        x = B.xs[i % B.n_x]
        sel = B.sel_all[i % B.sel_all.shape[0]]
        if path in ("fused", "fused_q"):
            K.router_logits_q8(B.logits, B.xq, x, b["router_w"], b["router_b"], s.hidden, s.n_expert, s.n_tok)
            K.moe_pair_routed(B.mid, B.ptrs, B.slot_w, sel, B.rw, B.logits, None, s.n_expert, s.k_used, 1.0, 1,
                              desc, sh, B.xq, s.hidden, s.ffn, s.n_tok, s.gate_row_bytes, s.gate_quant, s.act_op)
            if path == "fused":
                K.moe_down_f32(B.out, B.ptrs, B.slot_w, B.mid, s.ffn, s.hidden, n_slots, s.n_tok,
                               s.down_row_bytes, s.down_quant, s.biases)
            else:
                K.quantize_q8_k(B.midq, B.mid, s.ffn, s.n_tok * n_slots)
                K.moe_down_biased(B.out, B.ptrs, B.slot_w, B.midq, s.ffn, s.hidden, n_slots, s.n_tok,
                                  s.down_row_bytes, s.down_quant)
            return
        if path == "grouped":
            K.router_logits_q8(B.logits, B.xq, x, b["router_w"], b["router_b"], s.hidden, s.n_expert, s.n_tok)
            K.moe_route(sel, B.rw, B.ptrs, B.slot_w, B.active, B.logits, None, s.n_expert, s.k_used, 1.0, 1, desc,
                        sh, s.n_tok)
            K.moe_pair_swiglu_experts(B.mid, sel, B.active, B.slot_w, B.xq, desc, s.n_expert, sh, s.n_tok, s.k_used,
                                      s.hidden, s.ffn, s.gate_row_bytes, s.gate_quant, s.act_op)
            K.quantize_q8_k(B.midq, B.mid, s.ffn, s.n_tok * n_slots)
            K.moe_down_experts(B.partial, sel, B.active, B.midq, desc, s.n_expert, sh, s.n_tok, s.k_used, s.ffn,
                               s.hidden, s.down_row_bytes, s.down_quant)
            if s.biases:
                K.moe_slot_sum_bias(B.out, B.partial, B.ptrs, B.slot_w, s.hidden, n_slots, s.n_tok)
            else:
                K.moe_slot_sum(B.out, B.partial, s.hidden, n_slots, s.n_tok)
            return
        if path == "grouped_csr":
            K.router_logits_q8(B.logits, B.xq, x, b["router_w"], b["router_b"], s.hidden, s.n_expert, s.n_tok)
            K.moe_route_group(sel, B.rw, B.ptrs, B.slot_w, B.gptrs, B.starts, B.pairs, B.logits, None, s.n_expert,
                              s.k_used, 1.0, 1, desc, sh, s.n_tok, B.max_groups)
            K.moe_pair_swiglu_grouped(B.mid, B.gptrs, B.starts, B.pairs, B.slot_w, B.xq, s.hidden, s.ffn, n_slots,
                                      B.max_groups, s.gate_row_bytes, s.gate_quant, s.act_op)
            K.quantize_q8_k(B.midq, B.mid, s.ffn, s.n_tok * n_slots)
            B.partial.zero_()  # the CSR stage writes only listed pairs (the reference zeroes, elib:8481-8482)
            K.moe_down_grouped(B.partial, B.gptrs, B.starts, B.pairs, B.midq, s.ffn, s.hidden, n_slots,
                               B.max_groups, s.down_row_bytes, s.down_quant)
            if s.biases:
                K.moe_slot_sum_bias(B.out, B.partial, B.ptrs, B.slot_w, s.hidden, n_slots, s.n_tok)
            else:
                K.moe_slot_sum(B.out, B.partial, s.hidden, n_slots, s.n_tok)
            return
        K.matmul_f32(B.logits, b["router_w"], x, s.hidden, s.n_expert, s.n_tok)
        if b["router_b"] is not None:
            K.add_bias_rows(B.logits, b["router_b"], s.n_expert, s.n_tok)
        K.router_select(sel, B.rw, B.logits, B.zero_bias, s.n_expert, s.k_used, 1.0, s.n_tok, 1, 0)
        K.moe_route_ptrs(B.ptrs, B.slot_w, sel, B.rw, desc, s.n_expert, sh, s.n_tok, s.k_used)
        K.quantize_q8_k(B.xq, x, s.hidden, s.n_tok)
        if path == "grouped_split":
            K.moe_group_csr(B.gptrs, B.starts, B.pairs, B.ptrs, s.n_tok, n_slots, B.max_groups)
            K.moe_pair_swiglu_grouped(B.mid, B.gptrs, B.starts, B.pairs, B.slot_w, B.xq, s.hidden, s.ffn, n_slots,
                                      B.max_groups, s.gate_row_bytes, s.gate_quant, s.act_op)
            K.quantize_q8_k(B.midq, B.mid, s.ffn, s.n_tok * n_slots)
            B.partial.zero_()
            K.moe_down_grouped(B.partial, B.gptrs, B.starts, B.pairs, B.midq, s.ffn, s.hidden, n_slots,
                               B.max_groups, s.down_row_bytes, s.down_quant)
            K.moe_slot_sum(B.out, B.partial, s.hidden, n_slots, s.n_tok)
        else:
            K.moe_pair_swiglu(B.mid, B.ptrs, B.slot_w, B.xq, s.hidden, s.ffn, n_slots, s.n_tok, s.gate_row_bytes,
                              s.gate_quant, s.act_op)
            K.quantize_q8_k(B.midq, B.mid, s.ffn, s.n_tok * n_slots)
            K.moe_down(B.out, B.ptrs, B.midq, s.ffn, s.hidden, n_slots, s.n_tok, s.down_row_bytes, s.down_quant)
        if s.biases:
            K.moe_down_bias(B.out, B.ptrs, B.slot_w, s.hidden, n_slots, s.n_tok)

    return step


def layer_alg_bytes(s, fm, distinct: float) -> float:
    """Algorithmic bytes of one layer: each distinct expert's weights (and
    biases) once, the router weights, x in (f32, then its q8_K), out."""
    nb_in = fm.q8k_blocks(s.hidden)
    bias_bytes = 4 * (2 * s.ffn + s.hidden) if s.biases else 0
    act_bytes = s.n_tok * s.hidden * 4 * 2 + s.n_tok * nb_in * 292
    router_bytes = s.n_expert * s.hidden * 4 + (s.n_expert * 4 if s.biases else 0)
    return distinct * (s.expert_bytes + bias_bytes) + router_bytes + act_bytes


def expected_distinct(s) -> float:
    """E[distinct experts] of a chunk whose tokens each pick k of E uniformly."""
    return s.n_expert * (1 - (1 - s.k_used / s.n_expert) ** s.n_tok) + (1 if s.shared else 0)


def bench_moe(ctx, spec, steps, warmup, path: str, exact_steps: bool = False, stage_timing: bool = False):
    torch, K, fm = ctx["torch"], ctx["K"], ctx["fm"]
    s = spec
    bank_bytes = s.n_expert * s.expert_bytes
    n_banks = max(4, -(-ROTATE_BYTES // bank_bytes))
    L = DevLayer(ctx, spec, n_banks)
    descs = [L.bank_desc(K, b) for b in L.banks]
    shared = [[tuple(t.data_ptr() for t in b["sh"])] for b in L.banks] if s.shared else None
    est = layer_alg_bytes(s, fm, expected_distinct(s))
    n = steps if exact_steps else covering_steps(steps, est)
    B = LayerBufs(ctx, s, n + warmup, n_x=64)
    step = layer_step(ctx, s, L, B, descs, shared, path)
    tm = ctx["timer"].run(step, n, warmup)
    ms = tm["ms"]
    sel_h = B.sel_all[warmup:warmup + n].cpu().numpy()
    distinct = np.array([len(np.unique(sel_h[i])) for i in range(n)]) + (1 if s.shared else 0)
    alg = layer_alg_bytes(s, fm, float(np.mean(distinct)))
    res = {
        "path": path,
        "n_tok": s.n_tok,
        "us_per_layer": ms * 1e3,
        "us_per_token": ms * 1e3 / s.n_tok,
        "us_per_layer_eager": tm["ms_eager"] * 1e3,
        "mean_distinct_experts": float(np.mean(distinct)),
        "alg_bytes": alg,
        "GBps": alg / (ms * 1e-3) / 1e9,
        "layer_banks": n_banks,
        "layers_per_replay": n,
        "us_per_layer_replays": [round(t * 1e3, 3) for t in tm["ms_replays"]],
    }
    res["pct_of_peak"] = 100 * res["GBps"] / HBM_PEAK_GBS
    if stage_timing:
        res["stages"] = grouped_stage_timing(ctx, s, L, descs, shared, steps, warmup)
    del L, B
    torch.cuda.empty_cache()
    return res


def grouped_stage_timing(ctx, s, L, descs, shared, steps, warmup):
    """The grouped gate/up and down stages timed alone: max(`steps`,
    STAGE_LAUNCHES) launches of each per replay over chunks routed beforehand (one routing per bank and token batch,
    so consecutive launches read different experts of different banks), HIP
    events around a graph replay of the launches. Algorithmic bytes per
    launch: the gate and up (down) matrices of every distinct expert of the
    chunk once, each pair's activation row in (q8_K), its output row out."""
    torch, K, fm = ctx["torch"], ctx["K"], ctx["fm"]
    n_banks = len(L.banks)
    n_route = max(2 * n_banks, 8)
    Bs = [LayerBufs(ctx, s, 1, n_x=1) for _ in range(n_route)]
    xs = ctx["synth"].activations(n_route * s.n_tok, s.hidden, ctx["synth"].rng_for(47, s.name))
    xs = torch.from_numpy(xs).cuda().view(n_route, s.n_tok, s.hidden)
    distinct = []
    sh_of = (lambda i: shared[i % n_banks]) if shared else (lambda i: None)
    for i, B in enumerate(Bs):
        b = L.banks[i % n_banks]
        K.router_logits_q8(B.logits, B.xq, xs[i], b["router_w"], b["router_b"], s.hidden, s.n_expert, s.n_tok)
        K.moe_route(B.sel_all[0], B.rw, B.ptrs, B.slot_w, B.active, B.logits, None, s.n_expert, s.k_used, 1.0, 1,
                    descs[i % n_banks], sh_of(i), s.n_tok)
        K.moe_pair_swiglu_experts(B.mid, B.sel_all[0], B.active, B.slot_w, B.xq, descs[i % n_banks], s.n_expert,
                                  sh_of(i), s.n_tok, s.k_used, s.hidden, s.ffn, s.gate_row_bytes, s.gate_quant,
                                  s.act_op)
        K.quantize_q8_k(B.midq, B.mid, s.ffn, s.n_tok * B.n_slots)
        distinct.append(len(np.unique(B.sel_all[0].cpu().numpy())) + (1 if s.shared else 0))
    d = float(np.mean(distinct))
    n_pairs = s.n_tok * s.n_slots
    nb_in, nb_mid = fm.q8k_blocks(s.hidden), fm.q8k_blocks(s.ffn)
    out = {}

    def pair(i):
        B = Bs[i % n_route]
        K.moe_pair_swiglu_experts(B.mid, B.sel_all[0], B.active, B.slot_w, B.xq, descs[i % n_route % n_banks],
                                  s.n_expert, sh_of(i % n_route), s.n_tok, s.k_used, s.hidden, s.ffn,
                                  s.gate_row_bytes, s.gate_quant, s.act_op)

    def down(i):
        B = Bs[i % n_route]
        K.moe_down_experts(B.partial, B.sel_all[0], B.active, B.midq, descs[i % n_route % n_banks], s.n_expert,
                           sh_of(i % n_route), s.n_tok, s.k_used, s.ffn, s.hidden, s.down_row_bytes, s.down_quant)

    q = s.gate_quant
    stages = (("gate_up", pair, f"pk::moe_grouped_mmq_kq_kernel<{q}u, true, pk::ExpertGroups>",
               d * 2 * s.ffn * s.gate_row_bytes + n_pairs * nb_in * 292 + n_pairs * s.ffn * 4),
              ("down", down, f"pk::moe_grouped_mmq_kq_kernel<{s.down_quant}u, false, pk::ExpertGroups>",
               d * s.hidden * s.down_row_bytes + n_pairs * nb_mid * 292 + n_pairs * s.hidden * 4))
    # launches per timed replay: a replay's host launch call (25-75 us before
    # the first kernel can start) is the host's, not the kernel's, so it is
    # spread over STAGE_LAUNCHES launches rather than `steps`
    n_launch = max(steps, n_route, STAGE_LAUNCHES)
    for name, fn, kernel, alg in stages:
        tm = ctx["timer"].run(fn, n_launch, warmup)
        us = tm["ms"] * 1e3
        out[name] = {"kernel": kernel, "alg_bytes_per_launch": alg, "us_per_launch": us,
                     "us_per_launch_eager": tm["ms_eager"] * 1e3, "GBps": alg / (us * 1e-6) / 1e9,
                     "launches_timed": n_launch, "mean_distinct_experts": d}
        out[name]["frac"] = out[name]["GBps"] / HBM_PEAK_GBS
    del Bs
    return out


def stream_chain(ctx, sizes, reps: int = 20) -> dict:
    """The size-matched streaming ceiling of a chain of launches: pulsar_bw_read
    over `sizes` bytes, one launch per size in order (the bytes and launch
    count of a decode configuration's kernels), rotating over >= 2.2 GB of
    regions per size so no launch reads cached data. Returns the chain's
    time and its GB/s."""
    torch, K = ctx["torch"], ctx["K"]
    sizes = [max(256, int(n) // 256 * 256) for n in sizes]
    total = sum(sizes)
    n_reg = max(2, -(-ROTATE_BYTES // total))
    bufs = [torch.ones(n_reg * n // 4, dtype=torch.float32, device="cuda") for n in sizes]
    sink = torch.zeros(4, dtype=torch.float32, device="cuda")

    def step(i):
        for b, n in zip(bufs, sizes):
            K.bw_read(b.data_ptr() + (i % n_reg) * n, n, sink)

    ms = ctx["timer"].run(step, max(reps, n_reg), 3)["ms"]
    del bufs
    return {"bytes": total, "launches": len(sizes), "us": ms * 1e3, "GBps": total / (ms * 1e-3) / 1e9}


def stream_ceiling(ctx, nbytes: int, reps: int = 10) -> float:
    """GB/s of the streaming-read probe (pulsar_bw_read) over `nbytes`
    regions, rotating so consecutive launches read different memory."""
    torch, K = ctx["torch"], ctx["K"]
    nbytes = max(256, nbytes // 256 * 256)  # whole 16-byte loads, regions 256-byte aligned
    n_reg = max(2, -(-ROTATE_BYTES // nbytes)) if nbytes < ROTATE_BYTES else 1
    buf = torch.ones(n_reg * nbytes // 4, dtype=torch.float32, device="cuda")
    sink = torch.zeros(4, dtype=torch.float32, device="cuda")
    base = buf.data_ptr()
    ms = ctx["timer"].run(lambda i: K.bw_read(base + (i % n_reg) * nbytes, nbytes, sink), max(reps, n_reg), 3)["ms"]
    del buf
    return nbytes / (ms * 1e-3) / 1e9


# ------------------------------------------------------------ CPU baseline --

def cpu_info() -> dict:
    info = {"model": "unknown", "physical_cores": None, "logical_cpus": os.cpu_count()}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = {k.strip(): v.strip() for k, v in (ln.split(":", 1) for ln in txt.splitlines() if ":" in ln)}
        info["model"] = kv.get("Model name", info["model"])
        if "Core(s) per socket" in kv and "Socket(s)" in kv:
            info["physical_cores"] = int(kv["Core(s) per socket"]) * int(kv["Socket(s)"])
        # a virtualised host often reports only "AMD EPYC": family / model /
        # stepping name the generation (family 25 = Zen 3 / 4, 26 = Zen 5)
        info["family_model_stepping"] = "/".join(kv.get(k, "?") for k in ("CPU family", "Model", "Stepping"))
        flags = set(kv.get("Flags", "").split())
        info["simd"] = [f for f in ("avx2", "avx512f", "avx512_vnni", "avx512_bf16", "avx_vnni") if f in flags]
        if "L3 cache" in kv:
            info["l3"] = kv["L3 cache"]
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    if info["model"] == "unknown":
        try:
            with open("/proc/cpuinfo") as f:
                info["model"] = next(ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name"))
        except (OSError, StopIteration):
            pass
    return info


def cpu_baseline(seconds: float, ctx) -> dict:
    """The oracle's threaded restatement of the reference CPU lane
    (po_lane_moe: per token q8_K quantize, gate/up/GLU jobs over 256-row
    chunks, mid quantize, down jobs over 512-row chunks, crates/engine/src/
    lib.rs:1994-2100; AVX2 Q2_K dots, cpu_dot.rs:626-671) on the headline
    layer: config 4, 16 tokens routed top-8 of 128 Q2_K experts, each layer a
    different seeded token batch over one 793 MB host bank (a layer touches
    ~510 MB, far beyond the last-level cache). Timed at the lane's default
    pool, (logical / 2) - 2 threads (elib:1896), and at this process's whole
    CPU share. The reference lane takes at most 8 tokens (elib:7900-7908), so
    a 16-token chunk is a restatement of lane semantics."""
    import oracle

    synth, fm = ctx["synth"], ctx["fm"]
    s = synth.C4_Q2K
    bank = synth.moe_bank(s, seed=21)
    n_x = 8
    xs = synth.activations(n_x * s.n_tok, s.hidden, synth.rng_for(31, s.name)).reshape(n_x, s.n_tok, s.hidden)
    routed = []
    for i in range(n_x):
        lg = oracle.matmul_f32(bank.router_w, xs[i], s.hidden, s.n_expert, s.n_tok)
        sel, rw = oracle.router_select(lg, None, s.n_expert, s.k_used, 1.0, s.n_tok, 1, 0)
        ptrs = oracle.host_ptrs([(bank.gate[e], bank.up[e], bank.down[e]) for e in sel.reshape(-1)])
        routed.append((ptrs, rw, np.ascontiguousarray(xs[i]), len(np.unique(sel))))
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = max(1, min(16, avail))  # this process's CPU share (16 on the GPU boxes)
    lane_threads = max(1, threads // 2 - 2)
    prev = oracle.set_simd(True)

    def timed(nt, budget):
        oracle.lane_moe(*routed[0][:3], s.hidden, s.ffn, s.hidden, s.k_used, s.n_tok, s.gate_row_bytes,
                        s.gate_quant, s.down_row_bytes, s.down_quant, s.act_op, nt)  # warm the pool
        t0, n, d = time.perf_counter(), 0, 0
        while time.perf_counter() - t0 < budget or n == 0:
            ptrs, rw, x, nd = routed[n % n_x]
            oracle.lane_moe(ptrs, rw, x, s.hidden, s.ffn, s.hidden, s.k_used, s.n_tok, s.gate_row_bytes,
                            s.gate_quant, s.down_row_bytes, s.down_quant, s.act_op, nt)
            n += 1
            d += nd
        dt = time.perf_counter() - t0
        alg = layer_alg_bytes(s, fm, d / n)
        return {"threads": nt, "layers": n, "seconds": round(dt, 2), "us_per_layer": dt / n * 1e6,
                "value": alg / (dt / n) / 1e9, "unit": "GB/s"}

    try:
        full = timed(threads, seconds * 0.55)
        lane = timed(lane_threads, seconds * 0.45)
    finally:
        oracle.set_simd(prev)
    info = cpu_info()
    return {
        "value": full["value"],
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{full['layers']} config-4 Q2_K layers (16 tokens, top-8 of 128) on the AVX2 lane "
                  f"restatement in {full['seconds']} s with {threads} threads; 793 MB host bank, "
                  f"{n_x} token batches in rotation; expert FFN only (router on the GPU in the reference)",
        "us_per_layer": full["us_per_layer"],
        "avx2": oracle.avx2_supported(),
        "lane_default": lane,
        "cpu_model": info["model"],
        "cpu_family_model_stepping": info.get("family_model_stepping"),
        "cpu_simd": info.get("simd"),
        "cpu_l3": info.get("l3"),
        "physical_cores": info["physical_cores"],
        "logical_cpus_visible": info["logical_cpus"],
        "threads_available": avail,
    }


# --------------------------------------------------------------- PMC runs --

def topk_j(n_expert: int) -> int:
    """Experts per top-k lane of the routed pair kernel (its J template
    argument, as pulsar_moe_pair_routed picks it)."""
    return 1 if n_expert <= 64 else 2 if n_expert <= 128 else 4 if n_expert <= 256 else 8 if n_expert <= 512 else 16


def pmc_run(ctx, which: str):
    """Workloads of the rocprofv3 --pmc passes: ten eager steps of each named
    configuration on rotating weights, then five copies of a 256 MiB device
    buffer (reads 256 MiB, writes 256 MiB: the calibration of FETCH_SIZE and
    WRITE_SIZE). Prints one `pmc-alg {json}` line per configuration with the
    algorithmic bytes per dispatch of its main kernels, the figures the
    counters are compared with."""
    torch, K, synth, fm = ctx["torch"], ctx["K"], ctx["synth"], ctx["fm"]
    names = (["c1", "c2_chunk16", "c3", "c4_q2k", "c4_iq2xxs", "c5_b1", "c5_b64"] if which == "all"
             else which.split(","))
    specs = {"c3": (synth.C3, "fused"), "c4_q2k": (synth.C4_Q2K, "grouped"),
             "c4_iq2xxs": (synth.C4_IQ2, "grouped"), "c5_b1": (synth.C5_B1, "fused_q"),
             "c5_b64": (synth.C5_B64, "grouped")}
    for name in names:
        print(f"pmc-run {name}", flush=True)
        if name in ("c1", "c2_chunk16"):
            q, rows, cols = (fm.QUANT_Q4_K, 4096, 4096) if name == "c1" else (fm.QUANT_Q6_K, 8192, 4096)
            w = synth.quant_matrix(q, rows, cols, synth.rng_for(11, "pmc"))
            copies = dev_copies(torch, w, 1_000_000_000)
            rb = fm.row_bytes(q, cols)
            alg = {}
            runs = (((1, "pk::matvec_kernel<2u, 1u, 1u, 1u, 6u>"),) if name == "c1" else
                    ((1, "pk::matvec_kernel<4u, 1u, 1u, 1u, 6u>"), (16, "pk::mmq_gemm_kernel<4u, 2u, 4u, 1u, 2u>")))
            for n_tok, kern in runs:
                x = torch.from_numpy(synth.activations(n_tok, cols, synth.rng_for(12, "pmc"))).cuda()
                xq = torch.zeros(n_tok * fm.q8k_blocks(cols) * 292, dtype=torch.uint8, device="cuda")
                K.quantize_q8_k(xq, x, cols, n_tok)
                out = torch.zeros((n_tok, rows), dtype=torch.float32, device="cuda")
                for i in range(20):
                    K.matmul_kq(out, copies[i % copies.shape[0]], xq, cols, rows, n_tok, rb, q)
                alg[kern] = w.nbytes + xq.numel() + out.numel() * 4
            torch.cuda.synchronize()
            del copies
            print("pmc-alg " + json.dumps({"workload": name, "alg": alg}), flush=True)
            continue
        s, path = specs[name]
        n_banks = max(4, -(-ROTATE_BYTES // (s.n_expert * s.expert_bytes)))
        L = DevLayer(ctx, s, n_banks)
        descs = [L.bank_desc(K, b) for b in L.banks]
        shared = [[tuple(t.data_ptr() for t in b["sh"])] for b in L.banks] if s.shared else None
        B = LayerBufs(ctx, s, 10, n_x=10)
        step = layer_step(ctx, s, L, B, descs, shared, path)
        for i in range(10):
            step(i)
        torch.cuda.synchronize()
        sel = B.sel_all.cpu().numpy()
        d = float(np.mean([len(np.unique(sel[i])) for i in range(10)])) + (1 if s.shared else 0)
        n_pairs = s.n_tok * s.n_slots
        nb_in, nb_mid = fm.q8k_blocks(s.hidden), fm.q8k_blocks(s.ffn)
        gu = d * 2 * s.ffn * s.gate_row_bytes + (d * 2 * s.ffn * 4 if s.biases else 0)
        dn = d * s.hidden * s.down_row_bytes
        router = s.n_expert * s.hidden * 4 + s.n_tok * s.hidden * 4 + s.n_tok * s.n_expert * 4 + s.n_tok * nb_in * 292
        if path == "grouped":
            alg = {f"pk::router_logits_q8_kernel<2u>": router,
                   f"pk::moe_grouped_mmq_kq_kernel<{s.gate_quant}u, true, pk::ExpertGroups>":
                       gu + n_pairs * nb_in * 292 + n_pairs * s.ffn * 4,
                   f"pk::moe_grouped_mmq_kq_kernel<{s.down_quant}u, false, pk::ExpertGroups>":
                       dn + n_pairs * nb_mid * 292 + n_pairs * s.hidden * 4}
        elif path == "fused_q":
            bias_d = d * s.hidden * 4 if s.biases else 0
            alg = {"pk::router_logits_q8_kernel<1u>": router + (s.n_expert * 4 if s.biases else 0),
                   f"pk::moe_pair_routed_kernel<{s.gate_quant}u, 1u, {topk_j(s.n_expert)}u, 2u, 1u>":
                       gu + s.n_tok * nb_in * 292 + s.n_tok * s.n_expert * 4 + n_pairs * s.ffn * 4,
                   f"pk::moe_down_kernel<{s.down_quant}u, 1u, 2u, true>":
                       dn + bias_d + n_pairs * nb_mid * 292 + s.n_tok * s.hidden * 4}
        else:
            alg = {"pk::router_logits_q8_kernel<1u>": router,
                   f"pk::moe_pair_routed_kernel<{s.gate_quant}u, 1u, {topk_j(s.n_expert)}u, 0u, 1u>":
                       gu + s.n_tok * nb_in * 292 + s.n_tok * s.n_expert * 4 + n_pairs * s.ffn * 4,
                   f"pk::moe_down_f32_kernel<{s.down_quant}u, 1u, 0u>": dn + n_pairs * s.ffn * 4 + s.n_tok * s.hidden * 4}
        print("pmc-alg " + json.dumps({"workload": name, "mean_distinct_experts": d, "alg": alg}), flush=True)
        del L, B
        torch.cuda.empty_cache()
    src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc-run done", flush=True)


def pmc_summary(kernel: str):
    """Per-dispatch counters of `kernel` from the committed rocprofv3 --pmc
    summary (profiles/pmc_counters.json), if any."""
    p = ROOT / "profiles" / "pmc_counters.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(kernel)
    except (ValueError, OSError):
        return None


def rounded(v):
    if isinstance(v, float):
        return round(v, 4)
    if isinstance(v, dict):
        return {k: rounded(x) for k, x in v.items()}
    return v


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every box in this run has one GPU, and the path "
              f"is benchmarked on one GPU's share (got --gpus {args.gpus})", file=sys.stderr)
        sys.exit(2)
    import torch

    from pulsar_amd import _lib, synth
    from pulsar_amd import formats as fm
    from pulsar_amd import kernels as K

    _lib.load()
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    ctx = {"torch": torch, "K": K, "synth": synth, "fm": fm, "timer": Timer(torch, K)}
    if args.pmc_run:
        pmc_run(ctx, args.pmc_run)
        return
    steps, warmup = args.steps, args.warmup
    want = set(args.only) if args.only else None

    def on(name):
        return want is None or name in want

    results = {}
    if on(HEADLINE):
        results[HEADLINE] = bench_moe(ctx, synth.C4_Q2K, steps, warmup, "grouped", exact_steps=True,
                                      stage_timing=True)
    if on("c1_q4k_4096x4096_decode"):
        results["c1_q4k_4096x4096_decode"] = bench_matvec(ctx, "c1", fm.QUANT_Q4_K, 4096, 4096, 1, steps, warmup)
    if on("c2_q6k_8192x4096_decode"):
        results["c2_q6k_8192x4096_decode"] = bench_matvec(ctx, "c2_q6k_8192x4096_decode", fm.QUANT_Q6_K, 8192,
                                                          4096, 1, steps, warmup)
    if on("c2_q6k_8192x4096_chunk16"):
        results["c2_q6k_8192x4096_chunk16"] = bench_matvec(ctx, "c2c", fm.QUANT_Q6_K, 8192, 4096, 16, steps,
                                                           warmup)
    for spec, path in ((synth.C3, "fused"), (synth.C4_IQ2, "grouped"), (synth.C5_B1, "fused_q"),
                       (synth.C5_B64, "grouped")):
        if on(spec.name):
            results[spec.name] = bench_moe(ctx, spec, steps, warmup, path,
                                           stage_timing=spec is synth.C4_IQ2 or spec is synth.C5_B64)
        # the same layer through the reference's own (unfused) entry points
        if path.startswith("fused") and on(spec.name + "_unfused"):
            results[spec.name + "_unfused"] = bench_moe(ctx, spec, steps, warmup, "plain")
    if on(HEADLINE + "_csr"):
        results[HEADLINE + "_csr"] = bench_moe(ctx, synth.C4_Q2K, steps, warmup, "grouped_csr")
    if on(HEADLINE + "_split"):
        results[HEADLINE + "_split"] = bench_moe(ctx, synth.C4_Q2K, steps, warmup, "grouped_split")

    head = results.get(HEADLINE)
    ceilings = None
    if want is None and head:
        roof = head["stages"]["gate_up"]
        ceilings = {"stream_read_4GiB_GBps": stream_ceiling(ctx, 4 << 30),
                    "stream_read_at_roofline_kernel_bytes_GBps": stream_ceiling(ctx, int(roof["alg_bytes_per_launch"])),
                    "roofline_kernel_bytes": int(roof["alg_bytes_per_launch"])}
    if want is None:
        # size-matched ceilings of the decode configurations: the same bytes
        # in the same number of dependent launches, streamed by bw_read
        c3, c5 = synth.C3, synth.C5_B1
        chains = {
            "c1_q4k_4096x4096_decode": [9_458_240],
            "c2_q6k_8192x4096_decode": [27_562_560],
            "c3_moe_decode_q4k_q6k": [c3.n_expert * c3.hidden * 4,
                                      c3.n_slots * 2 * c3.ffn * c3.gate_row_bytes,
                                      c3.n_slots * c3.hidden * c3.down_row_bytes],
            "c5_moe_mxfp4_b1": [c5.n_expert * c5.hidden * 4, c5.n_slots * 2 * c5.ffn * c5.gate_row_bytes,
                                c5.n_slots * c5.ffn * 4, c5.n_slots * c5.hidden * c5.down_row_bytes],
        }
        ceilings = dict(ceilings or {})
        for name, sizes in chains.items():
            ch = stream_chain(ctx, sizes)
            ceilings[name] = ch
            r = results.get(name)
            if r:
                us = r.get("us_per_layer", r.get("us_per_launch"))
                r["ceiling_us"] = ch["us"]
                r["pct_of_ceiling"] = 100 * ch["us"] / us
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds, ctx)
    if head is None:  # a subset run without the headline
        name, head = next(iter(results.items()))
        print(json.dumps({"metric": METRIC, "partial_run": name, "results": rounded(results)}))
        return
    roof = head["stages"]["gate_up"]
    pmc = pmc_summary(ROOF_KERNEL) or {}
    line = {
        "metric": METRIC,
        "value": round(head["GBps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": head["us_per_layer"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random blocks of the stated formats; no checkpoints)",
        "config": {
            "workload": "BASELINE configs[3]: routed-MoE chunk layer, 16 tokens, hidden 4096, 128 Q2_K experts "
                        "of FFN 1536, top-8 softmax router, grouped path (6 launches); "
                        f"{head['layer_banks']} rotating layer banks of 793 MB",
            "us_per_layer": round(head["us_per_layer"], 3),
            "us_per_token": round(head["us_per_token"], 3),
            "mean_distinct_experts": head["mean_distinct_experts"],
            "alg_bytes_per_layer": head["alg_bytes"],
            "format": "Q2_K", "activation": "q8_K", "n_tok": 16,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(roof["GBps"], 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(roof["GBps"] / HBM_PEAK_GBS, 4),
            "traffic": (round(pmc["traffic_over_alg"] * roof["alg_bytes_per_launch"])
                        if pmc.get("traffic_over_alg") else None),
            "kernel": ROOF_KERNEL,
            "alg_bytes_per_launch": round(roof["alg_bytes_per_launch"]),
            "us_per_launch": round(roof["us_per_launch"], 3),
            "traffic_over_alg": pmc.get("traffic_over_alg"),
            "mfma_busy_frac": pmc.get("mfma_busy_frac"),
            "counters_source": ("profiles/pmc_counters.json (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE and SQ counters of "
                                "this kernel under `bench.py --pmc-run c4_q2k`, scaled by a 256 MiB copy's counts); "
                                "traffic = that run's HBM/algorithmic ratio x this run's algorithmic bytes"),
        },
        "cpu_baseline": rounded(cpu),
        "stream_ceilings": rounded(ceilings),
        "results": rounded(results),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
