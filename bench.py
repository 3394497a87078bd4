"""Benchmark of the quantized expert-matvec hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME ...] [--no-cpu]

Prints ONE JSON line. The headline (`value`) is BASELINE config 2's decode
matvec: Q6_K 8192 x 4096 against one q8_K token, as algorithmic HBM GB/s
(weight bytes + activation bytes + output bytes, per launch, / time). Every
other configuration is reported under "results":
  c1  Q4_K 4096x4096 matvec, batch 1
  c2  Q6_K 8192x4096 matvec, batch 1 (headline) and 16-token chunk
  c3  routed-MoE decode layer (Q4_K gate/up, Q6_K down, top-8 of 256 + shared)
  c4  routed-MoE 16-token chunk layer (Q2_K and IQ2_XXS, top-8 of 128, grouped)
  c5  gpt-oss MXFP4 MoE layer (top-4 of 32, biases, swiglu_oai), batch 1 and 64
A "step" is one pass of the path over one batch: one matvec launch (c1, c2)
or one whole layer (c3-c5: router GEMV, top-k, device pointer build, q8_K
quantize, gate/up/combine, mid quantize, down [+ grouping, bias]). Inputs are
resident in HBM before the timed region; weights rotate over >= 2 GB of
distinct copies / layer banks so the 256 MB Infinity Cache cannot serve them,
and each layer step routes a different seeded token batch. Timing: HIP events
on the per-thread default stream (the stream every pulsar_* launch uses) bracketing exactly
K steps after W warm-up steps, with a device synchronize on both sides.

cpu_baseline: the oracle's C restatement of the reference CPU lane
(oracle/pulsar_oracle.c) timed on this host's cores on a bounded sample of the
headline workload; it is a reported baseline, not the target.
"""
from __future__ import annotations

import argparse
import json
import os
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
HEADLINE = "c2_q6k_8192x4096_decode"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", nargs="*", default=None, help="subset of result names")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--pmc-run", action="store_true",
                    help="only the workload of the rocprofv3 --pmc traffic passes (no timing, no JSON)")
    return ap.parse_args()


class Timer:
    """HIP events on the launch stream (the per-thread default stream every
    pulsar_* launch uses) around K steps, two ways: eager launches from
    Python, and one replay of a HIP graph holding the same K steps, captured
    on that stream as the reference's decode graphs are
    (crates/kernels/src/lib.rs:755-811)."""

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
        g.launch()  # warm replay
        rt.sync()
        e0.record()
        g.launch()
        e1.record()
        e1.synchronize()
        graph = e0.elapsed_ms(e1) / steps
        del g
        rt.sync()
        return {"ms": graph, "ms_eager": eager}


def dev_copies(torch, host: np.ndarray, min_total: int, slack: int = 256):
    """Distinct device copies of `host` (+slack bytes each) totalling >= min_total."""
    n = max(1, -(-min_total // host.nbytes))
    base = torch.from_numpy(np.ascontiguousarray(host).view(np.uint8).reshape(-1)).cuda()
    buf = torch.empty((n, host.nbytes + slack), dtype=torch.uint8, device="cuda")
    buf.zero_()
    for i in range(n):
        buf[i, : host.nbytes].copy_(base)
    return buf


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

    tm = ctx["timer"].run(step, steps, warmup)
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
    }
    res["pct_of_peak"] = 100 * res["GBps"] / HBM_PEAK_GBS
    if n_tok > 1:
        res["int_ops"] = 2 * rows * cols * n_tok
        # int8 MFMA roofline: dense 5.0 POP/s on MI355X
        res["TOPS"] = res["int_ops"] / (ms * 1e-3) / 1e12
        res["mfma_frac"] = res["TOPS"] / INT8_PEAK_TOPS
    del copies
    return res


# ------------------------------------------------------------- MoE layers --

class DevLayer:
    """`n_banks` device copies of one layer's weights plus its router."""

    def __init__(self, ctx, spec, n_banks):
        torch, synth = ctx["torch"], ctx["synth"]
        bank = synth.moe_bank(spec, seed=21)
        self.spec, self.host = spec, bank
        E = spec.n_expert
        gsz, dsz = spec.ffn * spec.gate_row_bytes, spec.hidden * spec.down_row_bytes
        self.gsz, self.dsz = gsz, dsz
        self.banks = []
        for _ in range(n_banks):
            g = dev_copies(torch, bank.gate, 0)
            u = dev_copies(torch, bank.up, 0)
            d = dev_copies(torch, bank.down, 0)
            b = {"gate": g, "up": u, "down": d}
            b["router_w"] = torch.from_numpy(bank.router_w).cuda()
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


def bench_moe(ctx, spec, steps, warmup, path: str):
    """One whole layer per step. path: "plain" (reference entry points with
    device routing), "grouped" (router_logits_q8 + moe_route_group + the
    grouped stages + moe_slot_sum[_bias]: six launches), "grouped_split"
    (the same grouped stages behind the reference's separate router, select,
    pointer and CSR entry points: nine or ten), "fused" (router_logits_q8 +
    moe_pair_routed + moe_down_f32: three launches) or "fused_q"
    (router_logits_q8 + moe_pair_routed + quantize_q8_k + moe_down_biased:
    four; for wide mid rows, where every fused-down block re-quantizing the
    token's whole mid costs more than one quantize launch)."""
    torch, K, fm = ctx["torch"], ctx["K"], ctx["fm"]
    s = spec
    bank_bytes = s.n_expert * s.expert_bytes
    n_banks = max(4, -(-ROTATE_BYTES // bank_bytes))
    L = DevLayer(ctx, spec, n_banks)
    descs = [L.bank_desc(K, b) for b in L.banks]
    shared = [[tuple(t.data_ptr() for t in b["sh"])] for b in L.banks] if s.shared else None
    n_x = 16  # distinct seeded token batches, one per step in rotation
    xs = torch.from_numpy(ctx["synth"].activations(n_x * s.n_tok, s.hidden, ctx["synth"].rng_for(31, s.name))).cuda()
    xs = xs.view(n_x, s.n_tok, s.hidden)
    n_slots = s.n_slots
    nb_in, nb_mid = fm.q8k_blocks(s.hidden), fm.q8k_blocks(s.ffn)
    f32 = dict(dtype=torch.float32, device="cuda")
    logits = torch.zeros((s.n_tok, s.n_expert), **f32)
    zero_bias = torch.zeros(s.n_expert, **f32)
    sel_all = torch.zeros((steps + warmup, s.n_tok, s.k_used), dtype=torch.int32, device="cuda")
    rw = torch.zeros((s.n_tok, s.k_used), **f32)
    ptrs = torch.zeros(s.n_tok * n_slots * 48, dtype=torch.uint8, device="cuda")
    slot_w = torch.zeros((s.n_tok, n_slots), **f32)
    xq = torch.zeros(s.n_tok * nb_in * 292, dtype=torch.uint8, device="cuda")
    mid = torch.zeros((s.n_tok * n_slots, s.ffn), **f32)
    midq = torch.zeros(s.n_tok * n_slots * nb_mid * 292, dtype=torch.uint8, device="cuda")
    out = torch.zeros((s.n_tok, s.hidden), **f32)
    max_groups = min(s.n_expert, s.n_tok * n_slots)
    gptrs = torch.zeros(max_groups * 48, dtype=torch.uint8, device="cuda")
    starts = torch.zeros(max_groups + 1, dtype=torch.int32, device="cuda")
    pairs = torch.zeros(s.n_tok * n_slots, dtype=torch.int32, device="cuda")
    partial = torch.zeros((s.n_tok * n_slots, s.hidden), **f32)

    def step(i):
        b = L.banks[i % n_banks]
        x = xs[i % n_x]
        sel = sel_all[i]
        if path in ("fused", "fused_q"):
            K.router_logits_q8(logits, xq, x, b["router_w"], b["router_b"], s.hidden, s.n_expert, s.n_tok)
            K.moe_pair_routed(mid, ptrs, slot_w, sel, rw, logits, None, s.n_expert, s.k_used, 1.0, 1,
                              descs[i % n_banks], shared[i % n_banks] if shared else None, xq, s.hidden, s.ffn,
                              s.n_tok, s.gate_row_bytes, s.gate_quant, s.act_op)
            if path == "fused":
                K.moe_down_f32(out, ptrs, slot_w, mid, s.ffn, s.hidden, n_slots, s.n_tok, s.down_row_bytes,
                               s.down_quant, s.biases)
            else:
                K.quantize_q8_k(midq, mid, s.ffn, s.n_tok * n_slots)
                K.moe_down_biased(out, ptrs, slot_w, midq, s.ffn, s.hidden, n_slots, s.n_tok, s.down_row_bytes,
                                  s.down_quant)
            return
        if path == "grouped":
            K.router_logits_q8(logits, xq, x, b["router_w"], b["router_b"], s.hidden, s.n_expert, s.n_tok)
            K.moe_route_group(sel, rw, ptrs, slot_w, gptrs, starts, pairs, logits, None, s.n_expert, s.k_used, 1.0,
                              1, descs[i % n_banks], shared[i % n_banks] if shared else None, s.n_tok, max_groups)
            K.moe_pair_swiglu_grouped(mid, gptrs, starts, pairs, slot_w, xq, s.hidden, s.ffn, n_slots,
                                      max_groups, s.gate_row_bytes, s.gate_quant, s.act_op)
            K.quantize_q8_k(midq, mid, s.ffn, s.n_tok * n_slots)
            K.moe_down_grouped(partial, gptrs, starts, pairs, midq, s.ffn, s.hidden, n_slots, max_groups,
                               s.down_row_bytes, s.down_quant)
            if s.biases:
                K.moe_slot_sum_bias(out, partial, ptrs, slot_w, s.hidden, n_slots, s.n_tok)
            else:
                K.moe_slot_sum(out, partial, s.hidden, n_slots, s.n_tok)
            return
        K.matmul_f32(logits, b["router_w"], x, s.hidden, s.n_expert, s.n_tok)
        if b["router_b"] is not None:
            K.add_bias_rows(logits, b["router_b"], s.n_expert, s.n_tok)
        K.router_select(sel, rw, logits, zero_bias, s.n_expert, s.k_used, 1.0, s.n_tok, 1, 0)
        K.moe_route_ptrs(ptrs, slot_w, sel, rw, descs[i % n_banks], s.n_expert,
                         shared[i % n_banks] if shared else None, s.n_tok, s.k_used)
        K.quantize_q8_k(xq, x, s.hidden, s.n_tok)
        if path == "grouped_split":
            K.moe_group_csr(gptrs, starts, pairs, ptrs, s.n_tok, n_slots, max_groups)
            K.moe_pair_swiglu_grouped(mid, gptrs, starts, pairs, slot_w, xq, s.hidden, s.ffn, n_slots,
                                      max_groups, s.gate_row_bytes, s.gate_quant, s.act_op)
            K.quantize_q8_k(midq, mid, s.ffn, s.n_tok * n_slots)
            K.moe_down_grouped(partial, gptrs, starts, pairs, midq, s.ffn, s.hidden, n_slots, max_groups,
                               s.down_row_bytes, s.down_quant)
            K.moe_slot_sum(out, partial, s.hidden, n_slots, s.n_tok)
        else:
            K.moe_pair_swiglu(mid, ptrs, slot_w, xq, s.hidden, s.ffn, n_slots, s.n_tok, s.gate_row_bytes,
                              s.gate_quant, s.act_op)
            K.quantize_q8_k(midq, mid, s.ffn, s.n_tok * n_slots)
            K.moe_down(out, ptrs, midq, s.ffn, s.hidden, n_slots, s.n_tok, s.down_row_bytes, s.down_quant)
        if s.biases:
            K.moe_down_bias(out, ptrs, slot_w, s.hidden, n_slots, s.n_tok)

    tm = ctx["timer"].run(step, steps, warmup)
    ms = tm["ms"]
    sel_h = sel_all[warmup:].cpu().numpy()
    distinct = np.array([len(np.unique(sel_h[i])) for i in range(steps)]) + (1 if s.shared else 0)
    bias_bytes = 4 * (2 * s.ffn + s.hidden) if s.biases else 0
    act_bytes = s.n_tok * s.hidden * 4 * 2 + s.n_tok * nb_in * 292
    router_bytes = s.n_expert * s.hidden * 4 + (s.n_expert * 4 if s.biases else 0)
    alg = float(np.mean(distinct)) * (s.expert_bytes + bias_bytes) + router_bytes + act_bytes
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
    }
    res["pct_of_peak"] = 100 * res["GBps"] / HBM_PEAK_GBS
    del L
    torch.cuda.empty_cache()
    return res


def stream_peak(ctx) -> float:
    torch, K = ctx["torch"], ctx["K"]
    nbytes = 4 << 30
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    sink = torch.zeros(4, dtype=torch.float32, device="cuda")
    ms = ctx["timer"].run(lambda i: K.bw_read(buf, nbytes, sink), 10, 3)["ms"]
    del buf
    return nbytes / (ms * 1e-3) / 1e9


# ------------------------------------------------------------ CPU baseline --

def cpu_baseline(seconds: float) -> dict:
    """The oracle's threaded lane restatement on the headline workload
    (Q6_K 8192 x 4096 decode), rotating over >= 1 GB of host copies so the
    working set exceeds the last-level cache. Q6_K is not a lane format in
    the reference (crates/engine/src/lib.rs:2103-2114): this is a
    restatement of lane semantics."""
    import oracle
    from pulsar_amd import synth
    from pulsar_amd.formats import QUANT_Q6_K, row_bytes

    rows, cols = 8192, 4096
    w = synth.quant_matrix(QUANT_Q6_K, rows, cols, synth.rng_for(11, HEADLINE))
    n_copies = max(1, -(-1_000_000_000 // w.nbytes))
    copies = [w.copy() for _ in range(n_copies)]
    x = synth.activations(1, cols, synth.rng_for(12, HEADLINE))
    xq = oracle.quantize_q8_k(x)
    out = np.zeros((1, rows), np.float32)
    # this process's CPU share (16 threads on the GPU boxes, whatever nproc says)
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = max(1, min(16, avail))
    lane_threads = max(1, threads // 2 - 2)  # the lane's default pool, (logical / 2) - 2 (elib:1896)
    rb = row_bytes(QUANT_Q6_K, cols)
    alg = w.nbytes + xq.nbytes + out.nbytes

    def timed(nt, budget):
        oracle.matmul_kq_mt(copies[0], xq, cols, rows, 1, rb, QUANT_Q6_K, nt, out)  # warm the pool
        t0 = time.perf_counter()
        n = 0
        while time.perf_counter() - t0 < budget:
            oracle.matmul_kq_mt(copies[n % n_copies], xq, cols, rows, 1, rb, QUANT_Q6_K, nt, out)
            n += 1
        return n, time.perf_counter() - t0

    n, dt = timed(threads, seconds * 0.6)
    n_l, dt_l = timed(lane_threads, seconds * 0.4)
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next(l.split(":", 1)[1].strip() for l in f if l.startswith("model name"))
    except (OSError, StopIteration):
        pass
    return {
        "value": alg * n / dt / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n} passes of the Q6_K 8192x4096 decode matvec in {dt:.1f} s, {threads} threads, "
                  f"{n_copies} rotating host copies ({n_copies * w.nbytes / 1e9:.1f} GB)",
        "us_per_pass": dt / n * 1e6,
        "lane_default": {"threads": lane_threads, "value": alg * n_l / dt_l / 1e9, "unit": "GB/s",
                         "us_per_pass": dt_l / n_l * 1e6},
        "cpu_model": model,
        "logical_cpus_visible": os.cpu_count(),
    }


def pmc_run(ctx):
    """Workload of the `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE`
    passes: 20 eager launches each of the c2 decode matvec and the c2
    16-token MFMA matvec over rotating weight copies, then five copies of a
    256 MiB device buffer (reads 256 MiB, writes 256 MiB: the calibration of
    both counters)."""
    torch, K, synth, fm = ctx["torch"], ctx["K"], ctx["synth"], ctx["fm"]
    q, rows, cols = fm.QUANT_Q6_K, 8192, 4096
    w = synth.quant_matrix(q, rows, cols, synth.rng_for(11, "pmc"))
    copies = dev_copies(torch, w, 1_000_000_000)
    rb = fm.row_bytes(q, cols)
    for n_tok in (1, 16):
        x = torch.from_numpy(synth.activations(n_tok, cols, synth.rng_for(12, "pmc"))).cuda()
        xq = torch.zeros(n_tok * fm.q8k_blocks(cols) * 292, dtype=torch.uint8, device="cuda")
        K.quantize_q8_k(xq, x, cols, n_tok)
        out = torch.zeros((n_tok, rows), dtype=torch.float32, device="cuda")
        for i in range(20):
            K.matmul_kq(out, copies[i % copies.shape[0]], xq, cols, rows, n_tok, rb, q)
        torch.cuda.synchronize()
    del copies
    src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc-run done", flush=True)


def pmc_traffic(name: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    p = ROOT / "profiles" / "pmc_traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get(name)
    except (ValueError, OSError):
        return None


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
        pmc_run(ctx)
        return
    steps, warmup = args.steps, args.warmup
    want = set(args.only) if args.only else None

    def on(name):
        return want is None or name in want

    results = {}
    if on(HEADLINE):
        results[HEADLINE] = bench_matvec(ctx, HEADLINE, fm.QUANT_Q6_K, 8192, 4096, 1, steps, warmup)
    if on("c1_q4k_4096x4096_decode"):
        results["c1_q4k_4096x4096_decode"] = bench_matvec(ctx, "c1", fm.QUANT_Q4_K, 4096, 4096, 1, steps, warmup)
    if on("c2_q6k_8192x4096_chunk16"):
        results["c2_q6k_8192x4096_chunk16"] = bench_matvec(ctx, "c2c", fm.QUANT_Q6_K, 8192, 4096, 16, steps,
                                                           warmup)
    layer_steps = max(20, steps // 2)
    for spec, path in ((synth.C3, "fused"), (synth.C4_Q2K, "grouped"), (synth.C4_IQ2, "grouped"),
                       (synth.C5_B1, "fused_q"), (synth.C5_B64, "grouped")):
        if on(spec.name):
            results[spec.name] = bench_moe(ctx, spec, layer_steps, warmup, path)
        # the same layer through the reference's own (unfused) entry points
        if path.startswith("fused") and on(spec.name + "_unfused"):
            results[spec.name + "_unfused"] = bench_moe(ctx, spec, layer_steps, warmup, "plain")
        if spec is synth.C4_Q2K and on(spec.name + "_split"):
            results[spec.name + "_split"] = bench_moe(ctx, spec, layer_steps, warmup, "grouped_split")
    peak = stream_peak(ctx) if want is None else None

    head = results.get(HEADLINE) or next(iter(results.values()))
    head_name = HEADLINE if HEADLINE in results else next(iter(results))
    cpu = None if args.no_cpu else cpu_baseline(args.cpu_seconds)
    achieved = head.get("GBps")
    line = {
        "metric": METRIC,
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": head.get("us_per_launch", head.get("us_per_layer", 0.0)) / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random blocks of the stated formats; no checkpoints)",
        "config": {
            "workload": "Q6_K matvec 8192x4096, decode batch 1 (BASELINE configs[1]); weights rotate over "
                        f"{head.get('rotation_copies', 0)} HBM copies",
            "rows": 8192, "cols": 4096, "n_tok": 1, "format": "Q6_K", "activation": "q8_K",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": pmc_traffic(head_name),
            "kernel": head.get("kernel"),
            "alg_bytes_per_launch": head.get("alg_bytes"),
            "us_per_launch": round(head.get("us_per_launch", 0.0), 3),
        },
        "cpu_baseline": cpu,
        "stream_read_peak_GBps": None if peak is None else round(peak, 1),
        "results": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                    for k, v in results.items()},
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
