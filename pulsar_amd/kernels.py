"""Host-side mirror of the reference's kernel wrappers (crates/kernels/src/lib.rs).

Each function has the reference wrapper's name and argument order, takes
device buffers (torch CUDA tensors or raw device addresses as ints) and raises
KernelError(op) where the Rust wrapper returns Err(Error(op)) (the C entry
point returned 0; crates/kernels/src/lib.rs:212-218). Launches are
asynchronous on the calling thread's per-thread default stream (the
reference's --default-stream=per-thread); call runtime.sync() or
torch.cuda.synchronize() (the reference's kernels::sync) before reading
results on the host.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .formats import EXPERT_PTRS_BYTES


class KernelError(RuntimeError):
    """A kernel entry point returned 0 (crates/kernels/src/lib.rs:8-20)."""

    def __init__(self, op: str):
        super().__init__(f"hip kernel op failed: {op}")
        self.op = op


def _ptr(buf) -> int:
    if buf is None:
        return 0
    if isinstance(buf, int):
        return buf
    if hasattr(buf, "data_ptr"):
        if not buf.is_cuda:
            raise ValueError("device buffer expected (got a host tensor)")
        return buf.data_ptr()
    raise TypeError(f"cannot take a device address of {type(buf)!r}")


def _check(ret: int, op: str) -> None:
    if ret == 0:
        raise KernelError(op)


def quantize_q8_k(out, x, in_dim: int, n_rows: int) -> None:
    _check(_lib.load().pulsar_quantize_q8_K(_ptr(out), _ptr(x), in_dim, n_rows), "quantize_q8_k")


def matmul_kq(out, w, xq, in_dim: int, out_dim: int, n_tok: int, row_bytes: int, quant: int) -> None:
    _check(
        _lib.load().pulsar_matmul_kq(_ptr(out), _ptr(w), _ptr(xq), in_dim, out_dim, n_tok, row_bytes, quant),
        "matmul_kq",
    )


def moe_pair_swiglu(mid, ptrs, weights, x, in_dim: int, mid_dim: int, n_used: int, n_tok: int,
                    row_bytes: int, quant: int, act_op: int) -> None:
    _check(
        _lib.load().pulsar_moe_pair_swiglu(_ptr(mid), _ptr(ptrs), _ptr(weights), _ptr(x), in_dim, mid_dim,
                                           n_used, n_tok, row_bytes, quant, act_op),
        "moe_pair_swiglu",
    )


def moe_down(out, ptrs, mid, mid_dim: int, out_dim: int, n_used: int, n_tok: int, row_bytes: int,
             quant: int) -> None:
    _check(
        _lib.load().pulsar_moe_down(_ptr(out), _ptr(ptrs), _ptr(mid), mid_dim, out_dim, n_used, n_tok,
                                    row_bytes, quant),
        "moe_down",
    )


def moe_pair_swiglu_grouped(mid, gptrs, starts, pairs, weights, xq, in_dim: int, mid_dim: int,
                            n_used: int, n_group: int, row_bytes: int, quant: int, act_op: int) -> None:
    _check(
        _lib.load().pulsar_moe_pair_swiglu_grouped(_ptr(mid), _ptr(gptrs), _ptr(starts), _ptr(pairs),
                                                   _ptr(weights), _ptr(xq), in_dim, mid_dim, n_used,
                                                   n_group, row_bytes, quant, act_op),
        "moe_pair_swiglu_grouped",
    )


def moe_down_grouped(partial, gptrs, starts, pairs, midq, mid_dim: int, out_dim: int, n_used: int,
                     n_group: int, row_bytes: int, quant: int) -> None:
    _check(
        _lib.load().pulsar_moe_down_grouped(_ptr(partial), _ptr(gptrs), _ptr(starts), _ptr(pairs),
                                            _ptr(midq), mid_dim, out_dim, n_used, n_group, row_bytes,
                                            quant),
        "moe_down_grouped",
    )


def moe_slot_sum(out, partial, out_dim: int, n_used: int, n_tok: int) -> None:
    _check(_lib.load().pulsar_moe_slot_sum(_ptr(out), _ptr(partial), out_dim, n_used, n_tok), "moe_slot_sum")


def moe_down_bias(out, ptrs, weights, out_dim: int, n_used: int, n_tok: int) -> None:
    _check(
        _lib.load().pulsar_moe_down_bias(_ptr(out), _ptr(ptrs), _ptr(weights), out_dim, n_used, n_tok),
        "moe_down_bias",
    )


def add_bias_rows(x, bias, dim: int, rows: int) -> None:
    _check(_lib.load().pulsar_add_bias_rows(_ptr(x), _ptr(bias), dim, rows), "add_bias_rows")


def router_select(selected, weights, logits, bias, n_expert: int, k_used: int, weight_scale: float,
                  n_tok: int, mode: int, n_shexp: int) -> None:
    _check(
        _lib.load().pulsar_router_select(_ptr(selected), _ptr(weights), _ptr(logits), _ptr(bias), n_expert,
                                         k_used, weight_scale, n_tok, mode, n_shexp),
        "router_select",
    )


def matmul_f32(out, w, x, in_dim: int, out_dim: int, n_tok: int) -> None:
    _check(_lib.load().pulsar_matmul_f32(_ptr(out), _ptr(w), _ptr(x), in_dim, out_dim, n_tok), "matmul_f32")


class ExpertBank(ctypes.Structure):
    """pulsar_expert_bank (include/pulsar_moe.h): expert e's projection starts
    at base + e * stride bytes, its bias at b_base + e * b_stride floats."""

    _fields_ = [
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
        ("gate_b", ctypes.c_void_p), ("up_b", ctypes.c_void_p), ("down_b", ctypes.c_void_p),
        ("gate_stride", ctypes.c_uint64), ("up_stride", ctypes.c_uint64), ("down_stride", ctypes.c_uint64),
        ("gate_b_stride", ctypes.c_uint64), ("up_b_stride", ctypes.c_uint64), ("down_b_stride", ctypes.c_uint64),
    ]


class _Ptrs6(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("gate", "up", "down", "gate_b", "up_b", "down_b")]


def moe_route_ptrs(ptrs, slot_weights, selected, router_weights, bank: ExpertBank, n_expert: int,
                   shared, n_tok: int, k_used: int) -> None:
    """Device-side pointer build (no reference counterpart entry point; it
    replaces the host build of crates/engine/src/lib.rs:8255-8344).
    `shared` is a list of (gate, up, down[, biases]) address tuples."""
    shared = list(shared or [])
    arr = (_Ptrs6 * max(1, len(shared)))()
    for i, e in enumerate(shared):
        e = tuple(e) + (0,) * (6 - len(e))
        arr[i] = _Ptrs6(*[int(v) or None for v in e])
    _check(
        _lib.load().pulsar_moe_route_ptrs(_ptr(ptrs), _ptr(slot_weights), _ptr(selected), _ptr(router_weights),
                                          ctypes.byref(bank), n_expert, ctypes.cast(arr, ctypes.c_void_p),
                                          len(shared), n_tok, k_used),
        "moe_route_ptrs",
    )


def moe_group_csr(gptrs, starts, pairs, ptrs, n_tok: int, n_used: int, max_groups: int) -> None:
    """Device-side CSR by expert (replaces crates/engine/src/lib.rs:8357-8392)."""
    _check(
        _lib.load().pulsar_moe_group_csr(_ptr(gptrs), _ptr(starts), _ptr(pairs), _ptr(ptrs), n_tok, n_used,
                                         max_groups),
        "moe_group_csr",
    )


def moe_slot_sum_bias(out, partial, ptrs, weights, out_dim: int, n_used: int, n_tok: int) -> None:
    """moe_slot_sum + moe_down_bias in one launch (bit-identical)."""
    _check(_lib.load().pulsar_moe_slot_sum_bias(_ptr(out), _ptr(partial), _ptr(ptrs), _ptr(weights), out_dim,
                                                n_used, n_tok), "moe_slot_sum_bias")


def moe_route_group(selected, weights, ptrs, slot_weights, gptrs, starts, pairs, logits, router_bias,
                    n_expert: int, k_used: int, weight_scale: float, softmax_mode: int, bank: "ExpertBank", shared,
                    n_tok: int, max_groups: int) -> None:
    """router_select (modes 0/1) + moe_route_ptrs + moe_group_csr in one launch."""
    arr, n_shared = _shared_array(shared)
    _check(_lib.load().pulsar_moe_route_group(
        _ptr(selected), _ptr(weights), _ptr(ptrs), _ptr(slot_weights), _ptr(gptrs), _ptr(starts), _ptr(pairs),
        _ptr(logits), _ptr(router_bias), n_expert, k_used, weight_scale, softmax_mode, ctypes.byref(bank),
        ctypes.cast(arr, ctypes.c_void_p), n_shared, n_tok, max_groups), "moe_route_group")


def moe_route(selected, weights, ptrs, slot_weights, active, logits, router_bias, n_expert: int, k_used: int,
              weight_scale: float, softmax_mode: int, bank: "ExpertBank", shared, n_tok: int) -> None:
    """router_select (modes 0/1) + moe_route_ptrs in one launch (equal
    outputs), plus `active` (uint32 [2 + n_expert]): the count of distinct
    selected experts, the count of NULL slots, the expert ids in order of
    first appearance in (token, slot) order."""
    arr, n_shared = _shared_array(shared)
    _check(_lib.load().pulsar_moe_route(
        _ptr(selected), _ptr(weights), _ptr(ptrs), _ptr(slot_weights), _ptr(active), _ptr(logits), _ptr(router_bias),
        n_expert, k_used, weight_scale, softmax_mode, ctypes.byref(bank), ctypes.cast(arr, ctypes.c_void_p),
        n_shared, n_tok), "moe_route")


def moe_pair_swiglu_experts(mid, selected, active, slot_weights, xq, bank: "ExpertBank", n_expert: int, shared,
                            n_tok: int, k_used: int, in_dim: int, mid_dim: int, row_bytes: int, quant: int,
                            act_op: int) -> None:
    """The grouped gate/up stage with one group per selected expert, grouped
    on the device from moe_route's outputs (rows equal
    moe_pair_swiglu_grouped's; unrouted slots get rows of 0)."""
    arr, n_shared = _shared_array(shared)
    _check(_lib.load().pulsar_moe_pair_swiglu_experts(
        _ptr(mid), _ptr(selected), _ptr(active), _ptr(slot_weights), _ptr(xq), ctypes.byref(bank), n_expert,
        ctypes.cast(arr, ctypes.c_void_p), n_shared, n_tok, k_used, in_dim, mid_dim, row_bytes, quant, act_op),
        "moe_pair_swiglu_experts")


def moe_down_experts(partial, selected, active, midq, bank: "ExpertBank", n_expert: int, shared, n_tok: int,
                     k_used: int, mid_dim: int, out_dim: int, row_bytes: int, quant: int) -> None:
    """The grouped down stage with one group per selected expert; writes
    every row of partial (0 for unrouted slots)."""
    arr, n_shared = _shared_array(shared)
    _check(_lib.load().pulsar_moe_down_experts(
        _ptr(partial), _ptr(selected), _ptr(active), _ptr(midq), ctypes.byref(bank), n_expert,
        ctypes.cast(arr, ctypes.c_void_p), n_shared, n_tok, k_used, mid_dim, out_dim, row_bytes, quant),
        "moe_down_experts")


def _shared_array(shared):
    shared = list(shared or [])
    arr = (_Ptrs6 * max(1, len(shared)))()
    for i, e in enumerate(shared):
        e = tuple(e) + (0,) * (6 - len(e))
        arr[i] = _Ptrs6(*[int(v) or None for v in e])
    return arr, len(shared)


# ---- fused decode layer (extensions; each equals the separate calls it replaces)

def router_logits_q8(logits, xq, x, w_r, bias, in_dim: int, n_expert: int, n_tok: int) -> None:
    """matmul_f32 [+ add_bias_rows] + quantize_q8_k(x) in one launch."""
    _check(_lib.load().pulsar_router_logits_q8(_ptr(logits), _ptr(xq), _ptr(x), _ptr(w_r), _ptr(bias), in_dim,
                                               n_expert, n_tok), "router_logits_q8")


def moe_pair_routed(mid, ptrs, slot_weights, selected, weights, logits, router_bias, n_expert: int, k_used: int,
                    weight_scale: float, softmax_mode: int, bank: ExpertBank, shared, xq, in_dim: int,
                    mid_dim: int, n_tok: int, row_bytes: int, quant: int, act_op: int) -> None:
    """router_select (modes 0/1) + moe_route_ptrs + moe_pair_swiglu in one launch."""
    arr, n_shared = _shared_array(shared)
    _check(_lib.load().pulsar_moe_pair_routed(
        _ptr(mid), _ptr(ptrs), _ptr(slot_weights), _ptr(selected), _ptr(weights), _ptr(logits), _ptr(router_bias),
        n_expert, k_used, weight_scale, softmax_mode, ctypes.byref(bank), ctypes.cast(arr, ctypes.c_void_p),
        n_shared, _ptr(xq), in_dim, mid_dim, n_tok, row_bytes, quant, act_op), "moe_pair_routed")


def moe_down_f32(out, ptrs, slot_weights, mid, mid_dim: int, out_dim: int, n_used: int, n_tok: int,
                 row_bytes: int, quant: int, add_bias: bool) -> None:
    """quantize_q8_k(mid) + moe_down [+ moe_down_bias] in one launch."""
    _check(_lib.load().pulsar_moe_down_f32(_ptr(out), _ptr(ptrs), _ptr(slot_weights), _ptr(mid), mid_dim, out_dim,
                                           n_used, n_tok, row_bytes, quant, int(bool(add_bias))), "moe_down_f32")


def moe_down_biased(out, ptrs, weights, midq, mid_dim: int, out_dim: int, n_used: int, n_tok: int, row_bytes: int,
                    quant: int) -> None:
    """moe_down + moe_down_bias in one launch."""
    _check(_lib.load().pulsar_moe_down_biased(_ptr(out), _ptr(ptrs), _ptr(weights), _ptr(midq), mid_dim, out_dim,
                                              n_used, n_tok, row_bytes, quant), "moe_down_biased")


def moe_selftest() -> bool:
    """pulsar_moe_selftest (klib:1563): the MoE path per format against host mirrors."""
    return bool(_lib.load().pulsar_moe_selftest())


def router_selftest() -> bool:
    """pulsar_router_selftest (klib:1559)."""
    return bool(_lib.load().pulsar_router_selftest())


def set_stream(stream) -> None:
    """Routes later launches from this thread to `stream` (a torch Stream or
    a raw hipStream_t int); None (or torch's null stream) restores the
    per-thread default stream."""
    handle = 0 if stream is None else (stream if isinstance(stream, int) else stream.cuda_stream)
    _check(_lib.load().pulsar_set_stream(handle or None), "set_stream")


def bw_read(buf, nbytes: int, sink) -> None:
    _check(_lib.load().pulsar_bw_read(_ptr(buf), nbytes, _ptr(sink)), "bw_read")


EXPERT_PTRS_DTYPE = np.dtype(
    [("gate", "<u8"), ("up", "<u8"), ("down", "<u8"), ("gate_b", "<u8"), ("up_b", "<u8"), ("down_b", "<u8")]
)
assert EXPERT_PTRS_DTYPE.itemsize == EXPERT_PTRS_BYTES


def expert_ptrs(entries) -> np.ndarray:
    """Packs (gate, up, down[, gate_b, up_b, down_b]) address tuples (0 = NULL)
    into the 48-byte pulsar_expert_ptrs layout (crates/kernels/src/lib.rs:21-49)."""
    arr = np.zeros(len(entries), dtype=EXPERT_PTRS_DTYPE)
    for i, e in enumerate(entries):
        e = tuple(e) + (0,) * (6 - len(e))
        arr[i] = tuple(int(v) for v in e)
    return arr
