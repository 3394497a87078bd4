"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker and the timed CPU baseline.
Nothing under pulsar_amd/ imports it.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
Q8K = 292
EXPERT_PTRS_DTYPE = np.dtype(
    [("gate", "<u8"), ("up", "<u8"), ("down", "<u8"), ("gate_b", "<u8"), ("up_b", "<u8"), ("down_b", "<u8")]
)

_lib = None
_vp, _u32, _u64, _f32, _int = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_int


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    sig = {
        "po_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "po_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
        "po_quantize_q8_K": (None, [_vp, _vp, _u32, _u32]),
        "po_row_bytes": (_u64, [_u32, _u32]),
        "po_block_dot": (_f32, [_u32, _vp, _u32, _vp, _u32, _vp, _vp, _vp]),
        "po_vec_dot": (_f32, [_u32, _vp, _vp, _u32, _vp]),
        "po_dequant_row": (None, [_u32, _vp, _u32, _vp]),
        "po_matmul_kq": (_int, [_vp, _vp, _vp, _u32, _u32, _u32, _u64, _u32]),
        "po_glu": (_f32, [_f32, _f32, _u32]),
        "po_moe_pair_swiglu": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u64, _u32, _u32]),
        "po_moe_down": (_int, [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u64, _u32]),
        "po_moe_down_bias": (_int, [_vp, _vp, _vp, _u32, _u32, _u32]),
        "po_matmul_f32": (_int, [_vp, _vp, _vp, _u32, _u32, _u32]),
        "po_add_bias_rows": (_int, [_vp, _vp, _u32, _u32]),
        "po_router_select": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _f32, _u32, _u32, _u32]),
        "po_lcg": (_f32, [ctypes.POINTER(ctypes.c_uint64)]),
        "po_lane_moe": (_int, [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u32, _u64, _u32, _u64, _u32, _u32, _u32]),
        "po_matmul_kq_mt": (_int, [_vp, _vp, _vp, _u32, _u32, _u32, _u64, _u32, _u32, _vp]),
        "po_set_simd": (_int, [_int]),
        "po_rows_dot": (_int, [_vp, _vp, _u64, _u32, _vp, _u32, _u32, _u32, _u32, _vp]),
        "po_avx2_supported": (_int, []),
        "po_avx2_vec_dot": (_f32, [_u32, _vp, _vp, _u32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _p(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data


def f16_to_f32(h: int) -> float:
    return load().po_f16_to_f32(h)


def f32_to_f16(f: float) -> int:
    return load().po_f32_to_f16(f)


def quantize_q8_k(x: np.ndarray) -> np.ndarray:
    """f32 [rows, n] -> uint8 [rows, ceil(n/256) * 292]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None]
    rows, n = x.shape
    nb = -(-n // 256)
    out = np.zeros((rows, nb * Q8K), dtype=np.uint8)
    load().po_quantize_q8_K(_p(out), _p(x), n, rows)
    return out


def q8k_fields(xq: np.ndarray):
    """Splits q8_K bytes [..., nb*292] into (d f32 [..., nb], qs i8 [..., nb, 256], bsums i16 [..., nb, 16])."""
    shp = xq.shape[:-1]
    b = np.ascontiguousarray(xq).reshape(*shp, -1, Q8K)
    d = b[..., 0:4].copy().view(np.float32)[..., 0]
    qs = b[..., 4:260].copy().view(np.int8)
    bs = b[..., 260:292].copy().view(np.int16)
    return d, qs, bs


def block_dot(quant: int, row: np.ndarray, b: int, yblock: np.ndarray, n_valid32: int = 8):
    """(f, i0, i1, sumi[8]) of super-block b of `row` against one q8_K block."""
    i0 = ctypes.c_int32()
    i1 = ctypes.c_int32()
    sumi = np.zeros(8, dtype=np.int32)
    row = np.ascontiguousarray(row, dtype=np.uint8)
    yblock = np.ascontiguousarray(yblock, dtype=np.uint8)
    f = load().po_block_dot(quant, _p(row), b, _p(yblock), n_valid32, ctypes.addressof(i0),
                            ctypes.addressof(i1), _p(sumi))
    return f, i0.value, i1.value, sumi


def vec_dot(quant: int, row: np.ndarray, xq: np.ndarray, n: int, abs_sum: bool = True):
    """(row dot, sum_b |f_b|) of one row against one q8_K row.

    With abs_sum=False no magnitude sum is requested (None is returned for
    it), which lets po_vec_dot take its AVX2 row dots where they exist; with
    a magnitude sum it always walks the scalar per-block dots."""
    row = np.ascontiguousarray(row, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    if not abs_sum:
        return load().po_vec_dot(quant, _p(row), _p(xq), n, None), None
    a = ctypes.c_double()
    f = load().po_vec_dot(quant, _p(row), _p(xq), n, ctypes.addressof(a))
    return f, a.value


def dequant_row(quant: int, row: np.ndarray, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float64)
    load().po_dequant_row(quant, _p(np.ascontiguousarray(row, dtype=np.uint8)), n, _p(out))
    return out


def matmul_kq(w: np.ndarray, xq: np.ndarray, in_dim: int, out_dim: int, n_tok: int, row_bytes: int,
              quant: int) -> np.ndarray | None:
    out = np.zeros((n_tok, out_dim), dtype=np.float32)
    ok = load().po_matmul_kq(_p(out), _p(np.ascontiguousarray(w)), _p(np.ascontiguousarray(xq)), in_dim,
                             out_dim, n_tok, row_bytes, quant)
    return out if ok else None


def matmul_kq_mt(w, xq, in_dim, out_dim, n_tok, row_bytes, quant, threads, out=None, abs_sum=None):
    """The threaded dense matvec (256-row jobs); `abs_sum` (f64 [n_tok,
    out_dim], optional) receives each output's sum_b |f_b|."""
    if out is None:
        out = np.zeros((n_tok, out_dim), dtype=np.float32)
    ok = load().po_matmul_kq_mt(_p(out), _p(w), _p(xq), in_dim, out_dim, n_tok, row_bytes, quant, threads,
                                _p(abs_sum))
    return out if ok else None


def rows_dot(w, row_bytes, rows, xq, n, n_tok, quant, threads):
    """(values f32 [n_tok, rows], sum_b |f_b| f64 [n_tok, rows]) of every row
    of `w` (any format) against n_tok q8_K rows, on `threads` threads."""
    out = np.zeros((n_tok, rows), dtype=np.float32)
    abs_sum = np.zeros((n_tok, rows), dtype=np.float64)
    ok = load().po_rows_dot(_p(out), _p(np.ascontiguousarray(w)), row_bytes, rows, _p(np.ascontiguousarray(xq)),
                            n, n_tok, quant, threads, _p(abs_sum))
    if not ok:
        raise ValueError("po_rows_dot rejected its arguments")
    return out, abs_sum


def set_simd(on: bool) -> bool:
    """AVX2 row dots for Q4_K / Q2_K / IQ2_XXS on (the default where the CPU
    has AVX2) or off; returns the previous setting."""
    return bool(load().po_set_simd(1 if on else 0))


def avx2_supported() -> bool:
    return bool(load().po_avx2_supported())


def avx2_vec_dot(quant: int, row: np.ndarray, xq: np.ndarray, n: int) -> float:
    """The AVX2 row dot itself (oracle/lane_avx2.c), whatever the SIMD
    setting; Q4_K / Q2_K / IQ2_XXS, n a multiple of 256, AVX2 hosts only."""
    row = np.ascontiguousarray(row, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    return load().po_avx2_vec_dot(quant, _p(row), _p(xq), n)


def glu(g: float, u: float, op: int) -> float:
    return load().po_glu(g, u, op)


def host_ptrs(entries) -> np.ndarray:
    """Expert pointer records from (gate, up, down, gate_b, up_b, down_b)
    numpy arrays (None = NULL). The caller keeps the arrays alive."""
    arr = np.zeros(len(entries), dtype=EXPERT_PTRS_DTYPE)
    for i, e in enumerate(entries):
        e = tuple(e) + (None,) * (6 - len(e))
        arr[i] = tuple(0 if a is None else a.ctypes.data for a in e)
    return arr


def moe_pair_swiglu(ptrs, weights, xq, in_dim, mid_dim, n_used, n_tok, row_bytes, quant, act_op):
    mid = np.zeros((n_tok * n_used, mid_dim), dtype=np.float32)
    ok = load().po_moe_pair_swiglu(_p(mid), _p(ptrs), _p(np.ascontiguousarray(weights, dtype=np.float32)),
                                   _p(np.ascontiguousarray(xq)), in_dim, mid_dim, n_used, n_tok, row_bytes,
                                   quant, act_op)
    return mid if ok else None


def moe_down(ptrs, midq, mid_dim, out_dim, n_used, n_tok, row_bytes, quant):
    out = np.zeros((n_tok, out_dim), dtype=np.float32)
    ok = load().po_moe_down(_p(out), _p(ptrs), _p(np.ascontiguousarray(midq)), mid_dim, out_dim, n_used,
                            n_tok, row_bytes, quant)
    return out if ok else None


def moe_down_bias(out, ptrs, weights, out_dim, n_used, n_tok):
    out = np.ascontiguousarray(out, dtype=np.float32).copy()
    ok = load().po_moe_down_bias(_p(out), _p(ptrs), _p(np.ascontiguousarray(weights, dtype=np.float32)),
                                 out_dim, n_used, n_tok)
    return out if ok else None


def matmul_f32(w, x, in_dim, out_dim, n_tok):
    out = np.zeros((n_tok, out_dim), dtype=np.float32)
    ok = load().po_matmul_f32(_p(out), _p(np.ascontiguousarray(w, dtype=np.float32)),
                              _p(np.ascontiguousarray(x, dtype=np.float32)), in_dim, out_dim, n_tok)
    return out if ok else None


def add_bias_rows(x, bias, dim, rows):
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    ok = load().po_add_bias_rows(_p(x), _p(np.ascontiguousarray(bias, dtype=np.float32)), dim, rows)
    return x if ok else None


def router_select(logits, bias, n_expert, k_used, scale, n_tok, mode, n_shexp=0):
    n_slot = k_used + (n_shexp if mode == 2 else 0)
    sel = np.zeros((n_tok, n_slot), dtype=np.int32)
    w = np.zeros((n_tok, n_slot), dtype=np.float32)
    ok = load().po_router_select(_p(sel), _p(w), _p(np.ascontiguousarray(logits, dtype=np.float32)),
                                 _p(None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)),
                                 n_expert, k_used, scale, n_tok, mode, n_shexp)
    return (sel, w) if ok else None


def lcg_stream(seed: int, count: int) -> np.ndarray:
    """`count` draws of the reference test LCG (crates/quant/src/cpu_dot.rs:819-822)."""
    st = ctypes.c_uint64(seed)
    fn = load().po_lcg
    return np.array([fn(ctypes.byref(st)) for _ in range(count)], dtype=np.float32)


def lane_moe(ptrs, weights, x, in_dim, mid_dim, out_dim, n_used, n_tok, grb, gq, drb, dq, act_op, threads):
    out = np.zeros((n_tok, out_dim), dtype=np.float32)
    ok = load().po_lane_moe(_p(out), _p(ptrs), _p(np.ascontiguousarray(weights, dtype=np.float32)),
                            _p(np.ascontiguousarray(x, dtype=np.float32)), in_dim, mid_dim, out_dim, n_used,
                            n_tok, grb, gq, drb, dq, act_op, threads)
    return out if ok else None
