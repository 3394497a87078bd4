"""Loads libpulsar_moe.so and declares its C ABI (include/pulsar_moe.h).

torch is imported first on purpose: torch ships its own libamdhip64.so.7,
and loading this library afterwards makes the dynamic linker bind it to that
already-loaded runtime (same SONAME), so the process holds one HIP runtime.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

try:  # noqa: SIM105 - import order matters, see the module docstring
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - the library itself does not need torch
    torch = None

LIB_PATH = Path(__file__).resolve().parent / "libpulsar_moe.so"

_u32, _u64, _f32, _vp, _int = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p, ctypes.c_int

# name -> argument types (return type is int: 1 ok, 0 failure)
SIGNATURES = {
    "pulsar_quantize_q8_K": [_vp, _vp, _u32, _u32],
    "pulsar_matmul_kq": [_vp, _vp, _vp, _u32, _u32, _u32, _u64, _u32],
    "pulsar_moe_pair_swiglu": [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u64, _u32, _u32],
    "pulsar_moe_down": [_vp, _vp, _vp, _u32, _u32, _u32, _u32, _u64, _u32],
    "pulsar_moe_pair_swiglu_grouped": [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u64, _u32, _u32],
    "pulsar_moe_down_grouped": [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u64, _u32],
    "pulsar_moe_slot_sum": [_vp, _vp, _u32, _u32, _u32],
    "pulsar_moe_down_bias": [_vp, _vp, _vp, _u32, _u32, _u32],
    "pulsar_router_select": [_vp, _vp, _vp, _vp, _u32, _u32, _f32, _u32, _u32, _u32],
    "pulsar_matmul_f32": [_vp, _vp, _vp, _u32, _u32, _u32],
    "pulsar_add_bias_rows": [_vp, _vp, _u32, _u32],
    "pulsar_bw_read": [_vp, _u64, _vp],
    "pulsar_moe_route_ptrs": [_vp, _vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32],
    "pulsar_moe_group_csr": [_vp, _vp, _vp, _vp, _u32, _u32, _u32],
    "pulsar_moe_route_group": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _f32, _u32, _vp, _vp,
                               _u32, _u32, _u32],
    "pulsar_moe_slot_sum_bias": [_vp, _vp, _vp, _vp, _u32, _u32, _u32],
    "pulsar_moe_route": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _f32, _u32, _vp, _vp, _u32, _u32],
    "pulsar_moe_pair_swiglu_experts": [_vp, _vp, _vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32, _u32, _u32,
                                       _u64, _u32, _u32],
    "pulsar_moe_down_experts": [_vp, _vp, _vp, _vp, _vp, _u32, _vp, _u32, _u32, _u32, _u32, _u32, _u64, _u32],
    "pulsar_set_stream": [_vp],
    "pulsar_router_logits_q8": [_vp, _vp, _vp, _vp, _vp, _u32, _u32, _u32],
    "pulsar_moe_pair_routed": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _u32, _f32, _u32, _vp, _vp, _u32,
                               _vp, _u32, _u32, _u32, _u64, _u32, _u32],
    "pulsar_moe_down_f32": [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u64, _u32, _u32],
    "pulsar_moe_down_biased": [_vp, _vp, _vp, _vp, _u32, _u32, _u32, _u32, _u64, _u32],
    "pulsar_moe_selftest": [],
    "pulsar_router_selftest": [],
}

_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Returns the loaded library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m pulsar_amd.build` "
            "(there is no fallback implementation)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _int
    _lib = lib
    return lib
