"""Helpers shared by the GPU parity tests: device upload/download through
torch (plumbing only; all compute goes through libpulsar_moe.so) and the
fp32 tolerance the parity claims are stated in.

Tolerance (stated once, used by every fp32 comparison of a row dot): the
HIP kernels sum the per-super-block fp32 values in a different order than
the CPU lane, so |gpu - oracle| <= TOL_REL * sum_b |f_b| (+ TOL_ABS), with
sum_b |f_b| the oracle's condition-aware scale and TOL_REL = 1e-5.
"""
import json
import os

import numpy as np
import torch

import oracle

TOL_REL = 1e-5
TOL_ABS = 1e-30


def up(a: np.ndarray, dev="cuda:0") -> torch.Tensor:
    a = np.ascontiguousarray(a)
    t = torch.from_numpy(a.view(np.uint8).reshape(-1).copy())
    return t.to(dev)


def up_f32(a: np.ndarray, dev="cuda:0") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32).copy()).to(dev)


def zeros_f32(shape, dev="cuda:0") -> torch.Tensor:
    return torch.zeros(shape, dtype=torch.float32, device=dev)


def zeros_u8(n, dev="cuda:0") -> torch.Tensor:
    return torch.zeros(int(n), dtype=torch.uint8, device=dev)


def down(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def oracle_rows(quant, mat: np.ndarray, xq_row: np.ndarray, n: int):
    """(values, abs sums) of every row of `mat` against one q8_K row."""
    vals = np.zeros(mat.shape[0], np.float32)
    scale = np.zeros(mat.shape[0], np.float64)
    for r in range(mat.shape[0]):
        vals[r], scale[r] = oracle.vec_dot(quant, mat[r], xq_row, n)
    return vals, scale


def assert_rows_close(got, want, scale, what=""):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bound = TOL_REL * scale + TOL_ABS
    bad = np.argwhere(err > bound)
    assert bad.size == 0, (
        f"{what}: {bad.shape[0]} values outside 1e-5 * sum|f_b|; first {bad[:3].tolist()}, "
        f"max err {err.max():.3e}, max rel {(err / np.maximum(scale, 1e-30)).max():.3e}"
    )
    return float(err.max()), float((err / np.maximum(scale, 1e-30)).max())


def parity_stats(got, want, scale) -> dict:
    """Achieved error of fp32 outputs against the oracle: max |gpu - oracle|,
    max |delta| / sum_b |f_b| (the bound the tests assert) and the
    reference's own |delta| / max(|ref|, 1) (crates/kernels/src/lib.rs:2054)."""
    g = np.asarray(got, np.float64).reshape(-1)
    w = np.asarray(want, np.float64).reshape(-1)
    sc = np.asarray(scale, np.float64).reshape(-1)
    err = np.abs(g - w)
    return {"n": int(err.size), "max_abs": float(err.max()),
            "max_rel_sum_abs": float((err / np.maximum(sc, 1e-30)).max()),
            "max_rel_ref": float((err / np.maximum(np.abs(w), 1.0)).max())}


def record_parity(config: str, stats: dict) -> None:
    """Appends one JSON line {config, stats} to $PULSAR_PARITY_LOG when set
    (the achieved-error table of the parity runs)."""
    path = os.environ.get("PULSAR_PARITY_LOG")
    if path:
        with open(path, "a") as f:
            f.write(json.dumps({"config": config, **stats}) + "\n")
