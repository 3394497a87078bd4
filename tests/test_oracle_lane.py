"""Pins of the oracle's lane pieces that the kernels and the CPU baseline
rest on (CPU only):

- the AVX2 row dots equal the scalar dots bit for bit (the reference asserts
  the same of its AVX2 lane: crates/quant/src/cpu_dot.rs:902, 987, 1076,
  1081-1096);
- the threaded matvec po_matmul_kq_mt (the timed baseline and the checker of
  the full-size GPU tests) equals the serial po_matmul_kq bit for bit, and its
  sum_b |f_b| outputs equal po_vec_dot's;
- router_select mode 2 (sigmoid + bias selection, weights softmax(logsigmoid)
  over the winners' raw logits and the sink logits,
  crates/kernels/cuda/pulsar_kernels.cu:927-936, 1020-1037) against an f64
  numpy closed form written from that description.
"""
import numpy as np
import pytest

import oracle
from pulsar_amd import synth
from pulsar_amd.formats import QUANT_IQ2_XXS, QUANT_Q2_K, QUANT_Q4_K, QUANT_Q6_K, row_bytes

LANE_FORMATS = [QUANT_Q4_K, QUANT_Q2_K, QUANT_IQ2_XXS]
needs_avx2 = pytest.mark.skipif(not oracle.avx2_supported(), reason="host CPU has no AVX2")


@pytest.fixture
def scalar_then_restore():
    prev = oracle.set_simd(False)
    yield
    oracle.set_simd(prev)


def _rows_and_acts(quant, rows, n, seed):
    w = synth.quant_matrix(quant, rows, n, synth.rng_for(seed, "avx2"))
    # activations from the reference test generator (cpu_dot.rs:819-822),
    # scaled, plus one extreme row whose quants reach +-127
    x = oracle.lcg_stream(seed, 3 * n).reshape(3, n) * np.float32(3.0)
    x[2, ::7] = np.float32(1e4) * np.sign(x[2, ::7] + np.float32(1e-9))
    return w, oracle.quantize_q8_k(x)


@needs_avx2
@pytest.mark.parametrize("quant", LANE_FORMATS)
@pytest.mark.parametrize("n,seed", [(256, 42), (2048, 99), (5120, 7331), (4096, 424242)])
def test_avx2_dots_equal_scalar_bits(quant, n, seed):
    """Three routes to each row dot: po_vec_dot with SIMD off (scalar
    per-block dots), po_vec_dot with SIMD on and no magnitude sum requested
    (the dispatch to the AVX2 dots), and the AVX2 dot called directly. All
    three must agree bit for bit, including the activation row whose quants
    reach +-127."""
    w, xq = _rows_and_acts(quant, 24, n, seed)
    assert np.abs(oracle.q8k_fields(xq[2])[1].astype(int)).max() == 127

    def dots(fn):
        return np.array([[fn(w[r], xq[t]) for r in range(w.shape[0])] for t in range(xq.shape[0])], np.float32)

    got = {}
    for simd in (False, True):
        prev = oracle.set_simd(simd)
        try:
            got[simd] = dots(lambda row, x: oracle.vec_dot(quant, row, x, n, abs_sum=False)[0])
        finally:
            oracle.set_simd(prev)
    direct = dots(lambda row, x: oracle.avx2_vec_dot(quant, row, x, n))
    assert np.abs(got[False]).max() > 0
    assert np.array_equal(got[False].view(np.uint32), got[True].view(np.uint32))
    assert np.array_equal(got[False].view(np.uint32), direct.view(np.uint32))


@needs_avx2
@pytest.mark.parametrize("quant", LANE_FORMATS)
def test_avx2_threaded_lane_equals_scalar_lane(quant):
    """The threaded matvec with AVX2 dots equals the serial scalar one, on
    all three activation rows (the third reaches +-127)."""
    rows, n = 600, 1024
    w, xq = _rows_and_acts(quant, rows, n, 555)
    n_tok = xq.shape[0]
    rb = row_bytes(quant, n)
    prev = oracle.set_simd(False)
    try:
        want = oracle.matmul_kq(w, xq, n, rows, n_tok, rb, quant)
    finally:
        oracle.set_simd(prev)
    oracle.set_simd(True)
    try:
        got = oracle.matmul_kq_mt(w, xq, n, rows, n_tok, rb, quant, 5)
    finally:
        oracle.set_simd(prev)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("quant", [QUANT_Q6_K, QUANT_Q4_K, QUANT_Q2_K, QUANT_IQ2_XXS])
@pytest.mark.parametrize("threads", [1, 3, 8])
def test_matmul_mt_equals_serial(quant, threads, scalar_then_restore):
    rows, n, n_tok = 777, 1280, 3
    w = synth.quant_matrix(quant, rows, n, synth.rng_for(threads, "mt"))
    xq = oracle.quantize_q8_k(np.random.default_rng(threads).standard_normal((n_tok, n)).astype(np.float32))
    rb = row_bytes(quant, n)
    want = oracle.matmul_kq(w, xq, n, rows, n_tok, rb, quant)
    abs_sum = np.zeros((n_tok, rows), np.float64)
    got = oracle.matmul_kq_mt(w, xq, n, rows, n_tok, rb, quant, threads, abs_sum=abs_sum)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for t in (0, n_tok - 1):
        for r in (0, 255, 256, rows - 1):  # job boundaries
            v, a = oracle.vec_dot(quant, w[r], xq[t], n)
            assert np.float32(v) == got[t, r] and a == abs_sum[t, r]


def _sigmoid32(x):
    # f32 sigmoid with the reference's two branches (cu:913-921)
    x = np.float32(x)
    if x >= 0:
        return np.float32(1.0) / (np.float32(1.0) + np.exp(-x, dtype=np.float32))
    e = np.exp(x, dtype=np.float32)
    return e / (np.float32(1.0) + e)


def _mode2_closed_form(raw, sink, bias, k, scale):
    """ids by sigmoid(raw) + bias (higher wins, lower index on ties); weights
    softmax(logsigmoid([raw winners] ++ sink)) * scale in f64."""
    score = np.array([_sigmoid32(v) + np.float32(b) for v, b in zip(raw, bias)], np.float32)
    order = sorted(range(len(raw)), key=lambda e: (-float(score[e]), e))
    ids = order[:k]
    z = np.concatenate([raw[ids].astype(np.float64), sink.astype(np.float64)])
    ls = -np.logaddexp(0.0, -z)  # log(sigmoid(z)), by another route than softplus
    w = np.exp(ls - ls.max())
    return ids, w / w.sum() * scale


@pytest.mark.parametrize("n_expert,k,n_sh,seed", [(16, 4, 1, 0), (64, 8, 2, 1), (200, 6, 3, 2), (9, 9, 1, 3)])
def test_router_mode2_matches_closed_form(n_expert, k, n_sh, seed):
    rng = np.random.default_rng(seed)
    n_tok = 4
    # logits spread apart so f32/f64 rounding cannot reorder near-ties ...
    raw = (rng.permutation(n_expert)[None, :] * 0.37 - n_expert * 0.15 + rng.integers(-2, 3, (n_tok, 1))).astype(
        np.float32)
    raw[1] = raw[1][::-1]
    sink = rng.uniform(-4, 4, (n_tok, n_sh)).astype(np.float32)
    sink[3, 0] = 35.0  # softplus branches: large positive and negative inputs
    raw[3, 0] = -40.0
    bias = (rng.permutation(n_expert) * 0.011).astype(np.float32)
    # ... except exact ties: equal raw logits and biases -> the lower index wins
    raw[2, 5 % n_expert] = raw[2, 2]
    bias[5 % n_expert] = bias[2]
    logits = np.ascontiguousarray(np.concatenate([raw, sink], axis=1))
    sel, w = oracle.router_select(logits, bias, n_expert, k, 1.5, n_tok, 2, n_sh)
    for t in range(n_tok):
        ids, want = _mode2_closed_form(raw[t], sink[t], bias, k, 1.5)
        assert list(sel[t, :k]) == ids, t
        assert list(sel[t, k:]) == list(range(n_expert, n_expert + n_sh))
        np.testing.assert_allclose(w[t].astype(np.float64), want, rtol=2e-6, atol=1e-7)
        assert abs(float(w[t].astype(np.float64).sum()) - 1.5) < 1e-5


def test_router_mode2_closed_form_catches_plausible_mistakes():
    """The closed form separates the reference's weights from two plausible
    misreadings: weighting by sigmoid(raw) instead of logsigmoid(raw), or
    leaving the sink logits out of the softmax."""
    raw = np.array([1.5, -0.5, 0.25, 2.0], np.float32)
    sink = np.array([0.75], np.float32)
    bias = np.zeros(4, np.float32)
    ids, want = _mode2_closed_form(raw, sink, bias, 2, 1.0)
    z = np.concatenate([raw[ids], sink]).astype(np.float64)
    sig = 1 / (1 + np.exp(-z))
    wrong1 = np.exp(sig - sig.max())
    wrong1 /= wrong1.sum()
    ls = -np.logaddexp(0.0, -z[:2])
    wrong2 = np.exp(ls - ls.max())
    wrong2 /= wrong2.sum()
    assert np.abs(wrong1 - want).max() > 1e-3
    assert np.abs(wrong2 - want[:2]).max() > 1e-3
