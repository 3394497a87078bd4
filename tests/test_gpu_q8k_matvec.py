"""GPU parity: q8_K quantizer (bit-exact) and pulsar_matmul_kq (integer
stages exact, fp32 within 1e-5 * sum_b |f_b|) against the oracle."""
import numpy as np
import pytest
import torch

import oracle
from pulsar_amd import kernels as K
from pulsar_amd import formats as fm
from pulsar_amd import synth
from pulsar_amd.formats import QUANT_IQ2_XXS, QUANT_MXFP4, QUANT_Q2_K, QUANT_Q4_K, QUANT_Q6_K, row_bytes
from tests.gpu_util import assert_rows_close, down, up, up_f32, zeros_f32, zeros_u8

pytestmark = pytest.mark.gpu
rng = np.random.default_rng(99)
DENSE = [QUANT_Q4_K, QUANT_Q6_K, QUANT_Q2_K, QUANT_IQ2_XXS]


def gpu_quantize(x: np.ndarray) -> np.ndarray:
    rows, n = x.shape
    nb = -(-n // 256)
    out = zeros_u8(rows * nb * 292)
    K.quantize_q8_k(out, up_f32(x), n, rows)
    return down(out).reshape(rows, nb * 292)


@pytest.mark.parametrize("rows,n", [(1, 256), (3, 512), (2, 300), (5, 2880), (16, 4096), (1, 1)])
def test_q8k_bit_exact(dev, rows, n):
    x = (rng.standard_normal((rows, n)) * rng.uniform(0.01, 100)).astype(np.float32)
    if n >= 512:
        x[0, 256:512] = 0.0  # an all-zero block
    assert np.array_equal(gpu_quantize(x), oracle.quantize_q8_k(x))


def test_q8k_ties_and_extremes(dev):
    x = np.zeros((2, 512), np.float32)
    x[0, 0] = 127.0
    x[0, 1:9] = [0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 126.5, -126.5]  # ties under inv = 1
    x[0, 256:] = rng.standard_normal(256).astype(np.float32) * 1e-30  # tiny magnitudes
    x[1, :256] = 3.0e38 * rng.choice([-1, 1], 256)  # near float max
    x[1, 256:] = rng.integers(-127, 128, 256).astype(np.float32)
    x2 = np.zeros((2, 256), np.float32)
    x2[0, ::3] = rng.standard_normal(86).astype(np.float32) * 1e-40  # subnormal inputs
    x2[1, 0] = 2e-38  # 127/amax overflows to inf: 0 * inf quantizes to 0
    x2[1, 5] = -1e-38
    assert np.array_equal(gpu_quantize(x2), oracle.quantize_q8_k(x2))
    got = gpu_quantize(x)
    assert np.array_equal(got, oracle.quantize_q8_k(x))
    _, qs, _ = oracle.q8k_fields(got)
    assert list(qs[0, 0, :9]) == [127, 1, -1, 2, -2, 3, -3, 127, -127]


def unit_scale_xq(n_tok: int, n: int) -> np.ndarray:
    """q8_K rows with d = 1 and random quants (consistent bsums): with unit
    weight scales every dot is an exact integer."""
    nb = n // 256
    qs = rng.integers(-60, 61, (n_tok, nb, 256)).astype(np.int8)
    blk = np.zeros((n_tok, nb, 292), np.uint8)
    blk[..., 0:4] = np.array([1.0], np.float32).view(np.uint8)
    blk[..., 4:260] = qs.view(np.uint8)
    blk[..., 260:292] = qs.reshape(n_tok, nb, 16, 16).astype(np.int16).sum(-1).astype(np.int16).view(np.uint8).reshape(n_tok, nb, 32)
    return blk.reshape(n_tok, nb * 292)


def unit_scale_matrix(quant, rows, n, seed):
    w = synth.quant_matrix(quant, rows, n, synth.rng_for(seed, "unit"))
    bb = fm.BLOCK_LAYOUT[quant][1]
    blk = w.reshape(rows, -1, bb)
    d_off, m_off, d_val = {QUANT_Q4_K: (0, 2, 0x3C00), QUANT_Q2_K: (80, 82, 0x3C00), QUANT_Q6_K: (208, None, 0x3C00),
                           QUANT_IQ2_XXS: (0, None, 0x4800), fm.QUANT_Q5_K: (0, 2, 0x3C00),
                           fm.QUANT_Q3_K: (108, None, 0x3C00)}[quant]
    blk[..., d_off], blk[..., d_off + 1] = d_val & 0xFF, d_val >> 8
    if m_off is not None:
        blk[..., m_off], blk[..., m_off + 1] = 0x00, 0x3C  # dmin = 1
    return w


@pytest.mark.parametrize("quant", DENSE)
@pytest.mark.parametrize("n,rows,n_tok", [(256, 37, 1), (2048, 64, 1), (4096, 33, 3), (12288, 9, 1),
                                          (256, 21, 7), (4096, 37, 16), (2048, 50, 20), (1024, 16, 5),
                                          (1024, 50, 64), (512, 33, 100), (768, 70, 40)])
def test_matvec_integer_stage_exact(dev, quant, n, rows, n_tok):
    w = unit_scale_matrix(quant, rows, n, n + rows)
    xq = unit_scale_xq(n_tok, n)
    rb = row_bytes(quant, n)
    out = zeros_f32((n_tok, rows))
    K.matmul_kq(out, up(w), up(xq), n, rows, n_tok, rb, quant)
    got = down(out)
    want = oracle.matmul_kq(w, xq, n, rows, n_tok, rb, quant)
    assert np.abs(want).max() < 2**24  # every partial sum is an exact integer in fp32
    assert np.array_equal(got, want)


@pytest.mark.parametrize("quant", DENSE)
@pytest.mark.parametrize("n,rows,n_tok", [(256, 5, 1), (2048, 130, 1), (4096, 77, 2), (4096, 40, 5),
                                          (4096, 24, 16), (8192, 19, 1), (20480, 7, 1),
                                          (2816, 33, 9), (4096, 70, 33), (2048, 36, 70)])
def test_matvec_fp32_parity(dev, quant, n, rows, n_tok):
    w = synth.quant_matrix(quant, rows, n, synth.rng_for(n * rows + n_tok, "mv"))
    x = rng.standard_normal((n_tok, n)).astype(np.float32)
    xq = oracle.quantize_q8_k(x)
    rb = row_bytes(quant, n)
    out = zeros_f32((n_tok, rows))
    K.matmul_kq(out, up(w), up(xq), n, rows, n_tok, rb, quant)
    got = down(out)
    for t in range(n_tok):
        vals, scale = zip(*(oracle.vec_dot(quant, w[r], xq[t], n) for r in range(rows)))
        assert_rows_close(got[t], np.array(vals, np.float32), np.array(scale), f"q{quant} n{n} t{t}")


@pytest.mark.parametrize("quant,n_tok", [(QUANT_Q6_K, 1), (QUANT_Q6_K, 16), (QUANT_Q4_K, 16), (QUANT_Q4_K, 64)])
def test_matvec_padded_row_stride(dev, quant, n_tok):
    # row_bytes larger than the packed row: rows start row_bytes apart
    # (n_tok >= 5 runs the MFMA kernels)
    n, rows = 1024, 21
    rb = row_bytes(quant, n)
    w = synth.quant_matrix(quant, rows, n, synth.rng_for(5, "pad"))
    padded = np.zeros((rows, rb + 46), np.uint8)
    padded[:, :rb] = w
    xq = oracle.quantize_q8_k(rng.standard_normal((n_tok, n)).astype(np.float32))
    out = zeros_f32((n_tok, rows))
    K.matmul_kq(out, up(padded), up(xq), n, rows, n_tok, rb + 46, quant)
    want = oracle.matmul_kq(padded, xq, n, rows, n_tok, rb + 46, quant)
    for t in range(n_tok):
        vals, scale = zip(*(oracle.vec_dot(quant, w[r], xq[t], n) for r in range(rows)))
        assert_rows_close(down(out)[t], want[t], np.array(scale), f"padded stride t{t}")


def test_matvec_linearity_exact(dev):
    """Scaling x by 2 doubles q8_K d exactly and leaves the quants alone, so
    every output doubles bit-exactly (size-independent property)."""
    n, rows, quant = 4096, 256, QUANT_Q4_K
    w = up(synth.quant_matrix(quant, rows, n, synth.rng_for(3, "lin")))
    x = rng.standard_normal((1, n)).astype(np.float32)
    outs = []
    for s in (1.0, 2.0):
        xq = zeros_u8(16 * 292)
        K.quantize_q8_k(xq, up_f32(x * s), n, 1)
        o = zeros_f32((1, rows))
        K.matmul_kq(o, w, xq, n, rows, 1, row_bytes(quant, n), quant)
        outs.append(down(o))
    assert np.array_equal(outs[1], 2 * outs[0])


def test_matvec_error_contract(dev):
    buf = zeros_u8(1 << 16)
    out = zeros_f32(64)
    with pytest.raises(K.KernelError):
        K.matmul_kq(out, buf, buf, 200, 4, 1, 144, QUANT_Q4_K)  # in_dim % 256
    with pytest.raises(K.KernelError):
        K.matmul_kq(out, buf, buf, 256, 4, 1, 136, QUANT_MXFP4)  # not a dense format
    with pytest.raises(K.KernelError):
        K.matmul_kq(out, buf, buf, 256, 0, 1, 144, QUANT_Q4_K)
    with pytest.raises(K.KernelError):
        K.quantize_q8_k(out, buf, 0, 1)
    # A4_OK is accepted and ignored
    xq = zeros_u8(292)
    K.matmul_kq(out, buf, xq, 256, 4, 1, 144, QUANT_Q4_K | 0x8000_0000)
    torch.cuda.synchronize()


MORE_DENSE = [fm.QUANT_Q5_K, fm.QUANT_Q3_K, fm.QUANT_IQ4_XS, fm.QUANT_IQ4_NL, fm.QUANT_NVFP4]


@pytest.mark.parametrize("quant", [fm.QUANT_Q5_K, fm.QUANT_Q3_K], ids=lambda q: fm.NAMES[q])
@pytest.mark.parametrize("n,rows,n_tok", [(256, 37, 1), (2048, 64, 1), (4096, 33, 3), (1024, 16, 5), (512, 33, 40)])
def test_matvec_more_formats_integer_exact(dev, quant, n, rows, n_tok):
    """Q5_K and Q3_K dense dots at unit scales: exact integers, bit-exact."""
    w = unit_scale_matrix(quant, rows, n, n + rows)
    xq = unit_scale_xq(n_tok, n)
    rb = row_bytes(quant, n)
    out = zeros_f32((n_tok, rows))
    K.matmul_kq(out, up(w), up(xq), n, rows, n_tok, rb, quant)
    want = oracle.matmul_kq(w, xq, n, rows, n_tok, rb, quant)
    assert np.abs(want).max() < 2**24
    assert np.array_equal(down(out), want)


@pytest.mark.parametrize("quant", MORE_DENSE, ids=lambda q: fm.NAMES[q])
@pytest.mark.parametrize("n,rows,n_tok", [(256, 5, 1), (2048, 130, 1), (4096, 40, 3), (4096, 24, 16), (1024, 50, 64)])
def test_matvec_more_formats_fp32_parity(dev, quant, n, rows, n_tok):
    """The other dense formats of pulsar_kernels.cu:5090-5142 against the
    oracle, decode and token chunks."""
    w = synth.quant_matrix(quant, rows, n, synth.rng_for(n * rows + n_tok, "mv2"))
    x = rng.standard_normal((n_tok, n)).astype(np.float32)
    xq = oracle.quantize_q8_k(x)
    rb = row_bytes(quant, n)
    out = zeros_f32((n_tok, rows))
    K.matmul_kq(out, up(w), up(xq), n, rows, n_tok, rb, quant)
    got = down(out)
    for t in range(n_tok):
        vals, scale = zip(*(oracle.vec_dot(quant, w[r], xq[t], n) for r in range(rows)))
        assert_rows_close(got[t], np.array(vals, np.float32), np.array(scale), f"q{quant} n{n} t{t}")


def test_matvec_rejects_moe_only_formats(dev):
    """Q4_0, Q5_1, Q8_0 and the IQ1-3 formats are expert formats only: the
    dense entry point returns 0 for them (pulsar_kernels.cu:5110, 5139)."""
    buf = up(np.zeros(1 << 16, np.uint8))
    for q in (fm.QUANT_Q4_0, fm.QUANT_Q5_1, fm.QUANT_Q8_0, fm.QUANT_IQ2_XS, fm.QUANT_IQ3_XXS, fm.QUANT_IQ3_S,
              fm.QUANT_IQ2_S, fm.QUANT_IQ1_S, fm.QUANT_MXFP4):
        with pytest.raises(K.KernelError):
            K.matmul_kq(buf, buf, buf, 256, 4, 1, row_bytes(q, 256), q)


@pytest.mark.parametrize("quant", [QUANT_Q4_K, QUANT_Q6_K, QUANT_Q2_K, QUANT_IQ2_XXS, fm.QUANT_IQ4_NL, fm.QUANT_Q3_K],
                         ids=lambda q: fm.NAMES[q])
@pytest.mark.parametrize("n,rows,n_tok", [(36864, 9, 1), (40960, 13, 3), (33024, 6, 6)])
def test_matvec_rows_wider_than_32768(dev, quant, n, rows, n_tok):
    """Rows of more than 32768 values (the reference accepts any multiple of
    256, pulsar_kernels.cu:4904): the lane path walks them in 16-super-block
    slices (n_tok >= 5 on Q4_K / Q6_K goes to the MFMA GEMM). Seeded
    weights within 1e-5 * sum_b |f_b|, and unit scales bit-exact."""
    w = synth.quant_matrix(quant, rows, n, synth.rng_for(n + rows, "wide"))
    x = rng.standard_normal((n_tok, n)).astype(np.float32)
    xq = oracle.quantize_q8_k(x)
    rb = row_bytes(quant, n)
    out = zeros_f32((n_tok, rows))
    K.matmul_kq(out, up(w), up(xq), n, rows, n_tok, rb, quant)
    got = down(out)
    for t in range(n_tok):
        vals, scale = zip(*(oracle.vec_dot(quant, w[r], xq[t], n) for r in range(rows)))
        assert_rows_close(got[t], np.array(vals, np.float32), np.array(scale), f"q{quant} n{n} t{t}")
    if quant in (QUANT_Q4_K, QUANT_Q6_K, QUANT_Q2_K, QUANT_IQ2_XXS, fm.QUANT_Q3_K):
        wu = unit_scale_matrix(quant, rows, n, n)
        nb = n // 256  # q8_K rows with d = 1 and quants in [-12, 12]: sums stay exact in fp32
        qs = rng.integers(-12, 13, (n_tok, nb, 256)).astype(np.int8)
        blk = np.zeros((n_tok, nb, 292), np.uint8)
        blk[..., 0:4] = np.array([1.0], np.float32).view(np.uint8)
        blk[..., 4:260] = qs.view(np.uint8)
        blk[..., 260:292] = qs.reshape(n_tok, nb, 16, 16).astype(np.int16).sum(-1).astype(np.int16).view(
            np.uint8).reshape(n_tok, nb, 32)
        xu = blk.reshape(n_tok, nb * 292)
        out.zero_()
        K.matmul_kq(out, up(wu), up(xu), n, rows, n_tok, rb, quant)
        want = oracle.matmul_kq(wu, xu, n, rows, n_tok, rb, quant)
        assert np.abs(want).max() < 2**24
        assert np.array_equal(down(out), want)
