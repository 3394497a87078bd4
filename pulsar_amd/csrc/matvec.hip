// matvec.hip - pulsar_matmul_kq: dense K-quant / IQ matvec on q8_K rows.
//
// Decode shape (n_tok small): each wave streams rows (grid-stride over row
// passes), lanes over the row's units, the token's activation slices held in
// registers for the whole kernel. Weight loads are 16-byte loads at the
// formats' native (unaligned) offsets; consecutive lanes read consecutive
// bytes of a row, so every wave-wide load is one contiguous span.
#include "pk_rowdot.h"

namespace pk {

template <uint32_t Q, uint32_t T, uint32_t UPLMAX>
__global__ __launch_bounds__(256) void matvec_kernel(float *__restrict__ out,
                                                     const uint8_t *__restrict__ w,
                                                     const pulsar_block_q8_K *__restrict__ xq,
                                                     uint32_t n_units, uint32_t nblk32,
                                                     uint32_t lpr_log2, uint32_t in_blocks,
                                                     uint32_t out_dim, uint32_t n_tok,
                                                     uint64_t row_bytes, uint32_t n_pass) {
    __shared__ uint2 lut[Q == PULSAR_QUANT_IQ2_XXS ? 256 : 1];
    if (Q == PULSAR_QUANT_IQ2_XXS) {
        fill_iq2xxs_lut(lut);
        __syncthreads();
    }
    const RowGeom rg = row_geom(n_units, nblk32, lpr_log2);
    const uint32_t rpp = 64u >> lpr_log2;
    const uint32_t t0 = blockIdx.y * T;
    Act a[T][UPLMAX];
#pragma unroll
    for (uint32_t t = 0; t < T; t++) {
        const uint32_t tok = t0 + t < n_tok ? t0 + t : n_tok - 1u;
        load_row_acts<Q, UPLMAX>(xq + (uint64_t)tok * in_blocks, rg, a[t]);
    }
    const uint32_t waves = blockDim.x / 64u;
    const uint32_t n_waves = gridDim.x * waves;
    for (uint32_t pass = blockIdx.x * waves + threadIdx.x / 64u; pass < n_pass; pass += n_waves) {
        const uint32_t row = pass * rpp + rg.rip;
        const bool row_ok = row < out_dim;
        typename Fmt<Q>::W wu[UPLMAX];
        load_row_w<Q, UPLMAX>(w + (uint64_t)row * row_bytes, row_ok, rg, wu);
#pragma unroll
        for (uint32_t t = 0; t < T; t++) {
            float acc = row_partial<Q, UPLMAX>(row_ok, rg, wu, a[t], lut);
            acc = row_finish(acc, rg);
            if (row_ok && rg.lir == 0 && t0 + t < n_tok) out[(uint64_t)(t0 + t) * out_dim + row] = acc;
        }
    }
}

template <uint32_t Q, uint32_t T, uint32_t UPLMAX>
static void launch_matvec(float *out, const uint8_t *w, const pulsar_block_q8_K *xq, uint32_t n_units,
                          uint32_t nblk32, uint32_t lpr_log2, uint32_t in_blocks, uint32_t out_dim,
                          uint32_t n_tok, uint64_t row_bytes) {
    const uint32_t rpp = 64u >> lpr_log2;
    const uint32_t n_pass = (out_dim + rpp - 1u) / rpp;
    // one wave per row pass up to 8192 waves (8 per SIMD on 256 CUs), then
    // each wave loops
    const uint32_t waves = n_pass < 8192u ? n_pass : 8192u;
    const dim3 grid((waves + 3u) / 4u, (n_tok + T - 1u) / T);
    hipLaunchKernelGGL((matvec_kernel<Q, T, UPLMAX>), grid, dim3(256), 0, pk::stream(), out, w, xq, n_units,
                       nblk32, lpr_log2, in_blocks, out_dim, n_tok, row_bytes, n_pass);
}

template <uint32_t Q>
static int dispatch_matvec(float *out, const uint8_t *w, const pulsar_block_q8_K *xq, uint32_t in_dim,
                           uint32_t out_dim, uint32_t n_tok, uint64_t row_bytes) {
    const uint32_t n_units = units_per_row(Q, in_dim);
    const uint32_t l2 = lpr_log2_for(n_units);
    const uint32_t upl = (n_units + (1u << l2) - 1u) >> l2;
    const uint32_t in_blocks = (in_dim + 255u) / 256u;
    const uint32_t nblk32 = (in_dim + 31u) / 32u;
    if (upl <= 1u) {
        if (n_tok == 1u)
            launch_matvec<Q, 1, 1>(out, w, xq, n_units, nblk32, l2, in_blocks, out_dim, n_tok, row_bytes);
        else if (n_tok == 2u)
            launch_matvec<Q, 2, 1>(out, w, xq, n_units, nblk32, l2, in_blocks, out_dim, n_tok, row_bytes);
        else
            launch_matvec<Q, 4, 1>(out, w, xq, n_units, nblk32, l2, in_blocks, out_dim, n_tok, row_bytes);
    } else if (upl <= 2u) {
        if (n_tok == 1u)
            launch_matvec<Q, 1, 2>(out, w, xq, n_units, nblk32, l2, in_blocks, out_dim, n_tok, row_bytes);
        else
            launch_matvec<Q, 2, 2>(out, w, xq, n_units, nblk32, l2, in_blocks, out_dim, n_tok, row_bytes);
    } else if (upl <= 4u) {
        launch_matvec<Q, 1, 4>(out, w, xq, n_units, nblk32, l2, in_blocks, out_dim, n_tok, row_bytes);
    } else if (upl <= 8u) {
        launch_matvec<Q, 1, 8>(out, w, xq, n_units, nblk32, l2, in_blocks, out_dim, n_tok, row_bytes);
    } else {
        return reject("matmul_kq (in_dim above 32768)");
    }
    return launch_ok("matmul_kq launch");
}

}  // namespace pk

// pulsar_kernels.cu:4895-4906 contract: in_dim a multiple of 256, nonzero
// dims, quant one of the dense K-quant/IQ codes (MXFP4 is not a dense
// matmul_kq format in the reference either). QUANT_A4_OK is accepted and
// ignored (it selects an NVFP4 path there).
extern "C" int pulsar_matmul_kq(void *out, const void *w, const void *xq, uint32_t in_dim,
                                uint32_t out_dim, uint32_t n_tok, uint64_t row_bytes,
                                uint32_t quant) {
    quant &= ~PULSAR_QUANT_A4_OK;
    if (!out || !w || !xq || in_dim == 0 || in_dim % 256u != 0 || out_dim == 0 || n_tok == 0 ||
        row_bytes == 0)
        return pk::reject("matmul_kq");
    float *o = (float *)out;
    const uint8_t *wb = (const uint8_t *)w;
    const pulsar_block_q8_K *x = (const pulsar_block_q8_K *)xq;
    switch (quant) {
    case PULSAR_QUANT_Q4_K: return pk::dispatch_matvec<PULSAR_QUANT_Q4_K>(o, wb, x, in_dim, out_dim, n_tok, row_bytes);
    case PULSAR_QUANT_Q6_K: return pk::dispatch_matvec<PULSAR_QUANT_Q6_K>(o, wb, x, in_dim, out_dim, n_tok, row_bytes);
    case PULSAR_QUANT_Q2_K: return pk::dispatch_matvec<PULSAR_QUANT_Q2_K>(o, wb, x, in_dim, out_dim, n_tok, row_bytes);
    case PULSAR_QUANT_IQ2_XXS: return pk::dispatch_matvec<PULSAR_QUANT_IQ2_XXS>(o, wb, x, in_dim, out_dim, n_tok, row_bytes);
    default: return pk::reject("matmul_kq (quant)");
    }
}
