// matvec.hip - pulsar_matmul_kq: dense K-quant / IQ matvec on q8_K rows.
//
// Decode shape (n_tok small): each wave streams rows (grid-stride over row
// passes), lanes over the row's units, the token's activation slices held in
// registers for the whole kernel. Weight loads are 16-byte loads at the
// formats' native (unaligned) offsets; consecutive lanes read consecutive
// bytes of a row, so every wave-wide load is one contiguous span.
#include "pk_rowdot.h"

// token chunks of at least this many tokens go to the MFMA kernel
#ifndef PK_MMQ_MIN_TOK
#define PK_MMQ_MIN_TOK 5u
#endif

namespace pk {

// mmq.hip: MFMA kernel for token chunks; returns -1 when it has no kernel
// for the format (the caller then uses the lane kernels)
int launch_gemm(uint32_t quant, float *out, const uint8_t *w, const pulsar_block_q8_K *xq, uint32_t in_dim,
                uint32_t out_dim, uint32_t n_tok, uint64_t row_bytes);

// Each wave streams row passes pass0, pass0 + n_waves, ...: the row's
// weight units are requested first, then (once per wave) the token's
// activation slices, so the HBM latency of the first row overlaps the L2
// latency of the activations.
#ifndef PK_MV_TPB
#define PK_MV_TPB 256u
#endif
template <uint32_t Q, uint32_t T, uint32_t UPLMAX, uint32_t RPW, uint32_t L2>
__global__ __launch_bounds__(PK_MV_TPB) void matvec_kernel(float *__restrict__ out,
                                                     const uint8_t *__restrict__ w,
                                                     const pulsar_block_q8_K *__restrict__ xq,
                                                     uint32_t n_units, uint32_t nblk32,
                                                     uint32_t lpr_log2, uint32_t in_blocks,
                                                     uint32_t out_dim, uint32_t n_tok,
                                                     uint64_t row_bytes, uint32_t n_pass) {
    PK_FMT_LUT(Q)
    const RowGeom rg = row_geom<L2>(n_units, nblk32, lpr_log2);
    const uint32_t rpp = 64u >> rg.lpr_log2;
    const uint32_t t0 = blockIdx.y * T;
    const uint32_t waves = blockDim.x / 64u;
    const uint32_t n_waves = gridDim.x * waves;
    uint32_t base = (blockIdx.x * waves + threadIdx.x / 64u) * RPW;
    if (base >= n_pass) return;  // whole wave
    typename Fmt<Q>::W wu[RPW][UPLMAX];
#pragma unroll
    for (uint32_t p = 0; p < RPW; p++) {
        const uint32_t row = (base + p) * rpp + rg.rip;
        load_row_w<Q, UPLMAX>(w + (uint64_t)(row < out_dim ? row : 0u) * row_bytes, rg, wu[p]);
    }
    Act a[T][UPLMAX];
#pragma unroll
    for (uint32_t t = 0; t < T; t++) {
        const uint32_t tok = t0 + t < n_tok ? t0 + t : n_tok - 1u;
        load_row_acts<Q, UPLMAX>(xq + (uint64_t)tok * in_blocks, rg, a[t]);
    }
    for (;;) {
#pragma unroll
        for (uint32_t p = 0; p < RPW; p++) {
            const uint32_t row = (base + p) * rpp + rg.rip;
            const bool row_ok = row < out_dim;
#pragma unroll
            for (uint32_t t = 0; t < T; t++) {
                float acc = row_partial<Q, UPLMAX>(row_ok, rg, wu[p], a[t], lut);
                acc = row_finish(acc, rg);
                if (row_ok && rg.holds_row() && t0 + t < n_tok) out[(uint64_t)(t0 + t) * out_dim + row] = acc;
            }
        }
        base += n_waves * RPW;
        if (base >= n_pass) break;
#pragma unroll
        for (uint32_t p = 0; p < RPW; p++) {
            const uint32_t row = (base + p) * rpp + rg.rip;
            load_row_w<Q, UPLMAX>(w + (uint64_t)(row < out_dim ? row : 0u) * row_bytes, rg, wu[p]);
        }
    }
}

// Rows wider than the register-resident unit layout holds (more than 8
// units per lane: in_dim > 32768). A wave takes one row and walks it in
// slices of 16 super-blocks (64 units, one per lane): each slice's weight
// units and activation slices are loaded, the lane's super-block values are
// added to its running sum, and the row total is the fixed tree of the
// lanes' sums. T tokens per launch row (grid.y covers the rest).
template <uint32_t Q, uint32_t T>
__global__ __launch_bounds__(256) void matvec_wide_kernel(float *__restrict__ out, const uint8_t *__restrict__ w,
                                                          const pulsar_block_q8_K *__restrict__ xq, uint32_t n_units,
                                                          uint32_t nblk32, uint32_t in_blocks, uint32_t out_dim,
                                                          uint32_t n_tok, uint64_t row_bytes) {
    PK_FMT_LUT(Q)
    const uint32_t row = blockIdx.x * 4u + threadIdx.x / 64u;
    if (row >= out_dim) return;  // whole wave
    const uint32_t t0 = blockIdx.y * T;
    const uint8_t *wr = w + (uint64_t)row * row_bytes;
    float acc[T];
#pragma unroll
    for (uint32_t t = 0; t < T; t++) acc[t] = 0.0f;
    for (uint32_t u0 = 0; u0 < n_units; u0 += 64u) {
        RowGeom rg = row_geom<6>(n_units - u0 < 64u ? n_units - u0 : 64u, nblk32, 6u);
        const uint32_t sb0 = u0 / 4u;
        typename Fmt<Q>::W wu[1];
        load_row_w<Q, 1>(wr + (uint64_t)sb0 * Fmt<Q>::kSbBytes, rg, wu);
#pragma unroll
        for (uint32_t t = 0; t < T; t++) {
            const uint32_t tok = t0 + t < n_tok ? t0 + t : n_tok - 1u;
            Act a[1];
            load_row_acts<Q, 1>(xq + (uint64_t)tok * in_blocks + sb0, rg, a);
            acc[t] += row_partial<Q, 1>(true, rg, wu, a, lut);
        }
    }
    const RowGeom rg = row_geom<6>(64u, nblk32, 6u);
#pragma unroll
    for (uint32_t t = 0; t < T; t++) {
        const float v = row_finish(acc[t], rg);
        if (rg.holds_row() && t0 + t < n_tok) out[(uint64_t)(t0 + t) * out_dim + row] = v;
    }
}

#ifndef PK_MV_RPW
#define PK_MV_RPW 1
#endif
#ifndef PK_MV_WAVES
#define PK_MV_WAVES 4096u
#endif
template <uint32_t Q, uint32_t T, uint32_t UPLMAX, uint32_t RPW>
static void launch_matvec(float *out, const uint8_t *w, const pulsar_block_q8_K *xq, uint32_t n_units,
                          uint32_t nblk32, uint32_t lpr_log2, uint32_t in_blocks, uint32_t out_dim,
                          uint32_t n_tok, uint64_t row_bytes) {
    const uint32_t rpp = 64u >> lpr_log2;
    const uint32_t n_pass = (out_dim + rpp - 1u) / rpp;
    // up to 4096 chunks one wave each; larger matrices loop over a wave
    // count measured per format on 8192-32768-row matrices: Q6_K (the
    // heaviest decode per byte) runs best on 3072 waves, 3 blocks per CU
    // (8192 x 4096: 7.6 -> 7.2 us; 16384 x 4096: 13.0 -> 11.8 us), Q4_K and
    // Q2_K on 6144 (Q4_K 12288 x 4096: 7.9 -> 7.4 us; Q2_K 16384 x 4096:
    // 7.6 -> 7.2 us), each slower on the other's count
    constexpr uint32_t kCap = Q == PULSAR_QUANT_Q6_K ? 3072u : 6144u;
    const uint32_t chunks = (n_pass + RPW - 1u) / RPW;
    const uint32_t waves = chunks <= PK_MV_WAVES ? chunks : chunks < kCap ? chunks : kCap;
    constexpr uint32_t wpb = PK_MV_TPB / 64u;
    const dim3 grid((waves + wpb - 1u) / wpb, (n_tok + T - 1u) / T);
    if (lpr_log2 == 6)
        hipLaunchKernelGGL((matvec_kernel<Q, T, UPLMAX, RPW, 6>), grid, dim3(PK_MV_TPB), 0, pk::stream(), out, w,
                           xq, n_units, nblk32, lpr_log2, in_blocks, out_dim, n_tok, row_bytes, n_pass);
    else
        hipLaunchKernelGGL((matvec_kernel<Q, T, UPLMAX, RPW, 0>), grid, dim3(PK_MV_TPB), 0, pk::stream(), out, w,
                           xq, n_units, nblk32, lpr_log2, in_blocks, out_dim, n_tok, row_bytes, n_pass);
}


template <uint32_t Q>
static int dispatch_matvec(float *out, const uint8_t *w, const pulsar_block_q8_K *xq, uint32_t in_dim,
                           uint32_t out_dim, uint32_t n_tok, uint64_t row_bytes) {
    const uint32_t n_units = units_per_row(Q, in_dim);
    const uint32_t l2 = lpr_log2_for(n_units);
    const uint32_t upl = (n_units + (1u << l2) - 1u) >> l2;
    const uint32_t in_blocks = (in_dim + 255u) / 256u;
    const uint32_t nblk32 = (in_dim + 31u) / 32u;
#define PK_MV(T, U, R) launch_matvec<Q, T, U, R>(out, w, xq, n_units, nblk32, l2, in_blocks, out_dim, n_tok, row_bytes)
    if (upl <= 1u) {
        if (n_tok == 1u)
            PK_MV(1, 1, PK_MV_RPW);
        else if (n_tok == 2u)
            PK_MV(2, 1, 2);
        else
            PK_MV(4, 1, 1);
    } else if (upl <= 2u) {
        if (n_tok == 1u)
            PK_MV(1, 2, 2);
        else
            PK_MV(2, 2, 1);
    } else if (upl <= 4u) {
        PK_MV(1, 4, 1);
    } else if (upl <= 8u) {
        PK_MV(1, 8, 1);
    } else {
        // wider rows: one wave per row, streamed in 16-super-block slices
        const dim3 grid((out_dim + 3u) / 4u, n_tok <= 1u ? 1u : (n_tok + 3u) / 4u);
        if (n_tok == 1u)
            hipLaunchKernelGGL((matvec_wide_kernel<Q, 1>), grid, dim3(256), 0, pk::stream(), out, w, xq, n_units,
                               nblk32, in_blocks, out_dim, n_tok, row_bytes);
        else
            hipLaunchKernelGGL((matvec_wide_kernel<Q, 4>), grid, dim3(256), 0, pk::stream(), out, w, xq, n_units,
                               nblk32, in_blocks, out_dim, n_tok, row_bytes);
    }
#undef PK_MV
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
    if (n_tok >= PK_MMQ_MIN_TOK) {
        const int r = pk::launch_gemm(quant, o, wb, x, in_dim, out_dim, n_tok, row_bytes);
        if (r >= 0) return r;
    }
    // the dense formats of pulsar_kernels.cu:5090-5142
#define PK_MVQ(Q) \
    case Q: return pk::dispatch_matvec<Q>(o, wb, x, in_dim, out_dim, n_tok, row_bytes);
    switch (quant) {
    PK_MVQ(PULSAR_QUANT_Q4_K)
    PK_MVQ(PULSAR_QUANT_Q6_K)
    PK_MVQ(PULSAR_QUANT_Q2_K)
    PK_MVQ(PULSAR_QUANT_IQ2_XXS)
    PK_MVQ(PULSAR_QUANT_Q5_K)
    PK_MVQ(PULSAR_QUANT_Q3_K)
    PK_MVQ(PULSAR_QUANT_IQ4_XS)
    PK_MVQ(PULSAR_QUANT_IQ4_NL)
    PK_MVQ(PULSAR_QUANT_NVFP4)
    default: return pk::reject("matmul_kq (quant)");
    }
#undef PK_MVQ
}
