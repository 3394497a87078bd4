/* pulsar_oracle.h - CPU restatement of the reference's expert-matvec path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker the HIP library is compared
 * against and the CPU baseline bench.py times; nothing in pulsar_amd/ links,
 * loads or calls it.
 *
 * Every function follows a reference file:line (cited at its definition in
 * pulsar_oracle.c). Pointers are host pointers; structs are the same byte
 * layouts as include/pulsar_moe.h. Build with -ffp-contract=off so the float
 * epilogues round exactly as the reference's Rust lane does (Rust never
 * contracts a*b+c into an FMA).
 */
#ifndef PULSAR_ORACLE_H
#define PULSAR_ORACLE_H

#include <stdint.h>

#include "../include/pulsar_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* f16 <-> f32 (crates/quant/src/cpu_dot.rs:52-64; crates/quant/src/lib.rs:51-82) */
float po_f16_to_f32(uint16_t h);
uint16_t po_f32_to_f16(float f);

/* q8_K quantizer of the CPU lane; in_dim need not be a multiple of 256
 * (tail zero-padded). out: n_rows * ceil(in_dim/256) blocks. */
void po_quantize_q8_K(pulsar_block_q8_K *out, const float *x, uint32_t in_dim, uint32_t n_rows);

/* Bytes one row of n values occupies in `quant` (GGUF row_bytes). */
uint64_t po_row_bytes(uint32_t quant, uint32_t n);
/* Bytes per 256-value super-block as the dots index them (MXFP4: 8 * 17). */
uint32_t po_sb_bytes(uint32_t quant);

/* Integer stage of one super-block b of a row against q8_K block y.
 * Writes the exact int32 sums the float epilogue consumes:
 *   Q4_K   : i0 = isum, i1 = msum
 *   Q2_K   : i0 = isum, i1 = summs
 *   Q6_K   : i0 = isum
 *   IQ2_XXS: i0 = bsum (sum over 32-groups of sumi * (2*scale+1))
 *   MXFP4  : sumi[0..7] per 32-block (blocks past n_valid32 are 0)
 * and returns the super-block's fp32 value in the reference's operation
 * order. n_valid32 = valid 32-value blocks in this super-block (8 except a
 * MXFP4 tail). */
float po_block_dot(uint32_t quant, const uint8_t *row, uint32_t b,
                   const pulsar_block_q8_K *y, uint32_t n_valid32,
                   int32_t *i0, int32_t *i1, int32_t sumi[8]);

/* Row dot: sequential fp32 sum over super-blocks (the lane's vec_dot_*).
 * abs_sum (nullable) receives sum_b |f_b| in f64, the scale the parity
 * tolerance is stated against. */
float po_vec_dot(uint32_t quant, const uint8_t *row, const pulsar_block_q8_K *xq,
                 uint32_t n, double *abs_sum);

/* f64 dequant of one row (the reference tests' f64 dequant references). */
void po_dequant_row(uint32_t quant, const uint8_t *row, uint32_t n, double *out);

/* Dense matvec: out[t][r] = po_vec_dot(row r, xq[t]). Returns 1/0 like the ABI. */
int po_matmul_kq(float *out, const uint8_t *w, const pulsar_block_q8_K *xq,
                 uint32_t in_dim, uint32_t out_dim, uint32_t n_tok,
                 uint64_t row_bytes, uint32_t quant);

/* Gated combine (pulsar_kernels.cu:124-141 == elib:2131-2157), ops 0 and 2. */
float po_glu(float g, float u, uint32_t op);

/* MoE stages on host pointers (ptrs hold HOST addresses). Same semantics and
 * return convention as the ABI entry points of the same name. */
int po_moe_pair_swiglu(float *mid, const pulsar_expert_ptrs *ptrs, const float *weights,
                       const pulsar_block_q8_K *xq, uint32_t in_dim, uint32_t mid_dim,
                       uint32_t n_used, uint32_t n_tok, uint64_t row_bytes,
                       uint32_t quant, uint32_t act_op);
int po_moe_down(float *out, const pulsar_expert_ptrs *ptrs, const pulsar_block_q8_K *midq,
                uint32_t mid_dim, uint32_t out_dim, uint32_t n_used, uint32_t n_tok,
                uint64_t row_bytes, uint32_t quant);
int po_moe_down_bias(float *out, const pulsar_expert_ptrs *ptrs, const float *weights,
                     uint32_t out_dim, uint32_t n_used, uint32_t n_tok);

/* Router pieces. */
int po_matmul_f32(float *out, const float *w, const float *x, uint32_t in_dim,
                  uint32_t out_dim, uint32_t n_tok);
int po_add_bias_rows(float *x, const float *bias, uint32_t dim, uint32_t rows);
int po_router_select(int32_t *selected, float *weights, const float *logits,
                     const float *bias, uint32_t n_expert, uint32_t k_used,
                     float weight_scale, uint32_t n_tok, uint32_t mode, uint32_t n_shexp);

/* The reference test generator (crates/quant/src/cpu_dot.rs:819-822):
 * state = state * 6364136223846793005 + 1442695040888963407;
 * returns ((state >> 33) as f32 / 2^31) - 1. */
float po_lcg(uint64_t *state);

/* CPU expert lane baseline: the reference Lane's job structure
 * (crates/engine/src/lib.rs:1994-2100) on `threads` pthreads: per token
 * quantize x, gate/up/glu jobs over 256-row chunks, quantize mids, down jobs
 * over 512-row chunks. ptrs hold host addresses; NULL gate/up/down slots are
 * skipped like the GPU path. out: f32 [n_tok][out_dim]. Returns 1/0. */
int po_lane_moe(float *out, const pulsar_expert_ptrs *ptrs, const float *weights,
                const float *x, uint32_t in_dim, uint32_t mid_dim, uint32_t out_dim,
                uint32_t n_used, uint32_t n_tok, uint64_t gate_row_bytes,
                uint32_t gate_quant, uint64_t down_row_bytes, uint32_t down_quant,
                uint32_t act_op, uint32_t threads);

/* Multi-threaded dense matvec (rows split in 256-row jobs, like the Lane's
 * gate/up jobs) for the baseline and for large parity checks; abs_sum
 * (nullable, f64 [n_tok][out_dim]) receives each output's sum_b |f_b|. */
int po_matmul_kq_mt(float *out, const uint8_t *w, const pulsar_block_q8_K *xq,
                    uint32_t in_dim, uint32_t out_dim, uint32_t n_tok,
                    uint64_t row_bytes, uint32_t quant, uint32_t threads, double *abs_sum);

/* The same for any format (MXFP4 rows included, n a multiple of 32 there,
 * of 256 otherwise): out[t][r] = po_vec_dot(row r, xq[t]) over `rows` rows
 * row_bytes apart. The checker of full-shape expert stages. */
int po_rows_dot(float *out, const uint8_t *w, uint64_t row_bytes, uint32_t rows,
                const pulsar_block_q8_K *xq, uint32_t n, uint32_t n_tok, uint32_t quant,
                uint32_t threads, double *abs_sum);

/* Selects the AVX2 row dots of the lane formats (Q4_K, Q2_K, IQ2_XXS) in
 * po_vec_dot when on != 0 and the CPU has AVX2 (the default), the scalar
 * dots otherwise; returns the previous setting. Both give the same bits. A
 * request for abs_sum always takes the scalar dots. */
int po_set_simd(int on);

#ifdef __cplusplus
}
#endif

#endif /* PULSAR_ORACLE_H */
