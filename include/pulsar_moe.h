/* pulsar_moe.h - C ABI of the MI355X (gfx950) quantized expert-matvec library.
 *
 * Every entry point keeps the name, argument order, argument meaning and
 * return convention of the reference kernel library it replaces, so the
 * reference's Rust FFI block (crates/kernels/src/lib.rs:78-194) binds this
 * library unchanged:
 *   - return 1 on success, 0 on failure (invalid arguments or a launch error);
 *     the reason is printed as "pulsar-kernels: <what>: <error>" on stderr
 *     (crates/kernels/cuda/pulsar_kernels.cu:25-29);
 *   - every pointer argument except the self-tests' is a DEVICE pointer the
 *     caller owns; the library allocates nothing on these paths;
 *   - launches are asynchronous on the calling thread's per-thread default
 *     stream (hipStreamPerThread), the stream the reference's
 *     --default-stream=per-thread build launches on
 *     (crates/kernels/build.rs:42-48), so a thread-local graph capture begun
 *     on it records them; pulsar_set_stream selects another stream. Nothing
 *     here synchronises.
 *
 * Byte layouts are the GGUF/ggml ones (crates/gguf/src/lib.rs:145-180):
 *   Q2_K 84 B / 256, Q4_K 144 B / 256, Q6_K 210 B / 256, IQ2_XXS 66 B / 256,
 *   MXFP4 17 B / 32 (rows pack whole 32-value blocks, not super-blocks),
 *   q8_K 292 B / 256.
 */
#ifndef PULSAR_MOE_H
#define PULSAR_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quant codes (crates/kernels/src/lib.rs:55-73; pulsar_kernels.cu:2649-2668),
 * every one the reference defines. Bytes per 256 values: Q2_K 84, IQ2_XXS 66,
 * Q4_K 144, Q5_K 176, Q6_K 210, Q3_K 110, IQ2_XS 74, IQ3_XXS 98, Q4_0 8 x 18,
 * Q5_1 8 x 24, Q8_0 8 x 34, IQ4_XS 136, MXFP4 8 x 17, IQ4_NL 8 x 18, IQ3_S
 * 110, IQ2_S 82, IQ1_S 50, NVFP4 4 x 36 (crates/gguf/src/lib.rs:145-172). */
#define PULSAR_QUANT_Q2_K     0u
#define PULSAR_QUANT_IQ2_XXS  1u
#define PULSAR_QUANT_Q4_K     2u
#define PULSAR_QUANT_Q5_K     3u
#define PULSAR_QUANT_Q6_K     4u
#define PULSAR_QUANT_Q3_K     5u
#define PULSAR_QUANT_IQ2_XS   6u
#define PULSAR_QUANT_IQ3_XXS  7u
#define PULSAR_QUANT_Q4_0     8u
#define PULSAR_QUANT_Q5_1     9u
#define PULSAR_QUANT_Q8_0    10u
#define PULSAR_QUANT_IQ4_XS  11u
#define PULSAR_QUANT_MXFP4   12u
#define PULSAR_QUANT_IQ4_NL  13u
#define PULSAR_QUANT_IQ3_S   14u
#define PULSAR_QUANT_IQ2_S   15u
#define PULSAR_QUANT_IQ1_S   16u
#define PULSAR_QUANT_NVFP4   17u
/* OR'd into `quant` by callers that permit W4A4 (crates/kernels/src/lib.rs:51-55);
 * accepted and ignored here (it only selects an NVFP4 path in the reference). */
#define PULSAR_QUANT_A4_OK   0x80000000u

/* act_op codes of the gated combine (pulsar_kernels.cu:114-141) */
#define PULSAR_ACT_SILU        0u /* silu(g) * u */
#define PULSAR_ACT_SWIGLU_OAI  2u /* gpt-oss: clamp 7, alpha 1.702, (u + 1) */

#define PULSAR_QK_K 256u

/* q8_K activation block (pulsar_kernels.cu:1492-1496; lane Q8KRow,
 * crates/quant/src/cpu_dot.rs:19-23): d at byte 0, qs at 4, bsums at 260. */
typedef struct pulsar_block_q8_K {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} pulsar_block_q8_K;

/* Per-(token, slot) expert pointers (pulsar_kernels.cu:2555-2564;
 * crates/kernels/src/lib.rs:21-49). A NULL gate or up makes the pair stage
 * write 0 for that slot; a NULL down makes the down stage skip it; NULL
 * biases are skipped. gate_b/up_b hold mid_dim floats, down_b out_dim. */
typedef struct pulsar_expert_ptrs {
    const void *gate;
    const void *up;
    const void *down;
    const float *gate_b;
    const float *up_b;
    const float *down_b;
} pulsar_expert_ptrs;

#ifdef __cplusplus
static_assert(sizeof(pulsar_block_q8_K) == 292, "block_q8_K is 292 bytes");
static_assert(sizeof(pulsar_expert_ptrs) == 48, "pulsar_expert_ptrs is 48 bytes");
#else
_Static_assert(sizeof(pulsar_block_q8_K) == 292, "block_q8_K is 292 bytes");
_Static_assert(sizeof(pulsar_expert_ptrs) == 48, "pulsar_expert_ptrs is 48 bytes");
#endif

/* f32 rows [n_rows][in_dim] -> q8_K rows [n_rows][ceil(in_dim/256)].
 * Algorithm of the CPU lane (crates/quant/src/cpu_dot.rs:26-50): d = amax/127,
 * q = clamp(round_half_away(x * (127/amax)), -127, 127), bsums = 16-sums;
 * elements past in_dim in the tail block quantize to 0 (pulsar_kernels.cu:1499-1501).
 * Replaces pulsar_quantize_q8_K (pulsar_kernels.cu:1552). */
int pulsar_quantize_q8_K(void *out, const void *x, uint32_t in_dim, uint32_t n_rows);

/* out[t][r] = sum_b dot(w row r block b, xq[t] block b), fp32 [n_tok][out_dim].
 * quant: the reference's dense list (pulsar_kernels.cu:5090-5142) - Q2_K,
 * IQ2_XXS, Q4_K, Q5_K, Q6_K, Q3_K, IQ4_XS, IQ4_NL, NVFP4 (the expert-only
 * formats return 0, as there); in_dim % 256 == 0. 5 or more tokens on Q4_K,
 * Q5_K, Q6_K or NVFP4 run the int8 matrix-core GEMM.
 * Replaces pulsar_matmul_kq (pulsar_kernels.cu:4895). */
int pulsar_matmul_kq(void *out, const void *w, const void *xq, uint32_t in_dim,
                     uint32_t out_dim, uint32_t n_tok, uint64_t row_bytes,
                     uint32_t quant);

/* mid[t][s][r] = glu(gate_r . x_t + gate_b[r], up_r . x_t + up_b[r], act_op) * weights[t][s].
 * ptrs: pulsar_expert_ptrs[n_tok][n_used]; weights: f32 [n_tok][n_used];
 * xq: q8_K [n_tok][ceil(in_dim/256)]. Replaces pulsar_moe_pair_swiglu
 * (pulsar_kernels.cu:5149). */
int pulsar_moe_pair_swiglu(void *mid, const void *ptrs, const void *weights,
                           const void *xq, uint32_t in_dim, uint32_t mid_dim,
                           uint32_t n_used, uint32_t n_tok, uint64_t row_bytes,
                           uint32_t quant, uint32_t act_op);

/* out[t][r] = sum_s down_r(slot s) . midq[t][s], fp32 [n_tok][out_dim];
 * midq: q8_K [n_tok][n_used][ceil(mid_dim/256)]. Replaces pulsar_moe_down
 * (pulsar_kernels.cu:5289). */
int pulsar_moe_down(void *out, const void *ptrs, const void *midq,
                    uint32_t mid_dim, uint32_t out_dim, uint32_t n_used,
                    uint32_t n_tok, uint64_t row_bytes, uint32_t quant);

/* Grouped (CSR by expert) pair stage: gptrs [n_group], starts [n_group+1],
 * pairs [starts[n_group]] packing token << 4 | slot (n_used <= 16).
 * Writes mid[t][s][r] for every listed pair. Replaces
 * pulsar_moe_pair_swiglu_grouped (pulsar_kernels.cu:3483). */
int pulsar_moe_pair_swiglu_grouped(void *mid, const void *gptrs, const void *starts,
                                   const void *pairs, const void *weights,
                                   const void *xq, uint32_t in_dim, uint32_t mid_dim,
                                   uint32_t n_used, uint32_t n_group,
                                   uint64_t row_bytes, uint32_t quant,
                                   uint32_t act_op);

/* Grouped down stage: partial[t][s][r] = down_r(group of (t,s)) . midq[t][s]
 * for every listed pair; unlisted (t, s) are left untouched, so the caller
 * zeroes partial before every layer (crates/engine/src/lib.rs:8481-8482):
 * pulsar_moe_slot_sum reads every slot. Replaces pulsar_moe_down_grouped
 * (pulsar_kernels.cu:3537). */
int pulsar_moe_down_grouped(void *partial, const void *gptrs, const void *starts,
                            const void *pairs, const void *midq, uint32_t mid_dim,
                            uint32_t out_dim, uint32_t n_used, uint32_t n_group,
                            uint64_t row_bytes, uint32_t quant);

/* out[t][r] = sum_s partial[t][s][r] in slot order. Replaces
 * pulsar_moe_slot_sum (pulsar_kernels.cu:3651). */
int pulsar_moe_slot_sum(void *out, const void *partial, uint32_t out_dim,
                        uint32_t n_used, uint32_t n_tok);

/* out[t][r] += sum_s weights[t][s] * down_b(slot s)[r] (slots with a NULL
 * down_b skipped; nothing added where the sum is 0). Replaces
 * pulsar_moe_down_bias (pulsar_kernels.cu:3640). */
int pulsar_moe_down_bias(void *out, const void *ptrs, const void *weights,
                         uint32_t out_dim, uint32_t n_used, uint32_t n_tok);

/* Router top-k (pulsar_kernels.cu:938-1050): selected int32 and weights f32
 * [n_tok][k_used(+n_shexp)] from logits f32 [n_tok][n_expert(+n_shexp)].
 * mode 0 sigmoid + bias, normalised; mode 1 softmax over the k winners
 * (selection on raw logit + bias); mode 2 sigmoid+bias selection with the
 * shared "sink" logits appended, weights softmax(logsigmoid). Ties go to the
 * lower expert index. n_expert(+n_shexp) <= 1024. Replaces
 * pulsar_router_select (pulsar_kernels.cu:1052). */
int pulsar_router_select(void *selected, void *weights, const void *logits,
                         const void *bias, uint32_t n_expert, uint32_t k_used,
                         float weight_scale, uint32_t n_tok, uint32_t softmax_mode,
                         uint32_t n_shexp);

/* out[t][o] = sum_i w[o][i] * x[t][i] in fp32 (router logits). Replaces
 * pulsar_matmul_f32 (pulsar_kernels.cu:6526). */
int pulsar_matmul_f32(void *out, const void *w, const void *x, uint32_t in_dim,
                      uint32_t out_dim, uint32_t n_tok);

/* x[r][i] += bias[i] for rows rows of dim floats. Replaces
 * pulsar_add_bias_rows (pulsar_kernels.cu:3631). */
int pulsar_add_bias_rows(void *x, const void *bias, uint32_t dim, uint32_t rows);

/* ---- device-side routing (no counterpart entry point in the reference) ----
 * The reference builds the per-(token, slot) pointer array and the grouped
 * CSR on the host after reading the router's ids back
 * (crates/engine/src/lib.rs:7663-7670, 8255-8344, 8357-8392). These two
 * entry points do the same on the device, so a layer needs no host round
 * trip. */

/* One resident expert bank per projection: expert e's matrix starts at
 * base + e * stride bytes; its bias (NULL base = none) at b_base + e * b_stride
 * floats. Passed by host pointer, read at launch. */
typedef struct pulsar_expert_bank {
    const void *gate;
    const void *up;
    const void *down;
    const float *gate_b;
    const float *up_b;
    const float *down_b;
    uint64_t gate_stride;
    uint64_t up_stride;
    uint64_t down_stride;
    uint64_t gate_b_stride;
    uint64_t up_b_stride;
    uint64_t down_b_stride;
} pulsar_expert_bank;

/* ptrs[t][s] / slot_weights[t][s] for s < k_used from the router's
 * selected ids and weights ([n_tok][k_used]); an id outside [0, n_expert)
 * gives a NULL slot. Then n_shared always-on slots (s = k_used + i) with
 * pointers shared[i] (host array) and weight 1. Row stride of both outputs
 * is k_used + n_shared. Replaces the host pointer build at
 * crates/engine/src/lib.rs:8255-8344. */
int pulsar_moe_route_ptrs(void *ptrs, void *slot_weights, const void *selected,
                          const void *router_weights, const pulsar_expert_bank *bank,
                          uint32_t n_expert, const pulsar_expert_ptrs *shared,
                          uint32_t n_shared, uint32_t n_tok, uint32_t k_used);

/* Groups the (token, slot) pairs of ptrs [n_tok][n_used] by expert (equal
 * gate pointer, groups in order of first appearance, members in (token,
 * slot) order; NULL gates skipped), as crates/engine/src/lib.rs:8357-8392
 * does on the host. Writes gptrs [max_groups], starts [max_groups + 1] and
 * pairs (token << 4 | slot); group slots past the real count get NULL
 * pointers and empty ranges, so the grouped kernels can always be launched
 * with n_group = max_groups (which must be at least the number of distinct
 * experts, e.g. min(n_expert, n_tok * n_used)). n_used <= 16,
 * n_tok * n_used <= 2048. */
int pulsar_moe_group_csr(void *gptrs, void *starts, void *pairs, const void *ptrs,
                         uint32_t n_tok, uint32_t n_used, uint32_t max_groups);

/* pulsar_router_select (softmax_mode 0 or 1, no sink slots) +
 * pulsar_moe_route_ptrs + pulsar_moe_group_csr in one launch (no reference
 * counterpart: the reference selects on the device, then builds pointers
 * and the CSR on the host, crates/engine/src/lib.rs:7663-7670,
 * 8255-8392). Outputs equal those three calls': selected / weights
 * [n_tok][k_used], ptrs / slot_weights [n_tok][k_used + n_shared], gptrs,
 * starts, pairs. k_used + n_shared <= 16, n_tok * (k_used + n_shared) <=
 * 2048, k_used <= n_expert <= 1024; bank and shared are host pointers read
 * at launch. */
int pulsar_moe_route_group(void *selected, void *weights, void *ptrs, void *slot_weights,
                           void *gptrs, void *starts, void *pairs, const void *logits,
                           const void *router_bias, uint32_t n_expert, uint32_t k_used,
                           float weight_scale, uint32_t softmax_mode,
                           const pulsar_expert_bank *bank, const pulsar_expert_ptrs *shared,
                           uint32_t n_shared, uint32_t n_tok, uint32_t max_groups);

/* pulsar_router_select (softmax_mode 0 or 1, no sink slots) +
 * pulsar_moe_route_ptrs in one launch (no reference counterpart: the
 * reference selects on the device and builds the pointers on the host,
 * crates/engine/src/lib.rs:7663-7670, 8255-8344). Outputs equal those two
 * calls': selected / weights [n_tok][k_used], ptrs / slot_weights
 * [n_tok][k_used + n_shared]. It also writes active, uint32 [2 + n_expert]
 * (the grouped stages below may read all of it): active[0] = the number of
 * distinct experts the chunk selects,
 * active[1] = the number of NULL slots (ids outside [0, n_expert)),
 * active[2 ..] = the selected expert ids in order of first appearance in
 * (token, slot) order; the expert-indexed grouped stages below read it.
 * k_used + n_shared <= 16, k_used <= n_expert <= 1024, n_tok * (k_used +
 * n_shared) <= 2048; bank and shared are host pointers read at launch. */
int pulsar_moe_route(void *selected, void *weights, void *ptrs, void *slot_weights, void *active,
                     const void *logits, const void *router_bias, uint32_t n_expert, uint32_t k_used,
                     float weight_scale, uint32_t softmax_mode, const pulsar_expert_bank *bank,
                     const pulsar_expert_ptrs *shared, uint32_t n_shared, uint32_t n_tok);

/* The grouped stages with one group per expert the chunk selects, found
 * on the device from pulsar_moe_route's selected and active outputs
 * instead of a CSR (no reference counterpart: the reference groups on the
 * host, crates/engine/src/lib.rs:8357-8392). Each routed (token, slot)
 * pair runs in the group of its expert, shared slot i (s = k_used + i,
 * weight 1) of every token in a group of its own, exactly as
 * pulsar_moe_pair_swiglu_grouped / pulsar_moe_down_grouped would for the
 * same pairs, so the rows they write are bit-identical to those calls'.
 * Slots whose id is outside [0, n_expert) get rows of 0 in mid (partial),
 * so every row of mid [n_tok][k_used + n_shared][mid_dim] (partial
 * [..][out_dim]) is written and partial needs no zeroing. slot_weights
 * [n_tok][k_used + n_shared]. k_used + n_shared <= 16, n_tok * (k_used +
 * n_shared) <= 2048, n_expert <= 1024; bank and shared are host pointers. */
int pulsar_moe_pair_swiglu_experts(void *mid, const void *selected, const void *active,
                                   const void *slot_weights, const void *xq, const pulsar_expert_bank *bank,
                                   uint32_t n_expert, const pulsar_expert_ptrs *shared, uint32_t n_shared,
                                   uint32_t n_tok, uint32_t k_used, uint32_t in_dim, uint32_t mid_dim,
                                   uint64_t row_bytes, uint32_t quant, uint32_t act_op);
int pulsar_moe_down_experts(void *partial, const void *selected, const void *active, const void *midq,
                            const pulsar_expert_bank *bank, uint32_t n_expert, const pulsar_expert_ptrs *shared,
                            uint32_t n_shared, uint32_t n_tok, uint32_t k_used, uint32_t mid_dim,
                            uint32_t out_dim, uint64_t row_bytes, uint32_t quant);

/* pulsar_moe_slot_sum + pulsar_moe_down_bias in one launch (no reference
 * counterpart; the same sums in the same order, bit-identical to the two
 * calls). */
int pulsar_moe_slot_sum_bias(void *out, const void *partial, const void *ptrs,
                             const void *weights, uint32_t out_dim, uint32_t n_used,
                             uint32_t n_tok);

/* Self-checks: small device runs of the entry points compared with host
 * mirrors (q8_K bit-exact; every stage of the MoE path for Q2_K, IQ2_XXS,
 * Q4_K, Q6_K and MXFP4; router modes 0, 1 and 2). They allocate and
 * synchronise, print one line per case to stderr and return 1 when all pass.
 * Replace pulsar_kernels.cu:6421-6460 and 1271-1285. */
int pulsar_moe_selftest(void);
int pulsar_router_selftest(void);

/* ---- fused decode layer (no reference counterpart: the reference runs
 * these steps as separate launches with a host round trip in between,
 * crates/engine/src/lib.rs:7663-7670, 8416-8510). Each call produces
 * exactly the bytes of the separate calls it replaces. */

/* pulsar_matmul_f32(logits, w_r, x) [+ pulsar_add_bias_rows(logits, bias)
 * when bias != NULL] + pulsar_quantize_q8_K(xq, x, in_dim, n_tok), one
 * launch. */
int pulsar_router_logits_q8(void *logits, void *xq, const void *x, const void *w_r,
                            const void *bias, uint32_t in_dim, uint32_t n_expert,
                            uint32_t n_tok);

/* pulsar_router_select (softmax_mode 0 or 1, no sink slots) +
 * pulsar_moe_route_ptrs + pulsar_moe_pair_swiglu, one launch: every block
 * routes its token itself. Writes selected / weights [n_tok][k_used],
 * ptrs / slot_weights [n_tok][k_used + n_shared] and mid
 * [n_tok][k_used + n_shared][mid_dim]. k_used + n_shared <= 64,
 * n_shared <= 4; bank and shared are host pointers read at launch. */
int pulsar_moe_pair_routed(void *mid, void *ptrs, void *slot_weights, void *selected,
                           void *weights, const void *logits, const void *router_bias,
                           uint32_t n_expert, uint32_t k_used, float weight_scale,
                           uint32_t softmax_mode, const pulsar_expert_bank *bank,
                           const pulsar_expert_ptrs *shared, uint32_t n_shared,
                           const void *xq, uint32_t in_dim, uint32_t mid_dim, uint32_t n_tok,
                           uint64_t row_bytes, uint32_t quant, uint32_t act_op);

/* pulsar_quantize_q8_K(midq, mid, mid_dim, n_tok * n_used) +
 * pulsar_moe_down(out, ptrs, midq, ...) [+ pulsar_moe_down_bias(out, ptrs,
 * slot_weights) when add_bias], one launch; mid is f32
 * [n_tok][n_used][mid_dim]. The token's staged q8_K rows must fit 64 KiB
 * (n_used * ceil(mid_dim / 256) <= 215). */
int pulsar_moe_down_f32(void *out, const void *ptrs, const void *slot_weights, const void *mid,
                        uint32_t mid_dim, uint32_t out_dim, uint32_t n_used, uint32_t n_tok,
                        uint64_t row_bytes, uint32_t quant, uint32_t add_bias);

/* pulsar_moe_down + pulsar_moe_down_bias(out, ptrs, weights), one launch. */
int pulsar_moe_down_biased(void *out, const void *ptrs, const void *weights, const void *midq,
                           uint32_t mid_dim, uint32_t out_dim, uint32_t n_used, uint32_t n_tok,
                           uint64_t row_bytes, uint32_t quant);

/* Selects the stream every later launch from the calling thread goes to
 * (NULL restores the per-thread default stream, the default). No
 * counterpart in the reference, whose launches always use the per-thread
 * default stream (crates/kernels/build.rs:42-48); it lets a caller capture
 * the path into a graph on a stream of its own. Returns 1. */
int pulsar_set_stream(void *stream);

/* Streaming-read probe: reads `bytes` (a multiple of 16) from buf through
 * the compute units; `sink` receives nothing unless the data sums to an
 * impossible value. Replaces pulsar_bw_read (pulsar_kernels.cu:4889). */
int pulsar_bw_read(void *buf, uint64_t bytes, void *sink);

#ifdef __cplusplus
}
#endif

#endif /* PULSAR_MOE_H */
