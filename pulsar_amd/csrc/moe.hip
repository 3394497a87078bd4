// moe.hip - routed-expert FFN stages on q8_K activations.
//
// Plain path (per (token, slot) expert pointers, pulsar_kernels.cu:2566-2647):
//   pair : one block per (row group, slot, token); each wave streams the
//          gate and the up rows of its rows once and applies the combine
//          and the router weight;
//   down : one block per (row group, token); the block's 4 waves split the
//          token's slots, each slot's row dot lands in LDS and the slots
//          are summed in slot order.
// Grouped path (pulsar_kernels.cu:2689-2789): one block per (row block,
// expert group). Groups come from the CSR of moe_group_csr / route_group
// (CsrGroups) or straight from the router's selected ids and the touched-
// expert list of pulsar_moe_route (ExpertGroups). Q2_K, IQ2_XXS, MXFP4,
// Q4_K, Q5_K and Q6_K experts run on the int8 matrix cores (mmq.hip); the
// other formats here: the group's pair activations are staged in LDS once,
// and each wave streams row passes of the expert, dotting each pass with
// every pair.
#include "pk_rowdot.h"
#include "pk_route.h"

namespace pk {

constexpr uint32_t kWaves = 4;      // waves per block
#ifndef PK_PAIR_ONE_ROUND
#define PK_PAIR_ONE_ROUND 2048u
#endif
constexpr uint32_t kPairOneRoundBlocks = PK_PAIR_ONE_ROUND;
constexpr uint32_t kSlotChunk = 32; // down-stage slots staged in LDS per round


// One block per (RPW row-pass groups, slot, token); each wave takes RPW
// consecutive passes, the next pass's loads in flight while one is
// computed. NPL > 0: MXFP4 rows staged through LDS (SpanStage).
template <uint32_t Q, uint32_t UPLMAX, uint32_t NPL, uint32_t RPW>
__global__ __launch_bounds__(256) void moe_pair_kernel(float *__restrict__ mid,
                                                       const pulsar_expert_ptrs *__restrict__ ptrs,
                                                       const float *__restrict__ weights,
                                                       const pulsar_block_q8_K *__restrict__ xq,
                                                       uint32_t n_units, uint32_t nblk32,
                                                       uint32_t lpr_log2, uint32_t in_blocks,
                                                       uint32_t mid_dim, uint32_t n_used,
                                                       uint64_t row_bytes, uint32_t act_op) {
    PK_FMT_LUT(Q)
    const uint32_t slot = blockIdx.y, token = blockIdx.z;
    const uint64_t so = (uint64_t)token * n_used + slot;
    const pulsar_expert_ptrs p = ptrs[so];
    const RowGeom rg = row_geom(n_units, nblk32, lpr_log2);
    const uint32_t rpp = 64u >> lpr_log2;
    const uint32_t pass0 = (blockIdx.x * kWaves + threadIdx.x / 64u) * RPW;
    if (!p.gate || !p.up) {  // unrouted slot contributes zero (pulsar_kernels.cu:2587-2590)
#pragma unroll
        for (uint32_t k = 0; k < RPW; k++) {
            const uint32_t row = (pass0 + k) * rpp + rg.rip;
            if (row < mid_dim && rg.holds_row()) mid[so * mid_dim + row] = 0.0f;
        }
        return;
    }
    Act a[UPLMAX];
    load_row_acts<Q, UPLMAX>(xq + (uint64_t)token * in_blocks, rg, a);
    pair_passes<Q, UPLMAX, NPL, RPW>(mid + so * mid_dim, p, weights[so], a, rg, pass0, mid_dim, row_bytes, act_op,
                                     lut);
}

// BIAS: the row total then gets sum_s weights[s] * down_b_s[row] added when
// that sum is non-zero, as moe_down_bias does after the down stage.
template <uint32_t Q, uint32_t UPLMAX, uint32_t NPL, bool BIAS>
__global__ __launch_bounds__(256) void moe_down_kernel(float *__restrict__ out,
                                                       const pulsar_expert_ptrs *__restrict__ ptrs,
                                                       const pulsar_block_q8_K *__restrict__ midq,
                                                       uint32_t n_units, uint32_t nblk32,
                                                       uint32_t lpr_log2, uint32_t mid_blocks,
                                                       uint32_t out_dim, uint32_t n_used,
                                                       uint64_t row_bytes, const float *__restrict__ weights) {
    PK_FMT_LUT(Q)
    __shared__ float part[kSlotChunk][16];
    __shared__ float bpart[BIAS ? kSlotChunk : 1][16];
    const uint32_t token = blockIdx.y;
    const uint32_t wave = threadIdx.x / 64u;
    const RowGeom rg = row_geom(n_units, nblk32, lpr_log2);
    const uint32_t rpp = 64u >> lpr_log2;
    const uint32_t row = blockIdx.x * rpp + rg.rip;
    const bool row_ok = row < out_dim;
    float total = 0.0f, b = 0.0f;
    for (uint32_t base = 0; base < n_used; base += kSlotChunk) {
        const uint32_t end = base + kSlotChunk < n_used ? base + kSlotChunk : n_used;
        for (uint32_t s = base + wave; s < end; s += kWaves) {
            const uint64_t so = (uint64_t)token * n_used + s;
            const pulsar_expert_ptrs p = ptrs[so];
            // the slot's bias term w_s down_b_s[row], requested with the
            // slot's weights (a NULL bias adds +0, which leaves the bias sum,
            // never -0, as skipping it would)
            float bt = 0.0f;
            if (BIAS && p.down_b) bt = weights[so] * ldwf(p.down_b + (row_ok ? row : 0u));
            // -0.0 is the additive identity for every float, so a skipped
            // slot (NULL down, pulsar_kernels.cu:2635) leaves the sum as is
            float v = -0.0f;
            if (p.down) {
                Act a[UPLMAX];
                load_row_acts<Q, UPLMAX>(midq + so * mid_blocks, rg, a);
                typename Fmt<Q>::W w[UPLMAX];
                load_one_row<Q, UPLMAX, NPL>(as_global(p.down) + (uint64_t)(row_ok ? row : 0u) * row_bytes, rg, w);
                v = row_finish(row_partial<Q, UPLMAX>(row_ok, rg, w, a, lut), rg);
            }
            if (rg.holds_row()) {
                part[s - base][rg.rip] = v;
                if (BIAS) bpart[s - base][rg.rip] = bt;
            }
        }
        __syncthreads();
        if (wave == 0 && rg.holds_row())
            for (uint32_t s = base; s < end; s++) {
                total += part[s - base][rg.rip];
                if (BIAS) b += bpart[s - base][rg.rip];  // slot order, as moe_down_bias sums
            }
        __syncthreads();
    }
    if (wave == 0 && rg.holds_row() && row_ok) {
        if (BIAS && b != 0.0f) total += b;
        out[(uint64_t)token * out_dim + row] = total;
    }
}

#ifndef PK_GRP_PPW
#define PK_GRP_PPW 8u  // row passes per wave in the grouped kernels
#endif
constexpr uint32_t kGrpActLds = 32768u;  // LDS bytes for a group's staged activations
constexpr uint32_t kGrpMaxPairs = 16u;   // pairs staged per round

// Copies the q8_K rows of pairs [c0, c0 + np) into LDS (load_act_lds
// layout, `blocks` super-blocks per row) and their pair ids into pr_l.
// DOWN: the row is the (token, slot)'s mid row, else the token's row.
// Ends with a block barrier.
template <bool DOWN, typename G>
PK_DEV void stage_pair_acts(uint8_t *acts, uint32_t *pr_l, const G &grp, const uint32_t *lst, uint32_t c0,
                            uint32_t np, const pulsar_block_q8_K *src, uint32_t blocks, uint32_t n_used) {
    for (uint32_t j = threadIdx.x; j < np; j += blockDim.x) pr_l[j] = grp.pair(c0 + j, lst);
    __syncthreads();
    stage_q8_rows<2>(acts, np, blocks, blocks * kActLdsPitch, [&](uint32_t j) {
        const uint32_t pr = pr_l[j];
        const uint64_t row = DOWN ? (uint64_t)(pr >> 4) * n_used + (pr & 15u) : (uint64_t)(pr >> 4);
        return src + row * blocks;
    });
    __syncthreads();
}

// The NULL group's pairs (ExpertGroups): output rows [r0, r0 + nr) of each
// written as 0.
template <typename G>
PK_DEV void zero_group_rows(float *out, const G &grp, const uint32_t *lst, uint32_t s0, uint32_t s1, uint32_t r0,
                            uint32_t nr, uint32_t n_rows, uint32_t n_used) {
    for (uint32_t it = threadIdx.x; it < (s1 - s0) * nr; it += blockDim.x) {
        const uint32_t pr = grp.pair(s0 + it / nr, lst), row = r0 + it % nr;
        if (row < n_rows) out[((uint64_t)(pr >> 4) * n_used + (pr & 15u)) * n_rows + row] = 0.0f;
    }
}

// Grouped kernels: one block per (row block, expert group). The group's
// pair activations are staged in LDS once (in rounds of `pmax` pairs);
// every wave streams PK_GRP_PPW row passes of the expert, the next pass's
// weight loads issued before the current pass is dotted with each pair.
template <uint32_t Q, uint32_t UPLMAX, typename G>
__global__ __launch_bounds__(256) void moe_pair_grouped_kernel(
        float *__restrict__ mid, const G grp, const float *__restrict__ weights,
        const pulsar_block_q8_K *__restrict__ xq, uint32_t n_units, uint32_t nblk32, uint32_t lpr_log2,
        uint32_t in_blocks, uint32_t mid_dim, uint32_t n_used, uint64_t row_bytes, uint32_t act_op, uint32_t pmax,
        uint32_t lst_off) {
    PK_FMT_LUT(Q)
    extern __shared__ __align__(16) uint8_t acts_lds[];
    __shared__ uint32_t pr_l[kGrpMaxPairs];
    const uint32_t group = blockIdx.y;
    const typename G::Group gr = grp.group(group);
    const pulsar_expert_ptrs &p = gr.p;
    const bool nul = gr.is_null();
    if (!nul && (!p.gate || !p.up)) return;
    uint32_t *lst = (uint32_t *)(acts_lds + lst_off);
    uint32_t s0, s1;
    grp.range(gr, lst, s0, s1);
    if (s0 >= s1) return;
    const RowGeom rg = row_geom(n_units, nblk32, lpr_log2);
    const uint32_t rpp = 64u >> lpr_log2;
    const uint32_t n_pass = (mid_dim + rpp - 1u) / rpp;
    if (nul) {
        const uint32_t nr = kWaves * PK_GRP_PPW * rpp;
        zero_group_rows(mid, grp, lst, s0, s1, blockIdx.x * nr, nr, mid_dim, n_used);
        return;
    }
    const uint32_t pass0 = (blockIdx.x * kWaves + threadIdx.x / 64u) * PK_GRP_PPW;
    const uint32_t act_bytes = in_blocks * kActLdsPitch;
    auto row_of = [&](uint32_t pass) {
        const uint32_t row = pass * rpp + rg.rip;
        return row < mid_dim ? row : 0u;
    };
    typename Fmt<Q>::W wg[UPLMAX], wu[UPLMAX];
    load_row_w<Q, UPLMAX>(as_global(p.gate) + (uint64_t)row_of(pass0) * row_bytes, rg, wg);
    load_row_w<Q, UPLMAX>(as_global(p.up) + (uint64_t)row_of(pass0) * row_bytes, rg, wu);
    for (uint32_t c0 = s0; c0 < s1; c0 += pmax) {
        const uint32_t np = s1 - c0 < pmax ? s1 - c0 : pmax;
        if (c0 != s0) {
            __syncthreads();  // the previous round's activations are consumed
            load_row_w<Q, UPLMAX>(as_global(p.gate) + (uint64_t)row_of(pass0) * row_bytes, rg, wg);
            load_row_w<Q, UPLMAX>(as_global(p.up) + (uint64_t)row_of(pass0) * row_bytes, rg, wu);
        }
        stage_pair_acts<false>(acts_lds, pr_l, grp, lst, c0, np, xq, in_blocks, n_used);
        for (uint32_t k = 0; k < PK_GRP_PPW; k++) {
            const uint32_t pass = pass0 + k;
            if (pass >= n_pass) break;  // wave-uniform
            const bool more = k + 1u < PK_GRP_PPW && pass + 1u < n_pass;
            typename Fmt<Q>::W ng[UPLMAX], nu[UPLMAX];
            if (more) {
                load_row_w<Q, UPLMAX>(as_global(p.gate) + (uint64_t)row_of(pass + 1u) * row_bytes, rg, ng);
                load_row_w<Q, UPLMAX>(as_global(p.up) + (uint64_t)row_of(pass + 1u) * row_bytes, rg, nu);
            }
            const uint32_t row = pass * rpp + rg.rip;
            const bool row_ok = row < mid_dim;
            const float gb = row_ok && p.gate_b ? ldwf(p.gate_b + row) : 0.0f;
            const float ub = row_ok && p.up_b ? ldwf(p.up_b + row) : 0.0f;
            for (uint32_t j = 0; j < np; j++) {
                const uint32_t pr = pr_l[j];
                const uint64_t so = (uint64_t)(pr >> 4) * n_used + (pr & 15u);
#pragma unroll
                for (uint32_t i = 0; i < UPLMAX; i++) {
                    opaque(wg[i]);
                    opaque(wu[i]);
                }
                Act a[UPLMAX];
                load_row_acts_lds<Q, UPLMAX>(acts_lds + j * act_bytes, rg, a);
                float g = row_finish(row_partial<Q, UPLMAX>(row_ok, rg, wg, a, lut), rg);
                float u = row_finish(row_partial<Q, UPLMAX>(row_ok, rg, wu, a, lut), rg);
                if (row_ok && rg.holds_row()) {
                    if (p.gate_b) g += gb;
                    if (p.up_b) u += ub;
                    mid[so * mid_dim + row] = glu(g, u, act_op) * weights[so];
                }
            }
            if (more) {
#pragma unroll
                for (uint32_t i = 0; i < UPLMAX; i++) {
                    wg[i] = ng[i];
                    wu[i] = nu[i];
                }
            }
        }
    }
}

template <uint32_t Q, uint32_t UPLMAX, typename G>
__global__ __launch_bounds__(256) void moe_down_grouped_kernel(
        float *__restrict__ partial, const G grp, const pulsar_block_q8_K *__restrict__ midq, uint32_t n_units,
        uint32_t nblk32, uint32_t lpr_log2, uint32_t mid_blocks, uint32_t out_dim, uint32_t n_used,
        uint64_t row_bytes, uint32_t pmax, uint32_t lst_off) {
    PK_FMT_LUT(Q)
    extern __shared__ __align__(16) uint8_t acts_lds[];
    __shared__ uint32_t pr_l[kGrpMaxPairs];
    const uint32_t group = blockIdx.y;
    const typename G::Group gr = grp.group(group);
    const pulsar_expert_ptrs &p = gr.p;
    const bool nul = gr.is_null();
    if (!nul && !p.down) return;
    uint32_t *lst = (uint32_t *)(acts_lds + lst_off);
    uint32_t s0, s1;
    grp.range(gr, lst, s0, s1);
    if (s0 >= s1) return;
    const RowGeom rg = row_geom(n_units, nblk32, lpr_log2);
    const uint32_t rpp = 64u >> lpr_log2;
    const uint32_t n_pass = (out_dim + rpp - 1u) / rpp;
    if (nul) {
        const uint32_t nr = kWaves * PK_GRP_PPW * rpp;
        zero_group_rows(partial, grp, lst, s0, s1, blockIdx.x * nr, nr, out_dim, n_used);
        return;
    }
    const uint32_t pass0 = (blockIdx.x * kWaves + threadIdx.x / 64u) * PK_GRP_PPW;
    const uint32_t act_bytes = mid_blocks * kActLdsPitch;
    auto row_of = [&](uint32_t pass) {
        const uint32_t row = pass * rpp + rg.rip;
        return row < out_dim ? row : 0u;
    };
    typename Fmt<Q>::W w[UPLMAX];
    load_row_w<Q, UPLMAX>(as_global(p.down) + (uint64_t)row_of(pass0) * row_bytes, rg, w);
    for (uint32_t c0 = s0; c0 < s1; c0 += pmax) {
        const uint32_t np = s1 - c0 < pmax ? s1 - c0 : pmax;
        if (c0 != s0) {
            __syncthreads();
            load_row_w<Q, UPLMAX>(as_global(p.down) + (uint64_t)row_of(pass0) * row_bytes, rg, w);
        }
        stage_pair_acts<true>(acts_lds, pr_l, grp, lst, c0, np, midq, mid_blocks, n_used);
        for (uint32_t k = 0; k < PK_GRP_PPW; k++) {
            const uint32_t pass = pass0 + k;
            if (pass >= n_pass) break;  // wave-uniform
            const bool more = k + 1u < PK_GRP_PPW && pass + 1u < n_pass;
            typename Fmt<Q>::W nw[UPLMAX];
            if (more) load_row_w<Q, UPLMAX>(as_global(p.down) + (uint64_t)row_of(pass + 1u) * row_bytes, rg, nw);
            const uint32_t row = pass * rpp + rg.rip;
            const bool row_ok = row < out_dim;
            for (uint32_t j = 0; j < np; j++) {
                const uint32_t pr = pr_l[j];
                const uint64_t so = (uint64_t)(pr >> 4) * n_used + (pr & 15u);
#pragma unroll
                for (uint32_t i = 0; i < UPLMAX; i++) opaque(w[i]);
                Act a[UPLMAX];
                load_row_acts_lds<Q, UPLMAX>(acts_lds + j * act_bytes, rg, a);
                const float v = row_finish(row_partial<Q, UPLMAX>(row_ok, rg, w, a, lut), rg);
                if (row_ok && rg.holds_row()) partial[so * out_dim + row] = v;
            }
            if (more) {
#pragma unroll
                for (uint32_t i = 0; i < UPLMAX; i++) w[i] = nw[i];
            }
        }
    }
}

// Pairs staged per round for rows of `blocks` super-blocks.
static uint32_t grouped_pmax(uint32_t blocks) {
    const uint32_t per = blocks * kActLdsPitch;
    uint32_t pm = kGrpActLds / per;
    if (pm < 1u) pm = 1u;
    return pm < kGrpMaxPairs ? pm : kGrpMaxPairs;
}

// Deterministic slot reduce (pulsar_kernels.cu:2791-2806).
constexpr uint32_t kSumBatch = 8;
__global__ __launch_bounds__(256) void slot_sum_kernel(float *__restrict__ out,
                                                       const float *__restrict__ partial,
                                                       uint32_t out_dim, uint32_t n_used,
                                                       uint64_t total) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const uint64_t token = gid / out_dim;
    const uint64_t row = gid - token * out_dim;
    float acc = 0.0f;
    for (uint32_t s0 = 0; s0 < n_used; s0 += kSumBatch) {  // a batch's loads issued before its adds
        float pv[kSumBatch];
#pragma unroll
        for (uint32_t j = 0; j < kSumBatch; j++)
            pv[j] = partial[(token * n_used + (s0 + j < n_used ? s0 + j : n_used - 1u)) * out_dim + row];
#pragma unroll
        for (uint32_t j = 0; j < kSumBatch; j++)
            if (s0 + j < n_used) acc += pv[j];
    }
    out[gid] = acc;
}

// sum_s w_s down_b_s[row] over the token's slots in slot order, NULL biases
// skipped (pulsar_kernels.cu:3601-3619). Slots are taken kB at a time with
// every load of the batch issued first: the slot records, then the bias
// values (a NULL bias reads a valid dummy address and is not added).
constexpr uint32_t kBiasBatch = 8;
PK_DEV float slot_bias_sum(const pulsar_expert_ptrs *__restrict__ ptrs, const float *__restrict__ weights,
                           uint64_t token, uint32_t n_used, uint64_t row) {
    float b = 0.0f;
    for (uint32_t s0 = 0; s0 < n_used; s0 += kBiasBatch) {
        const float *db[kBiasBatch];
        float wv[kBiasBatch], bv[kBiasBatch];
#pragma unroll
        for (uint32_t j = 0; j < kBiasBatch; j++) {
            const uint64_t so = token * n_used + (s0 + j < n_used ? s0 + j : n_used - 1u);
            db[j] = ptrs[so].down_b;
            wv[j] = weights[so];
        }
#pragma unroll
        for (uint32_t j = 0; j < kBiasBatch; j++) bv[j] = ldwf(db[j] ? db[j] + row : weights + token * n_used);
#pragma unroll
        for (uint32_t j = 0; j < kBiasBatch; j++)
            if (s0 + j < n_used && db[j]) b += wv[j] * bv[j];
    }
    return b;
}

// slot_sum_kernel then down_bias_kernel in one pass: the same two sums in
// the same order, so the result is bit-identical to the two launches.
__global__ __launch_bounds__(256) void slot_sum_bias_kernel(float *__restrict__ out,
                                                            const float *__restrict__ partial,
                                                            const pulsar_expert_ptrs *__restrict__ ptrs,
                                                            const float *__restrict__ weights,
                                                            uint32_t out_dim, uint32_t n_used, uint64_t total) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const uint64_t token = gid / out_dim;
    const uint64_t row = gid - token * out_dim;
    float acc = 0.0f;
    for (uint32_t s0 = 0; s0 < n_used; s0 += kBiasBatch) {  // the partials of a batch loaded first
        float pv[kBiasBatch];
#pragma unroll
        for (uint32_t j = 0; j < kBiasBatch; j++)
            pv[j] = partial[(token * n_used + (s0 + j < n_used ? s0 + j : n_used - 1u)) * out_dim + row];
#pragma unroll
        for (uint32_t j = 0; j < kBiasBatch; j++)
            if (s0 + j < n_used) acc += pv[j];
    }
    const float b = slot_bias_sum(ptrs, weights, token, n_used, row);
    if (b != 0.0f) acc += b;
    out[gid] = acc;
}

// out += sum_s w_s * down_b_s (pulsar_kernels.cu:3601-3619).
__global__ __launch_bounds__(256) void down_bias_kernel(float *__restrict__ out,
                                                        const pulsar_expert_ptrs *__restrict__ ptrs,
                                                        const float *__restrict__ weights,
                                                        uint32_t out_dim, uint32_t n_used,
                                                        uint64_t total) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    const uint64_t token = gid / out_dim;
    const uint64_t row = gid - token * out_dim;
    const float b = slot_bias_sum(ptrs, weights, token, n_used, row);
    if (b != 0.0f) out[gid] += b;
}

// ------------------------------------------------------------ dispatch --

struct Geo {
    uint32_t n_units, nblk32, l2, upl, blocks;
};

static Geo geo_for(uint32_t quant, uint32_t k_dim) {
    Geo g;
    g.n_units = units_per_row(quant, k_dim);
    g.nblk32 = (k_dim + 31u) / 32u;
    g.l2 = lpr_log2_for(g.n_units);
    g.upl = (g.n_units + (1u << g.l2) - 1u) >> g.l2;
    g.blocks = (k_dim + 255u) / 256u;
    return g;
}

static bool quant_ok(uint32_t q) { return q <= PULSAR_QUANT_NVFP4; }

// Calls F::template run<Q, UPLMAX>() for the run-time (quant, upl);
// MAXU bounds the instantiated unit counts (the grouped kernels hold two
// weight rows in registers and would spill beyond 4 units per lane).
template <uint32_t MAXU, typename F>
static int with_format(uint32_t quant, uint32_t upl, F &&f) {
#define PK_UPL(Q)                                                   \
    if (upl <= 1u) return f.template run<Q, 1>();                   \
    if (upl <= 2u) return f.template run<Q, 2>();                   \
    if (upl <= 4u) return f.template run<Q, 4>();                   \
    if (MAXU >= 8u && upl <= 8u) return f.template run<Q, (MAXU >= 8u ? 8u : 4u)>(); \
    return reject("moe (row width above the supported maximum)");
#define PK_CASE(Q) \
    case Q: PK_UPL(Q)
    switch (quant) {
    PK_FOR_EACH_QUANT(PK_CASE)
    default: return reject("moe (quant)");
    }
#undef PK_CASE
#undef PK_UPL
}

struct PairLaunch {
    void *mid;
    const void *ptrs, *weights, *xq;
    uint32_t mid_dim, n_used, n_tok, act_op;
    uint64_t row_bytes;
    Geo g;
    template <uint32_t Q, uint32_t U>
    int run() {
        return with_stage<Q, U>(g, *this);
    }
    template <uint32_t Q, uint32_t U, uint32_t NPL>
    int go() {
        const uint32_t rpb = kWaves * (64u >> g.l2);
        // two passes per wave once the blocks would not all be resident at
        // once (8 per CU): then the waves run as one round
        const bool two = (uint64_t)((mid_dim + rpb - 1u) / rpb) * n_used * n_tok > kPairOneRoundBlocks;
        const uint32_t rpw = two ? 2u : 1u;
        const dim3 grid((mid_dim + rpw * rpb - 1u) / (rpw * rpb), n_used, n_tok);
#define PK_PAIR_GO(R)                                                                                          \
    hipLaunchKernelGGL((moe_pair_kernel<Q, U, NPL, R>), grid, dim3(256), 0, pk::stream(), (float *)mid,       \
                       (const pulsar_expert_ptrs *)ptrs, (const float *)weights, (const pulsar_block_q8_K *)xq, \
                       g.n_units, g.nblk32, g.l2, g.blocks, mid_dim, n_used, row_bytes, act_op)
        if (two)
            PK_PAIR_GO(2);
        else
            PK_PAIR_GO(1);
#undef PK_PAIR_GO
        return launch_ok("moe pair swiglu launch");
    }
};

struct DownLaunch {
    void *out;
    const void *ptrs, *midq;
    uint32_t out_dim, n_used, n_tok;
    uint64_t row_bytes;
    Geo g;
    const float *weights = nullptr;  // != NULL: bias epilogue (moe_down_kernel BIAS)
    template <uint32_t Q, uint32_t U>
    int run() {
        return with_stage<Q, U>(g, *this);
    }
    template <uint32_t Q, uint32_t U, uint32_t NPL>
    int go() {
        const uint32_t rpp = 64u >> g.l2;
        const dim3 grid((out_dim + rpp - 1u) / rpp, n_tok);
        if (weights)
            hipLaunchKernelGGL((moe_down_kernel<Q, U, NPL, true>), grid, dim3(256), 0, pk::stream(), (float *)out,
                               (const pulsar_expert_ptrs *)ptrs, (const pulsar_block_q8_K *)midq, g.n_units,
                               g.nblk32, g.l2, g.blocks, out_dim, n_used, row_bytes, weights);
        else
            hipLaunchKernelGGL((moe_down_kernel<Q, U, NPL, false>), grid, dim3(256), 0, pk::stream(), (float *)out,
                               (const pulsar_expert_ptrs *)ptrs, (const pulsar_block_q8_K *)midq, g.n_units,
                               g.nblk32, g.l2, g.blocks, out_dim, n_used, row_bytes, nullptr);
        return launch_ok("moe down launch");
    }
};

template <typename G>
struct PairGroupedLaunch {
    void *mid;
    G grp;
    const void *weights, *xq;
    uint32_t mid_dim, n_used, n_group, act_op;
    uint64_t row_bytes;
    Geo g;
    uint32_t lst_bytes;
    template <uint32_t Q, uint32_t U>
    int run() {
        const uint32_t rpb = kWaves * PK_GRP_PPW * (64u >> g.l2);
        const dim3 grid((mid_dim + rpb - 1u) / rpb, n_group);
        const uint32_t pmax = grouped_pmax(g.blocks);
        const uint32_t lst_off = pmax * g.blocks * kActLdsPitch;
        hipLaunchKernelGGL((moe_pair_grouped_kernel<Q, U, G>), grid, dim3(256), lst_off + lst_bytes, pk::stream(),
                           (float *)mid, grp, (const float *)weights, (const pulsar_block_q8_K *)xq, g.n_units,
                           g.nblk32, g.l2, g.blocks, mid_dim, n_used, row_bytes, act_op, pmax, lst_off);
        return launch_ok("moe pair swiglu grouped launch");
    }
};

template <typename G>
struct DownGroupedLaunch {
    void *partial;
    G grp;
    const void *midq;
    uint32_t out_dim, n_used, n_group;
    uint64_t row_bytes;
    Geo g;
    uint32_t lst_bytes;
    template <uint32_t Q, uint32_t U>
    int run() {
        const uint32_t rpb = kWaves * PK_GRP_PPW * (64u >> g.l2);
        const dim3 grid((out_dim + rpb - 1u) / rpb, n_group);
        const uint32_t pmax = grouped_pmax(g.blocks);
        const uint32_t lst_off = pmax * g.blocks * kActLdsPitch;
        hipLaunchKernelGGL((moe_down_grouped_kernel<Q, U, G>), grid, dim3(256), lst_off + lst_bytes, pk::stream(),
                           (float *)partial, grp, (const pulsar_block_q8_K *)midq, g.n_units, g.nblk32, g.l2,
                           g.blocks, out_dim, n_used, row_bytes, pmax, lst_off);
        return launch_ok("moe down grouped launch");
    }
};

}  // namespace pk

using namespace pk;

extern "C" int pulsar_moe_pair_swiglu(void *mid, const void *ptrs, const void *weights,
                                      const void *xq, uint32_t in_dim, uint32_t mid_dim,
                                      uint32_t n_used, uint32_t n_tok, uint64_t row_bytes,
                                      uint32_t quant, uint32_t act_op) {
    if (!mid || !ptrs || !weights || !xq || in_dim == 0 || mid_dim == 0 || n_used == 0 ||
        n_tok == 0 || row_bytes == 0 || (act_op != PULSAR_ACT_SILU && act_op != PULSAR_ACT_SWIGLU_OAI) ||
        n_used > 65535u || n_tok > 65535u)
        return reject("moe pair swiglu");
    const Geo g = geo_for(quant, in_dim);
    PairLaunch f{mid, ptrs, weights, xq, mid_dim, n_used, n_tok, act_op, row_bytes, g};
    if (!quant_ok(quant)) return reject("moe pair swiglu (quant)");
    return with_format<8>(quant, g.upl, f);
}

extern "C" int pulsar_moe_down(void *out, const void *ptrs, const void *midq, uint32_t mid_dim,
                               uint32_t out_dim, uint32_t n_used, uint32_t n_tok, uint64_t row_bytes,
                               uint32_t quant) {
    if (!out || !ptrs || !midq || mid_dim == 0 || out_dim == 0 || n_used == 0 || n_tok == 0 ||
        row_bytes == 0 || n_tok > 65535u)
        return reject("moe down");
    const Geo g = geo_for(quant, mid_dim);
    DownLaunch f{out, ptrs, midq, out_dim, n_used, n_tok, row_bytes, g};
    if (!quant_ok(quant)) return reject("moe down (quant)");
    return with_format<8>(quant, g.upl, f);
}

extern "C" int pulsar_moe_down_biased(void *out, const void *ptrs, const void *weights, const void *midq,
                                      uint32_t mid_dim, uint32_t out_dim, uint32_t n_used, uint32_t n_tok,
                                      uint64_t row_bytes, uint32_t quant) {
    quant &= ~PULSAR_QUANT_A4_OK;
    if (!out || !ptrs || !weights || !midq || mid_dim == 0 || out_dim == 0 || n_used == 0 || n_tok == 0 ||
        row_bytes == 0 || n_tok > 65535u)
        return reject("moe down biased");
    const Geo g = geo_for(quant, mid_dim);
    DownLaunch f{out, ptrs, midq, out_dim, n_used, n_tok, row_bytes, g};
    f.weights = (const float *)weights;
    if (!quant_ok(quant)) return reject("moe down biased (quant)");
    return with_format<8>(quant, g.upl, f);
}

// Grouped entry points keep the reference's argument contract
// (pulsar_kernels.cu:3488-3492, 3541-3547): in_dim (pair) and mid_dim (down)
// multiples of 256, n_used <= 16 (4-bit slot field in `pairs`).
namespace pk {
// mmq.hip: the grouped stages of Q2_K / IQ2_XXS / MXFP4 / Q4_K / Q5_K / Q6_K
// experts on the matrix cores; -1 for other formats
template <typename G>
int launch_grouped_mmq_kq(bool pair, uint32_t quant, float *out, const G &src, const float *weights,
                          const pulsar_block_q8_K *act, uint32_t k_dim, uint32_t n_rows, uint32_t n_used,
                          uint32_t n_group, uint64_t row_bytes, uint32_t act_op, uint32_t lst_bytes);
extern template int launch_grouped_mmq_kq<CsrGroups>(bool, uint32_t, float *, const CsrGroups &, const float *,
                                                     const pulsar_block_q8_K *, uint32_t, uint32_t, uint32_t,
                                                     uint32_t, uint64_t, uint32_t, uint32_t);
extern template int launch_grouped_mmq_kq<ExpertGroups>(bool, uint32_t, float *, const ExpertGroups &,
                                                        const float *, const pulsar_block_q8_K *, uint32_t, uint32_t,
                                                        uint32_t, uint32_t, uint64_t, uint32_t, uint32_t);

// The grouped gate / up stage for either group source: the matrix-core
// kernel where the format has one, else the lane kernels.
template <typename G>
static int pair_grouped(void *mid, const G &grp, const void *weights, const void *xq, uint32_t in_dim,
                        uint32_t mid_dim, uint32_t n_used, uint32_t n_group, uint64_t row_bytes, uint32_t quant,
                        uint32_t act_op, uint32_t lst_bytes) {
#ifndef PK_GRP_LANE_ONLY
    {
        const int r = launch_grouped_mmq_kq(true, quant, (float *)mid, grp, (const float *)weights,
                                            (const pulsar_block_q8_K *)xq, in_dim, mid_dim, n_used, n_group,
                                            row_bytes, act_op, lst_bytes);
        if (r >= 0) return r;
    }
#endif
    const Geo g = geo_for(quant, in_dim);
    PairGroupedLaunch<G> f{mid, grp, weights, xq, mid_dim, n_used, n_group, act_op, row_bytes, g, lst_bytes};
    if (!quant_ok(quant)) return reject("moe pair swiglu grouped (quant)");
    return with_format<4>(quant, g.upl, f);
}

template <typename G>
static int down_grouped(void *partial, const G &grp, const void *midq, uint32_t mid_dim, uint32_t out_dim,
                        uint32_t n_used, uint32_t n_group, uint64_t row_bytes, uint32_t quant, uint32_t lst_bytes) {
#ifndef PK_GRP_LANE_ONLY
    {
        const int r = launch_grouped_mmq_kq(false, quant, (float *)partial, grp, nullptr,
                                            (const pulsar_block_q8_K *)midq, mid_dim, out_dim, n_used, n_group,
                                            row_bytes, 0, lst_bytes);
        if (r >= 0) return r;
    }
#endif
    const Geo g = geo_for(quant, mid_dim);
    DownGroupedLaunch<G> f{partial, grp, midq, out_dim, n_used, n_group, row_bytes, g, lst_bytes};
    if (!quant_ok(quant)) return reject("moe down grouped (quant)");
    return with_format<4>(quant, g.upl, f);
}

// ExpertGroups from the entry points' arguments (bank and shared are host
// pointers read here).
static ExpertGroups expert_groups(const void *selected, const void *active, const pulsar_expert_bank *bank,
                                  uint32_t n_expert, const pulsar_expert_ptrs *shared, uint32_t n_shared,
                                  uint32_t n_tok, uint32_t k_used) {
    ExpertGroups G = {};
    G.sel = (const int32_t *)selected;
    G.active = (const uint32_t *)active;
    G.bank = *bank;
    for (uint32_t i = 0; i < n_shared; i++) G.shared.p[i] = shared[i];
    G.n_expert = n_expert;
    G.k_used = k_used;
    G.n_shared = n_shared;
    G.n_tok = n_tok;
    return G;
}
}  // namespace pk

extern "C" int pulsar_moe_pair_swiglu_grouped(void *mid, const void *gptrs, const void *starts,
                                              const void *pairs, const void *weights,
                                              const void *xq, uint32_t in_dim, uint32_t mid_dim,
                                              uint32_t n_used, uint32_t n_group,
                                              uint64_t row_bytes, uint32_t quant,
                                              uint32_t act_op) {
    quant &= ~PULSAR_QUANT_A4_OK;
    // MXFP4 rows need only whole 32-value blocks (a superset of the
    // reference's in_dim % 256 contract, which keeps gpt-oss's 2880 off the
    // grouped path, crates/engine/src/lib.rs:8354)
    const uint32_t k_mult = quant == PULSAR_QUANT_MXFP4 ? 32u : 256u;
    if (!mid || !gptrs || !starts || !pairs || !weights || !xq || in_dim == 0 ||
        in_dim % k_mult != 0 || mid_dim == 0 || n_used == 0 || n_used > 16u || n_group == 0 ||
        n_group > 65535u || row_bytes == 0 ||
        (act_op != PULSAR_ACT_SILU && act_op != PULSAR_ACT_SWIGLU_OAI))
        return reject("moe pair swiglu grouped");
    const CsrGroups grp{(const pulsar_expert_ptrs *)gptrs, (const uint32_t *)starts, (const uint32_t *)pairs};
    return pair_grouped(mid, grp, weights, xq, in_dim, mid_dim, n_used, n_group, row_bytes, quant, act_op, 0u);
}

extern "C" int pulsar_moe_down_grouped(void *partial, const void *gptrs, const void *starts,
                                       const void *pairs, const void *midq, uint32_t mid_dim,
                                       uint32_t out_dim, uint32_t n_used, uint32_t n_group,
                                       uint64_t row_bytes, uint32_t quant) {
    quant &= ~PULSAR_QUANT_A4_OK;
    const uint32_t k_mult = quant == PULSAR_QUANT_MXFP4 ? 32u : 256u;
    if (!partial || !gptrs || !starts || !pairs || !midq || mid_dim == 0 || mid_dim % k_mult != 0 ||
        out_dim == 0 || n_used == 0 || n_used > 16u || n_group == 0 || n_group > 65535u ||
        row_bytes == 0)
        return reject("moe down grouped");
    const CsrGroups grp{(const pulsar_expert_ptrs *)gptrs, (const uint32_t *)starts, (const uint32_t *)pairs};
    return down_grouped(partial, grp, midq, mid_dim, out_dim, n_used, n_group, row_bytes, quant, 0u);
}

// Shared checks of the expert-indexed grouped entry points.
static bool experts_args_ok(const void *selected, const void *active, const pulsar_expert_bank *bank,
                            uint32_t n_expert, const pulsar_expert_ptrs *shared, uint32_t n_shared, uint32_t n_tok,
                            uint32_t k_used) {
    return selected && active && bank && n_expert != 0 && n_expert <= 64u * kMaxPerLane && n_tok != 0 &&
           k_used != 0 && n_shared <= kMaxShared && (n_shared == 0 || shared) && k_used + n_shared <= 16u &&
           (uint64_t)n_tok * (k_used + n_shared) <= 2048u;
}

// The grid's group count: every expert the chunk can touch, the shared
// slots and the NULL group (groups past the touched count are empty).
static uint32_t expert_grid_groups(uint32_t n_expert, uint32_t n_shared, uint32_t n_tok, uint32_t k_used) {
    const uint32_t touch = n_tok * k_used < n_expert ? n_tok * k_used : n_expert;
    return touch + n_shared + 1u;
}

extern "C" int pulsar_moe_pair_swiglu_experts(void *mid, const void *selected, const void *active,
                                              const void *slot_weights, const void *xq,
                                              const pulsar_expert_bank *bank, uint32_t n_expert,
                                              const pulsar_expert_ptrs *shared, uint32_t n_shared,
                                              uint32_t n_tok, uint32_t k_used, uint32_t in_dim, uint32_t mid_dim,
                                              uint64_t row_bytes, uint32_t quant, uint32_t act_op) {
    quant &= ~PULSAR_QUANT_A4_OK;
    const uint32_t k_mult = quant == PULSAR_QUANT_MXFP4 ? 32u : 256u;
    if (!mid || !slot_weights || !xq ||
        !experts_args_ok(selected, active, bank, n_expert, shared, n_shared, n_tok, k_used) || !bank->gate ||
        !bank->up || in_dim == 0 || in_dim % k_mult != 0 || mid_dim == 0 || row_bytes == 0 ||
        (act_op != PULSAR_ACT_SILU && act_op != PULSAR_ACT_SWIGLU_OAI))
        return reject("moe pair swiglu experts");
    const ExpertGroups grp = expert_groups(selected, active, bank, n_expert, shared, n_shared, n_tok, k_used);
    return pair_grouped(mid, grp, slot_weights, xq, in_dim, mid_dim, k_used + n_shared,
                        expert_grid_groups(n_expert, n_shared, n_tok, k_used), row_bytes, quant, act_op,
                        4u * n_tok * k_used);
}

extern "C" int pulsar_moe_down_experts(void *partial, const void *selected, const void *active, const void *midq,
                                       const pulsar_expert_bank *bank, uint32_t n_expert,
                                       const pulsar_expert_ptrs *shared, uint32_t n_shared, uint32_t n_tok,
                                       uint32_t k_used, uint32_t mid_dim, uint32_t out_dim, uint64_t row_bytes,
                                       uint32_t quant) {
    quant &= ~PULSAR_QUANT_A4_OK;
    const uint32_t k_mult = quant == PULSAR_QUANT_MXFP4 ? 32u : 256u;
    if (!partial || !midq || !experts_args_ok(selected, active, bank, n_expert, shared, n_shared, n_tok, k_used) ||
        !bank->down || mid_dim == 0 || mid_dim % k_mult != 0 || out_dim == 0 || row_bytes == 0)
        return reject("moe down experts");
    const ExpertGroups grp = expert_groups(selected, active, bank, n_expert, shared, n_shared, n_tok, k_used);
    return down_grouped(partial, grp, midq, mid_dim, out_dim, k_used + n_shared,
                        expert_grid_groups(n_expert, n_shared, n_tok, k_used), row_bytes, quant,
                        4u * n_tok * k_used);
}

extern "C" int pulsar_moe_slot_sum(void *out, const void *partial, uint32_t out_dim, uint32_t n_used,
                                   uint32_t n_tok) {
    if (!out || !partial || out_dim == 0 || n_used == 0 || n_tok == 0) return reject("moe slot sum");
    const uint64_t total = (uint64_t)n_tok * out_dim;
    hipLaunchKernelGGL(slot_sum_kernel, dim3((uint32_t)((total + 255u) / 256u)), dim3(256), 0, pk::stream(),
                       (float *)out, (const float *)partial, out_dim, n_used, total);
    return launch_ok("moe slot sum launch");
}

extern "C" int pulsar_moe_down_bias(void *out, const void *ptrs, const void *weights,
                                    uint32_t out_dim, uint32_t n_used, uint32_t n_tok) {
    if (!out || !ptrs || !weights || out_dim == 0 || n_used == 0 || n_tok == 0)
        return reject("moe down bias");
    const uint64_t total = (uint64_t)n_tok * out_dim;
    hipLaunchKernelGGL(down_bias_kernel, dim3((uint32_t)((total + 255u) / 256u)), dim3(256), 0, pk::stream(),
                       (float *)out, (const pulsar_expert_ptrs *)ptrs, (const float *)weights,
                       out_dim, n_used, total);
    return launch_ok("moe down bias launch");
}

extern "C" int pulsar_moe_slot_sum_bias(void *out, const void *partial, const void *ptrs, const void *weights,
                                        uint32_t out_dim, uint32_t n_used, uint32_t n_tok) {
    if (!out || !partial || !ptrs || !weights || out_dim == 0 || n_used == 0 || n_tok == 0)
        return reject("moe slot sum bias");
    const uint64_t total = (uint64_t)n_tok * out_dim;
    hipLaunchKernelGGL(slot_sum_bias_kernel, dim3((uint32_t)((total + 255u) / 256u)), dim3(256), 0, pk::stream(),
                       (float *)out, (const float *)partial, (const pulsar_expert_ptrs *)ptrs, (const float *)weights,
                       out_dim, n_used, total);
    return launch_ok("moe slot sum bias launch");
}
