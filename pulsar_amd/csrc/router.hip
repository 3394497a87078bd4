// router.hip - the router pieces the routed-MoE layer runs before the
// experts: fp32 logits GEMV, row bias add, top-k select with weights.
#include "pk_route.h"

namespace pk {

// out[t][o] = sum_i w[o][i] * x[t][i]. One wave per output row; lanes
// stride the row with 16-byte loads; every token of the batch reuses the
// row from registers/L1 (pulsar_kernels.cu:6504-6524 computes the same
// sums, block-per-(row, token)).
template <uint32_t TG>
__global__ __launch_bounds__(256) void matmul_f32_kernel(float *__restrict__ out, const float *__restrict__ w,
                                                         const float *__restrict__ x, uint32_t in_dim,
                                                         uint32_t out_dim, uint32_t n_tok, uint32_t rb_log2) {
    gemv_block<TG>(out, w, x, nullptr, in_dim, out_dim, n_tok,
                   gemv_item(blockIdx.x, out_dim, gridDim.x / out_dim, rb_log2));
}

// x[r][i] += bias[i] (pulsar_kernels.cu:3621-3629)
__global__ __launch_bounds__(256) void add_bias_rows_kernel(float *__restrict__ x,
                                                            const float *__restrict__ bias,
                                                            uint32_t dim, uint64_t total) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    x[gid] += bias[gid % dim];
}

// One wave per token (pulsar_kernels.cu:938-1050 semantics). Lane l holds
// experts lJ .. lJ+J-1, so a lower lane means a lower expert index. Each of
// the k rounds takes the wave maximum of the lanes' best keys; the lowest
// lane holding it owns the winner (highest score, lowest index on ties),
// which it replaces by -inf like the reference, so an expert can win again
// once every remaining score is -inf. Weights are then normalised per the
// softmax mode, with the reference's sequential sums.
template <uint32_t J>
__global__ __launch_bounds__(64) void router_select_kernel(int32_t *__restrict__ selected,
                                                           float *__restrict__ weights,
                                                           const float *__restrict__ logits,
                                                           const float *__restrict__ bias,
                                                           uint32_t n_expert, uint32_t k_used,
                                                           float weight_scale, uint32_t mode,
                                                           uint32_t n_shexp) {
    __shared__ int32_t sel_l[64u * kMaxPerLane + 64u];
    __shared__ float w_l[64u * kMaxPerLane + 64u];
    __shared__ float es_l;
    const uint32_t token = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    const uint32_t sink = mode == 2u ? n_shexp : 0u;
    const uint32_t n_logit = n_expert + sink;
    const uint32_t n_slot = k_used + sink;
    const float *lg = logits + (uint64_t)token * n_logit;

    int32_t win[J];
    float wprob[J];
    float sum, wmax;
    topk_wave<J>(lg, bias, n_expert, k_used, mode, win, wprob, sum, wmax);
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
        const uint32_t k = lane + 64u * j;
        if (k < k_used) {
            sel_l[k] = win[j];
            w_l[k] = wprob[j];
        }
    }
    // mode 2: shared "sink" experts appended as always-on slots
    for (uint32_t sh = lane; sh < sink; sh += 64u) {
        sel_l[k_used + sh] = (int32_t)(n_expert + sh);
        w_l[k_used + sh] = lg[n_expert + sh];
    }
    __syncthreads();
    if (mode == 0u) {
        sum = fmaxf(sum, 6.103515625e-5f);
    } else {
        // mode 1: softmax over the k winners (== softmax -> top-k ->
        // renormalise); mode 2: softmax(logsigmoid(raw)) over winners ++ sinks
        float m = mode == 1u ? wmax : -INFINITY;
        for (uint32_t p = lane; p < n_slot; p += 64u) {
            float x = w_l[p];
            if (mode == 2u) {
                x = x < 0.0f ? x - log1pf(expf(x)) : -log1pf(expf(-x));
                m = fmaxf(m, x);
            }
            w_l[p] = x;
        }
        if (mode == 2u) m = wave_max(m);
        for (uint32_t p = lane; p < n_slot; p += 64u) w_l[p] = expf(w_l[p] - m);
        __syncthreads();
        if (lane == 0) {
            float es = 0.0f;
            for (uint32_t p = 0; p < n_slot; p++) es += w_l[p];
            es_l = es;
        }
        __syncthreads();
        sum = es_l;
    }
    int32_t *sel = selected + (uint64_t)token * n_slot;
    float *w = weights + (uint64_t)token * n_slot;
    for (uint32_t p = lane; p < n_slot; p += 64u) {
        sel[p] = sel_l[p];
        w[p] = w_l[p] / sum * weight_scale;
    }
}

}  // namespace pk

extern "C" int pulsar_matmul_f32(void *out, const void *w, const void *x, uint32_t in_dim,
                                 uint32_t out_dim, uint32_t n_tok) {
    if (!out || !w || !x || in_dim == 0 || out_dim == 0 || n_tok == 0) return pk::reject("matmul f32");
    // tokens in pairs (1 for a single token); one block per (row, pair): c4
    // layer 138.8 -> 137.5 us against groups of 4 (the same sums), 8 slower
    const uint32_t tg = n_tok == 1u ? 1u : 2u;
    const uint64_t work = (uint64_t)out_dim * ((n_tok + tg - 1u) / tg);
    if (work > 0x7fffffffull) return pk::reject("matmul f32 (size)");
    const dim3 grid((uint32_t)work);
    const uint32_t rbl = pk::gemv_xcd_split(out_dim, (n_tok + tg - 1u) / tg, tg);
    if (tg == 1u)
        hipLaunchKernelGGL(pk::matmul_f32_kernel<1>, grid, dim3(256), 0, pk::stream(), (float *)out,
                           (const float *)w, (const float *)x, in_dim, out_dim, n_tok, rbl);
    else
        hipLaunchKernelGGL(pk::matmul_f32_kernel<2>, grid, dim3(256), 0, pk::stream(), (float *)out,
                           (const float *)w, (const float *)x, in_dim, out_dim, n_tok, rbl);
    return pk::launch_ok("matmul f32 launch");
}

extern "C" int pulsar_add_bias_rows(void *x, const void *bias, uint32_t dim, uint32_t rows) {
    if (!x || !bias || dim == 0 || rows == 0) return pk::reject("add bias rows");
    const uint64_t total = (uint64_t)rows * dim;
    hipLaunchKernelGGL(pk::add_bias_rows_kernel, dim3((uint32_t)((total + 255u) / 256u)), dim3(256),
                       0, pk::stream(), (float *)x, (const float *)bias, dim, total);
    return pk::launch_ok("add bias rows launch");
}

// pulsar_kernels.cu:1052-1064 contract.
extern "C" int pulsar_router_select(void *selected, void *weights, const void *logits,
                                    const void *bias, uint32_t n_expert, uint32_t k_used,
                                    float weight_scale, uint32_t n_tok, uint32_t softmax_mode,
                                    uint32_t n_shexp) {
    if (!selected || !weights || !logits || n_expert == 0 || k_used == 0 || k_used > n_expert ||
        n_tok == 0 || softmax_mode > 2u || (softmax_mode != 2u && n_shexp != 0) ||
        n_expert + (softmax_mode == 2u ? n_shexp : 0u) > 1024u || n_expert > 64u * pk::kMaxPerLane)
        return pk::reject("router select");
#define PK_SELECT(J)                                                                                        \
    hipLaunchKernelGGL(pk::router_select_kernel<J>, dim3(n_tok), dim3(64), 0, pk::stream(), (int32_t *)selected, \
                       (float *)weights, (const float *)logits, (const float *)bias, n_expert, k_used,           \
                       weight_scale, softmax_mode, n_shexp)
    // the fewest experts per lane that hold them all (a lane's best is a
    // scan over its J entries in every round)
    if (n_expert <= 64u)
        PK_SELECT(1);
    else if (n_expert <= 128u)
        PK_SELECT(2);
    else if (n_expert <= 256u)
        PK_SELECT(4);
    else if (n_expert <= 512u)
        PK_SELECT(8);
    else
        PK_SELECT(16);
#undef PK_SELECT
    return pk::launch_ok("router select launch");
}
