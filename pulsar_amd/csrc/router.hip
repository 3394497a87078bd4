// router.hip - the router pieces the routed-MoE layer runs before the
// experts: fp32 logits GEMV, row bias add, top-k select with weights.
#include "pk_common.h"

namespace pk {

// out[t][o] = sum_i w[o][i] * x[t][i]. One wave per output row; lanes
// stride the row with 16-byte loads; every token of the batch reuses the
// row from registers/L1 (pulsar_kernels.cu:6504-6524 computes the same
// sums, block-per-(row, token)).
__global__ __launch_bounds__(64) void matmul_f32_kernel(float *__restrict__ out,
                                                        const float *__restrict__ w,
                                                        const float *__restrict__ x,
                                                        uint32_t in_dim, uint32_t out_dim,
                                                        uint32_t n_tok) {
    const uint32_t row = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    const float *wr = w + (uint64_t)row * in_dim;
    const uint32_t n4 = in_dim / 4u;
    for (uint32_t t = 0; t < n_tok; t++) {
        const float *xr = x + (uint64_t)t * in_dim;
        float acc = 0.0f;
        for (uint32_t i = lane; i < n4; i += 64u) {
            const uint4 a = ld128((const uint8_t *)(wr + 4u * i));
            const uint4 b = ld128((const uint8_t *)(xr + 4u * i));
            acc += __uint_as_float(a.x) * __uint_as_float(b.x);
            acc += __uint_as_float(a.y) * __uint_as_float(b.y);
            acc += __uint_as_float(a.z) * __uint_as_float(b.z);
            acc += __uint_as_float(a.w) * __uint_as_float(b.w);
        }
        for (uint32_t i = 4u * n4 + lane; i < in_dim; i += 64u) acc += wr[i] * xr[i];
        acc = group_sum<64>(acc);
        if (lane == 0) out[(uint64_t)t * out_dim + row] = acc;
    }
}

// x[r][i] += bias[i] (pulsar_kernels.cu:3621-3629)
__global__ __launch_bounds__(256) void add_bias_rows_kernel(float *__restrict__ x,
                                                            const float *__restrict__ bias,
                                                            uint32_t dim, uint64_t total) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    x[gid] += bias[gid % dim];
}

// sigmoid as pulsar_kernels.cu:913-921
PK_DEV float router_sigmoid(float x) {
    if (x >= 0.0f) {
        const float e = expf(-x);
        return 1.0f / (1.0f + e);
    }
    const float e = expf(x);
    return e / (1.0f + e);
}

// higher score wins; ties go to the lower expert index (pulsar_kernels.cu:922-925)
PK_DEV bool better(float av, uint32_t ai, float bv, uint32_t bi) {
    return av > bv || (av == bv && ai < bi);
}

constexpr uint32_t kMaxPerLane = 16;  // 64 lanes x 16 = 1024 routed logits

// One wave per token (pulsar_kernels.cu:938-1050 semantics): k rounds of a
// wave-wide arg-max over (score, index); lane 0 then normalises the k
// winners' weights in selection order.
__global__ __launch_bounds__(64) void router_select_kernel(int32_t *__restrict__ selected,
                                                           float *__restrict__ weights,
                                                           const float *__restrict__ logits,
                                                           const float *__restrict__ bias,
                                                           uint32_t n_expert, uint32_t k_used,
                                                           float weight_scale, uint32_t mode,
                                                           uint32_t n_shexp) {
    const uint32_t token = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    const uint32_t sink = mode == 2u ? n_shexp : 0u;
    const uint32_t n_logit = n_expert + sink;
    const uint32_t n_slot = k_used + sink;
    const float *lg = logits + (uint64_t)token * n_logit;
    int32_t *sel = selected + (uint64_t)token * n_slot;
    float *w = weights + (uint64_t)token * n_slot;

    float prob[kMaxPerLane], score[kMaxPerLane];
#pragma unroll
    for (uint32_t j = 0; j < kMaxPerLane; j++) {
        const uint32_t e = lane + 64u * j;
        if (e < n_expert) {
            const float raw = lg[e];
            const float p = mode == 1u ? raw : router_sigmoid(raw);
            prob[j] = mode == 2u ? raw : p;  // mode 2 weights use the raw winner logit
            score[j] = p + (bias ? bias[e] : 0.0f);
        } else {
            prob[j] = 0.0f;
            score[j] = -INFINITY;
        }
    }
    for (uint32_t k = 0; k < k_used; k++) {
        float bs = -INFINITY, bp = 0.0f;
        uint32_t bi = UINT32_MAX;
#pragma unroll
        for (uint32_t j = 0; j < kMaxPerLane; j++) {
            const uint32_t e = lane + 64u * j;
            if (e < n_expert && better(score[j], e, bs, bi)) {
                bs = score[j];
                bp = prob[j];
                bi = e;
            }
        }
#pragma unroll
        for (uint32_t m = 1; m < 64u; m <<= 1) {
            const float os = lane_xor(bs, m);
            const float op = lane_xor(bp, m);
            const uint32_t oi = (uint32_t)lane_xor((int32_t)bi, m);
            if (better(os, oi, bs, bi)) {
                bs = os;
                bp = op;
                bi = oi;
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < kMaxPerLane; j++)
            if (lane + 64u * j == bi) score[j] = -INFINITY;
        if (lane == 0) {
            sel[k] = (int32_t)bi;
            w[k] = bp;
        }
    }
    if (lane != 0) return;
    if (mode == 2u) {
        // shared "sink" experts appended as always-on slots; weights are
        // softmax(logsigmoid(raw)) * scale over winners ++ sinks
        for (uint32_t s = 0; s < sink; s++) {
            sel[k_used + s] = (int32_t)(n_expert + s);
            w[k_used + s] = lg[n_expert + s];
        }
        float m = -INFINITY;
        for (uint32_t k = 0; k < n_slot; k++) {
            const float x = w[k];
            w[k] = x < 0.0f ? x - log1pf(expf(x)) : -log1pf(expf(-x));
            m = fmaxf(m, w[k]);
        }
        float es = 0.0f;
        for (uint32_t k = 0; k < n_slot; k++) {
            w[k] = expf(w[k] - m);
            es += w[k];
        }
        for (uint32_t k = 0; k < n_slot; k++) w[k] = w[k] / es * weight_scale;
    } else if (mode == 1u) {
        // softmax -> top-k -> renormalise == softmax over the k winners
        float m = -INFINITY;
        for (uint32_t k = 0; k < k_used; k++) m = fmaxf(m, w[k]);
        float es = 0.0f;
        for (uint32_t k = 0; k < k_used; k++) {
            w[k] = expf(w[k] - m);
            es += w[k];
        }
        for (uint32_t k = 0; k < k_used; k++) w[k] = w[k] / es * weight_scale;
    } else {
        float sum = 0.0f;
        for (uint32_t k = 0; k < k_used; k++) sum += w[k];
        sum = fmaxf(sum, 6.103515625e-5f);
        for (uint32_t k = 0; k < k_used; k++) w[k] = w[k] / sum * weight_scale;
    }
}

}  // namespace pk

extern "C" int pulsar_matmul_f32(void *out, const void *w, const void *x, uint32_t in_dim,
                                 uint32_t out_dim, uint32_t n_tok) {
    if (!out || !w || !x || in_dim == 0 || out_dim == 0 || n_tok == 0) return pk::reject("matmul f32");
    hipLaunchKernelGGL(pk::matmul_f32_kernel, dim3(out_dim), dim3(64), 0, pk::stream(), (float *)out,
                       (const float *)w, (const float *)x, in_dim, out_dim, n_tok);
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
    hipLaunchKernelGGL(pk::router_select_kernel, dim3(n_tok), dim3(64), 0, pk::stream(), (int32_t *)selected,
                       (float *)weights, (const float *)logits, (const float *)bias, n_expert, k_used,
                       weight_scale, softmax_mode, n_shexp);
    return pk::launch_ok("router select launch");
}
