// router.hip - the router pieces the routed-MoE layer runs before the
// experts: fp32 logits GEMV, row bias add, top-k select with weights.
#include "pk_common.h"

namespace pk {

// out[t][o] = sum_i w[o][i] * x[t][i]. One wave per output row; lanes
// stride the row with 16-byte loads; every token of the batch reuses the
// row from registers/L1 (pulsar_kernels.cu:6504-6524 computes the same
// sums, block-per-(row, token)).
// One wave per (row, group of TG tokens): lanes stride over K with 16-byte
// loads of the row and of the TG token vectors, then a wave reduction per
// token. Waves of a block take consecutive rows of the same token group, so
// the token vectors are shared through the cache.
template <uint32_t TG>
__global__ __launch_bounds__(256) void matmul_f32_kernel(float *__restrict__ out, const float *__restrict__ w,
                                                         const float *__restrict__ x, uint32_t in_dim,
                                                         uint32_t out_dim, uint32_t n_tok, uint32_t n_work) {
    const uint32_t gw = blockIdx.x * 4u + (threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63u;
    if (gw >= n_work) return;  // wave-uniform
    const uint32_t row = gw % out_dim, t0 = (gw / out_dim) * TG;
    const float *wr = w + (uint64_t)row * in_dim;
    const float *xr[TG];
#pragma unroll
    for (uint32_t t = 0; t < TG; t++) xr[t] = x + (uint64_t)(t0 + t < n_tok ? t0 + t : n_tok - 1u) * in_dim;
    float acc[TG];
#pragma unroll
    for (uint32_t t = 0; t < TG; t++) acc[t] = 0.0f;
    const uint32_t n4 = in_dim / 4u;
    for (uint32_t i = lane; i < n4; i += 64u) {
        const uint4 a = ld128((const uint8_t *)(wr + 4u * i));
#pragma unroll
        for (uint32_t t = 0; t < TG; t++) {
            const uint4 b = ld128((const uint8_t *)(xr[t] + 4u * i));
            acc[t] += __uint_as_float(a.x) * __uint_as_float(b.x);
            acc[t] += __uint_as_float(a.y) * __uint_as_float(b.y);
            acc[t] += __uint_as_float(a.z) * __uint_as_float(b.z);
            acc[t] += __uint_as_float(a.w) * __uint_as_float(b.w);
        }
    }
    for (uint32_t i = 4u * n4 + lane; i < in_dim; i += 64u) {
#pragma unroll
        for (uint32_t t = 0; t < TG; t++) acc[t] += wr[i] * xr[t][i];
    }
#pragma unroll
    for (uint32_t t = 0; t < TG; t++) {
        const float v = group_sum<64>(acc[t]);
        if (lane == 0 && t0 + t < n_tok) out[(uint64_t)(t0 + t) * out_dim + row] = v;
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

constexpr uint32_t kMaxPerLane = 16;  // 64 lanes x 16 = 1024 routed logits

// Order-preserving key of a routing score: larger score <=> larger key,
// -0 and +0 equal, every non-NaN score >= 1 and NaN 0. The reference's
// comparator (pulsar_kernels.cu:922-925) lets the higher score win, ties
// going to the lower expert index, and never picks a NaN.
PK_DEV uint32_t score_key(float v) {
    if (v != v) return 0u;
    const uint32_t u = __builtin_bit_cast(uint32_t, v + 0.0f);  // -0 -> +0
    return ((u & 0x80000000u) ? ~u : (u | 0x80000000u)) + 1u;
}

PK_DEV uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (uint32_t s = 1; s < 64u; s <<= 1) {
        const uint32_t o = (uint32_t)partner((int32_t)v, s);
        v = o > v ? o : v;
    }
    return v;
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

    const uint32_t kNegInf = score_key(-INFINITY);
    uint32_t key[J];
    float prob[J];
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
        const uint32_t e = lane * J + j;
        if (e < n_expert) {
            const float raw = lg[e];
            const float p = mode == 1u ? raw : router_sigmoid(raw);
            prob[j] = mode == 2u ? raw : p;  // mode 2 weights use the raw winner logit
            key[j] = score_key(p + (bias ? bias[e] : 0.0f));
        } else {
            prob[j] = 0.0f;
            key[j] = 0u;
        }
    }
    // this lane's best: first (lowest index) maximal key
    uint32_t bk = 0u, bj = 0u;
    float bp = 0.0f;
    auto lane_best = [&]() {
        bk = 0u;
        bj = 0u;
        bp = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < J; j++)
            if (key[j] > bk) {
                bk = key[j];
                bj = j;
                bp = prob[j];
            }
    };
    lane_best();
    float sum = 0.0f, wmax = -INFINITY;
    for (uint32_t k = 0; k < k_used; k++) {
        const uint32_t m = wave_max_u32(bk);
        int32_t win = -1;  // no candidate: every routed score is NaN
        float wp = 0.0f;
        if (m != 0u) {
            const uint64_t bal = __ballot(bk == m);
            const int f = __builtin_ctzll(bal);
            win = __builtin_amdgcn_readlane((int)(lane * J + bj), f);
            wp = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bp), f));
            if ((int)lane == f) {
#pragma unroll
                for (uint32_t j = 0; j < J; j++)
                    if (j == bj) key[j] = kNegInf;
                lane_best();
            }
        }
        if (lane == 0) {
            sel_l[k] = win;
            w_l[k] = wp;
        }
        sum += wp;
        wmax = fmaxf(wmax, wp);
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
    // tokens in groups of 4 (1 for a single token); one wave per (row, group)
    const uint32_t tg = n_tok == 1u ? 1u : 4u;
    const uint64_t work = (uint64_t)out_dim * ((n_tok + tg - 1u) / tg);
    if (work > 0xffffffffull - 3u) return pk::reject("matmul f32 (size)");
    const dim3 grid((uint32_t)((work + 3u) / 4u));
    if (tg == 1u)
        hipLaunchKernelGGL(pk::matmul_f32_kernel<1>, grid, dim3(256), 0, pk::stream(), (float *)out,
                           (const float *)w, (const float *)x, in_dim, out_dim, n_tok, (uint32_t)work);
    else
        hipLaunchKernelGGL(pk::matmul_f32_kernel<4>, grid, dim3(256), 0, pk::stream(), (float *)out,
                           (const float *)w, (const float *)x, in_dim, out_dim, n_tok, (uint32_t)work);
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
    if (n_expert <= 256u)
        PK_SELECT(4);
    else if (n_expert <= 512u)
        PK_SELECT(8);
    else
        PK_SELECT(16);
#undef PK_SELECT
    return pk::launch_ok("router select launch");
}
