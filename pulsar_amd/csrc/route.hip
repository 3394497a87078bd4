// route.hip - device-side routing glue: per-(token, slot) expert pointers
// from the router's ids, and the grouped-path CSR built from those pointers.
// The reference does both on the host after a device->host copy of the ids
// (crates/engine/src/lib.rs:7663-7670, 8255-8344, 8357-8392).
#include "pk_common.h"

namespace pk {

constexpr uint32_t kMaxShared = 4;
constexpr uint32_t kMaxCsrPairs = 2048;

struct SharedSlots {
    pulsar_expert_ptrs p[kMaxShared];
};

__global__ __launch_bounds__(256) void route_ptrs_kernel(pulsar_expert_ptrs *__restrict__ ptrs,
                                                         float *__restrict__ slot_w,
                                                         const int32_t *__restrict__ selected,
                                                         const float *__restrict__ router_w,
                                                         pulsar_expert_bank bank, uint32_t n_expert,
                                                         SharedSlots shared, uint32_t n_shared,
                                                         uint32_t n_tok, uint32_t k_used) {
    const uint32_t n_slots = k_used + n_shared;
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n_tok * n_slots) return;
    const uint32_t t = (uint32_t)(i / n_slots), s = (uint32_t)(i % n_slots);
    pulsar_expert_ptrs p = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    float w = 1.0f;
    if (s < k_used) {
        const int32_t e = selected[(uint64_t)t * k_used + s];
        w = router_w[(uint64_t)t * k_used + s];
        if (e >= 0 && (uint32_t)e < n_expert) {
            const uint64_t ue = (uint64_t)e;
            p.gate = (const uint8_t *)bank.gate + ue * bank.gate_stride;
            p.up = (const uint8_t *)bank.up + ue * bank.up_stride;
            p.down = (const uint8_t *)bank.down + ue * bank.down_stride;
            if (bank.gate_b) p.gate_b = bank.gate_b + ue * bank.gate_b_stride;
            if (bank.up_b) p.up_b = bank.up_b + ue * bank.up_b_stride;
            if (bank.down_b) p.down_b = bank.down_b + ue * bank.down_b_stride;
        }
    } else {
        p = shared.p[s - k_used];
    }
    ptrs[i] = p;
    slot_w[i] = w;
}

// One block; every pair's group rank and destination are counted directly
// (n <= 2048 pairs, so the quadratic counts stay in the microseconds).
__global__ __launch_bounds__(1024) void group_csr_kernel(pulsar_expert_ptrs *__restrict__ gptrs,
                                                         uint32_t *__restrict__ starts,
                                                         uint32_t *__restrict__ pairs,
                                                         const pulsar_expert_ptrs *__restrict__ ptrs,
                                                         uint32_t n, uint32_t n_used,
                                                         uint32_t max_groups) {
    __shared__ uint64_t key[kMaxCsrPairs];
    __shared__ uint16_t first[kMaxCsrPairs];  // index of the first pair with the same gate
    __shared__ uint16_t grp[kMaxCsrPairs];    // group id (0xffff: NULL gate)
    __shared__ uint32_t n_groups, n_pairs;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    for (uint32_t i = tid; i < n; i += nt) key[i] = (uint64_t)(uintptr_t)ptrs[i].gate;
    if (tid == 0) {
        n_groups = 0;
        n_pairs = 0;
    }
    __syncthreads();
    for (uint32_t i = tid; i < n; i += nt) {
        uint32_t f = i;
        if (key[i] != 0)
            for (uint32_t j = 0; j < i; j++)
                if (key[j] == key[i]) {
                    f = j;
                    break;
                }
        first[i] = (uint16_t)f;
    }
    __syncthreads();
    // group id = number of distinct gates first seen before this group's first pair
    for (uint32_t i = tid; i < n; i += nt) {
        uint16_t g = 0xffffu;
        if (key[i] != 0) {
            const uint32_t f = first[i];
            uint32_t r = 0;
            for (uint32_t j = 0; j < f; j++) r += (key[j] != 0 && first[j] == j) ? 1u : 0u;
            g = (uint16_t)r;
        }
        grp[i] = g;
        if (key[i] != 0) {
            atomicAdd(&n_pairs, 1u);
            if (first[i] == i) atomicAdd(&n_groups, 1u);
        }
    }
    __syncthreads();
    for (uint32_t i = tid; i < n; i += nt) {
        const uint32_t g = grp[i];
        if (g == 0xffffu) continue;
        // destination = pairs ordered by (group, pair index)
        uint32_t dst = 0;
        for (uint32_t j = 0; j < n; j++) {
            const uint32_t gj = grp[j];
            dst += (gj != 0xffffu && (gj < g || (gj == g && j < i))) ? 1u : 0u;
        }
        pairs[dst] = ((i / n_used) << 4) | (i % n_used);
        if (first[i] == i && g < max_groups) {
            starts[g] = dst;
            gptrs[g] = ptrs[i];
        }
    }
    for (uint32_t g = n_groups + tid; g < max_groups; g += nt) {
        gptrs[g] = pulsar_expert_ptrs{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
        starts[g] = n_pairs;
    }
    if (tid == 0) starts[max_groups] = n_pairs;
}

}  // namespace pk

extern "C" int pulsar_moe_route_ptrs(void *ptrs, void *slot_weights, const void *selected,
                                     const void *router_weights, const pulsar_expert_bank *bank,
                                     uint32_t n_expert, const pulsar_expert_ptrs *shared,
                                     uint32_t n_shared, uint32_t n_tok, uint32_t k_used) {
    if (!ptrs || !slot_weights || !selected || !router_weights || !bank || n_tok == 0 ||
        k_used == 0 || n_shared > pk::kMaxShared || (n_shared && !shared))
        return pk::reject("moe route ptrs");
    pk::SharedSlots sh = {};
    for (uint32_t i = 0; i < n_shared; i++) sh.p[i] = shared[i];
    const uint64_t total = (uint64_t)n_tok * (k_used + n_shared);
    hipLaunchKernelGGL(pk::route_ptrs_kernel, dim3((uint32_t)((total + 255u) / 256u)), dim3(256), 0, pk::stream(),
                       (pulsar_expert_ptrs *)ptrs, (float *)slot_weights, (const int32_t *)selected,
                       (const float *)router_weights, *bank, n_expert, sh, n_shared, n_tok, k_used);
    return pk::launch_ok("moe route ptrs launch");
}

extern "C" int pulsar_moe_group_csr(void *gptrs, void *starts, void *pairs, const void *ptrs,
                                    uint32_t n_tok, uint32_t n_used, uint32_t max_groups) {
    if (!gptrs || !starts || !pairs || !ptrs || n_tok == 0 || n_used == 0 || n_used > 16u ||
        max_groups == 0 || (uint64_t)n_tok * n_used > pk::kMaxCsrPairs)
        return pk::reject("moe group csr");
    hipLaunchKernelGGL(pk::group_csr_kernel, dim3(1), dim3(1024), 0, pk::stream(), (pulsar_expert_ptrs *)gptrs,
                       (uint32_t *)starts, (uint32_t *)pairs, (const pulsar_expert_ptrs *)ptrs,
                       n_tok * n_used, n_used, max_groups);
    return pk::launch_ok("moe group csr launch");
}
