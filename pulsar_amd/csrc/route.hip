// route.hip - device-side routing glue: per-(token, slot) expert pointers
// from the router's ids, and the grouped-path CSR built from those pointers.
// The reference does both on the host after a device->host copy of the ids
// (crates/engine/src/lib.rs:7663-7670, 8255-8344, 8357-8392).
#include "pk_route.h"

namespace pk {

constexpr uint32_t kMaxCsrPairs = 2048;


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
    pulsar_expert_ptrs p;
    float w = 1.0f;
    if (s < k_used) {
        w = router_w[(uint64_t)t * k_used + s];
        p = bank_ptrs(bank, n_expert, selected[(uint64_t)t * k_used + s]);
    } else {
        p = shared.p[s - k_used];
    }
    ptrs[i] = p;
    slot_w[i] = w;
}

constexpr uint32_t kCsrThreads = 1024;  // two pairs per thread
constexpr uint32_t kHashSlots = 4096;    // open-addressing table, >= 2 x kMaxCsrPairs

// Exclusive block-wide scan of two consecutive elements per thread (2 tid,
// 2 tid + 1); returns the total. Contains two block barriers.
PK_DEV uint32_t block_scan2(uint32_t v0, uint32_t v1, uint32_t &e0, uint32_t &e1, uint32_t *wsum) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t own = v0 + v1;
    // inclusive wave scan by DPP: row_shr 1/2/4/8 within 16-lane rows (lanes
    // without a source add 0), then row_bcast 15 / 31 carry the row totals
    int32_t x = (int32_t)own;
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
    const uint32_t s = (uint32_t)x;
    if (lane == 63u) wsum[wave] = s;
    __syncthreads();
    uint32_t base = 0, total = 0;
#pragma unroll
    for (uint32_t w = 0; w < kCsrThreads / 64u; w++) {
        const uint32_t x = wsum[w];
        base += w < wave ? x : 0u;
        total += x;
    }
    e0 = base + s - own;
    e1 = e0 + v0;
    __syncthreads();
    return total;
}

PK_DEV uint32_t ptr_hash(uint64_t k) { return (uint32_t)(((k >> 4) * 0x9E3779B97F4A7C15ull) >> 52); }

// Groups the (token, slot) pairs by expert (gate pointer) in order of first
// appearance, pairs of a group in pair order, like the reference's host
// grouping (crates/engine/src/lib.rs:8357-8392). One block; every step has
// constant depth: first occurrences through an LDS hash table (atomic CAS
// insert, atomic min of the pair index), group ids and group starts by
// block scans, members scattered to their group's segment and put in pair
// order by counting the smaller pair indices in the segment.
// The CSR build's LDS tables (declared by the kernel, cleared by
// csr_clear before a block barrier that precedes csr_build).
struct CsrLds {
    unsigned long long tkey[kHashSlots];
    uint32_t tfirst[kHashSlots];
    uint32_t gid_of[kMaxCsrPairs];  // group id, at the index of the group's first pair
    uint32_t gstart[kMaxCsrPairs + 1];
    uint32_t fill[kMaxCsrPairs];
    uint32_t seg[kMaxCsrPairs];  // pair indices by group, unordered within a group
    uint32_t wsum[kCsrThreads / 64u];
};

PK_DEV void csr_clear(CsrLds &T) {
    for (uint32_t h = threadIdx.x; h < kHashSlots; h += kCsrThreads) {
        T.tkey[h] = 0ull;
        T.tfirst[h] = UINT32_MAX;
    }
    for (uint32_t g = threadIdx.x; g < kMaxCsrPairs; g += kCsrThreads) {
        T.gstart[g] = 0u;
        T.fill[g] = 0u;
    }
}

template <typename KeyFn, typename PtrFn>
PK_DEV void csr_build(CsrLds &T, pulsar_expert_ptrs *__restrict__ gptrs, uint32_t *__restrict__ starts,
                      uint32_t *__restrict__ pairs, KeyFn key_of, PtrFn ptrs_of, uint32_t n, uint32_t n_used,
                      uint32_t max_groups) {
    auto &tkey = T.tkey;
    auto &tfirst = T.tfirst;
    auto &gid_of = T.gid_of;
    auto &gstart = T.gstart;
    auto &fill = T.fill;
    auto &seg = T.seg;
    auto &wsum = T.wsum;
    const uint32_t tid = threadIdx.x;

    uint64_t key[2];
    uint32_t slot[2] = {0u, 0u};
#pragma unroll
    for (uint32_t e = 0; e < 2; e++) {
        const uint32_t i = 2u * tid + e;
        key[e] = i < n ? key_of(i) : 0ull;
        if (key[e] != 0ull) {
            uint32_t h = ptr_hash(key[e]);
            for (;;) {  // the table has more free slots than pairs: ends
                const unsigned long long prev = atomicCAS(&tkey[h], 0ull, (unsigned long long)key[e]);
                if (prev == 0ull || prev == key[e]) break;
                h = (h + 1u) & (kHashSlots - 1u);
            }
            atomicMin(&tfirst[h], i);
            slot[e] = h;
        }
    }
    __syncthreads();
    uint32_t first[2], isf[2];
#pragma unroll
    for (uint32_t e = 0; e < 2; e++) {
        first[e] = key[e] != 0ull ? tfirst[slot[e]] : UINT32_MAX;
        isf[e] = first[e] == 2u * tid + e ? 1u : 0u;
    }
    uint32_t g0, g1;
    const uint32_t n_groups = block_scan2(isf[0], isf[1], g0, g1, wsum);
    if (isf[0]) gid_of[2u * tid] = g0;
    if (isf[1]) gid_of[2u * tid + 1u] = g1;
    __syncthreads();
    uint32_t grp[2];
#pragma unroll
    for (uint32_t e = 0; e < 2; e++) {
        grp[e] = key[e] != 0ull ? gid_of[first[e]] : UINT32_MAX;
        if (key[e] != 0ull) atomicAdd(&gstart[grp[e]], 1u);  // member count for now
    }
    __syncthreads();
    uint32_t c0 = gstart[2u * tid], c1 = gstart[2u * tid + 1u], s0, s1;
    const uint32_t n_pairs = block_scan2(c0, c1, s0, s1, wsum);
    gstart[2u * tid] = s0;
    gstart[2u * tid + 1u] = s1;
    if (tid == 0) gstart[kMaxCsrPairs] = n_pairs;
    __syncthreads();
#pragma unroll
    for (uint32_t e = 0; e < 2; e++)
        if (key[e] != 0ull) seg[gstart[grp[e]] + atomicAdd(&fill[grp[e]], 1u)] = 2u * tid + e;
    __syncthreads();
#pragma unroll
    for (uint32_t e = 0; e < 2; e++) {
        if (key[e] == 0ull) continue;
        const uint32_t i = 2u * tid + e, g = grp[e], st = gstart[g], len = fill[g];
        uint32_t r = 0;
        for (uint32_t q = 0; q < len; q++) r += seg[st + q] < i ? 1u : 0u;
        pairs[st + r] = ((i / n_used) << 4) | (i % n_used);
        if (isf[e] && g < max_groups) {
            starts[g] = st;
            gptrs[g] = ptrs_of(i);
        }
    }
    // group slots past the last group: NULL with empty ranges. Groups past
    // max_groups (a too-small bound from the caller) are not reachable.
    const uint32_t end = n_groups > max_groups ? gstart[max_groups] : n_pairs;
    for (uint32_t g = n_groups + tid; g < max_groups; g += kCsrThreads) {
        gptrs[g] = pulsar_expert_ptrs{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
        starts[g] = end;
    }
    if (tid == 0) starts[max_groups] = end;
}

__global__ __launch_bounds__(kCsrThreads) void group_csr_kernel(pulsar_expert_ptrs *__restrict__ gptrs,
                                                               uint32_t *__restrict__ starts,
                                                               uint32_t *__restrict__ pairs,
                                                               const pulsar_expert_ptrs *__restrict__ ptrs,
                                                               uint32_t n, uint32_t n_used, uint32_t max_groups) {
    __shared__ CsrLds T;
    csr_clear(T);
    __syncthreads();
    csr_build(
            T, gptrs, starts, pairs, [&](uint32_t i) { return (uint64_t)(uintptr_t)ptrs[i].gate; },
            [&](uint32_t i) { return ptrs[i]; }, n, n_used, max_groups);
}

// Maximum over the lpt-lane group holding this lane (lpt a power of two,
// 4..64), in every lane of the group: butterfly steps quad_perm 1032 and
// 2301, row_half_mirror (8), row_mirror (16), a swizzle lane ^ 16 (32) and a
// permute lane ^ 32 (64).
PK_DEV uint32_t group_max_u32(uint32_t v, uint32_t lpt) {
    auto mx = [](int32_t a, int32_t b) { return (uint32_t)a > (uint32_t)b ? a : b; };
    int32_t x = (int32_t)v;
    x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
    x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
    if (lpt >= 8u) x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false));
    if (lpt >= 16u) x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false));
    if (lpt >= 32u) x = mx(x, __builtin_amdgcn_ds_swizzle(x, 0x401F));
    if (lpt >= 64u) x = mx(x, __shfl_xor(x, 32, 64));
    return (uint32_t)x;
}

// The routing of route_group_kernel / route_kernel: router_select (modes
// 0/1) + route_ptrs for every token of the chunk by one block. A wave
// routes 64 / lpt tokens at once, lpt lanes per token (lane kk of a group
// holds experts kk J .. kk J + J - 1): every top-k round is a group
// maximum, the winner is the group's lowest lane holding it (its lowest
// such expert), which records (expert, prob) for round k in LDS and drops
// that score to -inf, as topk_wave does for one token per wave. The router
// weights then follow route_lane's arithmetic from the recorded winners in
// round order. Every pair's expert goes to eid_l (routed id, -1 for a NULL
// slot, -2 - s for shared slot s); the caller's block barrier follows.
template <uint32_t J>
PK_DEV void route_tokens(int32_t *__restrict__ sel, float *__restrict__ rw, pulsar_expert_ptrs *__restrict__ ptrs,
                         float *__restrict__ slot_w, const float *__restrict__ logits, const float *__restrict__ rbias,
                         uint32_t n_expert, uint32_t k_used, float scale, uint32_t mode,
                         const pulsar_expert_bank &bank, const SharedSlots &shared, uint32_t n_shared, uint32_t n_tok,
                         uint32_t lpt, int32_t *eid_l) {
    __shared__ int32_t win_e[kMaxCsrPairs + 64];  // token t's round-k winner at t k_used + k (+ spare slots)
    __shared__ float win_p[kMaxCsrPairs + 64];    // ... and its prob
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t n_slots = k_used + n_shared;
    const uint32_t tpw = 64u / lpt, g0 = lane & ~(lpt - 1u), kk = lane - g0;
    const uint64_t gmask = lpt == 64u ? ~0ull : (1ull << lpt) - 1ull;
    const uint32_t kNegInf = score_key(-INFINITY);
    if (lpt == 64u) {  // a token per wave: route_lane's DPP wave maxima
        for (uint32_t t = wave; t < n_tok; t += kCsrThreads / 64u) {  // wave-uniform
            int32_t e;
            float w;
            route_lane<J>(logits + (uint64_t)t * n_expert, rbias, n_expert, k_used, scale, mode, e, w);
            const uint64_t i = (uint64_t)t * n_slots + lane;
            if (lane < k_used) {
                sel[(uint64_t)t * k_used + lane] = e;
                rw[(uint64_t)t * k_used + lane] = w;
                ptrs[i] = bank_ptrs(bank, n_expert, e);
                slot_w[i] = w;
                eid_l[i] = e < 0 ? -1 : e;
            } else if (lane < n_slots) {
                ptrs[i] = shared.p[lane - k_used];
                slot_w[i] = 1.0f;
                eid_l[i] = -2 - (int32_t)(lane - k_used);
            }
        }
        return;
    }
    for (uint32_t tb = wave * tpw; tb < n_tok; tb += (kCsrThreads / 64u) * tpw) {
        const uint32_t t = tb + lane / lpt;
        const bool t_ok = t < n_tok;
        const float *lg = logits + (uint64_t)(t_ok ? t : n_tok - 1u) * n_expert;
        const float *bsrc = rbias ? rbias : lg;
        float raw_l[J], bias_l[J];
#pragma unroll
        for (uint32_t j = 0; j < J; j++) {  // every load before any use, clamped indices
            const uint32_t e = kk * J + j, ec = e < n_expert ? e : n_expert - 1u;
            raw_l[j] = lg[ec];
            bias_l[j] = bsrc[ec];
        }
        uint32_t key[J];
        float prob[J];
#pragma unroll
        for (uint32_t j = 0; j < J; j++) {
            const float p = mode == 1u ? raw_l[j] : router_sigmoid(raw_l[j]);
            prob[j] = p;
            key[j] = kk * J + j < n_expert ? score_key(p + (rbias ? bias_l[j] : 0.0f)) : 0u;
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
        // no divergent section in a round: lanes that record nothing store
        // to their own spare slot, and the winner's update is a select
        for (uint32_t k = 0; k < k_used; k++) {
            const uint32_t m = group_max_u32(bk, lpt);  // 0: no candidate left (all NaN)
            const uint64_t gm = (__ballot(m != 0u && bk == m) >> g0) & gmask;
            const bool mine = gm != 0ull && kk == (uint32_t)__builtin_ctzll(gm);
            const bool rec = t_ok && (mine || (m == 0u && kk == 0u));
            const uint32_t at = rec ? t * k_used + k : kMaxCsrPairs + lane;
            win_e[at] = mine ? (int32_t)(kk * J + bj) : -1;
            win_p[at] = mine ? bp : 0.0f;
#pragma unroll
            for (uint32_t j = 0; j < J; j++) key[j] = mine && j == bj ? kNegInf : key[j];
            lane_best();
        }
        // the winners' LDS records visible to the wave's other lanes
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (!t_ok) continue;
        // route_lane's weights: sequential sum and max of the winners' probs
        // (all the token's records read at once, clamped to its k_used;
        // k_used <= 16, a CSR slot limit)
        float wp[16];
#pragma unroll
        for (uint32_t k = 0; k < 16u; k++) wp[k] = win_p[t * k_used + (k < k_used ? k : k_used - 1u)];
        float sum = 0.0f, wmax = -INFINITY;
#pragma unroll
        for (uint32_t k = 0; k < 16u; k++) {
            if (k >= k_used) break;  // wave-uniform
            sum += wp[k];
            wmax = fmaxf(wmax, wp[k]);
        }
        const uint32_t ks = kk < k_used ? kk : 0u;
        const int32_t e = win_e[t * k_used + ks];
        const float pk = win_p[t * k_used + ks];
        float w;
        if (mode == 1u) {
            float es = 0.0f;
#pragma unroll
            for (uint32_t k = 0; k < 16u; k++) {
                if (k >= k_used) break;
                es += expf(wp[k] - wmax);
            }
            w = expf(pk - wmax) / es * scale;
        } else {
            w = pk / fmaxf(sum, 6.103515625e-5f) * scale;
        }
        if (kk < k_used) {
            const uint64_t i = (uint64_t)t * n_slots + kk;
            sel[(uint64_t)t * k_used + kk] = e;
            rw[(uint64_t)t * k_used + kk] = w;
            ptrs[i] = bank_ptrs(bank, n_expert, e);
            slot_w[i] = w;
            eid_l[i] = e < 0 ? -1 : e;
        } else if (kk < n_slots) {
            const uint64_t i = (uint64_t)t * n_slots + kk;
            ptrs[i] = shared.p[kk - k_used];
            slot_w[i] = 1.0f;
            eid_l[i] = -2 - (int32_t)(kk - k_used);
        }
    }
}

// router_select (modes 0/1) + route_ptrs + group_csr in one block: the
// routing of route_tokens, then the CSR built from every pair's expert as
// group_csr_kernel does (the CSR tables are cleared first, while the
// logits load).
template <uint32_t J>
__global__ __launch_bounds__(kCsrThreads) void route_group_kernel(
        int32_t *__restrict__ sel, float *__restrict__ rw, pulsar_expert_ptrs *__restrict__ ptrs,
        float *__restrict__ slot_w, pulsar_expert_ptrs *__restrict__ gptrs, uint32_t *__restrict__ starts,
        uint32_t *__restrict__ pairs, const float *__restrict__ logits, const float *__restrict__ rbias,
        uint32_t n_expert, uint32_t k_used, float scale, uint32_t mode, pulsar_expert_bank bank,
        SharedSlots shared, uint32_t n_shared, uint32_t n_tok, uint32_t max_groups, uint32_t lpt) {
    __shared__ int32_t eid_l[kMaxCsrPairs];  // routed expert, or -2 - s for shared slot s
    __shared__ CsrLds T;
    csr_clear(T);
    route_tokens<J>(sel, rw, ptrs, slot_w, logits, rbias, n_expert, k_used, scale, mode, bank, shared, n_shared,
                    n_tok, lpt, eid_l);
    const uint32_t n_slots = k_used + n_shared;
    __syncthreads();
    auto ptrs_of = [&](uint32_t i) {
        const int32_t e = eid_l[i];
        return e >= -1 ? bank_ptrs(bank, n_expert, e) : shared.p[-2 - e];
    };
    csr_build(
            T, gptrs, starts, pairs, [&](uint32_t i) { return (uint64_t)(uintptr_t)ptrs_of(i).gate; }, ptrs_of,
            n_tok * n_slots, n_slots, max_groups);
}

// router_select (modes 0/1) + route_ptrs in one block (the routing of
// route_tokens: the same values as route_group_kernel and as the two
// separate calls), then the list of the experts the chunk touches, for the
// expert-indexed grouped stages: active[0] = their count, active[1] = the
// number of NULL slots (ids outside [0, n_expert)), active[2 ..] = the
// touched expert ids in order of first appearance in (token, slot) order,
// the group order of the reference's host CSR (crates/engine/src/lib.rs:
// 8357-8392). That order also streams faster than ascending ids, which
// keep the resident blocks on neighbouring experts, one contiguous slice
// of the bank (c4 gate / up 88.4 against 83.8 us on the same chunks).
template <uint32_t J>
__global__ __launch_bounds__(kCsrThreads) void route_kernel(
        int32_t *__restrict__ sel, float *__restrict__ rw, pulsar_expert_ptrs *__restrict__ ptrs,
        float *__restrict__ slot_w, uint32_t *__restrict__ active, const float *__restrict__ logits,
        const float *__restrict__ rbias, uint32_t n_expert, uint32_t k_used, float scale, uint32_t mode,
        pulsar_expert_bank bank, SharedSlots shared, uint32_t n_shared, uint32_t n_tok, uint32_t lpt) {
    __shared__ int32_t eid_l[kMaxCsrPairs];
    __shared__ uint32_t first_l[64u * kMaxPerLane];  // an expert's first pair index
    __shared__ uint32_t n_null, wcnt[kCsrThreads / 64u];
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    for (uint32_t i = threadIdx.x; i < n_expert; i += blockDim.x) first_l[i] = UINT32_MAX;
    if (threadIdx.x == 0) n_null = 0u;
    route_tokens<J>(sel, rw, ptrs, slot_w, logits, rbias, n_expert, k_used, scale, mode, bank, shared, n_shared,
                    n_tok, lpt, eid_l);
    __syncthreads();
    const uint32_t n = n_tok * (k_used + n_shared);
    uint32_t nulls = 0u;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const int32_t e = eid_l[i];
        if (e >= 0)
            atomicMin(&first_l[(uint32_t)e], i);
        else if (e == -1)
            nulls++;
    }
    if (nulls) atomicAdd(&n_null, nulls);
    __syncthreads();
    // pair i is its expert's first one: their ranks by ballots and wave offsets
    uint32_t base = 0u;
    for (uint32_t i0 = 0; i0 < n; i0 += blockDim.x) {  // block-uniform
        const uint32_t i = i0 + threadIdx.x;
        const int32_t e = i < n ? eid_l[i] : -1;
        const bool first = e >= 0 && first_l[(uint32_t)e] == i;
        const uint64_t bal = __ballot(first);
        if (lane == 0) wcnt[wave] = (uint32_t)__builtin_popcountll(bal);
        __syncthreads();
        uint32_t off = base, tot = 0u;
        for (uint32_t w = 0; w < kCsrThreads / 64u; w++) {
            off += w < wave ? wcnt[w] : 0u;
            tot += wcnt[w];
        }
        if (first) active[2u + off + (uint32_t)__builtin_popcountll(bal & ((1ull << lane) - 1ull))] = (uint32_t)e;
        base += tot;
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        active[0] = base;
        active[1] = n_null;
    }
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
    hipLaunchKernelGGL(pk::group_csr_kernel, dim3(1), dim3(pk::kCsrThreads), 0, pk::stream(), (pulsar_expert_ptrs *)gptrs,
                       (uint32_t *)starts, (uint32_t *)pairs, (const pulsar_expert_ptrs *)ptrs,
                       n_tok * n_used, n_used, max_groups);
    return pk::launch_ok("moe group csr launch");
}

extern "C" int pulsar_moe_route_group(void *selected, void *weights, void *ptrs, void *slot_weights, void *gptrs,
                                      void *starts, void *pairs, const void *logits, const void *router_bias,
                                      uint32_t n_expert, uint32_t k_used, float weight_scale, uint32_t softmax_mode,
                                      const pulsar_expert_bank *bank, const pulsar_expert_ptrs *shared,
                                      uint32_t n_shared, uint32_t n_tok, uint32_t max_groups) {
    const uint32_t n_slots = k_used + n_shared;
    if (!selected || !weights || !ptrs || !slot_weights || !gptrs || !starts || !pairs || !logits || !bank ||
        n_tok == 0 || k_used == 0 || k_used > n_expert || k_used > 64u || n_expert > 64u * pk::kMaxPerLane ||
        softmax_mode > 1u || n_shared > pk::kMaxShared || (n_shared && !shared) || n_slots > 16u ||
        max_groups == 0 || (uint64_t)n_tok * n_slots > pk::kMaxCsrPairs)
        return pk::reject("moe route group");
    pk::SharedSlots sh = {};
    for (uint32_t s = 0; s < n_shared; s++) sh.p[s] = shared[s];
    // lanes per token: a power of two holding the token's experts (J per
    // lane) and its slots, at least 4 (J = 8 for 128 experts, 16 lanes per
    // token, measured slower than J = 4 with 32: the longer per-lane scan
    // costs more than the LDS-routed exchange it saves)
    const uint32_t jl = n_expert <= 256u ? 4u : n_expert <= 512u ? 8u : 16u;
    const uint32_t need = (n_expert + jl - 1u) / jl > n_slots ? (n_expert + jl - 1u) / jl : n_slots;
    uint32_t lpt = 4u;
    while (lpt < need) lpt <<= 1;
#define PK_RG(J)                                                                                                 \
    hipLaunchKernelGGL(pk::route_group_kernel<J>, dim3(1), dim3(pk::kCsrThreads), 0, pk::stream(),              \
                       (int32_t *)selected, (float *)weights, (pulsar_expert_ptrs *)ptrs, (float *)slot_weights, \
                       (pulsar_expert_ptrs *)gptrs, (uint32_t *)starts, (uint32_t *)pairs, (const float *)logits, \
                       (const float *)router_bias, n_expert, k_used, weight_scale, softmax_mode, *bank, sh, n_shared, \
                       n_tok, max_groups, lpt)
    if (jl == 4u)
        PK_RG(4);
    else if (jl == 8u)
        PK_RG(8);
    else
        PK_RG(16);
#undef PK_RG
    return pk::launch_ok("moe route group launch");
}

extern "C" int pulsar_moe_route(void *selected, void *weights, void *ptrs, void *slot_weights, void *active,
                                const void *logits, const void *router_bias, uint32_t n_expert, uint32_t k_used,
                                float weight_scale, uint32_t softmax_mode, const pulsar_expert_bank *bank,
                                const pulsar_expert_ptrs *shared, uint32_t n_shared, uint32_t n_tok) {
    const uint32_t n_slots = k_used + n_shared;
    if (!selected || !weights || !ptrs || !slot_weights || !active || !logits || !bank || n_tok == 0 ||
        k_used == 0 || k_used > n_expert || n_expert > 64u * pk::kMaxPerLane || softmax_mode > 1u ||
        n_shared > pk::kMaxShared || (n_shared && !shared) || n_slots > 16u ||
        (uint64_t)n_tok * n_slots > pk::kMaxCsrPairs)
        return pk::reject("moe route");
    pk::SharedSlots sh = {};
    for (uint32_t s = 0; s < n_shared; s++) sh.p[s] = shared[s];
    // lanes per token: as many as let the block's 16 waves route every token
    // in one round (c4's 16 tokens: a wave each; c5's 64: 16 lanes each),
    // at least the token's slots, and enough that J = experts per lane <= 16
    auto pow2 = [](uint32_t v) {
        uint32_t p = 1u;
        while (p < v) p <<= 1;
        return p;
    };
    const uint32_t tpw = pow2((n_tok + pk::kCsrThreads / 64u - 1u) / (pk::kCsrThreads / 64u));
    uint32_t lpt = tpw >= 16u ? 4u : 64u / tpw;
    lpt = lpt > pow2(n_slots) ? lpt : pow2(n_slots);
    lpt = lpt > 4u ? lpt : 4u;
    while ((n_expert + lpt - 1u) / lpt > 16u) lpt <<= 1;
    const uint32_t jl = pow2((n_expert + lpt - 1u) / lpt);
#define PK_RT(J)                                                                                                 \
    hipLaunchKernelGGL(pk::route_kernel<J>, dim3(1), dim3(pk::kCsrThreads), 0, pk::stream(), (int32_t *)selected, \
                       (float *)weights, (pulsar_expert_ptrs *)ptrs, (float *)slot_weights, (uint32_t *)active,   \
                       (const float *)logits, (const float *)router_bias, n_expert, k_used, weight_scale,         \
                       softmax_mode, *bank, sh, n_shared, n_tok, lpt)
    if (jl == 1u)
        PK_RT(1);
    else if (jl == 2u)
        PK_RT(2);
    else if (jl == 4u)
        PK_RT(4);
    else if (jl == 8u)
        PK_RT(8);
    else
        PK_RT(16);
#undef PK_RT
    return pk::launch_ok("moe route launch");
}
