// pk_route.h - routing helpers shared by the router kernels and the fused
// decode-layer kernels: scores, the wave-wide top-k, expert pointers.
#pragma once

#include "pk_common.h"

namespace pk {

// sigmoid as pulsar_kernels.cu:913-921: x >= 0 gives 1 / (1 + exp(-x)),
// otherwise exp(x) / (1 + exp(x)). Both sides take exp(-|x|) (the same
// argument, -0 included), so one exp and one division with the numerator
// selected give the same bits without a divergent branch that would run
// both sides (NaN: exp(NaN) / (1 + NaN) = NaN either way).
PK_DEV float router_sigmoid(float x) {
    const float e = expf(-fabsf(x));
    return (x >= 0.0f ? 1.0f : e) / (1.0f + e);
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

// Wave maximum, returned wave-uniform: DPP moves carry it to lane 63
// (row_shr 1/2/4/8 within each 16-lane row, then row_bcast 15/31 across
// rows; lanes without a source read 0, the identity of an unsigned max),
// which is read back as a scalar. No LDS-routed permutes: a top-k round
// is latency-bound on this reduction.
PK_DEV uint32_t wave_max_u32(uint32_t v) {
    int32_t x = (int32_t)v;
    auto mx = [](int32_t a, int32_t b) { return (uint32_t)a > (uint32_t)b ? a : b; };
    x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true));
    x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true));
    x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true));
    x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true));
    x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false));
    x = mx(x, __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane(x, 63);
}

// The k rounds of the reference's top-k (pulsar_kernels.cu:938-1010) for
// one token, by one wave. Lane l holds experts lJ .. lJ+J-1, so a lower
// lane means a lower expert index. Each round takes the wave maximum of the
// lanes' best keys; the lowest lane holding it owns the winner (highest
// score, lowest index on ties), which it replaces by -inf like the
// reference, so an expert can win again once every remaining score is
// -inf. Winner number k lands in lane k % 64, slot k / 64 of win / wprob
// (index, or -1 when every score is NaN; its prob, the raw logit in mode
// 2). `sum` is the sequential sum of the winners' probs, `wmax` their max.
// KW record slots per lane hold winners 0 .. 64 KW - 1 (KW = 1 for callers
// with k_used <= 64: one select per round instead of J).
template <uint32_t J, uint32_t KW = J>
PK_DEV void topk_wave(const float *lg, const float *bias, uint32_t n_expert, uint32_t k_used, uint32_t mode,
                      int32_t (&win)[KW], float (&wprob)[KW], float &sum, float &wmax) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t kNegInf = score_key(-INFINITY);
    uint32_t key[J];
    float prob[J];
    // every load issued before any is used (clamped in-range indices, no
    // branch around them): a load under a branch makes the compiler wait
    // for it right there, and these come from memory the previous launch
    // wrote, at full memory latency each
    float raw_l[J], bias_l[J];
    const float *bsrc = bias ? bias : lg;
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
        const uint32_t e = lane * J + j, ec = e < n_expert ? e : n_expert - 1u;
        raw_l[j] = lg[ec];
        bias_l[j] = bsrc[ec];
    }
#pragma unroll
    for (uint32_t j = 0; j < KW; j++) {
        win[j] = -1;
        wprob[j] = 0.0f;
    }
#pragma unroll
    for (uint32_t j = 0; j < J; j++) {
        const uint32_t e = lane * J + j;
        if (e < n_expert) {
            const float raw = raw_l[j];
            const float p = mode == 1u ? raw : router_sigmoid(raw);
            prob[j] = mode == 2u ? raw : p;  // mode 2 weights use the raw winner logit
            key[j] = score_key(p + (bias ? bias_l[j] : 0.0f));
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
    sum = 0.0f;
    wmax = -INFINITY;
    // A round has no divergent section: the winner's update and the record
    // of winner k are selects on every lane (a round is one dependent chain,
    // and exec-mask branches lengthen it)
    for (uint32_t k = 0; k < k_used; k++) {
        const uint32_t m = wave_max_u32(bk);  // 0: no candidate, every routed score is NaN
        const int f = __builtin_ctzll(__ballot(bk == m));
        const int32_t e_f = __builtin_amdgcn_readlane((int)(lane * J + bj), f);
        const float p_f = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bp), f));
        const int32_t w_e = m != 0u ? e_f : -1;
        const float w_p = m != 0u ? p_f : 0.0f;
        const bool mine = m != 0u && (int)lane == f;
#pragma unroll
        for (uint32_t j = 0; j < J; j++) key[j] = mine && j == bj ? kNegInf : key[j];
        lane_best();
        const bool rec = lane == (k & 63u);
#pragma unroll
        for (uint32_t j = 0; j < KW; j++) {
            win[j] = rec && j == (k >> 6) ? w_e : win[j];
            wprob[j] = rec && j == (k >> 6) ? w_p : wprob[j];
        }
        sum += w_p;
        wmax = fmaxf(wmax, w_p);
    }
}

// Routing of one token by the calling wave (modes 0 and 1, no sink
// slots): lane k < k_used gets winner k (-1 if none) and its router weight,
// normalised as router_select_kernel does (mode 1: softmax over the
// winners with a sequential exp-sum; mode 0: probabilities over their
// sequential sum, floored at 2^-14). k_used <= 64.
template <uint32_t J>
PK_DEV void route_lane(const float *lg, const float *rbias, uint32_t n_expert, uint32_t k_used, float scale,
                       uint32_t mode, int32_t &e, float &w) {
    int32_t win[1];
    float wprob[1];
    float sum, wmax;
    topk_wave<J, 1>(lg, rbias, n_expert, k_used, mode, win, wprob, sum, wmax);
    // winner k sits in lane k, slot 0
    const uint32_t lane = threadIdx.x & 63u;
    if (mode == 1u) {
        const float ek = lane < k_used ? expf(wprob[0] - wmax) : 0.0f;
        float es = 0.0f;
        for (uint32_t k = 0; k < k_used; k++)
            es += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ek), (int)k));
        w = ek / es * scale;
    } else {
        w = wprob[0] / fmaxf(sum, 6.103515625e-5f) * scale;
    }
    e = win[0];
}

// Blocks go to the 8 XCDs round-robin (block b to XCD b % 8), each XCD with
// its own L2. gemv_item maps block b to the item (token group * out_dim +
// row) it computes so that the blocks of one XCD cover a band of out_dim /
// 2^rb_log2 rows times a band of n_grp / 2^(3 - rb_log2) token groups, each
// row and token of the band fetched into that L2 once; the host picks the
// split that fetches the fewest bytes (rows and tokens are in_dim floats
// each). rb_log2 = 3 is the plain order (rows interleaved over the XCDs,
// every token group on every XCD). Only the item each block computes
// changes, not how it computes it.
PK_DEV uint32_t gemv_item(uint32_t b, uint32_t out_dim, uint32_t n_grp, uint32_t rb_log2) {
    if (rb_log2 >= 3u) return b;
    const uint32_t xcd = b & 7u, j = b >> 3;
    const uint32_t tb_n = 8u >> rb_log2;                   // token-group bands
    const uint32_t rows = out_dim >> rb_log2, grps = n_grp / tb_n;  // band sizes (divisible, host-checked)
    const uint32_t rb = xcd / tb_n, tb = xcd % tb_n;
    const uint32_t row = rb * rows + j % rows, grp = tb * grps + j / rows;
    return grp * out_dim + row;
}

// The split gemv_item uses: rows in 2^r bands, token groups in 2^(3 - r),
// r chosen so that an XCD fetches the fewest rows plus tokens (out_dim / 2^r
// + n_grp tg / 2^(3 - r)); the plain order (3) on ties and where the bands
// would not divide evenly.
static inline uint32_t gemv_xcd_split(uint32_t out_dim, uint32_t n_grp, uint32_t tg) {
    uint32_t best = 3u;
    uint64_t best_cost = (uint64_t)(out_dim >> 3) + (uint64_t)n_grp * tg;
    for (int r = 2; r >= 0; r--) {
        const uint32_t tb = 8u >> r;
        if (out_dim % (1u << r) != 0u || n_grp % tb != 0u) continue;
        const uint64_t cost = (uint64_t)(out_dim >> r) + (uint64_t)(n_grp / tb) * tg;
        if (cost < best_cost) {
            best_cost = cost;
            best = (uint32_t)r;
        }
    }
    return out_dim % 8u == 0u || best < 3u ? best : 3u;
}

// f32 GEMV for router logits, one block of 256 threads per (row, group of
// TG tokens): the row's K is split over the block's threads (thread i takes
// float4 pieces i, i + 256, ... so every wave-wide load is one contiguous
// KiB), all of a batch's loads (4 pieces of the row and of each token)
// issued before any is used. Each thread sums its products in order, the
// wave sums its lanes by a fixed butterfly, and the block adds its 4 waves'
// sums in wave order; the bias (if any) is added to the finished sum, as a
// separate bias pass would. A router row is one memory round trip.
template <uint32_t TG>
PK_DEV void gemv_block(float *__restrict__ out, const float *__restrict__ w, const float *__restrict__ x,
                       const float *__restrict__ bias, uint32_t in_dim, uint32_t out_dim, uint32_t n_tok,
                       uint32_t item) {
    constexpr uint32_t B = 4;  // float4 pieces per thread per batch
    __shared__ float part[4][TG];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t row = item % out_dim, t0 = (item / out_dim) * TG;
    const float *wr = w + (uint64_t)row * in_dim;
    const float *xr[TG];
#pragma unroll
    for (uint32_t t = 0; t < TG; t++) xr[t] = x + (uint64_t)(t0 + t < n_tok ? t0 + t : n_tok - 1u) * in_dim;
    float acc[TG];
#pragma unroll
    for (uint32_t t = 0; t < TG; t++) acc[t] = 0.0f;
    const uint32_t n4 = in_dim / 4u;
    for (uint32_t base = 0; base < n4; base += 256u * B) {
        uint4 wv[B], xv[TG][B];
#pragma unroll
        for (uint32_t b = 0; b < B; b++) {
            const uint32_t i = base + tid + 256u * b, ic = i < n4 ? i : n4 - 1u;  // clamped: no branch
            wv[b] = ld128((const uint8_t *)(wr + 4u * ic));
#pragma unroll
            for (uint32_t t = 0; t < TG; t++) xv[t][b] = ld128((const uint8_t *)(xr[t] + 4u * ic));
        }
#pragma unroll
        for (uint32_t b = 0; b < B; b++) {
            if (base + tid + 256u * b >= n4) break;
            const uint4 a = wv[b];
#pragma unroll
            for (uint32_t t = 0; t < TG; t++) {
                const uint4 c = xv[t][b];
                acc[t] += __uint_as_float(a.x) * __uint_as_float(c.x);
                acc[t] += __uint_as_float(a.y) * __uint_as_float(c.y);
                acc[t] += __uint_as_float(a.z) * __uint_as_float(c.z);
                acc[t] += __uint_as_float(a.w) * __uint_as_float(c.w);
            }
        }
    }
    for (uint32_t i = 4u * n4 + tid; i < in_dim; i += 256u) {
#pragma unroll
        for (uint32_t t = 0; t < TG; t++) acc[t] += wr[i] * xr[t][i];
    }
#pragma unroll
    for (uint32_t t = 0; t < TG; t++) {
        const float v = group_sum<64>(acc[t]);
        if (lane == 0) part[wave][t] = v;
    }
    __syncthreads();
    if (tid < TG && t0 + tid < n_tok) {
        float v = part[0][tid];
        v += part[1][tid];
        v += part[2][tid];
        v += part[3][tid];
        if (bias) v += bias[row];
        out[(uint64_t)(t0 + tid) * out_dim + row] = v;
    }
}

constexpr uint32_t kMaxShared = 4;

struct SharedSlots {
    pulsar_expert_ptrs p[kMaxShared];
};

// Expert e's pointers in a bank (NULL record when e is out of range).
PK_DEV pulsar_expert_ptrs bank_ptrs(const pulsar_expert_bank &bank, uint32_t n_expert, int32_t e) {
    pulsar_expert_ptrs p = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    if (e >= 0 && (uint32_t)e < n_expert) {
        const uint64_t ue = (uint64_t)e;
        p.gate = (const uint8_t *)bank.gate + ue * bank.gate_stride;
        p.up = (const uint8_t *)bank.up + ue * bank.up_stride;
        p.down = (const uint8_t *)bank.down + ue * bank.down_stride;
        if (bank.gate_b) p.gate_b = bank.gate_b + ue * bank.gate_b_stride;
        if (bank.up_b) p.up_b = bank.up_b + ue * bank.up_b_stride;
        if (bank.down_b) p.down_b = bank.down_b + ue * bank.down_b_stride;
    }
    return p;
}

// Routing of one token for slot `slot`, computed by the calling wave (every
// wave of the block computes the same): the expert pointers and router
// weight of the slot, with the weight normalisation of router_select_kernel
// (mode 1: softmax over the winners with a sequential exp-sum; mode 0:
// probabilities over their sequential sum, floored at 2^-14).
struct SlotRoute {
    pulsar_expert_ptrs p;
    float w;
    int32_t e;
};

template <uint32_t J>
PK_DEV SlotRoute route_slot(const float *lg, const float *rbias, uint32_t n_expert, uint32_t k_used,
                            float scale, uint32_t mode, const pulsar_expert_bank &bank, const SharedSlots &shared,
                            uint32_t slot) {
    SlotRoute r;
    if (slot < k_used) {  // wave-uniform: a shared slot needs no routing
        int32_t e;
        float wk;
        route_lane<J>(lg, rbias, n_expert, k_used, scale, mode, e, wk);
        r.e = __builtin_amdgcn_readlane(e, (int)slot);
        r.w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), (int)slot));
        r.p = bank_ptrs(bank, n_expert, r.e);
    } else {
        r.e = -1;
        r.w = 1.0f;
        r.p = shared.p[slot - k_used];
    }
    return r;
}

// ---- how a grouped block finds its expert group --------------------------
// Both sources resolve group g to a Group (the expert's pointers and what
// the group is) with group(); range() then gives the group's (token, slot)
// pairs (token << 4 | slot, in pair order) through pair(), which a thread
// may call for any index in [b, e) right after range().

// The reference's grouped contract: a CSR by expert from the caller
// (gptrs [n_group], starts [n_group + 1], pairs), pulsar_kernels.cu:3483-3591.
struct CsrGroups {
    const pulsar_expert_ptrs *gptrs;
    const uint32_t *starts;
    const uint32_t *pairs;
#ifdef PK_CSR_PAD
    uint8_t pad_[296];
#endif
    struct Group {
        pulsar_expert_ptrs p;
        uint32_t g;
        PK_DEV bool is_null() const { return false; }
    };
    PK_DEV Group group(uint32_t g) const { return Group{gptrs[g], g}; }
    PK_DEV void range(const Group &G, uint32_t *, uint32_t &b, uint32_t &e) const {
        b = starts[G.g];
        e = starts[G.g + 1u];
    }
    PK_DEV uint32_t pair(uint32_t i, const uint32_t *) const { return pairs[i]; }
};

// One group per expert a chunk touches, in a resident bank, found from the
// router's selected ids (no CSR). active (written by the router,
// pulsar_moe_route): [0] = the number of touched experts, [1] = the number
// of NULL slots, [2 ..] = the touched expert ids (first appearance
// order). Group g < active[0] is
// bank expert active[2 + g], its pairs the (token, slot < k_used) whose id
// is that expert; the next n_shared groups are the shared slots k_used + i
// of every token; the next is the NULL group, the slots whose id is outside
// [0, n_expert), whose output rows the grouped kernels write as 0 (an
// unrouted slot contributes zero, pulsar_kernels.cu:2587-2590, 2635); later
// groups are empty. A block reads its group with one load and collects its
// pairs in pair order into an LDS list of up to n_tok * k_used entries.
// Every thread of the block calls range(), which has no block barrier; the
// list is read by the block only after its next barrier.
struct ExpertGroups {
    const int32_t *sel;      // [n_tok][k_used]
    const uint32_t *active;  // [2 + touched experts]
    pulsar_expert_bank bank;
    SharedSlots shared;
    uint32_t n_expert, k_used, n_shared, n_tok;
    struct Group {
        pulsar_expert_ptrs p;
        uint32_t kind, e;  // kind 0: routed expert e, 1: shared slot e, 2: NULL, 3: empty
        int32_t pf[2];     // this lane's selected ids q = lane, lane + 64
        PK_DEV bool is_null() const { return kind == 2u; }
    };
    // active[0], active[1], the group's id and the lane's first selected ids
    // are requested together (clamped indices; active holds 2 + n_expert
    // entries), so the block's pair list costs one memory round trip.
    PK_DEV Group group(uint32_t g) const {
        const uint32_t total = n_tok * k_used;
        const uint32_t lane = threadIdx.x & 63u;
        const uint32_t n_act = active[0], n_nul = active[1];
        const uint32_t e_g = active[2u + (g < n_expert ? g : n_expert - 1u)];
        Group G;
        G.pf[0] = sel[lane < total ? lane : total - 1u];
        G.pf[1] = sel[lane + 64u < total ? lane + 64u : total - 1u];
        G.p = pulsar_expert_ptrs{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
        G.e = 0u;
        if (g < n_act) {
            G.kind = 0u;
            G.e = e_g;
            G.p = bank_ptrs(bank, n_expert, (int32_t)e_g);
        } else if (g < n_act + n_shared) {
            G.kind = 1u;
            G.e = g - n_act;
            G.p = shared.p[G.e];
        } else {
            G.kind = g == n_act + n_shared && n_nul != 0u ? 2u : 3u;
        }
        return G;
    }
    // Every wave scans the selected ids and writes the same list to lst
    // (ballots, no block barrier); on return the calling wave's writes are
    // visible to the wave's lanes, so a thread may read any entry of the
    // list before the block's next barrier. lst holds the pairs [b, e).
    PK_DEV void range(const Group &G, uint32_t *lst, uint32_t &b, uint32_t &e) const {
        const uint32_t lane = threadIdx.x & 63u;
        b = e = 0u;
        if (G.kind == 3u) return;
        if (G.kind == 1u) {  // a shared slot: every token
            const uint32_t sl = k_used + G.e;
            for (uint32_t t = lane; t < n_tok; t += 64u) lst[t] = (t << 4) | sl;
            e = n_tok;
        } else {
            const bool nul = G.kind == 2u;
            const int32_t want = (int32_t)G.e;
            const uint32_t total = n_tok * k_used;
            uint32_t base = 0u;
            for (uint32_t q0 = 0; q0 < total; q0 += 64u) {  // wave-uniform
                const uint32_t q = q0 + lane;
                const int32_t id = q0 == 0u ? G.pf[0] : q0 == 64u ? G.pf[1] : sel[q < total ? q : total - 1u];
                const bool hit = q < total && (nul ? (id < 0 || (uint32_t)id >= n_expert) : id == want);
                const uint64_t bal = __ballot(hit);
                if (hit) {
                    const uint32_t t = q / k_used;
                    lst[base + (uint32_t)__builtin_popcountll(bal & ((1ull << lane) - 1ull))] =
                            (t << 4) | (q - t * k_used);
                }
                base += (uint32_t)__builtin_popcountll(bal);
            }
            e = base;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    PK_DEV uint32_t pair(uint32_t i, const uint32_t *lst) const { return lst[i]; }
};

}  // namespace pk
