// fused.hip - the routed-MoE decode layer in three launches instead of
// seven to nine (router GEMV, bias, top-k, pointer build, x quantize, gate/up,
// mid quantize, down, down bias). Each fused kernel computes exactly what
// the separate entry points compute, with the same arithmetic in the same
// order, so its outputs are bit-identical to theirs:
//   pulsar_router_logits_q8 = pulsar_matmul_f32 (+ pulsar_add_bias_rows)
//                             + pulsar_quantize_q8_K(x)
//   pulsar_moe_pair_routed  = pulsar_router_select (modes 0/1)
//                             + pulsar_moe_route_ptrs + pulsar_moe_pair_swiglu
//   pulsar_moe_down_f32     = pulsar_quantize_q8_K(mid) + pulsar_moe_down
//                             (+ pulsar_moe_down_bias)
// On this GPU every launch costs a few microseconds even when its work is
// tiny (a kernel boundary writes back and invalidates the per-XCD L2s), so
// a decode layer is launch-bound; the reference has the same sequence
// (crates/engine/src/lib.rs:8416-8510) with a host round trip in it.
#include "pk_q8k.h"
#include "pk_route.h"
#include "pk_rowdot.h"

namespace pk {

// Issue priority of the routing wave of a routed pair block while it
// routes: its top-k is one dependent chain, and the blocks that start in a
// later round route beside earlier blocks' decoding waves on the same SIMDs
// (c5 batch 1, 2880 blocks in two rounds: 33.45 -> 32.41 us; c3, one round:
// 16.99 -> 16.92 us; alternating libraries on one box).
#ifndef PK_ROUTE_PRIO
#define PK_ROUTE_PRIO 3
#endif
constexpr uint32_t kFusedMaxSlots = 64;    // k_used + n_shared
constexpr uint32_t kFusedMaxActLds = 65536; // staged mid rows of one token


// Blocks [0, gemv_blocks) compute logits (one block per (row, TG tokens),
// the same reduction as pulsar_matmul_f32 so the logits are bit-identical),
// the rest quantize x (one wave per 256-value block).
template <uint32_t TG>
__global__ __launch_bounds__(256) void router_logits_q8_kernel(
        float *__restrict__ logits, pulsar_block_q8_K *__restrict__ xq, const float *__restrict__ x,
        const float *__restrict__ w, const float *__restrict__ bias, uint32_t in_dim, uint32_t n_expert,
        uint32_t n_tok, uint32_t gemv_blocks, uint32_t nb, uint32_t rb_log2) {
    if (blockIdx.x < gemv_blocks) {
        gemv_block<TG>(logits, w, x, bias, in_dim, n_expert, n_tok,
                       gemv_item(blockIdx.x, n_expert, gemv_blocks / n_expert, rb_log2));
        return;
    }
    const uint32_t gblk = (blockIdx.x - gemv_blocks) * 4u + (threadIdx.x >> 6);
    if (gblk >= n_tok * nb) return;  // whole wave
    const uint32_t row = gblk / nb, b = gblk - row * nb;
    quantize_block_wave<4u, 260u>(x + (uint64_t)row * in_dim, in_dim, b, (uint8_t *)(xq + gblk));
}

// Waves per routed pair block (the first routes the token for all of them;
// the staging of MXFP4 rows takes 2 NPL KiB of LDS per wave). Blocks of 8
// waves, which route half as often per row, measured the same (c3 16.8 us,
// c5 batch 1 35.2 us).
template <uint32_t Q>
constexpr uint32_t kRoutedWaves = 4u;

// grid (row blocks, k_used + n_shared, n_tok); the pair stage of
// moe_pair_kernel for the slot's expert, routed in-block.
template <uint32_t Q, uint32_t UPLMAX, uint32_t J, uint32_t NPL, uint32_t RPW>
__global__ __launch_bounds__(64 * kRoutedWaves<Q>) void moe_pair_routed_kernel(
        float *__restrict__ mid, pulsar_expert_ptrs *__restrict__ ptrs_out, float *__restrict__ slot_w_out,
        int32_t *__restrict__ sel_out, float *__restrict__ w_out, const float *__restrict__ logits,
        const float *__restrict__ rbias, uint32_t n_expert, uint32_t k_used, float scale, uint32_t mode,
        pulsar_expert_bank bank, SharedSlots shared, const pulsar_block_q8_K *__restrict__ xq, uint32_t n_units,
        uint32_t nblk32, uint32_t lpr_log2, uint32_t in_blocks, uint32_t mid_dim, uint64_t row_bytes,
        uint32_t act_op) {
    PK_FMT_LUT(Q)
    const uint32_t slot = blockIdx.y, token = blockIdx.z, n_slots = gridDim.y;
    const uint64_t so = (uint64_t)token * n_slots + slot;
    const RowGeom rg = row_geom(n_units, nblk32, lpr_log2);
    // the token's activation slices do not depend on the routing: in flight
    // while the wave routes
    Act a[UPLMAX];
    load_row_acts<Q, UPLMAX>(xq + (uint64_t)token * in_blocks, rg, a);
    // one wave routes the token for the whole block (every block of the
    // slot computes the same route)
    __shared__ SlotRoute route_l;
    if (threadIdx.x < 64u) {
#if PK_ROUTE_PRIO
        __builtin_amdgcn_s_setprio(PK_ROUTE_PRIO);
#endif
        const SlotRoute rr = route_slot<J>(logits + (uint64_t)token * n_expert, rbias, n_expert, k_used, scale,
                                           mode, bank, shared, slot);
        if (threadIdx.x == 0) route_l = rr;
#if PK_ROUTE_PRIO
        __builtin_amdgcn_s_setprio(0);
#endif
    }
    __syncthreads();
    const SlotRoute r = route_l;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        ptrs_out[so] = r.p;
        slot_w_out[so] = r.w;
        if (slot < k_used) {
            sel_out[(uint64_t)token * k_used + slot] = r.e;
            w_out[(uint64_t)token * k_used + slot] = r.w;
        }
    }
    const pulsar_expert_ptrs &p = r.p;
    const uint32_t rpp = 64u >> lpr_log2;
    const uint32_t pass0 = (blockIdx.x * kRoutedWaves<Q> + threadIdx.x / 64u) * RPW;
    if (!p.gate || !p.up) {  // unrouted slot contributes zero (pulsar_kernels.cu:2587-2590)
#pragma unroll
        for (uint32_t k = 0; k < RPW; k++) {
            const uint32_t row = (pass0 + k) * rpp + rg.rip;
            if (row < mid_dim && rg.holds_row()) mid[so * mid_dim + row] = 0.0f;
        }
        return;
    }
    pair_passes<Q, UPLMAX, NPL, RPW, kRoutedWaves<Q>>(mid + so * mid_dim, p, r.w, a, rg, pass0, mid_dim, row_bytes,
                                                      act_op, lut);
}

constexpr uint32_t kFusedMaxPass = 8;  // row passes per block in the fused down
#ifndef PK_FUSED_DOWN_ROWS
#define PK_FUSED_DOWN_ROWS 8u
#endif
#ifndef PK_FUSED_DOWN_WAVES
#define PK_FUSED_DOWN_WAVES 16u
#endif
// waves of a fused-down block: the token's (pass, slot) dots all in flight
// at once, and the mid blocks quantized a few per wave
constexpr uint32_t kFusedDownWaves = PK_FUSED_DOWN_WAVES;

// grid (row blocks, n_tok), a row block = n_pass passes of rpp rows. The
// block quantizes the token's n_used mid rows into LDS (the q8_K bytes the
// quantize kernel would write); its waves then take the (pass, slot) dots
// round-robin into LDS partials, and each row's slots are summed in slot
// order from +0 (NULL down: -0, the additive identity) as moe_down_kernel
// does, then the optional bias term sum_s w_s down_b_s[row] is added when
// non-zero (moe_down_bias).
template <uint32_t Q, uint32_t UPLMAX, uint32_t NPL>
__global__ __launch_bounds__(1024) void moe_down_f32_kernel(
        float *__restrict__ out, const pulsar_expert_ptrs *__restrict__ ptrs, const float *__restrict__ slot_w,
        const float *__restrict__ mid, uint32_t n_units, uint32_t nblk32, uint32_t lpr_log2,
        uint32_t mid_blocks, uint32_t mid_dim, uint32_t out_dim, uint32_t n_used, uint64_t row_bytes,
        uint32_t add_bias, uint32_t n_pass) {
    PK_FMT_LUT(Q)
    extern __shared__ __align__(16) uint8_t acts_lds[];
    __shared__ pulsar_expert_ptrs p_l[kFusedMaxSlots];
    __shared__ float w_l[kFusedMaxSlots];
    const uint32_t token = blockIdx.y, wave = threadIdx.x / 64u, nw = blockDim.x / 64u;
    const uint32_t n_blk = n_used * mid_blocks;
    float *part = (float *)(acts_lds + n_blk * kActLdsPitch);  // [n_pass][n_used][16]
    const RowGeom rg = row_geom(n_units, nblk32, lpr_log2);
    const uint32_t rpp = 64u >> lpr_log2;
    const uint32_t pass0 = blockIdx.x * n_pass;
    // the slot records are requested first (every thread, clamped index: a
    // load under a branch would be waited for right there) and stored to
    // LDS after the mid rows are quantized, so the two round trips overlap
    const uint32_t s_mine = threadIdx.x < n_used ? threadIdx.x : n_used - 1u;
    const pulsar_expert_ptrs p_mine = ptrs[(uint64_t)token * n_used + s_mine];
    const float w_mine = slot_w ? slot_w[(uint64_t)token * n_used + s_mine] : 0.0f;
    // the wave's mid blocks blk = wave + nw i, loaded four at a time before
    // use and quantized two at a time (their reductions interleave)
    auto load_batch = [&](uint32_t base, float (&v)[4][4]) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i++) {
            const uint32_t blk = base + nw * i;
            if (blk < n_blk) {
                const uint32_t s = blk / mid_blocks, b = blk - s * mid_blocks;
                load_block4(mid + ((uint64_t)token * n_used + s) * mid_dim, mid_dim, b, v[i]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) v[i][j] = 0.0f;
            }
        }
    };
    auto quantize_batch = [&](uint32_t base, const float (&v)[4][4]) {
#pragma unroll
        for (uint32_t i = 0; i < 4; i += 2) {
            const uint32_t blk = base + nw * i;
            if (blk < n_blk)
                quantize_vals_wave2<16u, 272u>(v[i], v[i + 1], acts_lds + blk * kActLdsPitch,
                                               acts_lds + (blk + nw) * kActLdsPitch, blk + nw < n_blk);
        }
    };
    // the first batch is requested before the first weight row, whose
    // address waits for the slot record (a round trip of its own). Unstaged
    // rows: the wave's first (pass, slot) item then has its weights in
    // flight while the mid rows are quantized. A NULL expert reads the
    // token's mid row instead (in bounds: a weight row is shorter than 4
    // bytes per value) and is not used.
    float v0[4][4];
    load_batch(wave, v0);
    typename Fmt<Q>::W w_first[UPLMAX];
    if constexpr (NPL == 0) {
        const uint32_t ks = wave < n_pass * n_used ? wave : 0u;
        const uint32_t k = ks / n_used, s = ks - k * n_used;
        const uint32_t row = (pass0 + k) * rpp + rg.rip;
        const uint8_t *dp = (const uint8_t *)ptrs[(uint64_t)token * n_used + s].down;
        const uint8_t *src = dp ? dp + (uint64_t)(row < out_dim ? row : 0u) * row_bytes
                                : (const uint8_t *)(mid + (uint64_t)token * n_used * mid_dim);
        load_row_w<Q, UPLMAX>(as_global(src), rg, w_first);
    }
    quantize_batch(wave, v0);
    for (uint32_t base = wave + 4u * nw; base < n_blk; base += 4u * nw) {
        float v[4][4];
        load_batch(base, v);
        quantize_batch(base, v);
    }
    if (threadIdx.x < n_used) {
        p_l[threadIdx.x] = p_mine;
        w_l[threadIdx.x] = w_mine;
    }
    __syncthreads();
    const uint32_t act_bytes = mid_blocks * kActLdsPitch;
    for (uint32_t ks = wave; ks < n_pass * n_used; ks += nw) {
        const uint32_t k = ks / n_used, s = ks - k * n_used;
        const uint32_t row = (pass0 + k) * rpp + rg.rip;
        if ((pass0 + k) * rpp >= out_dim) break;  // wave-uniform; later items are later passes
        const bool row_ok = row < out_dim;
        float v = -0.0f;
        if (p_l[s].down) {
            typename Fmt<Q>::W w[UPLMAX];
            if (NPL == 0 && ks == wave) {
#pragma unroll
                for (uint32_t u = 0; u < UPLMAX; u++) w[u] = w_first[u];
            } else {
                load_one_row<Q, UPLMAX, NPL, kFusedDownWaves>(
                        as_global(p_l[s].down) + (uint64_t)(row_ok ? row : 0u) * row_bytes, rg, w);
            }
            Act a[UPLMAX];
            load_row_acts_lds<Q, UPLMAX>(acts_lds + s * act_bytes, rg, a);
            v = row_finish(row_partial<Q, UPLMAX>(row_ok, rg, w, a, lut), rg);
        }
        if (rg.holds_row()) part[(k * n_used + s) * 16u + rg.rip] = v;
    }
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < n_pass * rpp; t += blockDim.x) {
        const uint32_t k = t / rpp, rip = t - k * rpp;
        const uint32_t row = (pass0 + k) * rpp + rip;
        if (row >= out_dim) continue;
        float total = 0.0f;
        for (uint32_t s = 0; s < n_used; s++) total += part[(k * n_used + s) * 16u + rip];
        if (add_bias) {
            float b = 0.0f;
            for (uint32_t s = 0; s < n_used; s++)
                if (p_l[s].down_b) b += w_l[s] * ldwf(p_l[s].down_b + row);
            if (b != 0.0f) total += b;
        }
        out[(uint64_t)token * out_dim + row] = total;
    }
}

// ------------------------------------------------------------ dispatch --

// F::template run<Q, UPLMAX>() for the run-time (quant, upl), up to 4
// units per lane.
template <typename F>
static int fused_format(uint32_t quant, uint32_t upl, F &&f) {
#define PK_FUPL(Q)                                       \
    if (upl <= 1u) return f.template run<Q, 1>();        \
    if (upl <= 2u) return f.template run<Q, 2>();        \
    if (upl <= 4u) return f.template run<Q, 4>();        \
    return reject("fused moe (row width above the supported maximum)");
#define PK_FCASE(Q) \
    case Q: PK_FUPL(Q)
    switch (quant) {
    PK_FOR_EACH_QUANT(PK_FCASE)
    default: return reject("fused moe (quant)");
    }
#undef PK_FCASE
#undef PK_FUPL
}

struct PairRoutedLaunch {
    void *mid, *ptrs_out, *slot_w_out, *sel_out, *w_out;
    const void *logits, *rbias, *xq;
    uint32_t n_expert, k_used, mode, n_slots, n_tok, mid_dim, act_op;
    float scale;
    pulsar_expert_bank bank;
    SharedSlots shared;
    uint64_t row_bytes;
    FGeo g;
    uint32_t j_per_lane;
    template <uint32_t Q, uint32_t U, uint32_t NPL>
    int go() {
        if (j_per_lane == 1u) return go_j<Q, U, 1, NPL>();
        if (j_per_lane == 2u) return go_j<Q, U, 2, NPL>();
        if (j_per_lane == 4u) return go_j<Q, U, 4, NPL>();
        if (j_per_lane == 8u) return go_j<Q, U, 8, NPL>();
        return go_j<Q, U, 16, NPL>();
    }
    // one row pass per wave: two (as the plain pair kernel takes on large
    // launches) measured slower here, the routing being on every block's path
    template <uint32_t Q, uint32_t U, uint32_t J, uint32_t NPL>
    int go_j() {
        const uint32_t rpb = kRoutedWaves<Q> * (64u >> g.l2);
        const dim3 grid((mid_dim + rpb - 1u) / rpb, n_slots, n_tok);
        hipLaunchKernelGGL((moe_pair_routed_kernel<Q, U, J, NPL, 1>), grid, dim3(64u * kRoutedWaves<Q>), 0, pk::stream(),
                           (float *)mid, (pulsar_expert_ptrs *)ptrs_out, (float *)slot_w_out, (int32_t *)sel_out,
                           (float *)w_out, (const float *)logits, (const float *)rbias, n_expert, k_used, scale,
                           mode, bank, shared, (const pulsar_block_q8_K *)xq, g.n_units, g.nblk32, g.l2,
                           g.blocks, mid_dim, row_bytes, act_op);
        return launch_ok("moe pair routed launch");
    }
    template <uint32_t Q, uint32_t U>
    int run() {
        // experts per lane of the top-k: the fewest that hold them all (a
        // lane's best is a scan over its J entries in every round)
        j_per_lane = n_expert <= 64u ? 1u : n_expert <= 128u ? 2u : n_expert <= 256u ? 4u : n_expert <= 512u ? 8u : 16u;
        return with_stage<Q, U>(g, *this);
    }
};

struct DownF32Launch {
    void *out;
    const void *ptrs, *slot_w, *mid;
    uint32_t mid_dim, out_dim, n_used, n_tok, add_bias;
    uint64_t row_bytes;
    FGeo g;
    template <uint32_t Q, uint32_t U>
    int run() {
        return with_stage<Q, U>(g, *this);
    }
    template <uint32_t Q, uint32_t U, uint32_t NPL>
    int go() {
        const uint32_t rpp = 64u >> g.l2;
        uint32_t n_pass = PK_FUSED_DOWN_ROWS / rpp;  // ~PK_FUSED_DOWN_ROWS rows per block
        n_pass = n_pass < 1u ? 1u : n_pass > kFusedMaxPass ? kFusedMaxPass : n_pass;
        const uint32_t rpb = n_pass * rpp;
        const dim3 grid((out_dim + rpb - 1u) / rpb, n_tok);
        const size_t lds = (size_t)n_used * g.blocks * kActLdsPitch + (size_t)n_pass * n_used * 16u * 4u;
        uint32_t nw = n_pass * n_used;  // one (pass, slot) dot per wave where it fits
        nw = nw < 4u ? 4u : nw > kFusedDownWaves ? kFusedDownWaves : nw;
        hipLaunchKernelGGL((moe_down_f32_kernel<Q, U, NPL>), grid, dim3(64u * nw), lds, pk::stream(), (float *)out,
                           (const pulsar_expert_ptrs *)ptrs, (const float *)slot_w, (const float *)mid, g.n_units,
                           g.nblk32, g.l2, g.blocks, mid_dim, out_dim, n_used, row_bytes, add_bias, n_pass);
        return launch_ok("moe down f32 launch");
    }
};

}  // namespace pk

using namespace pk;

extern "C" int pulsar_router_logits_q8(void *logits, void *xq, const void *x, const void *w_r, const void *bias,
                                       uint32_t in_dim, uint32_t n_expert, uint32_t n_tok) {
    if (!logits || !xq || !x || !w_r || in_dim == 0 || n_expert == 0 || n_tok == 0)
        return reject("router logits q8");
    const uint32_t tg = n_tok == 1u ? 1u : 2u;
    const uint64_t work = (uint64_t)n_expert * ((n_tok + tg - 1u) / tg);
    const uint32_t nb = (in_dim + 255u) / 256u;
    const uint64_t qblocks = ((uint64_t)n_tok * nb + 3u) / 4u;
    const uint64_t gemv_blocks = work;
    if (gemv_blocks + qblocks > 0x7fffffffull) return reject("router logits q8 (size)");
    const dim3 grid((uint32_t)(gemv_blocks + qblocks));
    const uint32_t rbl = gemv_xcd_split(n_expert, (n_tok + tg - 1u) / tg, tg);
    if (tg == 1u)
        hipLaunchKernelGGL(router_logits_q8_kernel<1>, grid, dim3(256), 0, pk::stream(), (float *)logits,
                           (pulsar_block_q8_K *)xq, (const float *)x, (const float *)w_r, (const float *)bias,
                           in_dim, n_expert, n_tok, (uint32_t)gemv_blocks, nb, rbl);
    else
        hipLaunchKernelGGL(router_logits_q8_kernel<2>, grid, dim3(256), 0, pk::stream(), (float *)logits,
                           (pulsar_block_q8_K *)xq, (const float *)x, (const float *)w_r, (const float *)bias,
                           in_dim, n_expert, n_tok, (uint32_t)gemv_blocks, nb, rbl);
    return launch_ok("router logits q8 launch");
}

extern "C" int pulsar_moe_pair_routed(void *mid, void *ptrs, void *slot_weights, void *selected, void *weights,
                                      const void *logits, const void *router_bias, uint32_t n_expert,
                                      uint32_t k_used, float weight_scale, uint32_t softmax_mode,
                                      const pulsar_expert_bank *bank, const pulsar_expert_ptrs *shared,
                                      uint32_t n_shared, const void *xq, uint32_t in_dim, uint32_t mid_dim,
                                      uint32_t n_tok, uint64_t row_bytes, uint32_t quant, uint32_t act_op) {
    quant &= ~PULSAR_QUANT_A4_OK;
    if (!mid || !ptrs || !slot_weights || !selected || !weights || !logits || !bank || !xq || in_dim == 0 ||
        mid_dim == 0 || n_tok == 0 || k_used == 0 || k_used > n_expert || n_expert > 64u * kMaxPerLane ||
        softmax_mode > 1u || n_shared > kMaxShared || (n_shared && !shared) ||
        k_used + n_shared > kFusedMaxSlots || (act_op != 0u && act_op != 2u) || n_tok > 65535u)
        return reject("moe pair routed");
    PairRoutedLaunch l;
    l.mid = mid;
    l.ptrs_out = ptrs;
    l.slot_w_out = slot_weights;
    l.sel_out = selected;
    l.w_out = weights;
    l.logits = logits;
    l.rbias = router_bias;
    l.xq = xq;
    l.n_expert = n_expert;
    l.k_used = k_used;
    l.mode = softmax_mode;
    l.n_slots = k_used + n_shared;
    l.n_tok = n_tok;
    l.mid_dim = mid_dim;
    l.act_op = act_op;
    l.scale = weight_scale;
    l.bank = *bank;
    for (uint32_t s = 0; s < kMaxShared; s++)
        l.shared.p[s] = s < n_shared ? shared[s] : pulsar_expert_ptrs{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    l.row_bytes = row_bytes;
    l.g = fgeo_for(quant, in_dim);
    return fused_format(quant, l.g.upl, l);
}

extern "C" int pulsar_moe_down_f32(void *out, const void *ptrs, const void *slot_weights, const void *mid,
                                   uint32_t mid_dim, uint32_t out_dim, uint32_t n_used, uint32_t n_tok,
                                   uint64_t row_bytes, uint32_t quant, uint32_t add_bias) {
    quant &= ~PULSAR_QUANT_A4_OK;
    const FGeo g = fgeo_for(quant, mid_dim);
    if (!out || !ptrs || !mid || mid_dim == 0 || out_dim == 0 || n_used == 0 || n_tok == 0 ||
        n_used > kFusedMaxSlots || (add_bias && !slot_weights) || n_tok > 65535u ||
        (uint64_t)n_used * g.blocks * kActLdsPitch > kFusedMaxActLds)
        return reject("moe down f32");
    DownF32Launch l;
    l.out = out;
    l.ptrs = ptrs;
    l.slot_w = slot_weights;
    l.mid = mid;
    l.mid_dim = mid_dim;
    l.out_dim = out_dim;
    l.n_used = n_used;
    l.n_tok = n_tok;
    l.add_bias = add_bias;
    l.row_bytes = row_bytes;
    l.g = g;
    return fused_format(quant, g.upl, l);
}
