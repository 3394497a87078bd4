// pk_rowdot.h - one wave computes the dot products of `rpp` rows with q8_K
// activations, lanes spread over the row's units.
//
// Lane layout: a row is covered by `lpr` lanes (a power of two, >= 4 and
// >= the unit count, capped at 64), so a wave holds rpp = 64 / lpr rows.
// Lane `lir` of a row owns units lir, lir + lpr, lir + 2 lpr, ... (UPLMAX
// at most). The four lanes of a super-block are adjacent; their exact
// int32 partials meet in the quad's last lane (two DPP row_shr adds), which
// forms the super-block's fp32 value in the reference's operation order.
// Those values are then summed into the row group's last lane with DPP
// row_shr / row_bcast adds, a fixed fp32 tree.
#pragma once

#include "pk_formats.h"

namespace pk {

struct RowGeom {
    uint32_t n_units;   // units per row
    uint32_t nblk32;    // 32-value blocks per row (MXFP4 tail bound)
    uint32_t lpr_log2;  // lanes per row = 1 << lpr_log2
    uint32_t lir;       // this lane's index within its row group
    uint32_t rip;       // this lane's row within the wave (0 .. rpp-1)
    // the lane that ends with the row's value (the group's last lane)
    PK_DEV bool holds_row() const { return lir == (1u << lpr_log2) - 1u; }
};

// Chooses the lane layout for a row of n_units units.
static inline uint32_t lpr_log2_for(uint32_t n_units) {
    uint32_t l = 2;
    while ((1u << l) < n_units && l < 6) l++;
    return l;
}
static inline uint32_t units_per_row(uint32_t quant, uint32_t in_dim) {
    if (quant == PULSAR_QUANT_MXFP4) return (in_dim + 63u) / 64u;
    return 4u * ((in_dim + 255u) / 256u);
}

// Row geometry of a matrix stage: units per row, 32-value blocks, lanes
// per row (log2), units per lane and q8_K blocks per activation row.
struct FGeo {
    uint32_t n_units, nblk32, l2, upl, blocks;
};
static FGeo fgeo_for(uint32_t quant, uint32_t k_dim) {
    FGeo g;
    g.n_units = units_per_row(quant, k_dim);
    g.nblk32 = (k_dim + 31u) / 32u;
    g.l2 = lpr_log2_for(g.n_units);
    g.upl = (g.n_units + (1u << g.l2) - 1u) >> g.l2;
    g.blocks = (k_dim + 255u) / 256u;
    return g;
}

// L2 > 0 fixes lanes-per-row at compile time (1 << L2); with L2 == 6 a
// wave holds one row, so row addresses stay wave-uniform (scalar).
template <uint32_t L2 = 0>
PK_DEV RowGeom row_geom(uint32_t n_units, uint32_t nblk32, uint32_t lpr_log2_rt) {
    const uint32_t lpr_log2 = L2 ? L2 : lpr_log2_rt;
    const uint32_t lane = threadIdx.x & 63u;
    RowGeom g;
    g.n_units = n_units;
    g.nblk32 = nblk32;
    g.lpr_log2 = lpr_log2;
    g.lir = lane & ((1u << lpr_log2) - 1u);
    g.rip = lane >> lpr_log2;
    return g;
}

template <uint32_t Q>
PK_DEV void load_unit_act(const pulsar_block_q8_K *xq_row, uint32_t g, Act &a) {
    load_act<Fmt<Q>::kStride32, Fmt<Q>::kBsMode>(xq_row, g, a);
}

// Loads this lane's activation slices (UPLMAX units) of one q8_K row. A
// slice is loaded whenever its super-block exists, also for the missing
// units of a MXFP4 tail super-block: q8_K blocks are always whole (their
// tail is zero), and the quad's epilogue needs the block scale on every lane.
template <uint32_t Q, uint32_t UPLMAX>
PK_DEV void load_row_acts(const pulsar_block_q8_K *xq_row, const RowGeom &rg, Act (&a)[UPLMAX]) {
#pragma unroll
    for (uint32_t i = 0; i < UPLMAX; i++) {
        const uint32_t g = rg.lir + (i << rg.lpr_log2);
        if ((g & ~3u) < rg.n_units) load_unit_act<Q>(xq_row, g, a[i]);
    }
}

// The same from an LDS copy of the row (load_act_lds layout).
template <uint32_t Q, uint32_t UPLMAX>
PK_DEV void load_row_acts_lds(const uint8_t *row, const RowGeom &rg, Act (&a)[UPLMAX]) {
#pragma unroll
    for (uint32_t i = 0; i < UPLMAX; i++) {
        const uint32_t g = rg.lir + (i << rg.lpr_log2);
        if ((g & ~3u) < rg.n_units) load_act_lds<Fmt<Q>::kStride32, Fmt<Q>::kBsMode>(row, g, a[i]);
    }
}

// Two bsums (int16 halves of x) and two more (y) -> their low 7 bits
// (high = false, l = b & 127) or the rest (high = true, h = b >> 7), one
// byte each: b = 128 h + l exactly, l in [0, 128), |h| <= 16 for the sums
// of 16 int8 the quantizer writes. Both splits are formed and one kept by
// a select (a divergent branch here would split the caller's hot loop).
typedef short pk_short2 __attribute__((ext_vector_type(2)));
PK_DEV uint32_t bsum_bytes(uint32_t x, uint32_t y, bool high) {
    const uint32_t hx = __builtin_bit_cast(uint32_t, __builtin_bit_cast(pk_short2, x) >> (short)7);  // h = b >> 7
    const uint32_t hy = __builtin_bit_cast(uint32_t, __builtin_bit_cast(pk_short2, y) >> (short)7);
    const uint32_t lx = x & 0x007f007fu, ly = y & 0x007f007fu;  // l = b & 127
    return __builtin_amdgcn_perm(high ? hy : ly, high ? hx : lx, 0x06040200u);  // bytes 0, 2 of x, then of y
}

// Block-wide copy of m q8_K rows (k_blocks blocks each) into LDS in the
// load_act_lds layout, row j at byte j * row_pitch; row j comes from the
// global q8_K row src_row(j).
// A block is copied as 16 + 2 16-byte pieces (qs, bsums) and its d, all
// loads of a batch of B per thread issued before their stores (B trades
// registers for loads in flight). SPLIT: each bsums piece (8 int16) is
// stored as the int8 bytes of its 128 h + l split instead, l bytes of the
// 8 sums then h bytes (the operands of the grouped Q2_K min-term MFMAs).
template <uint32_t B, bool SPLIT = false, typename RowFn>
PK_DEV void stage_q8_rows(uint8_t *lds, uint32_t m, uint32_t k_blocks, uint32_t row_pitch, RowFn src_row) {
    const uint32_t per_row = k_blocks * 19u, total = m * per_row;
    for (uint32_t base = threadIdx.x; base < total; base += B * blockDim.x) {
        uint4 v[B];
        uint32_t dst[B];
        bool is_d[B], is_bs[B];
#pragma unroll
        for (uint32_t u = 0; u < B; u++) {
            const uint32_t it = base + u * blockDim.x;
            dst[u] = UINT32_MAX;
            is_d[u] = is_bs[u] = false;
            if (it < total) {
                const uint32_t j = it / per_row, r = it - j * per_row, sb = r / 19u, c = r - sb * 19u;
                const uint8_t *src = (const uint8_t *)src_row(j) + (uint64_t)sb * 292u;
                // pieces 0..15: qs (source 4 + 16c), 16, 17: bsums (260, 276), 18: d (0)
                const uint32_t so = c < 16u ? 4u + 16u * c : c == 16u ? 260u : c == 17u ? 276u : 0u;
                const uint32_t dofs = c < 16u ? 16u + 16u * c : c == 16u ? 272u : c == 17u ? 288u : 0u;
                dst[u] = j * row_pitch + sb * kActLdsPitch + dofs;
                is_d[u] = c == 18u;
                is_bs[u] = c == 16u || c == 17u;
                v[u] = c < 18u ? ld128(src + so) : make_uint4(ld32(src), 0u, 0u, 0u);
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < B; u++) {
            if (dst[u] == UINT32_MAX) continue;
            if (is_d[u]) {
                *(uint32_t *)(lds + dst[u]) = v[u].x;  // d
            } else {
                uint4 x = v[u];
                if (SPLIT && is_bs[u])
                    x = make_uint4(bsum_bytes(v[u].x, v[u].y, false), bsum_bytes(v[u].z, v[u].w, false),
                                   bsum_bytes(v[u].x, v[u].y, true), bsum_bytes(v[u].z, v[u].w, true));
                *(uint4 *)(lds + dst[u]) = x;
            }
        }
    }
}

// Row value pieces (defined below): row_partial leaves each super-block's
// value in its quad's last lane, row_finish sums them into the row group's
// last lane.
template <uint32_t Q, uint32_t UPLMAX>
PK_DEV float row_partial(bool row_ok, const RowGeom &rg, const typename Fmt<Q>::W (&w)[UPLMAX],
                         const Act (&a)[UPLMAX], const uint2 *lut);
PK_DEV float row_finish(float acc, const RowGeom &rg);

// Loads this lane's weight units of one row. Loads are unconditional: a
// lane whose unit does not exist reads the row's last unit instead (in
// bounds) and row_partial masks its contribution; callers likewise pass a
// valid row for rows past the matrix. No predicated loads in the hot loop.
template <uint32_t Q, uint32_t UPLMAX>
PK_DEV void load_row_w(const uint8_t *row, const RowGeom &rg, typename Fmt<Q>::W (&w)[UPLMAX]) {
#pragma unroll
    for (uint32_t i = 0; i < UPLMAX; i++) {
        // no branch around the loads, not even a uniform one: every call
        // issues the same loads, so the waits that follow count exactly
        const uint32_t g = rg.lir + (i << rg.lpr_log2);
        w[i] = Fmt<Q>::load(row, g < rg.n_units ? g : rg.n_units - 1u, rg.nblk32);
    }
}

// ------------------------------------------------ MXFP4 row staging --
// MXFP4 rows are runs of 17-byte blocks, so a lane's unit (two blocks)
// starts at an odd byte and its 16-byte loads straddle 16-byte lines: on
// 2880-wide expert rows such loads move the slab at ~3.0 TB/s where aligned
// 16-byte pieces of the same rows move at ~4.7 TB/s. A wave that holds one
// row (64 lanes per row) copies the row's byte span into its LDS area as
// aligned pieces, NPL per lane (clamped to the span, so every lane issues
// every load), and its lanes then read their units from LDS.
template <uint32_t NPL>
struct SpanStage {
    uint4 v[NPL];
    uint32_t skew, np;
    PK_DEV void issue(const uint8_t *row, uint32_t nbytes) {
        const uintptr_t a = (uintptr_t)row;
        skew = (uint32_t)(a & 15u);
        np = (skew + nbytes + 15u) >> 4;
        const uint8_t *a0 = row - skew;
        const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
        for (uint32_t j = 0; j < NPL; j++) {
            const uint32_t p = lane + 64u * j;
            v[j] = ldw128(a0 + 16u * (p < np ? p : np - 1u));
        }
    }
    // Writes the pieces to the wave's area (NPL KiB, 16-byte aligned) and
    // returns the LDS address of the row's first byte.
    PK_DEV const uint8_t *store(uint8_t *lds) const {
        const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
        for (uint32_t j = 0; j < NPL; j++) {
            const uint32_t p = lane + 64u * j;
            if (p < np) *(uint4 *)(lds + 16u * p) = v[j];
        }
        return lds + skew;
    }
};

// Stores of a wave to its own LDS area become visible to its other lanes.
PK_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The lane's units of a row staged by SpanStage (load_row_w's unit choice).
template <uint32_t UPLMAX>
PK_DEV void load_row_w_lds(const uint8_t *row, const RowGeom &rg, Fmt<PULSAR_QUANT_MXFP4>::W (&w)[UPLMAX]) {
#pragma unroll
    for (uint32_t i = 0; i < UPLMAX; i++) {
        const uint32_t g = rg.lir + (i << rg.lpr_log2);
        w[i] = Fmt<PULSAR_QUANT_MXFP4>::load_lds(row, g < rg.n_units ? g : rg.n_units - 1u, rg.nblk32);
    }
}

// The lane's units of one row (NPL == 0: load_row_w; else staged through
// the wave's NPL KiB of LDS; blocks of at most MAXW waves).
template <uint32_t Q, uint32_t UPLMAX, uint32_t NPL, uint32_t MAXW = 4>
PK_DEV void load_one_row(const uint8_t *row, const RowGeom &rg, typename Fmt<Q>::W (&w)[UPLMAX]) {
    if constexpr (NPL == 0) {
        load_row_w<Q, UPLMAX>(row, rg, w);
    } else {
        __shared__ __align__(16) uint8_t stage[MAXW][NPL * 1024u];
        SpanStage<NPL> st;
        st.issue(row, 17u * rg.nblk32);
        const uint8_t *l = st.store(stage[threadIdx.x / 64u]);
        wave_lds_sync();
        load_row_w_lds<UPLMAX>(l, rg, w);
        wave_lds_sync();  // read before the wave's next staging overwrites them
    }
}

// A wave's gate / up row pair, one pass ahead: issue() starts the loads
// of the next pass (into registers: the units, or for NPL > 0 the aligned
// pieces of the MXFP4 rows), land() makes them the current units wg / wu
// (through the wave's 2 NPL KiB of LDS when staged; blocks of at most MAXW
// waves). The loads of pass k+1 are in flight while pass k is computed.
template <uint32_t Q, uint32_t UPLMAX, uint32_t NPL, uint32_t MAXW = 4>
struct PairRowPipe {
    typename Fmt<Q>::W wg[UPLMAX], wu[UPLMAX];
    typename Fmt<Q>::W ng[NPL ? 1 : UPLMAX], nu[NPL ? 1 : UPLMAX];
    SpanStage<NPL ? NPL : 1> sg, su;
    PK_DEV void issue(const uint8_t *grow, const uint8_t *urow, const RowGeom &rg) {
        if constexpr (NPL == 0) {
            load_row_w<Q, UPLMAX>(grow, rg, ng);
            load_row_w<Q, UPLMAX>(urow, rg, nu);
        } else {
            sg.issue(grow, 17u * rg.nblk32);
            su.issue(urow, 17u * rg.nblk32);
        }
    }
    PK_DEV void land(const RowGeom &rg) {
        if constexpr (NPL == 0) {
#pragma unroll
            for (uint32_t i = 0; i < UPLMAX; i++) {
                wg[i] = ng[i];
                wu[i] = nu[i];
            }
        } else {
            __shared__ __align__(16) uint8_t stage[MAXW][2][NPL * 1024u];
            uint8_t(&mine)[2][NPL * 1024u] = stage[threadIdx.x / 64u];
            const uint8_t *lg = sg.store(mine[0]);
            const uint8_t *lu = su.store(mine[1]);
            wave_lds_sync();
            load_row_w_lds<UPLMAX>(lg, rg, wg);
            load_row_w_lds<UPLMAX>(lu, rg, wu);
            wave_lds_sync();  // read before the next land() overwrites them
        }
    }
};

// The pair stage of RPW consecutive row passes of one (token, slot):
// mid_row[row] = glu(gate . x + gate_b, up . x + up_b) * w for the wave's
// rows (pulsar_kernels.cu:2606-2612: bias on the projection output, then
// the combine, then the router weight). Blocks of at most MAXW waves.
template <uint32_t Q, uint32_t UPLMAX, uint32_t NPL, uint32_t RPW, uint32_t MAXW = 4>
PK_DEV void pair_passes(float *mid_row, const pulsar_expert_ptrs &p, float w, const Act (&a)[UPLMAX],
                        const RowGeom &rg, uint32_t pass0, uint32_t mid_dim, uint64_t row_bytes, uint32_t act_op,
                        const uint2 *lut) {
    const uint32_t rpp = 64u >> rg.lpr_log2;
    PairRowPipe<Q, UPLMAX, NPL, MAXW> pipe;
    auto off = [&](uint32_t k) {
        const uint32_t row = (pass0 + k) * rpp + rg.rip;
        return (uint64_t)(row < mid_dim ? row : 0u) * row_bytes;
    };
    pipe.issue(as_global(p.gate) + off(0), as_global(p.up) + off(0), rg);
    pipe.land(rg);
#pragma unroll
    for (uint32_t k = 0; k < RPW; k++) {
        if (k + 1u < RPW) pipe.issue(as_global(p.gate) + off(k + 1u), as_global(p.up) + off(k + 1u), rg);
        const uint32_t row = (pass0 + k) * rpp + rg.rip;
        const bool row_ok = row < mid_dim;
        float g = row_finish(row_partial<Q, UPLMAX>(row_ok, rg, pipe.wg, a, lut), rg);
        float u = row_finish(row_partial<Q, UPLMAX>(row_ok, rg, pipe.wu, a, lut), rg);
        if (row_ok && rg.holds_row()) {
            if (p.gate_b) g += ldwf(p.gate_b + row);
            if (p.up_b) u += ldwf(p.up_b + row);
            mid_row[row] = glu(g, u, act_op) * w;
        }
        if (k + 1u < RPW) pipe.land(rg);
    }
}

// Pieces per lane for staging an MXFP4 row of nblk32 blocks with UPLMAX
// units per lane, or 0 when the row is not staged (several rows per wave,
// or wider than the instantiated staging).
static inline uint32_t mx_stage_npl(uint32_t quant, uint32_t lpr_log2, uint32_t upl, uint32_t nblk32) {
    if (quant != PULSAR_QUANT_MXFP4 || lpr_log2 != 6u || upl > 2u) return 0;
    const uint32_t need = (17u * nblk32 + 30u + 1023u) / 1024u;
    return need <= 2u * upl ? 2u * upl : need <= 2u * upl + 1u ? 2u * upl + 1u : 0u;
}

// F::template go<Q, U, NPL>() with the MXFP4 staging depth for the
// geometry g (l2, nblk32; NPL 0: units loaded from global memory directly).
template <uint32_t Q, uint32_t U, typename G, typename F>
static int with_stage(const G &g, F &f) {
    if constexpr (Q == PULSAR_QUANT_MXFP4 && U <= 2u) {
        const uint32_t npl = mx_stage_npl(Q, g.l2, U, g.nblk32);
        if (npl == 2u * U) return f.template go<Q, U, 2u * U>();
        if (npl == 2u * U + 1u) return f.template go<Q, U, 2u * U + 1u>();
    }
    return f.template go<Q, U, 0>();
}

// This lane's share of the row value: the last lane of each super-block
// quad holds that super-block's value, every other lane 0. All lanes must
// call it (it exchanges across lanes).
template <uint32_t Q, uint32_t UPLMAX>
PK_DEV float row_partial(bool row_ok, const RowGeom &rg, const typename Fmt<Q>::W (&w)[UPLMAX],
                         const Act (&a)[UPLMAX], const uint2 *lut) {
    float acc = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < UPLMAX; i++) {
        const uint32_t g = rg.lir + (i << rg.lpr_log2);
        if ((i << rg.lpr_log2) >= rg.n_units) continue;  // uniform: no unit of this lane set exists
        const bool ok = row_ok && g < rg.n_units;
        // the super-block exists when its first unit does (a MXFP4 tail
        // super-block may hold fewer than 4 units)
        const bool sb_ok = row_ok && (g & ~3u) < rg.n_units && (g & 3u) == 3u;
        // computed on every lane (missing units hold zeroed weights) and
        // masked afterwards: no divergent branch in the hot loop
        Part p = Fmt<Q>::part(w[i], a[i], g & 3u, lut);
        p.i0 = ok ? p.i0 : 0;
        p.i0 += dpp_shr<1>(p.i0);
        p.i0 += dpp_shr<2>(p.i0);
        if (Fmt<Q>::kHasI1) {
            p.i1 = ok ? p.i1 : 0;
            p.i1 += dpp_shr<1>(p.i1);
            p.i1 += dpp_shr<2>(p.i1);
        }
        if (kFloatPart<Q>) {
            p.f = ok ? p.f : 0.0f;
            p.f += dpp_shr<1>(p.f);
            p.f += dpp_shr<2>(p.f);
        }
        const float v = Fmt<Q>::sb_value(w[i], a[i].yd, p);
        acc += sb_ok ? v : 0.0f;
    }
    return acc;
}

// Completes the row value in the row group's last lane (rg.holds_row()),
// from quads whose last lane holds a value.
PK_DEV float row_finish(float acc, const RowGeom &rg) {
    const uint32_t l2 = rg.lpr_log2;  // uniform
    if (l2 >= 3) acc += dpp_shr<4>(acc);
    if (l2 >= 4) acc += dpp_shr<8>(acc);
    if (l2 >= 5) acc += dpp_bcast15(acc);
    if (l2 >= 6) acc += dpp_bcast31(acc);
    return acc;
}

}  // namespace pk
