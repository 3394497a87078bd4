// pk_rowdot.h - one wave computes the dot products of `rpp` rows with q8_K
// activations, lanes spread over the row's units.
//
// Lane layout: a row is covered by `lpr` lanes (a power of two, >= 4 and
// >= the unit count, capped at 64), so a wave holds rpp = 64 / lpr rows.
// Lane `lir` of a row owns units lir, lir + lpr, lir + 2 lpr, ... (UPLMAX
// at most). The four lanes of a super-block are adjacent, their exact
// int32 partials meet in a 2-step DPP butterfly, and every lane of the quad
// forms the super-block's fp32 value in the reference's operation order.
// The quads' values are then summed over the row's lanes in a fixed fp32
// tree.
#pragma once

#include "pk_formats.h"

namespace pk {

struct RowGeom {
    uint32_t n_units;   // units per row
    uint32_t nblk32;    // 32-value blocks per row (MXFP4 tail bound)
    uint32_t lpr_log2;  // lanes per row = 1 << lpr_log2
    uint32_t lir;       // this lane's index within its row group
    uint32_t rip;       // this lane's row within the wave (0 .. rpp-1)
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

PK_DEV RowGeom row_geom(uint32_t n_units, uint32_t nblk32, uint32_t lpr_log2) {
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

// Loads this lane's weight units of one row.
template <uint32_t Q, uint32_t UPLMAX>
PK_DEV void load_row_w(const uint8_t *row, bool row_ok, const RowGeom &rg,
                       typename Fmt<Q>::W (&w)[UPLMAX]) {
#pragma unroll
    for (uint32_t i = 0; i < UPLMAX; i++) {
        const uint32_t g = rg.lir + (i << rg.lpr_log2);
        if (row_ok && g < rg.n_units) w[i] = Fmt<Q>::load(row, g, rg.nblk32);
    }
}

// This lane's share of the row value: every lane of a super-block's quad
// ends with that super-block's value (the quad's integer sums meet in the
// butterfly, and each lane forms the same fp32 epilogue from them). All
// lanes must call it (it exchanges across lanes).
template <uint32_t Q, uint32_t UPLMAX>
PK_DEV float row_partial(bool row_ok, const RowGeom &rg, const typename Fmt<Q>::W (&w)[UPLMAX],
                         const Act (&a)[UPLMAX], const uint2 *lut) {
    float acc = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < UPLMAX; i++) {
        const uint32_t g = rg.lir + (i << rg.lpr_log2);
        if ((i << rg.lpr_log2) >= rg.n_units) break;  // uniform: no unit of this lane set exists
        const bool ok = row_ok && g < rg.n_units;
        // the super-block exists when its first unit does (a MXFP4 tail
        // super-block may hold fewer than 4 units)
        const bool sb_ok = row_ok && (g & ~3u) < rg.n_units;
        Part p = {0, 0, 0.0f};
        if (ok) p = Fmt<Q>::part(w[i], a[i], g & 3u, lut);
        p.i0 = group_sum<4>(p.i0);
        p.i1 = group_sum<4>(p.i1);
        if (Q == PULSAR_QUANT_MXFP4) p.f = group_sum<4>(p.f);
        if (sb_ok) acc += Fmt<Q>::sb_value(w[i], a[i].yd, p);
    }
    return acc;
}

// Completes the row value across the row's lanes, starting from quads that
// each hold one value (result in every lane of the row group).
PK_DEV float row_finish(float acc, const RowGeom &rg) {
    return group_sum_from(acc, 4u, 1u << rg.lpr_log2);
}

}  // namespace pk
