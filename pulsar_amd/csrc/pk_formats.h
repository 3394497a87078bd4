// pk_formats.h - per-format decode of one "unit" (64 weights) against the
// matching 64 q8_K activations.
//
// Every super-block of 256 values splits into 4 units, so a row of in_dim
// values has 4 * ceil(in_dim/256) units (MXFP4: ceil(in_dim/64)). A lane owns
// whole units; the 4 lanes of a super-block sit next to each other, so the
// super-block's exact int32 sums are a 2-step butterfly and the super-block
// epilogue runs in the reference's fp32 operation order on lane u == 0.
//
// Unit u of a super-block, per format (reference layout citations inline):
//   Q4_K    : chunk j = u of qs (low nibbles = values 64u..+31, high = +32..+63)
//   Q6_K    : half h = u>>1, i-range k = u&1: values 128h + 32q + 16k + i
//   Q2_K    : k = u>>1, half = u&1: values 128k + 32s + 16half + i
//   IQ2_XXS : 32-groups 2u, 2u+1 (values 64u..64u+63)
//   MXFP4   : 32-blocks 2u, 2u+1 of the row (values 64u..64u+63)
// For Q6_K and Q2_K the unit's activations are four 16-value runs 32 apart;
// for the others one 64-value run.
#pragma once

#include "pk_common.h"
#include "../../include/pulsar_iq2xxs_grid.h"

namespace pk {

// Activation slice of one unit: 64 int8 as 16 words, 4 group sums, scale.
struct Act {
    uint4 q[4];
    int32_t bs[4];
    float yd;
};

// Per-unit partial: exact integers (format-specific meaning) and, for
// MXFP4, the unit's share of the super-block's float sum.
struct Part {
    int32_t i0;
    int32_t i1;
    float f;
};

PK_DEV uint32_t byte_of(uint32_t w, uint32_t i) { return (w >> (8u * i)) & 0xffu; }
PK_DEV uint32_t byte_of(uint4 v, uint32_t i) {
    const uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return byte_of(w, i & 3u);
}
PK_DEV uint32_t byte_of(uint2 v, uint32_t i) { return byte_of(i < 4 ? v.x : v.y, i & 3u); }
PK_DEV uint32_t word_of(uint4 v, uint32_t i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}
PK_DEV int32_t sext16(uint32_t v) { return (int32_t)(int16_t)(uint16_t)v; }

// 16 activation bytes (one uint4) dotted with 16 weight bytes (4 words).
PK_DEV int32_t dot16(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, uint4 a, int32_t acc) {
    acc = dot4(w0, a.x, acc);
    acc = dot4(w1, a.y, acc);
    acc = dot4(w2, a.z, acc);
    acc = dot4(w3, a.w, acc);
    return acc;
}

// Loads the activation slice of unit g (super-block g>>2, unit g&3) of a
// q8_K row laid out with PITCH bytes per super-block, d at 0, qs at QOFF
// and bsums at BOFF. ACT_STRIDE32 selects the 4 x 16 runs 32 apart (Q6_K,
// Q2_K).
// ALIGNED: the fields sit at their natural alignment (LDS copies).
template <bool ALIGNED>
PK_DEV uint4 ldf128(const uint8_t *p) {
    if (ALIGNED) return *(const uint4 *)p;
    return ld128(p);
}
template <bool ALIGNED>
PK_DEV uint2 ldf64(const uint8_t *p) {
    if (ALIGNED) return *(const uint2 *)p;
    return ld64(p);
}

template <bool ACT_STRIDE32, int BS_MODE, uint32_t PITCH, uint32_t QOFF, uint32_t BOFF, bool ALIGNED = false>
PK_DEV void load_act_at(const uint8_t *row, uint32_t g, Act &a) {
    const uint8_t *blk = row + (uint64_t)(g >> 2) * PITCH;
    const uint32_t u = g & 3u;
    a.yd = ALIGNED ? *(const float *)blk : __builtin_bit_cast(float, ld32(blk));
    const uint8_t *qs = blk + QOFF;
    if (ACT_STRIDE32) {
        const uint32_t base = 128u * (u >> 1) + 16u * (u & 1u);
#pragma unroll
        for (int s = 0; s < 4; s++) a.q[s] = ldf128<ALIGNED>(qs + base + 32u * s);
    } else {
#pragma unroll
        for (int s = 0; s < 4; s++) a.q[s] = ldf128<ALIGNED>(qs + 64u * u + 16u * s);
    }
    const uint8_t *bs = blk + BOFF;
    if (BS_MODE == 1) {  // Q4_K: bsums[4u .. 4u+3]
        const uint2 v = ldf64<ALIGNED>(bs + 8u * u);
        a.bs[0] = sext16(v.x);
        a.bs[1] = sext16(v.x >> 16);
        a.bs[2] = sext16(v.y);
        a.bs[3] = sext16(v.y >> 16);
    } else if (BS_MODE == 2) {  // Q2_K / Q6_K: bsums[8(u>>1) + (u&1) + 2s]
        const uint4 v = ldf128<ALIGNED>(bs + 16u * (u >> 1));
        const uint32_t o = u & 1u;
        a.bs[0] = sext16(word_of(v, 0) >> (16u * o));
        a.bs[1] = sext16(word_of(v, 1) >> (16u * o));
        a.bs[2] = sext16(word_of(v, 2) >> (16u * o));
        a.bs[3] = sext16(word_of(v, 3) >> (16u * o));
    } else {
        a.bs[0] = a.bs[1] = a.bs[2] = a.bs[3] = 0;
    }
}

// From a q8_K row in global memory (292-byte blocks).
template <bool ACT_STRIDE32, int BS_MODE>
PK_DEV void load_act(const pulsar_block_q8_K *xq_row, uint32_t g, Act &a) {
    load_act_at<ACT_STRIDE32, BS_MODE, 292u, 4u, 260u>((const uint8_t *)xq_row, g, a);
}

// LDS copy of a q8_K row: 304-byte blocks, d at 0, qs at 16 (16-byte
// aligned), bsums at 272. Source dword k of a block lands at byte
// (k == 0 ? 0 : 4k + 12).
constexpr uint32_t kActLdsPitch = 304u;
PK_DEV uint32_t act_lds_offset(uint32_t k) { return k == 0 ? 0u : 4u * k + 12u; }
// Bytes between consecutive staged rows that the 16 lanes of an MFMA operand
// read together (one row per lane): the row's blocks plus 16 bytes when their
// count is even. The stride is then 4 (mod 8) dwords, so the 16 rows start in
// 16 distinct groups of 4 of the LDS's 64 four-byte banks; an even count
// alone makes it a multiple of 8 dwords (16 blocks: a multiple of 64, every
// row on the same banks).
__host__ __device__ constexpr uint32_t act_row_pitch(uint32_t k_blocks) {
    return k_blocks * kActLdsPitch + (k_blocks % 2u == 0u ? 16u : 0u);
}

template <bool ACT_STRIDE32, int BS_MODE>
PK_DEV void load_act_lds(const uint8_t *row, uint32_t g, Act &a) {
    load_act_at<ACT_STRIDE32, BS_MODE, kActLdsPitch, 16u, 272u, true>(row, g, a);
}

template <uint32_t Q>
struct Fmt;

// ---------------------------------------------------------------- Q4_K ---
// block_q4_K (pulsar_kernels.cu:1323-1328): f16 d @0, f16 dmin @2,
// scales[12] @4, qs[128] @16. Lane dot: cpu_dot.rs:250-279.
template <>
struct Fmt<PULSAR_QUANT_Q4_K> {
    static constexpr bool kHasI1 = true;  // second exact sum (min terms) in use
    static constexpr uint32_t kSbBytes = 144;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 1;
    struct W {
        uint4 hdr;     // d, dmin, scales[12]
        uint4 qa, qb;  // qs[32u .. 32u+31]
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u;
        W w;
        w.hdr = ldw128(blk);
        w.qa = ldw128(blk + 16 + 32u * u);
        w.qb = ldw128(blk + 32 + 32u * u);
        return w;
    }
    // get_scale_min_k4 (cpu_dot.rs:147-156) for j = 2u and 2u + 1
    PK_DEV static void scale_min(uint4 hdr, uint32_t j, int32_t &sc, int32_t &m) {
        // scale bytes q[i] are header bytes 4 + i
        if (j < 4) {
            sc = (int32_t)(byte_of(hdr, 4 + j) & 63u);
            m = (int32_t)(byte_of(hdr, 8 + j) & 63u);
        } else {
            sc = (int32_t)((byte_of(hdr, 8 + j) & 0x0fu) | ((byte_of(hdr, j) >> 6) << 4));
            m = (int32_t)((byte_of(hdr, 8 + j) >> 4) | ((byte_of(hdr, 4 + j) >> 6) << 4));
        }
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t u, const uint2 *) {
        const uint32_t lo = 0x0f0f0f0fu;
        int32_t s1 = 0, s2 = 0;
        s1 = dot16(w.qa.x & lo, w.qa.y & lo, w.qa.z & lo, w.qa.w & lo, a.q[0], s1);
        s1 = dot16(w.qb.x & lo, w.qb.y & lo, w.qb.z & lo, w.qb.w & lo, a.q[1], s1);
        s2 = dot16((w.qa.x >> 4) & lo, (w.qa.y >> 4) & lo, (w.qa.z >> 4) & lo, (w.qa.w >> 4) & lo, a.q[2], s2);
        s2 = dot16((w.qb.x >> 4) & lo, (w.qb.y >> 4) & lo, (w.qb.z >> 4) & lo, (w.qb.w >> 4) & lo, a.q[3], s2);
        int32_t sc1, m1, sc2, m2;
        scale_min(w.hdr, 2 * u, sc1, m1);
        scale_min(w.hdr, 2 * u + 1, sc2, m2);
        Part p;
        // every factor fits 24 bits signed: full-rate v_mul_i32_i24
        p.i0 = __mul24(sc1, s1) + __mul24(sc2, s2);
        p.i1 = __mul24(m1, a.bs[0] + a.bs[1]) + __mul24(m2, a.bs[2] + a.bs[3]);
        p.f = 0.0f;
        return p;
    }
    // total += xd*yd*isum - xmin*yd*msum  (cpu_dot.rs:276)
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        const float xd = f16f((uint16_t)w.hdr.x);
        const float xmin = f16f((uint16_t)(w.hdr.x >> 16));
        return xd * yd * (float)p.i0 - xmin * yd * (float)p.i1;
    }
};

// ---------------------------------------------------------------- Q6_K ---
// block_q6_K (pulsar_kernels.cu:1330-1335): ql[128] @0, qh[64] @128,
// int8 scales[16] @192, f16 d @208. Dot: pulsar_kernels.cu:5920-5948.
// Unit (h, k): ql[64h + 16k ..+16) carries quarters 0 (low nibble) and 2
// (high), ql[64h + 32 + 16k ..+16) quarters 1 and 3, qh[32h + 16k ..+16)
// bits 2q..2q+1 the high 2 bits; scale of quarter q is sc[8h + 2q + k].
// The 6-bit code c is used unsigned and the -32 offset folded through the
// q8_K group sum: sum (c - 32) * x = sum c * x - 32 * bsum (exact).
template <>
struct Fmt<PULSAR_QUANT_Q6_K> {
    static constexpr bool kHasI1 = false;  // second exact sum (min terms) in use
    static constexpr uint32_t kSbBytes = 210;
    static constexpr bool kStride32 = true;
    static constexpr int kBsMode = 2;
    struct W {
        uint4 la, lb, qh;
        uint2 sc;  // scales[8h .. 8h+7]
        uint32_t d;
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u, h = u >> 1, k = u & 1u;
        W w;
        w.la = ldw128(blk + 64u * h + 16u * k);
        w.lb = ldw128(blk + 64u * h + 32u + 16u * k);
        w.qh = ldw128(blk + 128u + 32u * h + 16u * k);
        w.sc = ldw64(blk + 192u + 8u * h);
        w.d = ldw16(blk + 208u);
        return w;
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t u, const uint2 *) {
        const uint32_t k = u & 1u;
        const uint32_t lo4 = 0x0f0f0f0fu, hi2 = 0x30303030u;
        // code c = low nibble | (2 high bits << 4): the high bits of quarter
        // q sit at bits 2q..2q+1 of each qh byte and move to bits 4..5
        const uint32_t qh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
        const uint32_t la[4] = {w.la.x, w.la.y, w.la.z, w.la.w};
        const uint32_t lb[4] = {w.lb.x, w.lb.y, w.lb.z, w.lb.w};
        uint32_t c[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            c[0][i] = (la[i] & lo4) | ((qh[i] << 4) & hi2);
            c[1][i] = (lb[i] & lo4) | ((qh[i] << 2) & hi2);
            c[2][i] = ((la[i] >> 4) & lo4) | (qh[i] & hi2);
            c[3][i] = ((lb[i] >> 4) & lo4) | ((qh[i] >> 2) & hi2);
        }
        // scales of this unit: bytes k, k+2, k+4, k+6 of scales[8h..8h+7]
        const uint32_t s0 = __builtin_amdgcn_alignbyte(w.sc.y, w.sc.x, k);
        const uint32_t s1 = __builtin_amdgcn_alignbyte(0u, w.sc.y, k);
        const int32_t sc[4] = {(int32_t)(s0 << 24) >> 24, (int32_t)(s0 << 8) >> 24,
                               (int32_t)(s1 << 24) >> 24, (int32_t)(s1 << 8) >> 24};
        int32_t isum = 0;
#pragma unroll
        for (int q = 0; q < 4; q++)
            isum += __mul24(sc[q], dot16(c[q][0], c[q][1], c[q][2], c[q][3], a.q[q], 0) - 32 * a.bs[q]);
        return Part{isum, 0, 0.0f};
    }
    // d * y->d * isum with d = x->d (pulsar_kernels.cu:5946)
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        const float xd = f16f((uint16_t)w.d);
        return xd * yd * (float)p.i0;
    }
};

// ---------------------------------------------------------------- Q2_K ---
// block_q2_K (pulsar_kernels.cu:1296-1301): scales[16] @0 (low nibble
// scale, high nibble min), qs[64] @16, f16 d @80, f16 dmin @82.
// Dot: cpu_dot.rs:732-767. Unit (k, half): qs[32k + 16half ..+16) shifted
// by 2s gives values 128k + 32s + 16half + i under scale byte 8k + 2s + half.
template <>
struct Fmt<PULSAR_QUANT_Q2_K> {
    static constexpr bool kHasI1 = true;  // second exact sum (min terms) in use
    static constexpr uint32_t kSbBytes = 84;
    static constexpr bool kStride32 = true;
    static constexpr int kBsMode = 2;
    struct W {
        uint4 qs;
        uint2 sc;  // scales[8k .. 8k+7]
        uint32_t dd;  // d | dmin << 16
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u, k = u >> 1, half = u & 1u;
        W w;
        w.qs = ldw128(blk + 16u + 32u * k + 16u * half);
        w.sc = ldw64(blk + 8u * k);
        w.dd = ldw32(blk + 80u);
        return w;
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t u, const uint2 *) {
        const uint32_t half = u & 1u;
        const uint32_t m2 = 0x03030303u;
        int32_t isum = 0, summs = 0;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t sh = 2u * s;
            const int32_t d = dot16((w.qs.x >> sh) & m2, (w.qs.y >> sh) & m2, (w.qs.z >> sh) & m2,
                                    (w.qs.w >> sh) & m2, a.q[s], 0);
            const uint32_t scb = byte_of(w.sc, 2u * s + half);
            isum += __mul24((int32_t)(scb & 0x0fu), d);
            summs += __mul24(a.bs[s], (int32_t)(scb >> 4));
        }
        return Part{isum, summs, 0.0f};
    }
    // yd*xd*isum - yd*xmin*summs (cpu_dot.rs:764-765)
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        const float xd = f16f((uint16_t)w.dd);
        const float xmin = f16f((uint16_t)(w.dd >> 16));
        return yd * xd * (float)p.i0 - yd * xmin * (float)p.i1;
    }
};

// ------------------------------------------------------------- IQ2_XXS ---
// block_iq2_xxs (pulsar_kernels.cu:1303-1306): f16 d @0, then per 32-group
// aux0 (4 grid indices) and aux1 (4 x 7 sign bits, 4-bit scale in 28..31).
// Dot: cpu_dot.rs:92-122. The grid lives in LDS as 256 x 8 magnitude bytes.
// The LDS table holds the 256 grid rows (8 magnitude bytes each) and, at
// kIq2SignRow + s7, the 8-byte mask of the 7-bit sign field s7: 0xff in
// byte j when value j is negated.
constexpr uint32_t kIq2SignRow = 256u, kIq2LutRows = 256u + 128u;
PK_DEV void iq2_signed8(const uint2 *lut, uint32_t idx, uint32_t s7, uint32_t &w0, uint32_t &w1) {
    const uint2 g = lut[idx];
    const uint2 m = lut[kIq2SignRow + s7];
    // per-byte two's-complement negation where the mask is set; magnitudes
    // are 8, 25 or 43, so (~g + 1) never carries into the next byte
    w0 = (g.x ^ m.x) + (m.x & 0x01010101u);
    w1 = (g.y ^ m.y) + (m.y & 0x01010101u);
}

template <>
struct Fmt<PULSAR_QUANT_IQ2_XXS> {
    static constexpr bool kHasI1 = false;  // second exact sum (min terms) in use
    static constexpr uint32_t kSbBytes = 66;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    struct W {
        uint4 aux;  // aux0_a, aux1_a, aux0_b, aux1_b
        uint32_t d;
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        W w;
        w.aux = ldw128(blk + 2u + 16u * (g & 3u));
        w.d = ldw16(blk);
        return w;
    }
    PK_DEV static int32_t group(const uint2 *lut, uint32_t aux0, uint32_t aux1, uint4 a0, uint4 a1) {
        uint32_t w[8];
#pragma unroll
        for (int k = 0; k < 4; k++)
            iq2_signed8(lut, (aux0 >> (8 * k)) & 0xffu, (aux1 >> (7 * k)) & 127u, w[2 * k], w[2 * k + 1]);
        int32_t sumi = dot16(w[0], w[1], w[2], w[3], a0, 0);
        sumi = dot16(w[4], w[5], w[6], w[7], a1, sumi);
        return __mul24(sumi, (int32_t)(2u * (aux1 >> 28) + 1u));
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *lut) {
        const int32_t b0 = group(lut, w.aux.x, w.aux.y, a.q[0], a.q[1]);
        const int32_t b1 = group(lut, w.aux.z, w.aux.w, a.q[2], a.q[3]);
        return Part{b0 + b1, 0, 0.0f};
    }
    // 0.125 * xd * yd * bsum (cpu_dot.rs:120)
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        const float xd = f16f((uint16_t)w.d);
        return 0.125f * xd * yd * (float)p.i0;
    }
};

// Fills an LDS copy of the IQ2_XXS grid (256 x 8 bytes) from the base-3
// codes and the 128 sign masks after it (kIq2LutRows rows in all); call
// from all threads of the block, then __syncthreads().
__device__ static const uint16_t k_iq2xxs_codes[256] = {PULSAR_IQ2XXS_GRID_CODES};
PK_DEV void fill_iq2xxs_lut(uint2 *lut) {
    for (uint32_t i = threadIdx.x; i < 256u; i += blockDim.x) {
        uint32_t c = k_iq2xxs_codes[i];
        uint32_t b[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t dgt = c % 3u;
            c /= 3u;
            b[j] = dgt == 0 ? 8u : dgt == 1 ? 25u : 43u;
        }
        lut[i] = make_uint2(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24),
                            b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24));
    }
    for (uint32_t s7 = threadIdx.x; s7 < 128u; s7 += blockDim.x) {
        // sign_mask (cpu_dot.rs:66-70): bit 7 completes even parity
        const uint32_t s = s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7);
        uint32_t m[2] = {0u, 0u};
#pragma unroll
        for (int j = 0; j < 8; j++)
            if ((s >> j) & 1u) m[j >> 2] |= 0xffu << (8 * (j & 3));
        lut[kIq2SignRow + s7] = make_uint2(m[0], m[1]);
    }
}

// --------------------------------------------------------------- MXFP4 ---
// block_mxfp4 (pulsar_kernels.cu:1424-1430): E8M0 e @0, qs[16] @1 (low
// nibble = value i, high = i + 16). Rows pack 17-byte blocks. Dot:
// pulsar_kernels.cu:5715-5741 with the doubled E2M1 table and the
// 2^(e-128) scale (e < 2 flushes to 0).
// Doubled E2M1 values {0,1,2,3,4,6,8,12} and their negatives, selected per
// byte by v_perm_b32 on the code's low 3 bits and blended on its sign bit.
// The blend mask comes from v_perm_b32 too: selectors 8, 9, 10, 11 give
// 0xff / 0x00 from bit 15 / 31 of the low source word and bit 15 / 31 of
// the high one, so each byte's sign bit is first moved to one of those.
PK_DEV uint32_t mxfp4_pick(uint32_t sel, uint32_t m) {
    const uint32_t pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, sel);
    const uint32_t neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, sel);
    return (neg & m) | (pos & ~m);
}
// codes in bits 0..3 of each byte of n (bits 4..7 ignored)
PK_DEV uint32_t mxfp4_kv4(uint32_t n) {
    // byte k's sign (bit 8k + 3) -> bit 15 / 31 of (n << 12) for k = 0, 2
    // and of (n << 4) for k = 1, 3
    const uint32_t m = __builtin_amdgcn_perm(n << 12, n << 4, 0x090B080Au);
    return mxfp4_pick(n & 0x07070707u, m);
}
// codes in bits 4..7 of each byte of q
PK_DEV uint32_t mxfp4_kv4_hi(uint32_t q) {
    // byte k's sign (bit 8k + 7) -> bit 15 / 31 of (q << 8) for k = 0, 2
    // and of q for k = 1, 3
    const uint32_t m = __builtin_amdgcn_perm(q << 8, q, 0x090B080Au);
    return mxfp4_pick((q >> 4) & 0x07070707u, m);
}
PK_DEV float mxfp4_scale_half(uint32_t e) {
    return e < 2u ? 0.0f : __builtin_bit_cast(float, (e - 1u) << 23);
}
PK_DEV int32_t mxfp4_block(uint4 q, uint4 a0, uint4 a1) {
    int32_t s = dot16(mxfp4_kv4(q.x), mxfp4_kv4(q.y), mxfp4_kv4(q.z), mxfp4_kv4(q.w), a0, 0);
    s = dot16(mxfp4_kv4_hi(q.x), mxfp4_kv4_hi(q.y), mxfp4_kv4_hi(q.z), mxfp4_kv4_hi(q.w), a1, s);
    return s;
}

template <>
struct Fmt<PULSAR_QUANT_MXFP4> {
    static constexpr bool kHasI1 = false;  // second exact sum (min terms) in use
    static constexpr uint32_t kSbBytes = 136;  // 8 blocks per 256 values
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    struct W {
        uint4 q0, q1;
        uint32_t e;  // e0 | e1 << 8; e1 = 0 when the second block is absent
        uint32_t two;  // 1 when the unit holds two blocks
    };
    // n_blocks = valid 32-blocks in the row
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t n_blocks) {
        const uint8_t *p = row + 34ull * g;
        W w;
        w.two = 2u * g + 1u < n_blocks ? 1u : 0u;
        // a unit without a second block (odd block count) re-reads its
        // first block instead of reading past the row
        const uint8_t *p1 = w.two ? p + 17 : p;
        w.q0 = ldw128(p + 1);
        w.q1 = ldw128(p1 + 1);
        w.e = ldw8(p) | ((w.two ? ldw8(p1) : 0u) << 8);
        return w;
    }
    // the same unit from an LDS copy of the row (row = the row's first byte)
    PK_DEV static W load_lds(const uint8_t *row, uint32_t g, uint32_t n_blocks) {
        const uint8_t *p = row + 34u * g;
        W w;
        w.two = 2u * g + 1u < n_blocks ? 1u : 0u;
        const uint8_t *p1 = w.two ? p + 17 : p;
        w.q0 = lds128u(p + 1);
        w.q1 = lds128u(p1 + 1);
        w.e = lds8(p) | ((w.two ? lds8(p1) : 0u) << 8);
        return w;
    }
    // sumf += scale_half(e) * sumi for each block with sumi != 0, in block order
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *) {
        const int32_t s0 = mxfp4_block(w.q0, a.q[0], a.q[1]);
        const int32_t s1 = w.two ? mxfp4_block(w.q1, a.q[2], a.q[3]) : 0;  // select, both computed
        // fma == the reference's multiply-add here (exact product of a power
        // of two and an int < 2^24), and a zero sum adds +0, which leaves a
        // sum that is never -0 unchanged: no test on s0 / s1 needed
        float f = __builtin_fmaf(mxfp4_scale_half(w.e & 0xffu), (float)s0, 0.0f);
        f = __builtin_fmaf(mxfp4_scale_half(w.e >> 8), (float)s1, f);
        return Part{s0, s1, f};
    }
    // y->d * sumf
    PK_DEV static float sb_value(const W &, float yd, const Part &p) { return yd * p.f; }
};

}  // namespace pk

#include "pk_formats_ext.h"

namespace pk {

// Per-format LDS table of the lane kernels (kRows uint2 rows; 1 = none)
// and its fill, by all threads of the block before a __syncthreads().
template <uint32_t Q, typename = void>
struct FmtLut {
    static constexpr uint32_t kRows = 1;
    PK_DEV static void fill(uint2 *) {}
};
template <>
struct FmtLut<PULSAR_QUANT_IQ2_XXS> {
    static constexpr uint32_t kRows = kIq2LutRows;
    PK_DEV static void fill(uint2 *lut) { fill_iq2xxs_lut(lut); }
};
template <uint32_t Q>
struct FmtLut<Q, decltype((void)Fmt<Q>::kLutRows)> {
    static constexpr uint32_t kRows = Fmt<Q>::kLutRows;
    PK_DEV static void fill(uint2 *lut) { Fmt<Q>::fill_lut(lut); }
};

// Formats whose super-block value is a float sum of per-block terms (the
// unit's float partial is reduced across the quad instead of integers).
template <uint32_t Q>
constexpr bool kFloatPart = Q == PULSAR_QUANT_MXFP4 || Q == PULSAR_QUANT_Q8_0 || Q == PULSAR_QUANT_Q4_0 ||
                            Q == PULSAR_QUANT_Q5_1 || Q == PULSAR_QUANT_IQ4_NL || Q == PULSAR_QUANT_NVFP4;

}  // namespace pk

// Declares and fills the format's LDS table `lut` (every thread of the
// block must reach it).
#define PK_FMT_LUT(Q)                                   \
    __shared__ uint2 lut[pk::FmtLut<Q>::kRows];         \
    if constexpr (pk::FmtLut<Q>::kRows > 1) {           \
        pk::FmtLut<Q>::fill(lut);                       \
        __syncthreads();                                \
    }

// Switch over every expert format: F(Q) per code.
#define PK_FOR_EACH_QUANT(F)                                                                    \
    F(PULSAR_QUANT_Q2_K) F(PULSAR_QUANT_IQ2_XXS) F(PULSAR_QUANT_Q4_K) F(PULSAR_QUANT_Q5_K)      \
    F(PULSAR_QUANT_Q6_K) F(PULSAR_QUANT_Q3_K) F(PULSAR_QUANT_IQ2_XS) F(PULSAR_QUANT_IQ3_XXS)    \
    F(PULSAR_QUANT_Q4_0) F(PULSAR_QUANT_Q5_1) F(PULSAR_QUANT_Q8_0) F(PULSAR_QUANT_IQ4_XS)       \
    F(PULSAR_QUANT_MXFP4) F(PULSAR_QUANT_IQ4_NL) F(PULSAR_QUANT_IQ3_S) F(PULSAR_QUANT_IQ2_S)    \
    F(PULSAR_QUANT_IQ1_S) F(PULSAR_QUANT_NVFP4)
