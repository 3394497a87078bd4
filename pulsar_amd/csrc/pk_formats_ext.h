// pk_formats_ext.h - the unit decoders of the remaining expert formats
// (pulsar_kernels.cu:2649-2668 codes 3, 5-11, 13-17), in the framework of
// pk_formats.h: a unit is 64 values of one super-block, the lane's exact
// integer partials (i0, i1) or, for formats with a float scale per 32 or
// 16 values, its float partial (f) meet in the quad's last lane, and
// sb_value forms the super-block value.
//
// Unit u of a super-block, per format:
//   Q5_K    : chunk u (values 64u..64u+63), as Q4_K plus qh bits 2u, 2u+1
//   Q3_K    : half h = u>>1, l-half = u&1: values 128h + 32s + 16(u&1) + i
//   IQ2_XS, IQ3_XXS, IQ3_S, IQ2_S, IQ1_S : 32-groups 2u, 2u+1
//   IQ4_XS  : sub-blocks 2u, 2u+1
//   Q8_0, Q4_0, Q5_1, IQ4_NL : 32-value blocks 2u, 2u+1
//   NVFP4   : 64-value block u (four 16-value sub-blocks)
#pragma once

#include "../../include/pulsar_iq_grids.h"

namespace pk {

// ------------------------------------------------------- shared helpers --

// Spreads the 4 low bits of x to bit 0 of bytes 0..3 (the shifted copies
// of x do not overlap, so the product has no carries between them).
PK_DEV uint32_t spread4(uint32_t x) { return ((x & 0xfu) * 0x00204081u) & 0x01010101u; }

// Per-byte negation of 8 magnitude bytes g where the 8-byte mask m is 0xff
// (magnitudes are below 128: ~g + 1 never carries across bytes).
PK_DEV uint2 apply_signs(uint2 g, uint2 m) {
    return make_uint2((g.x ^ m.x) + (m.x & 0x01010101u), (g.y ^ m.y) + (m.y & 0x01010101u));
}

// 8-byte mask of a sign byte s: 0xff in byte j when bit j of s is set.
PK_DEV uint2 sign_bytes_mask(uint32_t s) {
    return make_uint2(spread4(s) * 0xffu, spread4(s >> 4) * 0xffu);
}

// kvalues_iq4nl (pulsar_kernels.cu:5602-5603, 5840-5841) per byte by
// v_perm_b32 on the code's low 3 bits, blended on bit 3: codes in bits
// 0..3 of each byte of n (bits 4..7 ignored).
PK_DEV uint32_t iq4nl_kv4(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    // {-127,-104,-83,-65} {-49,-35,-22,-10} / {1,13,25,38} {53,69,89,113}
    const uint32_t lo = __builtin_amdgcn_perm(0xF6EADDCFu, 0xBFAD9881u, sel);
    const uint32_t hi = __builtin_amdgcn_perm(0x71594535u, 0x26190D01u, sel);
    const uint32_t m = ((n >> 3) & 0x01010101u) * 0xffu;
    return (hi & m) | (lo & ~m);
}

// ------------------------------------------------------------ IQ grids --
// LDS tables (uint2 rows): grids expanded from include/pulsar_iq_grids.h,
// sign masks of the 7-bit ksigns index (cpu_dot.rs:66-70) or of an
// explicit sign byte. Filled by all threads of the block before use.

__device__ static const uint16_t k_iq2xs_codes[512] = {PULSAR_IQ2XS_GRID_CODES};
__device__ static const uint16_t k_iq2s_codes[1024] = {PULSAR_IQ2S_GRID_CODES};
__device__ static const uint16_t k_iq3xxs_codes[256] = {PULSAR_IQ3XXS_GRID_CODES};
__device__ static const uint16_t k_iq3s_codes[512] = {PULSAR_IQ3S_GRID_CODES};
__device__ static const uint16_t k_iq1s_codes[2048] = {PULSAR_IQ1S_GRID_CODES};

// 8 bytes of a base-3 code: digit j -> v[digit] in byte j
PK_DEV uint2 base3_row(uint32_t c, uint32_t v0, uint32_t v1, uint32_t v2) {
    uint32_t b[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const uint32_t d = c % 3u;
        c /= 3u;
        b[j] = d == 0 ? v0 : d == 1 ? v1 : v2;
    }
    return make_uint2(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24), b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24));
}
// 4 bytes of a 3-bit-per-byte code through an 8-entry byte table (two words)
PK_DEV uint32_t bits3_row(uint32_t c, uint32_t t_hi, uint32_t t_lo) {
    const uint32_t sel = (c & 7u) | (((c >> 3) & 7u) << 8) | (((c >> 6) & 7u) << 16) | (((c >> 9) & 7u) << 24);
    return __builtin_amdgcn_perm(t_hi, t_lo, sel);
}
// ksigns masks for the 128 7-bit indices at rows [row0, row0 + 128)
PK_DEV void fill_ksign_rows(uint2 *lut, uint32_t row0) {
    for (uint32_t s7 = threadIdx.x; s7 < 128u; s7 += blockDim.x)
        lut[row0 + s7] = sign_bytes_mask(s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7));
}
// masks of the 256 sign bytes at rows [row0, row0 + 256)
PK_DEV void fill_sbyte_rows(uint2 *lut, uint32_t row0) {
    for (uint32_t s = threadIdx.x; s < 256u; s += blockDim.x) lut[row0 + s] = sign_bytes_mask(s);
}

// ----------------------------------------------------------------- Q5_K --
// block_q5_K (pulsar_kernels.cu:1324-1330): f16 d @0, f16 dmin @2,
// scales[12] @4, qh[32] @16, qs[128] @48. Dot: pulsar_kernels.cu:5892-5918
// (Q4_K's, with value 64u + i gaining bit 2u of qh[i] as its fifth bit,
// value 64u + 32 + i bit 2u + 1).
template <>
struct Fmt<PULSAR_QUANT_Q5_K> {
    static constexpr bool kHasI1 = true;
    static constexpr uint32_t kSbBytes = 176;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 1;
    struct W {
        uint4 hdr;     // d, dmin, scales[12]
        uint4 qa, qb;  // qs[32u .. 32u+31]
        uint4 ha, hb;  // qh[0 .. 31]
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u;
        W w;
        w.hdr = ldw128(blk);
        w.ha = ldw128(blk + 16);
        w.hb = ldw128(blk + 32);
        w.qa = ldw128(blk + 48 + 32u * u);
        w.qb = ldw128(blk + 64 + 32u * u);
        return w;
    }
    PK_DEV static uint32_t c5(uint32_t q, uint32_t h, uint32_t qsh, uint32_t hsh) {
        return ((q >> qsh) & 0x0f0f0f0fu) | (((h >> hsh) & 0x01010101u) << 4);
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t u, const uint2 *) {
        const uint32_t h1 = 2u * u, h2 = 2u * u + 1u;
        int32_t s1 = dot16(c5(w.qa.x, w.ha.x, 0, h1), c5(w.qa.y, w.ha.y, 0, h1), c5(w.qa.z, w.ha.z, 0, h1),
                           c5(w.qa.w, w.ha.w, 0, h1), a.q[0], 0);
        s1 = dot16(c5(w.qb.x, w.hb.x, 0, h1), c5(w.qb.y, w.hb.y, 0, h1), c5(w.qb.z, w.hb.z, 0, h1),
                   c5(w.qb.w, w.hb.w, 0, h1), a.q[1], s1);
        int32_t s2 = dot16(c5(w.qa.x, w.ha.x, 4, h2), c5(w.qa.y, w.ha.y, 4, h2), c5(w.qa.z, w.ha.z, 4, h2),
                           c5(w.qa.w, w.ha.w, 4, h2), a.q[2], 0);
        s2 = dot16(c5(w.qb.x, w.hb.x, 4, h2), c5(w.qb.y, w.hb.y, 4, h2), c5(w.qb.z, w.hb.z, 4, h2),
                   c5(w.qb.w, w.hb.w, 4, h2), a.q[3], s2);
        int32_t sc1, m1, sc2, m2;
        Fmt<PULSAR_QUANT_Q4_K>::scale_min(w.hdr, 2 * u, sc1, m1);
        Fmt<PULSAR_QUANT_Q4_K>::scale_min(w.hdr, 2 * u + 1, sc2, m2);
        Part p;
        p.i0 = __mul24(sc1, s1) + __mul24(sc2, s2);
        p.i1 = __mul24(m1, a.bs[0] + a.bs[1]) + __mul24(m2, a.bs[2] + a.bs[3]);
        p.f = 0.0f;
        return p;
    }
    // d * y->d * isum - dmin * y->d * msum (pulsar_kernels.cu:5916-5917)
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        return Fmt<PULSAR_QUANT_Q4_K>::sb_value(Fmt<PULSAR_QUANT_Q4_K>::W{w.hdr, w.qa, w.qb}, yd, p);
    }
};

// ----------------------------------------------------------------- Q3_K --
// block_q3_K (pulsar_kernels.cu:1309-1315): hmask[32] @0, qs[64] @32,
// scales[12] @96 (16 6-bit, minus 32), f16 d @108. Lane dot: cpu_dot.rs:
// 166-204. Unit (h, half): qs[32h + 16half ..+16) shifted by 2s and bit
// 4h + s of hmask[16half ..+16) give the 3-bit code c of values 128h + 32s +
// 16half + i; the value is c - 4 under scale 8h + 2s + half. The -4 offset
// folds through the q8_K 16-value sums: sum (c - 4) x = sum c x - 4 bsum.
template <>
struct Fmt<PULSAR_QUANT_Q3_K> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 110;
    static constexpr bool kStride32 = true;
    static constexpr int kBsMode = 2;
    struct W {
        uint4 qs, hm;
        uint2 sl;     // scales[0 .. 7]
        uint32_t sh;  // scales[8 .. 11]
        uint32_t d;
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u, h = u >> 1, half = u & 1u;
        W w;
        w.qs = ldw128(blk + 32u + 32u * h + 16u * half);
        w.hm = ldw128(blk + 16u * half);
        w.sl = ldw64(blk + 96);
        w.sh = ldw32(blk + 104);
        w.d = ldw16(blk + 108);
        return w;
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t u, const uint2 *) {
        const uint32_t h = u >> 1, half = u & 1u;
        const uint32_t q[4] = {w.qs.x, w.qs.y, w.qs.z, w.qs.w};
        const uint32_t m[4] = {w.hm.x, w.hm.y, w.hm.z, w.hm.w};
        int32_t isum = 0;
#pragma unroll
        for (uint32_t s = 0; s < 4; s++) {
            uint32_t c[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                c[i] = ((q[i] >> (2u * s)) & 0x03030303u) | (((m[i] >> (4u * h + s)) & 0x01010101u) << 2);
            const int32_t d = dot16(c[0], c[1], c[2], c[3], a.q[s], 0) - 4 * a.bs[s];
            // k3 scale j = 8h + 2s + half (cpu_dot.rs:133-145): low 4 bits
            // from nibble h of scales[2s + half], high 2 from scales[8 +
            // 2(s & 1) + half] bits 2(2h + s/2)
            const uint32_t lo = (byte_of(w.sl, 2u * s + half) >> (4u * h)) & 0x0fu;
            const uint32_t hi = (byte_of(w.sh, 2u * (s & 1u) + half) >> (2u * (2u * h + (s >> 1)))) & 3u;
            isum += __mul24((int32_t)(lo | (hi << 4)) - 32, d);
        }
        return Part{isum, 0, 0.0f};
    }
    // xd * y.d * isum (cpu_dot.rs:201)
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        return f16f((uint16_t)w.d) * yd * (float)p.i0;
    }
};

// --------------------------------------------------------------- IQ2_XS --
// block_iq2_xs (pulsar_kernels.cu:1364-1368): f16 d @0, qs[32] u16 @2
// (9-bit grid index, 7-bit ksigns index), scales[8] @66. Lane dot:
// cpu_dot.rs:299-338. LDS: 512 grid rows, then 128 sign-mask rows.
constexpr uint32_t kIq2xsSignRow = 512u;
template <>
struct Fmt<PULSAR_QUANT_IQ2_XS> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 74;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    static constexpr uint32_t kLutRows = 512u + 128u;
    PK_DEV static void fill_lut(uint2 *lut) {
        for (uint32_t i = threadIdx.x; i < 512u; i += blockDim.x) lut[i] = base3_row(k_iq2xs_codes[i], 8u, 25u, 43u);
        fill_ksign_rows(lut, kIq2xsSignRow);
    }
    struct W {
        uint4 qs;     // qs[8u .. 8u+7]
        uint32_t sc;  // scales[2u], scales[2u+1] in the low 16 bits
        uint32_t d;
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u;
        W w;
        w.qs = ldw128(blk + 2u + 16u * u);
        w.sc = ldw16(blk + 66u + 2u * u);
        w.d = ldw16(blk);
        return w;
    }
    PK_DEV static int32_t eight(const uint2 *lut, uint32_t q, uint4 a, bool hi_half) {
        const uint2 w = apply_signs(lut[q & 511u], lut[kIq2xsSignRow + (q >> 9)]);
        return hi_half ? dot4(w.y, a.w, dot4(w.x, a.z, 0)) : dot4(w.y, a.y, dot4(w.x, a.x, 0));
    }
    PK_DEV static int32_t group(const uint2 *lut, uint32_t q01, uint32_t q23, uint32_t sc, uint4 a0, uint4 a1) {
        // entries 0, 1 under the low scale nibble, 2, 3 under the high one
        const int32_t s1 = eight(lut, q01 & 0xffffu, a0, false) + eight(lut, q01 >> 16, a0, true);
        const int32_t s2 = eight(lut, q23 & 0xffffu, a1, false) + eight(lut, q23 >> 16, a1, true);
        return __mul24((int32_t)(2u * (sc & 0x0fu) + 1u), s1) + __mul24((int32_t)(2u * (sc >> 4) + 1u), s2);
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *lut) {
        const int32_t b0 = group(lut, w.qs.x, w.qs.y, w.sc & 0xffu, a.q[0], a.q[1]);
        const int32_t b1 = group(lut, w.qs.z, w.qs.w, (w.sc >> 8) & 0xffu, a.q[2], a.q[3]);
        return Part{b0 + b1, 0, 0.0f};
    }
    // 0.125 * xd * y.d * bsum (cpu_dot.rs:336)
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        return 0.125f * f16f((uint16_t)w.d) * yd * (float)p.i0;
    }
};

// -------------------------------------------------------------- IQ3_XXS --
// block_iq3_xxs (pulsar_kernels.cu:1370-1373): f16 d @0, qs[64] grid
// indices @2, 8 u32 @66 (4 x 7-bit ksigns index, 4-bit scale at 28..31).
// Lane dot: cpu_dot.rs:349-390, whose per-group scale xd * (0.5 + s) *
// 0.5 is xd / 4 * (2s + 1): the integer sum of (2s + 1) * sumi is exact.
// LDS: the 256 u32 grid entries (128 rows), then 128 sign-mask rows.
constexpr uint32_t kIq3xxsSignRow = 128u;
template <>
struct Fmt<PULSAR_QUANT_IQ3_XXS> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 98;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    static constexpr uint32_t kLutRows = 128u + 128u;
    PK_DEV static void fill_lut(uint2 *lut) {
        uint32_t *g = (uint32_t *)lut;
        for (uint32_t i = threadIdx.x; i < 256u; i += blockDim.x)
            g[i] = bits3_row(k_iq3xxs_codes[i], 0x3E342C24u, 0x1C140C04u);  // {4,12,...,52,62}
        fill_ksign_rows(lut, kIq3xxsSignRow);
    }
    struct W {
        uint4 qs;   // grid indices of groups 2u, 2u+1
        uint2 aux;  // their aux words
        uint32_t d;
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u;
        W w;
        w.qs = ldw128(blk + 2u + 16u * u);
        w.aux = ldw64(blk + 66u + 8u * u);
        w.d = ldw16(blk);
        return w;
    }
    PK_DEV static int32_t group(const uint2 *lut, uint32_t i03, uint32_t i47, uint32_t aux, uint4 a0, uint4 a1) {
        const uint32_t *grid = (const uint32_t *)lut;
        const uint32_t idx[8] = {i03 & 0xffu, (i03 >> 8) & 0xffu, (i03 >> 16) & 0xffu, i03 >> 24,
                                 i47 & 0xffu, (i47 >> 8) & 0xffu, (i47 >> 16) & 0xffu, i47 >> 24};
        int32_t sumi = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) {
            const uint2 w = apply_signs(make_uint2(grid[idx[2 * j]], grid[idx[2 * j + 1]]),
                                        lut[kIq3xxsSignRow + ((aux >> (7u * j)) & 127u)]);
            const uint4 &a = j < 2 ? a0 : a1;
            const uint32_t ax = (j & 1u) ? a.z : a.x, ay = (j & 1u) ? a.w : a.y;
            sumi = dot4(w.y, ay, dot4(w.x, ax, sumi));
        }
        return __mul24(sumi, (int32_t)(2u * (aux >> 28) + 1u));
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *lut) {
        const int32_t b0 = group(lut, w.qs.x, w.qs.y, w.aux.x, a.q[0], a.q[1]);
        const int32_t b1 = group(lut, w.qs.z, w.qs.w, w.aux.y, a.q[2], a.q[3]);
        return Part{b0 + b1, 0, 0.0f};
    }
    // y.d * sum_g xd (2s + 1) / 4 * sumi_g
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        return 0.25f * f16f((uint16_t)w.d) * yd * (float)p.i0;
    }
};

// --------------------------------------------------------------- IQ4_XS --
// block_iq4_xs (pulsar_kernels.cu:1343-1347): f16 d @0, scales_h u16 @2,
// scales_l[4] @4, qs[128] @8. Dot: pulsar_kernels.cu:5843-5865. Sub-block
// ib: 6-bit scale ls (low 4 bits nibble ib&1 of scales_l[ib/2], high 2 bits
// 2ib of scales_h), values kvalues[nibble] * (ls - 32).
template <>
struct Fmt<PULSAR_QUANT_IQ4_XS> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 136;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    struct W {
        uint4 qa, qb;  // qs[32u .. 32u+31]
        uint2 hdr;     // d, scales_h, scales_l[4]
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u;
        W w;
        w.hdr = ldw64(blk);
        w.qa = ldw128(blk + 8u + 32u * u);
        w.qb = ldw128(blk + 24u + 32u * u);
        return w;
    }
    PK_DEV static int32_t sub(uint4 q, uint4 a_lo, uint4 a_hi) {
        int32_t s = dot16(iq4nl_kv4(q.x), iq4nl_kv4(q.y), iq4nl_kv4(q.z), iq4nl_kv4(q.w), a_lo, 0);
        return dot16(iq4nl_kv4(q.x >> 4), iq4nl_kv4(q.y >> 4), iq4nl_kv4(q.z >> 4), iq4nl_kv4(q.w >> 4), a_hi, s);
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t u, const uint2 *) {
        const uint32_t sh = w.hdr.x >> 16, sl = byte_of(w.hdr.y, u);
        const int32_t ls0 = (int32_t)((sl & 0x0fu) | (((sh >> (4u * u)) & 3u) << 4)) - 32;
        const int32_t ls1 = (int32_t)((sl >> 4) | (((sh >> (4u * u + 2u)) & 3u) << 4)) - 32;
        return Part{__mul24(ls0, sub(w.qa, a.q[0], a.q[1])) + __mul24(ls1, sub(w.qb, a.q[2], a.q[3])), 0, 0.0f};
    }
    // d * y.d * sum_ib ls_ib sumi_ib
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        return f16f((uint16_t)w.hdr.x) * yd * (float)p.i0;
    }
};

// ------------------------------------------- 32-value-block formats ------
// Q8_0 (34 B: f16 d, 32 int8), Q4_0 (18 B: f16 d, 16 nibble bytes, value
// nibble - 8), Q5_1 (24 B: f16 d, f16 m, u32 qh, 16 nibble bytes, value
// d (nibble | qh bit << 4) + m), IQ4_NL (18 B: f16 d, 16 nibble bytes,
// value d kvalues[nibble]): low nibble of byte i = value i, high = i + 16.
// Dots: pulsar_kernels.cu:5793-5805, 5773-5791, 5950-5975, 5605-5625, each
// sumf += (per-block float) over the 8 blocks of a super-block, then
// y.d * sumf. A unit holds blocks 2u, 2u+1; its float partial is their two
// terms in block order (a block contributing nothing when the reference
// skips it), and the super-block sums the units' partials.
PK_DEV uint32_t lo4(uint32_t v) { return v & 0x0f0f0f0fu; }
PK_DEV uint32_t hi4(uint32_t v) { return (v >> 4) & 0x0f0f0f0fu; }

template <>
struct Fmt<PULSAR_QUANT_Q8_0> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 272;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    struct W {
        uint4 q[4];   // block 2u values 0..31, block 2u+1 values 0..31
        uint32_t dd;  // d of block 2u | d of block 2u+1 << 16
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *bp = row + (uint64_t)(g >> 2) * kSbBytes + 68u * (g & 3u);
        W w;
        w.q[0] = ldw128(bp + 2);
        w.q[1] = ldw128(bp + 18);
        w.q[2] = ldw128(bp + 36);
        w.q[3] = ldw128(bp + 52);
        w.dd = ldw16(bp) | ((uint32_t)ldw16(bp + 34) << 16);
        return w;
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *) {
        const int32_t s0 = dot16(w.q[1].x, w.q[1].y, w.q[1].z, w.q[1].w, a.q[1],
                                 dot16(w.q[0].x, w.q[0].y, w.q[0].z, w.q[0].w, a.q[0], 0));
        const int32_t s1 = dot16(w.q[3].x, w.q[3].y, w.q[3].z, w.q[3].w, a.q[3],
                                 dot16(w.q[2].x, w.q[2].y, w.q[2].z, w.q[2].w, a.q[2], 0));
        float f = s0 != 0 ? f16f((uint16_t)w.dd) * (float)s0 : 0.0f;
        if (s1 != 0) f += f16f((uint16_t)(w.dd >> 16)) * (float)s1;
        return Part{s0, s1, f};
    }
    PK_DEV static float sb_value(const W &, float yd, const Part &p) { return yd * p.f; }
};

template <>
struct Fmt<PULSAR_QUANT_Q4_0> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 144;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 1;  // bs[0] + bs[1]: block 2u, bs[2] + bs[3]: block 2u+1
    struct W {
        uint4 q0, q1;
        uint32_t dd;
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *bp = row + (uint64_t)(g >> 2) * kSbBytes + 36u * (g & 3u);
        W w;
        w.q0 = ldw128(bp + 2);
        w.q1 = ldw128(bp + 20);
        w.dd = ldw16(bp) | ((uint32_t)ldw16(bp + 18) << 16);
        return w;
    }
    PK_DEV static int32_t nib_dot(uint4 q, uint4 a_lo, uint4 a_hi) {
        return dot16(hi4(q.x), hi4(q.y), hi4(q.z), hi4(q.w), a_hi,
                     dot16(lo4(q.x), lo4(q.y), lo4(q.z), lo4(q.w), a_lo, 0));
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *) {
        const int32_t s0 = nib_dot(w.q0, a.q[0], a.q[1]), s1 = nib_dot(w.q1, a.q[2], a.q[3]);
        const int32_t b0 = a.bs[0] + a.bs[1], b1 = a.bs[2] + a.bs[3];
        float f = (s0 != 0 || b0 != 0) ? f16f((uint16_t)w.dd) * (float)(s0 - 8 * b0) : 0.0f;
        if (s1 != 0 || b1 != 0) f += f16f((uint16_t)(w.dd >> 16)) * (float)(s1 - 8 * b1);
        return Part{s0 - 8 * b0, s1 - 8 * b1, f};
    }
    PK_DEV static float sb_value(const W &, float yd, const Part &p) { return yd * p.f; }
};

template <>
struct Fmt<PULSAR_QUANT_Q5_1> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 192;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 1;
    struct W {
        uint4 q0, q1;
        uint2 hd0, hd1;  // (d | m << 16, qh) of blocks 2u and 2u+1
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *bp = row + (uint64_t)(g >> 2) * kSbBytes + 48u * (g & 3u);
        W w;
        w.hd0 = ldw64(bp);
        w.q0 = ldw128(bp + 8);
        w.hd1 = ldw64(bp + 24);
        w.q1 = ldw128(bp + 32);
        return w;
    }
    // nibbles of 4 bytes plus their fifth bits (bits k .. k+3 of qh)
    PK_DEV static uint32_t c5(uint32_t nib, uint32_t qh, uint32_t k) { return nib | (spread4(qh >> k) << 4); }
    PK_DEV static int32_t blk_dot(uint4 q, uint32_t qh, uint4 a_lo, uint4 a_hi) {
        int32_t s = dot16(c5(lo4(q.x), qh, 0), c5(lo4(q.y), qh, 4), c5(lo4(q.z), qh, 8), c5(lo4(q.w), qh, 12), a_lo, 0);
        return dot16(c5(hi4(q.x), qh, 16), c5(hi4(q.y), qh, 20), c5(hi4(q.z), qh, 24), c5(hi4(q.w), qh, 28), a_hi, s);
    }
    PK_DEV static float term(uint32_t dm, int32_t s, int32_t b) {
        return (s != 0 || b != 0) ? f16f((uint16_t)dm) * (float)s + f16f((uint16_t)(dm >> 16)) * (float)b : 0.0f;
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *) {
        const int32_t s0 = blk_dot(w.q0, w.hd0.y, a.q[0], a.q[1]), s1 = blk_dot(w.q1, w.hd1.y, a.q[2], a.q[3]);
        float f = term(w.hd0.x, s0, a.bs[0] + a.bs[1]);
        f += term(w.hd1.x, s1, a.bs[2] + a.bs[3]);
        return Part{s0, s1, f};
    }
    PK_DEV static float sb_value(const W &, float yd, const Part &p) { return yd * p.f; }
};

template <>
struct Fmt<PULSAR_QUANT_IQ4_NL> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 144;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    using W = Fmt<PULSAR_QUANT_Q4_0>::W;
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t n) { return Fmt<PULSAR_QUANT_Q4_0>::load(row, g, n); }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *) {
        const int32_t s0 = Fmt<PULSAR_QUANT_IQ4_XS>::sub(w.q0, a.q[0], a.q[1]);
        const int32_t s1 = Fmt<PULSAR_QUANT_IQ4_XS>::sub(w.q1, a.q[2], a.q[3]);
        float f = s0 != 0 ? f16f((uint16_t)w.dd) * (float)s0 : 0.0f;
        if (s1 != 0) f += f16f((uint16_t)(w.dd >> 16)) * (float)s1;
        return Part{s0, s1, f};
    }
    PK_DEV static float sb_value(const W &, float yd, const Part &p) { return yd * p.f; }
};

// ---------------------------------------------------------------- IQ3_S --
// block_iq3_s (pulsar_kernels.cu:1390-1396): f16 d @0, qs[64] @2 (low 8
// index bits), qh[8] @66 (ninth bit of entry p of group g: bit p of qh[g]),
// signs[32] @74 (byte 4g + l: entries 2l, 2l+1), scales[4] @106 (nibble
// g&1 of byte g/2). Dot: pulsar_kernels.cu:5683-5713; db = d (1 + 2 sc) is
// integral in sc, so the sum of (1 + 2 sc) * sumi is exact. LDS: 512 u32
// grid entries (256 rows), then the 256 sign-byte masks.
constexpr uint32_t kIq3sSignRow = 256u;
template <>
struct Fmt<PULSAR_QUANT_IQ3_S> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 110;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    static constexpr uint32_t kLutRows = 256u + 256u;
    PK_DEV static void fill_lut(uint2 *lut) {
        uint32_t *g = (uint32_t *)lut;
        for (uint32_t i = threadIdx.x; i < 512u; i += blockDim.x)
            g[i] = bits3_row(k_iq3s_codes[i], 0x0F0D0B09u, 0x07050301u);  // 2d + 1
        fill_sbyte_rows(lut, kIq3sSignRow);
    }
    struct W {
        uint4 qs;      // qs[16u .. 16u+15]
        uint2 sg;      // signs[8u .. 8u+7]
        uint32_t qhs;  // qh[2u], qh[2u+1] | scales[u] << 16
        uint32_t d;
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u;
        W w;
        w.qs = ldw128(blk + 2u + 16u * u);
        w.sg = ldw64(blk + 74u + 8u * u);
        w.qhs = ldw16(blk + 66u + 2u * u) | (ldw8(blk + 106u + u) << 16);
        w.d = ldw16(blk);
        return w;
    }
    PK_DEV static int32_t group(const uint2 *lut, uint32_t i03, uint32_t i47, uint32_t qh, uint32_t sg, uint4 a0,
                                uint4 a1) {
        const uint32_t *grid = (const uint32_t *)lut;
        int32_t sumi = 0;
#pragma unroll
        for (uint32_t l = 0; l < 4; l++) {
            const uint32_t iw = l < 2 ? i03 : i47, sh = 16u * (l & 1u);
            const uint32_t e0 = ((iw >> sh) & 0xffu) | (((qh >> (2u * l)) & 1u) << 8);
            const uint32_t e1 = ((iw >> (sh + 8u)) & 0xffu) | (((qh >> (2u * l + 1u)) & 1u) << 8);
            const uint2 w = apply_signs(make_uint2(grid[e0], grid[e1]), lut[kIq3sSignRow + ((sg >> (8u * l)) & 0xffu)]);
            const uint4 &a = l < 2 ? a0 : a1;
            const uint32_t ax = (l & 1u) ? a.z : a.x, ay = (l & 1u) ? a.w : a.y;
            sumi = dot4(w.y, ay, dot4(w.x, ax, sumi));
        }
        return sumi;
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *lut) {
        const uint32_t sc = w.qhs >> 16;
        const int32_t s0 = group(lut, w.qs.x, w.qs.y, w.qhs & 0xffu, w.sg.x, a.q[0], a.q[1]);
        const int32_t s1 = group(lut, w.qs.z, w.qs.w, (w.qhs >> 8) & 0xffu, w.sg.y, a.q[2], a.q[3]);
        return Part{__mul24((int32_t)(1u + 2u * (sc & 0x0fu)), s0) + __mul24((int32_t)(1u + 2u * ((sc >> 4) & 0x0fu)), s1),
                    0, 0.0f};
    }
    // y.d * sum_g d (1 + 2 sc_g) sumi_g
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        return f16f((uint16_t)w.d) * yd * (float)p.i0;
    }
};

// ---------------------------------------------------------------- IQ2_S --
// block_iq2_s (pulsar_kernels.cu:1381-1385): f16 d @0, qs[32] @2 (low 8
// index bits), signs[32] @34, qh[8] @66 (bits 2j, 2j+1 of qh[g] are index
// bits 8, 9 of entry j), scales[8] @74 (entries 0, 1: low nibble n, 2, 3:
// high). Dot: pulsar_kernels.cu:5627-5657 with dl = d (0.5 + n) / 4 = d (2n
// + 1) / 8: the sum of (2n + 1) * acc is exact. LDS: 1024 grid rows, then
// the 256 sign-byte masks.
constexpr uint32_t kIq2sSignRow = 1024u;
template <>
struct Fmt<PULSAR_QUANT_IQ2_S> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 82;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    static constexpr uint32_t kLutRows = 1024u + 256u;
    PK_DEV static void fill_lut(uint2 *lut) {
        for (uint32_t i = threadIdx.x; i < 1024u; i += blockDim.x) lut[i] = base3_row(k_iq2s_codes[i], 8u, 25u, 43u);
        fill_sbyte_rows(lut, kIq2sSignRow);
    }
    struct W {
        uint2 qs, sg;   // qs[8u .. 8u+7], signs[8u .. 8u+7]
        uint32_t qhsc;  // qh[2u], qh[2u+1], scales[2u], scales[2u+1]
        uint32_t d;
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u;
        W w;
        w.qs = ldw64(blk + 2u + 8u * u);
        w.sg = ldw64(blk + 34u + 8u * u);
        w.qhsc = ldw16(blk + 66u + 2u * u) | ((uint32_t)ldw16(blk + 74u + 2u * u) << 16);
        w.d = ldw16(blk);
        return w;
    }
    PK_DEV static int32_t group(const uint2 *lut, uint32_t idx4, uint32_t sg4, uint32_t qh, uint32_t sc, uint4 a0,
                                uint4 a1) {
        int32_t s1 = 0, s2 = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) {
            const uint32_t e = ((idx4 >> (8u * j)) & 0xffu) | (((qh >> (2u * j)) & 3u) << 8);
            const uint2 w = apply_signs(lut[e], lut[kIq2sSignRow + ((sg4 >> (8u * j)) & 0xffu)]);
            const uint4 &a = j < 2 ? a0 : a1;
            const uint32_t ax = (j & 1u) ? a.z : a.x, ay = (j & 1u) ? a.w : a.y;
            if (j < 2)
                s1 = dot4(w.y, ay, dot4(w.x, ax, s1));
            else
                s2 = dot4(w.y, ay, dot4(w.x, ax, s2));
        }
        return __mul24((int32_t)(2u * (sc & 0x0fu) + 1u), s1) + __mul24((int32_t)(2u * (sc >> 4) + 1u), s2);
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *lut) {
        const int32_t b0 = group(lut, w.qs.x, w.sg.x, w.qhsc & 0xffu, (w.qhsc >> 16) & 0xffu, a.q[0], a.q[1]);
        const int32_t b1 = group(lut, w.qs.y, w.sg.y, (w.qhsc >> 8) & 0xffu, w.qhsc >> 24, a.q[2], a.q[3]);
        return Part{b0 + b1, 0, 0.0f};
    }
    // y.d * sum d (2n + 1) / 8 * acc
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        return 0.125f * f16f((uint16_t)w.d) * yd * (float)p.i0;
    }
};

// ---------------------------------------------------------------- IQ1_S --
// block_iq1_s (pulsar_kernels.cu:1404-1408): f16 d @0, qs[32] @2 (low 8
// index bits), qh[8] u16 @34 (bits 3j..3j+2: index bits 8..10 of entry j,
// 12..14: scale s, 15: delta sign). Values d (2s + 1) (g +- 1/8), g in
// {-1, 0, 1}. Dot: pulsar_kernels.cu:5659-5681. LDS: 2048 grid rows of
// int8 ternaries.
template <>
struct Fmt<PULSAR_QUANT_IQ1_S> {
    static constexpr bool kHasI1 = true;
    static constexpr uint32_t kSbBytes = 50;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 1;
    static constexpr uint32_t kLutRows = 2048u;
    PK_DEV static void fill_lut(uint2 *lut) {
        for (uint32_t i = threadIdx.x; i < 2048u; i += blockDim.x) lut[i] = base3_row(k_iq1s_codes[i], 0xffu, 0u, 1u);
    }
    struct W {
        uint2 qs;     // qs[8u .. 8u+7]
        uint32_t qh;  // qh[2u] | qh[2u+1] << 16
        uint32_t d;
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *blk = row + (uint64_t)(g >> 2) * kSbBytes;
        const uint32_t u = g & 3u;
        W w;
        w.qs = ldw64(blk + 2u + 8u * u);
        w.qh = ldw32(blk + 34u + 4u * u);
        w.d = ldw16(blk);
        return w;
    }
    PK_DEV static int32_t group(const uint2 *lut, uint32_t idx4, uint32_t qh, uint4 a0, uint4 a1) {
        int32_t s = 0;
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) {
            const uint2 w = lut[((idx4 >> (8u * j)) & 0xffu) | (((qh >> (3u * j)) & 7u) << 8)];
            const uint4 &a = j < 2 ? a0 : a1;
            const uint32_t ax = (j & 1u) ? a.z : a.x, ay = (j & 1u) ? a.w : a.y;
            s = dot4(w.y, ay, dot4(w.x, ax, s));
        }
        return s;
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *lut) {
        Part p;
        p.i0 = 0;
        p.i1 = 0;
#pragma unroll
        for (uint32_t k = 0; k < 2; k++) {
            const uint32_t qh = (w.qh >> (16u * k)) & 0xffffu;
            const int32_t ls = (int32_t)(2u * ((qh >> 12) & 7u) + 1u);
            const int32_t lsum = group(lut, k ? w.qs.y : w.qs.x, qh, a.q[2 * k], a.q[2 * k + 1]);
            const int32_t bsum = a.bs[2 * k] + a.bs[2 * k + 1];
            p.i0 += __mul24(ls, lsum);
            p.i1 += (qh & 0x8000u) ? -__mul24(ls, bsum) : __mul24(ls, bsum);
        }
        p.f = 0.0f;
        return p;
    }
    // d * y.d * (sumi + 0.125 * sumi1) (pulsar_kernels.cu:5680)
    PK_DEV static float sb_value(const W &w, float yd, const Part &p) {
        return f16f((uint16_t)w.d) * yd * ((float)p.i0 + 0.125f * (float)p.i1);
    }
};

// ---------------------------------------------------------------- NVFP4 --
// NVFP4 (crates/gguf/src/lib.rs:170: 64 values in 36 bytes): 4 UE4M3
// scale bytes, then per 16-value sub-block 8 bytes (low nibble = value i,
// high = value i + 8), E2M1 codes. Dot: pulsar_kernels.cu:5743-5771, the
// doubled E2M1 table of MXFP4 against half the UE4M3 scale, sumf over the
// sub-blocks in order.
// UE4M3 (ggml_ue4m3_to_fp32): 0 and 0x7F are zero, exponent field 0 is
// subnormal (m * 2^-9), else (1 + m/8) * 2^(e - 7); both exact in f32.
PK_DEV float ue4m3f(uint32_t e) {
    const uint32_t ex = (e >> 3) & 0xfu, man = e & 7u;
    if (e == 0u || e == 0x7fu) return 0.0f;
    return ex == 0u ? (float)man * 0.001953125f : __builtin_bit_cast(float, ((ex + 120u) << 23) | (man << 20));
}
template <>
struct Fmt<PULSAR_QUANT_NVFP4> {
    static constexpr bool kHasI1 = false;
    static constexpr uint32_t kSbBytes = 144;
    static constexpr bool kStride32 = false;
    static constexpr int kBsMode = 0;
    struct W {
        uint4 qa, qb;  // sub-blocks 0, 1 / 2, 3: 8 code bytes each
        uint32_t e;    // 4 scale bytes
    };
    PK_DEV static W load(const uint8_t *row, uint32_t g, uint32_t) {
        const uint8_t *bp = row + (uint64_t)(g >> 2) * kSbBytes + 36u * (g & 3u);
        W w;
        w.e = ldw32(bp);
        w.qa = ldw128(bp + 4);
        w.qb = ldw128(bp + 20);
        return w;
    }
    PK_DEV static int32_t sub(uint32_t c0, uint32_t c1, uint4 a) {
        int32_t s = dot4(mxfp4_kv4(c0), a.x, 0);
        s = dot4(mxfp4_kv4(c1), a.y, s);
        s = dot4(mxfp4_kv4_hi(c0), a.z, s);
        return dot4(mxfp4_kv4_hi(c1), a.w, s);
    }
    PK_DEV static Part part(const W &w, const Act &a, uint32_t, const uint2 *) {
        const int32_t s[4] = {sub(w.qa.x, w.qa.y, a.q[0]), sub(w.qa.z, w.qa.w, a.q[1]), sub(w.qb.x, w.qb.y, a.q[2]),
                              sub(w.qb.z, w.qb.w, a.q[3])};
        float f = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; k++) f += ue4m3f((w.e >> (8 * k)) & 0xffu) * 0.5f * (float)s[k];
        return Part{s[0] + s[1], s[2] + s[3], f};
    }
    PK_DEV static float sb_value(const W &, float yd, const Part &p) { return yd * p.f; }
};

}  // namespace pk
