/* pulsar_oracle.c - CPU restatement of the reference's quantized expert path.
 *
 * TEST INFRASTRUCTURE ONLY (see pulsar_oracle.h): the checker for the HIP
 * library and the CPU baseline that bench.py times. Build with
 * -O2 -ffp-contract=off (oracle/Makefile).
 *
 * Reference files this follows (all paths under the reference checkout):
 *   cpu   = crates/quant/src/cpu_dot.rs           (the CPU expert lane)
 *   cu    = crates/kernels/cuda/pulsar_kernels.cu  (host mirrors, kernels)
 *   elib  = crates/engine/src/lib.rs               (Lane composition)
 */
#include "pulsar_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "../include/pulsar_iq2xxs_grid.h"
#include "../include/pulsar_iq_grids.h"

/* ---------------------------------------------------------------- f16 -- */

/* cpu:52-64 (exact, including subnormals) */
float po_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    uint32_t bits;
    float f;
    if (exp == 0) {
        bits = sign | 0x38800000u; /* +-2^-14 */
        memcpy(&f, &bits, 4);
        return f * ((float)man / 1024.0f);
    }
    if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

/* crates/quant/src/lib.rs:51-82 (round to nearest even) */
uint16_t po_f32_to_f16(float x) {
    uint32_t bits;
    memcpy(&bits, &x, 4);
    const uint16_t s = (uint16_t)((bits >> 16) & 0x8000u);
    const int32_t e = (int32_t)((bits >> 23) & 0xffu);
    const uint32_t m = bits & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(s | 0x7c00u | (m ? 0x200u : 0u));
    const int32_t e16 = e - 127 + 15;
    if (e16 >= 0x1f) return (uint16_t)(s | 0x7c00u);
    if (e16 <= 0) {
        if (e16 < -10) return s;
        const uint32_t mm = m | 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e16);
        const uint32_t half = mm >> shift;
        const uint32_t rem = mm & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        const uint32_t rounded = half + ((rem > halfway) | ((rem == halfway) & (half & 1u)));
        return (uint16_t)(s | rounded);
    }
    const uint32_t half = (uint32_t)s | ((uint32_t)e16 << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    const uint32_t rounded = half + ((rem > 0x1000u) | ((rem == 0x1000u) & (half & 1u)));
    return (uint16_t)rounded;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t rd32(const uint8_t *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* --------------------------------------------------------------- q8_K -- */

/* cpu:26-50. amax folds with max from 0; an all-zero block gets d = 0 and
 * zero quants; otherwise d = amax/127, inv = 127/amax and
 * q = clamp(round(x*inv), -127, 127) with round = half away from zero.
 * The tail past in_dim is zero (cu:1499-1501), which leaves amax unchanged. */
void po_quantize_q8_K(pulsar_block_q8_K *out, const float *x, uint32_t in_dim, uint32_t n_rows) {
    const uint32_t nb = (in_dim + 255u) / 256u;
    for (uint32_t r = 0; r < n_rows; r++) {
        for (uint32_t b = 0; b < nb; b++) {
            pulsar_block_q8_K *yb = out + (uint64_t)r * nb + b;
            float v[256];
            for (uint32_t i = 0; i < 256; i++) {
                const uint64_t c = (uint64_t)b * 256u + i;
                v[i] = c < in_dim ? x[(uint64_t)r * in_dim + c] : 0.0f;
            }
            float amax = 0.0f;
            for (uint32_t i = 0; i < 256; i++) amax = fmaxf(amax, fabsf(v[i]));
            if (amax == 0.0f) {
                memset(yb, 0, sizeof(*yb));
                continue;
            }
            const float scale = amax / 127.0f;
            const float inv = 127.0f / amax;
            yb->d = scale;
            for (uint32_t i = 0; i < 256; i++) {
                /* Rust's `f32 as i8` saturates and maps NaN to 0; NaN arises
                 * only when 127/amax overflows (amax < ~3.7e-37) on a 0 */
                float q = roundf(v[i] * inv);
                if (q != q) q = 0.0f;
                if (q < -127.0f) q = -127.0f;
                if (q > 127.0f) q = 127.0f;
                yb->qs[i] = (int8_t)q;
            }
            for (uint32_t g = 0; g < 16; g++) {
                int32_t s = 0;
                for (uint32_t i = 0; i < 16; i++) s += yb->qs[16 * g + i];
                yb->bsums[g] = (int16_t)s;
            }
        }
    }
}

/* ------------------------------------------------------------ formats -- */

/* bytes per 256 values (crates/gguf/src/lib.rs:145-172) */
uint32_t po_sb_bytes(uint32_t quant) {
    switch (quant) {
    case PULSAR_QUANT_Q2_K: return 84;
    case PULSAR_QUANT_IQ2_XXS: return 66;
    case PULSAR_QUANT_Q4_K: return 144;
    case PULSAR_QUANT_Q5_K: return 176;
    case PULSAR_QUANT_Q6_K: return 210;
    case PULSAR_QUANT_Q3_K: return 110;
    case PULSAR_QUANT_IQ2_XS: return 74;
    case PULSAR_QUANT_IQ3_XXS: return 98;
    case PULSAR_QUANT_Q4_0: return 8 * 18;
    case PULSAR_QUANT_Q5_1: return 8 * 24;
    case PULSAR_QUANT_Q8_0: return 8 * 34;
    case PULSAR_QUANT_IQ4_XS: return 136;
    case PULSAR_QUANT_MXFP4: return 8 * 17;
    case PULSAR_QUANT_IQ4_NL: return 8 * 18;
    case PULSAR_QUANT_IQ3_S: return 110;
    case PULSAR_QUANT_IQ2_S: return 82;
    case PULSAR_QUANT_IQ1_S: return 50;
    case PULSAR_QUANT_NVFP4: return 4 * 36;
    default: return 0;
    }
}

/* crates/gguf/src/lib.rs:145-180: ceil(n / block) * block_bytes; MXFP4 is
 * (32, 17), so its rows pack exact 32-value blocks. Every other format's
 * rows here are whole 256-value super-blocks. */
uint64_t po_row_bytes(uint32_t quant, uint32_t n) {
    if (quant == PULSAR_QUANT_MXFP4) return (uint64_t)((n + 31u) / 32u) * 17u;
    return (uint64_t)((n + 255u) / 256u) * po_sb_bytes(quant);
}

/* cpu:133-145 (k3_unpack_scales): 16 6-bit scales from 12 bytes, minus 32 */
static void k3_scales(const uint8_t *s, int32_t sc[16]) {
    for (uint32_t j = 0; j < 16; j++) {
        const uint32_t hi = ((uint32_t)s[8 + j % 4] >> (2 * (j / 4))) & 3u;
        const uint32_t lo = j < 8 ? (s[j] & 0x0fu) : (uint32_t)(s[j - 8] >> 4);
        sc[j] = (int32_t)(lo | (hi << 4)) - 32;
    }
}

/* the IQ grids of include/pulsar_iq_grids.h, expanded (signed int8 bytes) */
static const uint16_t k_iq2xs_codes[512] = {PULSAR_IQ2XS_GRID_CODES};
static const uint16_t k_iq2s_codes[1024] = {PULSAR_IQ2S_GRID_CODES};
static const uint16_t k_iq3xxs_codes[256] = {PULSAR_IQ3XXS_GRID_CODES};
static const uint16_t k_iq3s_codes[512] = {PULSAR_IQ3S_GRID_CODES};
static const uint16_t k_iq1s_codes[2048] = {PULSAR_IQ1S_GRID_CODES};
static int32_t base3_digit(uint32_t c, uint32_t j) {
    for (uint32_t k = 0; k < j; k++) c /= 3u;
    return (int32_t)(c % 3u);
}
static int32_t iq2xs_mag(uint32_t idx, uint32_t j) {
    static const int32_t m[3] = {8, 25, 43};
    return m[base3_digit(k_iq2xs_codes[idx], j)];
}
static int32_t iq2s_mag(uint32_t idx, uint32_t j) {
    static const int32_t m[3] = {8, 25, 43};
    return m[base3_digit(k_iq2s_codes[idx], j)];
}
static int32_t iq3xxs_mag(uint32_t idx, uint32_t j) {
    static const int32_t m[8] = {4, 12, 20, 28, 36, 44, 52, 62};
    return m[(k_iq3xxs_codes[idx] >> (3 * j)) & 7u];
}
static int32_t iq3s_mag(uint32_t idx, uint32_t j) { return 2 * (int32_t)((k_iq3s_codes[idx] >> (3 * j)) & 7u) + 1; }
static int32_t iq1s_val(uint32_t idx, uint32_t j) { return base3_digit(k_iq1s_codes[idx], j) - 1; }

/* cu:5602-5603, 5843 (kvalues_iq4nl) */
static const int32_t k_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

/* cu:5762-5767 (ggml_ue4m3_to_fp32): unsigned E4M3, 0 and 0x7F are zero */
static float ue4m3(uint8_t e) {
    if (e == 0 || e == 0x7F) return 0.0f;
    const int ex = (e >> 3) & 0xF, man = e & 7;
    return ex == 0 ? ldexpf((float)man, -9) : ldexpf(1.0f + (float)man / 8.0f, ex - 7);
}

/* cpu:147-156 == cu:1349-1359 (ggml get_scale_min_k4) */
void po_k4_scale_min(uint32_t j, const uint8_t *q, int32_t *sc, int32_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* IQ2_XXS grid, expanded from the base-3 codes of include/pulsar_iq2xxs_grid.h
 * (digit d_j -> magnitude {8, 25, 43}[d_j] in byte j). */
static const uint16_t k_iq2xxs_codes[256] = {PULSAR_IQ2XXS_GRID_CODES};
uint32_t po_iq2xxs_mag(uint32_t idx, uint32_t j) {
    static const uint8_t mags[3] = {8, 25, 43};
    uint32_t c = k_iq2xxs_codes[idx];
    for (uint32_t k = 0; k < j; k++) c /= 3u;
    return mags[c % 3u];
}

/* cpu:66-70: 7 stored sign bits, bit 7 completes even parity */
static uint32_t sign_mask(uint32_t s7) {
    return s7 | ((uint32_t)(__builtin_popcount(s7) & 1) << 7);
}

/* cu:1424-1448: doubled E2M1 table and its compensating 2^(e-128) scale,
 * flushed to zero for e < 2 */
static const int32_t k_mxfp4_kv[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
static float mxfp4_scale_half(uint8_t e) {
    if (e < 2) return 0.0f;
    const uint32_t bits = (uint32_t)(e - 1u) << 23;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float po_block_dot(uint32_t quant, const uint8_t *row, uint32_t b,
                   const pulsar_block_q8_K *y, uint32_t n_valid32,
                   int32_t *i0, int32_t *i1, int32_t sumi_out[8]) {
    const int8_t *q8 = y->qs;
    const int16_t *bs = y->bsums;
    const float yd = y->d;
    int32_t d0 = 0, d1 = 0;
    float f = 0.0f;
    switch (quant) {
    case PULSAR_QUANT_Q4_K: {
        /* cpu:250-279 */
        const uint8_t *blk = row + (uint64_t)b * 144u;
        const float xd = po_f16_to_f32(rd16(blk));
        const float xmin = po_f16_to_f32(rd16(blk + 2));
        const uint8_t *scales = blk + 4;
        const uint8_t *q4 = blk + 16;
        int32_t isum = 0, msum = 0;
        for (uint32_t j = 0; j < 4; j++) {
            int32_t sc1, m1, sc2, m2;
            po_k4_scale_min(2 * j, scales, &sc1, &m1);
            po_k4_scale_min(2 * j + 1, scales, &sc2, &m2);
            int32_t s1 = 0, s2 = 0;
            for (uint32_t i = 0; i < 32; i++) {
                const uint8_t v = q4[32 * j + i];
                s1 += (int32_t)(v & 0x0f) * q8[64 * j + i];
                s2 += (int32_t)(v >> 4) * q8[64 * j + 32 + i];
            }
            isum += sc1 * s1 + sc2 * s2;
            msum += m1 * (bs[4 * j] + bs[4 * j + 1]) + m2 * (bs[4 * j + 2] + bs[4 * j + 3]);
        }
        d0 = isum;
        d1 = msum;
        f = xd * yd * (float)isum - xmin * yd * (float)msum;
        break;
    }
    case PULSAR_QUANT_Q2_K: {
        /* cpu:732-767 */
        const uint8_t *blk = row + (uint64_t)b * 84u;
        const uint8_t *sc = blk;
        const uint8_t *q2 = blk + 16;
        const float xd = po_f16_to_f32(rd16(blk + 80));
        const float xmin = po_f16_to_f32(rd16(blk + 82));
        int32_t summs = 0;
        for (uint32_t j = 0; j < 16; j++) summs += bs[j] * (int32_t)(sc[j] >> 4);
        int32_t isum = 0;
        uint32_t is = 0;
        for (uint32_t k = 0; k < 2; k++) {
            for (uint32_t shift = 0; shift < 8; shift += 2) {
                for (uint32_t half = 0; half < 2; half++) {
                    const int32_t d = sc[is] & 0x0f;
                    is++;
                    int32_t sumi = 0;
                    for (uint32_t i = 0; i < 16; i++) {
                        const int32_t q = (q2[32 * k + 16 * half + i] >> shift) & 3;
                        sumi += q * q8[128 * k + 32 * (shift / 2) + 16 * half + i];
                    }
                    isum += d * sumi;
                }
            }
        }
        d0 = isum;
        d1 = summs;
        f = yd * xd * (float)isum - yd * xmin * (float)summs;
        break;
    }
    case PULSAR_QUANT_Q6_K: {
        /* cu:5920-5948 (== cu:1830-1861, cu:3163-3188) */
        const uint8_t *blk = row + (uint64_t)b * 210u;
        const uint8_t *ql = blk;
        const uint8_t *qh = blk + 128;
        const int8_t *sc = (const int8_t *)(blk + 192);
        const float xd = po_f16_to_f32(rd16(blk + 208));
        int32_t isum = 0;
        for (uint32_t j = 0; j < 2; j++) {
            int32_t g[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (uint32_t i = 0; i < 32; i++) {
                const uint32_t sub = i >> 4;
                const int32_t v0 = ((ql[i] & 0x0f) | (((qh[i] >> 0) & 3) << 4)) - 32;
                const int32_t v1 = ((ql[32 + i] & 0x0f) | (((qh[i] >> 2) & 3) << 4)) - 32;
                const int32_t v2 = ((ql[i] >> 4) | (((qh[i] >> 4) & 3) << 4)) - 32;
                const int32_t v3 = ((ql[32 + i] >> 4) | (((qh[i] >> 6) & 3) << 4)) - 32;
                g[0 + sub] += v0 * q8[i];
                g[2 + sub] += v1 * q8[32 + i];
                g[4 + sub] += v2 * q8[64 + i];
                g[6 + sub] += v3 * q8[96 + i];
            }
            for (uint32_t k = 0; k < 8; k++) isum += (int32_t)sc[k] * g[k];
            sc += 8;
            ql += 64;
            qh += 32;
            q8 += 128;
        }
        d0 = isum;
        f = xd * yd * (float)isum;
        break;
    }
    case PULSAR_QUANT_IQ2_XXS: {
        /* cpu:92-122 */
        const uint8_t *blk = row + (uint64_t)b * 66u;
        const float xd = po_f16_to_f32(rd16(blk));
        int32_t bsum = 0;
        for (uint32_t ib32 = 0; ib32 < 8; ib32++) {
            const uint32_t aux0 = rd32(blk + 2 + 8 * ib32);
            const uint32_t aux1 = rd32(blk + 6 + 8 * ib32);
            const int32_t ls = (int32_t)(2u * (aux1 >> 28) + 1u);
            int32_t sumi = 0;
            for (uint32_t k = 0; k < 4; k++) {
                const uint32_t gi = (aux0 >> (8 * k)) & 0xffu;
                const uint32_t sm = sign_mask((aux1 >> (7 * k)) & 127u);
                for (uint32_t i = 0; i < 8; i++) {
                    const int32_t g = po_iq2xxs_mag(gi, i);
                    const int32_t w = ((sm >> i) & 1u) ? -g : g;
                    sumi += w * q8[32 * ib32 + 8 * k + i];
                }
            }
            bsum += sumi * ls;
        }
        d0 = bsum;
        f = 0.125f * xd * yd * (float)bsum;
        break;
    }
    case PULSAR_QUANT_MXFP4: {
        /* cu:5715-5741; blocks past the row's last valid 32-block are not
         * read (their activations are the zero-padded q8_K tail, so the
         * reference's sumi == 0 skip drops them anyway) */
        const uint8_t *base = row + (uint64_t)b * 136u;
        float sumf = 0.0f;
        for (uint32_t k = 0; k < 8; k++) {
            int32_t sumi = 0;
            if (k < n_valid32) {
                const uint8_t *bp = base + 17u * k;
                for (uint32_t i = 0; i < 16; i++) {
                    const uint8_t q = bp[1 + i];
                    sumi += k_mxfp4_kv[q & 0x0f] * q8[32 * k + i];
                    sumi += k_mxfp4_kv[q >> 4] * q8[32 * k + 16 + i];
                }
                if (sumi != 0) sumf += mxfp4_scale_half(bp[0]) * (float)sumi;
            }
            if (sumi_out) sumi_out[k] = sumi;
        }
        f = yd * sumf;
        break;
    }
    case PULSAR_QUANT_Q5_K: {
        /* cu:5892-5918: Q4_K with a fifth bit per value from qh (bit 2j of
         * qh[i] for value 64j + i, bit 2j + 1 for 64j + 32 + i) */
        const uint8_t *blk = row + (uint64_t)b * 176u;
        const float xd = po_f16_to_f32(rd16(blk));
        const float xmin = po_f16_to_f32(rd16(blk + 2));
        const uint8_t *qh = blk + 16, *q5 = blk + 48;
        int32_t isum = 0, msum = 0;
        for (uint32_t j = 0; j < 4; j++) {
            int32_t sc1, m1, sc2, m2;
            po_k4_scale_min(2 * j, blk + 4, &sc1, &m1);
            po_k4_scale_min(2 * j + 1, blk + 4, &sc2, &m2);
            int32_t s1 = 0, s2 = 0;
            for (uint32_t i = 0; i < 32; i++) {
                const int32_t h1 = (qh[i] >> (2 * j)) & 1, h2 = (qh[i] >> (2 * j + 1)) & 1;
                s1 += ((q5[32 * j + i] & 0x0f) | (h1 << 4)) * q8[64 * j + i];
                s2 += ((q5[32 * j + i] >> 4) | (h2 << 4)) * q8[64 * j + 32 + i];
            }
            isum += sc1 * s1 + sc2 * s2;
            msum += m1 * (bs[4 * j] + bs[4 * j + 1]) + m2 * (bs[4 * j + 2] + bs[4 * j + 3]);
        }
        d0 = isum;
        d1 = msum;
        f = xd * yd * (float)isum - xmin * yd * (float)msum;
        break;
    }
    case PULSAR_QUANT_Q3_K: {
        /* cpu:166-204 (== cu:5807-5838) */
        const uint8_t *blk = row + (uint64_t)b * 110u;
        const uint8_t *hm = blk, *q3 = blk + 32;
        const float xd = po_f16_to_f32(rd16(blk + 108));
        int32_t sc[16];
        k3_scales(blk + 96, sc);
        int32_t isum = 0;
        uint32_t hbit = 1u, is = 0;
        for (uint32_t k = 0; k < 2; k++) {
            for (uint32_t shift = 0; shift < 8; shift += 2) {
                for (uint32_t half = 0; half < 2; half++) {
                    int32_t s16 = 0;
                    for (uint32_t i = 0; i < 16; i++) {
                        const uint32_t l = 16 * half + i;
                        int32_t q = (q3[32 * k + l] >> shift) & 3;
                        if ((hm[l] & hbit) == 0u) q -= 4;
                        s16 += q * q8[128 * k + 32 * (shift / 2) + l];
                    }
                    isum += sc[is++] * s16;
                }
                hbit <<= 1;
            }
        }
        d0 = isum;
        f = xd * yd * (float)isum;
        break;
    }
    case PULSAR_QUANT_IQ2_XS: {
        /* cpu:299-338 */
        const uint8_t *blk = row + (uint64_t)b * 74u;
        const float xd = po_f16_to_f32(rd16(blk));
        int32_t bsum = 0;
        for (uint32_t g = 0; g < 8; g++) {
            const uint8_t sc = blk[66 + g];
            const int32_t ls1 = 2 * (sc & 0x0f) + 1, ls2 = 2 * (sc >> 4) + 1;
            int32_t s1 = 0, s2 = 0;
            for (uint32_t j = 0; j < 4; j++) {
                const uint32_t q = rd16(blk + 2 + 2 * (4 * g + j));
                const uint32_t sm = sign_mask(q >> 9);
                int32_t acc = 0;
                for (uint32_t i = 0; i < 8; i++) {
                    const int32_t gv = iq2xs_mag(q & 511u, i);
                    acc += ((sm >> i) & 1u ? -gv : gv) * q8[32 * g + 8 * j + i];
                }
                if (j < 2) s1 += acc; else s2 += acc;
            }
            bsum += ls1 * s1 + ls2 * s2;
        }
        d0 = bsum;
        f = 0.125f * xd * yd * (float)bsum;
        break;
    }
    case PULSAR_QUANT_IQ3_XXS: {
        /* cpu:349-390: per group db = xd * (0.5 + s) * 0.5 in f32;
         * d0 = sum_g (2 s + 1) * sumi_g, the same value in integers */
        const uint8_t *blk = row + (uint64_t)b * 98u;
        const float xd = po_f16_to_f32(rd16(blk));
        float sumf = 0.0f;
        int32_t isum = 0;
        for (uint32_t g = 0; g < 8; g++) {
            const uint32_t aux = rd32(blk + 66 + 4 * g);
            const float db = xd * (0.5f + (float)(aux >> 28)) * 0.5f;
            int32_t sumi = 0;
            for (uint32_t j = 0; j < 4; j++) {
                const uint32_t sm = sign_mask((aux >> (7 * j)) & 127u);
                const uint32_t i0 = blk[2 + 8 * g + 2 * j], i1 = blk[2 + 8 * g + 2 * j + 1];
                for (uint32_t i = 0; i < 4; i++) {
                    const int32_t w0 = iq3xxs_mag(i0, i), w1 = iq3xxs_mag(i1, i);
                    sumi += ((sm >> i) & 1u ? -w0 : w0) * q8[32 * g + 8 * j + i] +
                            ((sm >> (4 + i)) & 1u ? -w1 : w1) * q8[32 * g + 8 * j + 4 + i];
                }
            }
            sumf += db * (float)sumi;
            isum += (int32_t)(2u * (aux >> 28) + 1u) * sumi;
        }
        d0 = isum;
        f = yd * sumf;
        break;
    }
    case PULSAR_QUANT_IQ4_XS: {
        /* cu:5843-5865 */
        const uint8_t *blk = row + (uint64_t)b * 136u;
        const uint32_t sh = rd16(blk + 2);
        const uint8_t *qs = blk + 8;
        float sumf = 0.0f;
        int any = 0;
        int32_t isum = 0;
        for (uint32_t ib = 0; ib < 8; ib++) {
            const int32_t ls = (int32_t)(((blk[4 + ib / 2] >> (4 * (ib & 1))) & 0x0fu) | (((sh >> (2 * ib)) & 3u) << 4)) - 32;
            int32_t sumi = 0;
            for (uint32_t j = 0; j < 16; j++) {
                const uint8_t v = qs[16 * ib + j];
                sumi += k_iq4nl[v & 0x0f] * q8[32 * ib + j] + k_iq4nl[v >> 4] * q8[32 * ib + 16 + j];
            }
            if (sumi != 0) {
                sumf += (float)(ls * sumi);
                any = 1;
            }
            isum += ls * sumi;
        }
        d0 = isum;
        f = any ? po_f16_to_f32(rd16(blk)) * yd * sumf : 0.0f;
        break;
    }
    case PULSAR_QUANT_Q8_0: {
        /* cu:5793-5805: 8 blocks of f16 d + 32 int8 */
        float sumf = 0.0f;
        for (uint32_t k = 0; k < 8; k++) {
            const uint8_t *bp = row + (uint64_t)b * 272u + 34u * k;
            int32_t sumi = 0;
            for (uint32_t i = 0; i < 32; i++) sumi += (int8_t)bp[2 + i] * q8[32 * k + i];
            if (sumi != 0) sumf += po_f16_to_f32(rd16(bp)) * (float)sumi;
            if (sumi_out) sumi_out[k] = sumi;
        }
        f = yd * sumf;
        break;
    }
    case PULSAR_QUANT_Q4_0: {
        /* cu:5773-5791: value = nibble - 8, folded through the bsums */
        float sumf = 0.0f;
        for (uint32_t k = 0; k < 8; k++) {
            const uint8_t *bp = row + (uint64_t)b * 144u + 18u * k;
            int32_t sumi = 0;
            for (uint32_t i = 0; i < 16; i++)
                sumi += (bp[2 + i] & 0x0f) * q8[32 * k + i] + (bp[2 + i] >> 4) * q8[32 * k + 16 + i];
            const int32_t bsum = bs[2 * k] + bs[2 * k + 1];
            if (sumi != 0 || bsum != 0) sumf += po_f16_to_f32(rd16(bp)) * (float)(sumi - 8 * bsum);
            if (sumi_out) sumi_out[k] = sumi - 8 * bsum;
        }
        f = yd * sumf;
        break;
    }
    case PULSAR_QUANT_Q5_1: {
        /* cu:5950-5975: value = d * (nibble | qh bit << 4) + m */
        float sumf = 0.0f;
        for (uint32_t k = 0; k < 8; k++) {
            const uint8_t *bp = row + (uint64_t)b * 192u + 24u * k;
            const uint32_t qh = rd32(bp + 4);
            int32_t sumi = 0;
            for (uint32_t i = 0; i < 16; i++) {
                const int32_t lo = (bp[8 + i] & 0x0f) | (int32_t)(((qh >> i) & 1u) << 4);
                const int32_t hi = (bp[8 + i] >> 4) | (int32_t)(((qh >> (i + 16)) & 1u) << 4);
                sumi += lo * q8[32 * k + i] + hi * q8[32 * k + 16 + i];
            }
            const int32_t bsum = bs[2 * k] + bs[2 * k + 1];
            if (sumi != 0 || bsum != 0)
                sumf += po_f16_to_f32(rd16(bp)) * (float)sumi + po_f16_to_f32(rd16(bp + 2)) * (float)bsum;
            if (sumi_out) sumi_out[k] = sumi;
        }
        f = yd * sumf;
        break;
    }
    case PULSAR_QUANT_IQ4_NL: {
        /* cu:5605-5625 */
        float sumf = 0.0f;
        for (uint32_t k = 0; k < 8; k++) {
            const uint8_t *bp = row + (uint64_t)b * 144u + 18u * k;
            int32_t sumi = 0;
            for (uint32_t i = 0; i < 16; i++)
                sumi += k_iq4nl[bp[2 + i] & 0x0f] * q8[32 * k + i] + k_iq4nl[bp[2 + i] >> 4] * q8[32 * k + 16 + i];
            if (sumi != 0) sumf += po_f16_to_f32(rd16(bp)) * (float)sumi;
            if (sumi_out) sumi_out[k] = sumi;
        }
        f = yd * sumf;
        break;
    }
    case PULSAR_QUANT_IQ3_S: {
        /* cu:5683-5713; d0 = sum_g (1 + 2 sc) * sumi_g */
        const uint8_t *blk = row + (uint64_t)b * 110u;
        const float d = po_f16_to_f32(rd16(blk));
        const uint8_t *qs = blk + 2, *qhb = blk + 66, *sg = blk + 74, *scb = blk + 106;
        float sumf = 0.0f;
        int32_t isum = 0;
        for (uint32_t g = 0; g < 8; g++) {
            const int32_t sc = (g & 1) ? (scb[g >> 1] >> 4) : (scb[g >> 1] & 0x0f);
            const float db = d * (float)(1 + 2 * sc);
            const uint32_t qh = qhb[g];
            int32_t sumi = 0;
            for (uint32_t l = 0; l < 4; l++) {
                const uint32_t i0 = qs[8 * g + 2 * l] | ((qh << (8 - 2 * l)) & 256u);
                const uint32_t i1 = qs[8 * g + 2 * l + 1] | ((qh << (7 - 2 * l)) & 256u);
                const uint32_t s = sg[4 * g + l];
                for (uint32_t j = 0; j < 4; j++) {
                    const int32_t v0 = iq3s_mag(i0, j), v1 = iq3s_mag(i1, j);
                    sumi += ((s >> j) & 1u ? -v0 : v0) * q8[32 * g + 8 * l + j] +
                            ((s >> (j + 4)) & 1u ? -v1 : v1) * q8[32 * g + 8 * l + 4 + j];
                }
            }
            sumf += db * (float)sumi;
            isum += (1 + 2 * sc) * sumi;
        }
        d0 = isum;
        f = yd * sumf;
        break;
    }
    case PULSAR_QUANT_IQ2_S: {
        /* cu:5627-5657; d0 = sum (2 n + 1) * acc, dl = d (2 n + 1) / 8 */
        const uint8_t *blk = row + (uint64_t)b * 82u;
        const float d = po_f16_to_f32(rd16(blk));
        const uint8_t *qs = blk + 2, *sg = blk + 34, *qhb = blk + 66, *scb = blk + 74;
        float sumf = 0.0f;
        int32_t isum = 0;
        for (uint32_t g = 0; g < 8; g++) {
            const uint32_t qh = qhb[g];
            for (uint32_t j = 0; j < 4; j++) {
                const uint32_t idx = qs[4 * g + j] | ((qh << (8 - 2 * j)) & 0x300u);
                const uint32_t s = sg[4 * g + j];
                const int32_t n = j < 2 ? (scb[g] & 0x0f) : (scb[g] >> 4);
                const float dl = d * (0.5f + (float)n) * 0.25f;
                int32_t acc = 0;
                for (uint32_t k = 0; k < 8; k++) {
                    const int32_t gv = iq2s_mag(idx, k);
                    acc += ((s >> k) & 1u ? -gv : gv) * q8[32 * g + 8 * j + k];
                }
                sumf += dl * (float)acc;
                isum += (2 * n + 1) * acc;
            }
        }
        d0 = isum;
        f = yd * sumf;
        break;
    }
    case PULSAR_QUANT_IQ1_S: {
        /* cu:5659-5681 */
        const uint8_t *blk = row + (uint64_t)b * 50u;
        int32_t sumi = 0, sumi1 = 0;
        for (uint32_t g = 0; g < 8; g++) {
            const uint32_t qh = rd16(blk + 34 + 2 * g);
            const int32_t ls = 2 * (int32_t)((qh >> 12) & 7u) + 1;
            const int32_t dsign = (qh & 0x8000u) ? -1 : 1;
            int32_t lsum = 0;
            for (uint32_t j = 0; j < 4; j++) {
                const uint32_t idx = blk[2 + 4 * g + j] | (((qh >> (3 * j)) & 7u) << 8);
                for (uint32_t k = 0; k < 8; k++) lsum += iq1s_val(idx, k) * q8[32 * g + 8 * j + k];
            }
            sumi += ls * lsum;
            sumi1 += ls * dsign * (bs[2 * g] + bs[2 * g + 1]);
        }
        d0 = sumi;
        d1 = sumi1;
        f = po_f16_to_f32(rd16(blk)) * yd * ((float)sumi + 0.125f * (float)sumi1);
        break;
    }
    case PULSAR_QUANT_NVFP4: {
        /* cu:5743-5771: 4 blocks of 4 UE4M3 scales + 32 nibble bytes; per
         * 16-value sub-block the doubled E2M1 table and half the scale */
        float sumf = 0.0f;
        for (uint32_t k = 0; k < 4; k++) {
            const uint8_t *bp = row + (uint64_t)b * 144u + 36u * k;
            for (uint32_t sub = 0; sub < 4; sub++) {
                int32_t sumi = 0;
                for (uint32_t i = 0; i < 8; i++) {
                    const uint8_t q = bp[4 + 8 * sub + i];
                    sumi += k_mxfp4_kv[q & 0x0f] * q8[64 * k + 16 * sub + i] +
                            k_mxfp4_kv[q >> 4] * q8[64 * k + 16 * sub + 8 + i];
                }
                sumf += ue4m3(bp[sub]) * 0.5f * (float)sumi;
            }
        }
        f = yd * sumf;
        break;
    }
    default:
        break;
    }
    if (i0) *i0 = d0;
    if (i1) *i1 = d1;
    return f;
}

static uint32_t valid32_in_sb(uint32_t n, uint32_t b) {
    const uint32_t rem = n - 256u * b;
    return rem >= 256u ? 8u : (rem + 31u) / 32u;
}

/* AVX2 row dots of the lane formats (lane_avx2.c): on by default where the
 * CPU has AVX2, like the reference lane's dispatch (cpu:76-86, 242-247,
 * 721-726); bit-identical to the scalar dots. */
int po_avx2_supported(void);
int po_avx2_has_format(uint32_t quant);
float po_avx2_vec_dot(uint32_t quant, const uint8_t *row, const pulsar_block_q8_K *xq, uint32_t n);
static int g_simd = -1;

int po_set_simd(int on) {
    const int prev = g_simd < 0 ? po_avx2_supported() : g_simd;
    g_simd = on && po_avx2_supported();
    return prev;
}

/* cpu:242-279 (and siblings): total = 0; total += f_b for b in order */
float po_vec_dot(uint32_t quant, const uint8_t *row, const pulsar_block_q8_K *xq,
                 uint32_t n, double *abs_sum) {
    if (g_simd < 0) g_simd = po_avx2_supported();
    if (g_simd && !abs_sum && n % 256u == 0 && po_avx2_has_format(quant))
        return po_avx2_vec_dot(quant, row, xq, n);
    const uint32_t nb = (n + 255u) / 256u;
    float total = 0.0f;
    double as = 0.0;
    for (uint32_t b = 0; b < nb; b++) {
        const float f = po_block_dot(quant, row, b, xq + b, valid32_in_sb(n, b), NULL, NULL, NULL);
        total += f;
        as += fabs((double)f);
    }
    if (abs_sum) *abs_sum = as;
    return total;
}

/* f64 element-wise dequant, straight from the format descriptions (the
 * reference tests' dequant references: cpu:848-872, 925-947, 971-989). */
void po_dequant_row(uint32_t quant, const uint8_t *row, uint32_t n, double *out) {
    const uint32_t nb = (n + 255u) / 256u;
    for (uint32_t b = 0; b < nb; b++) {
        double v[256];
        memset(v, 0, sizeof(v));
        switch (quant) {
        case PULSAR_QUANT_Q4_K: {
            const uint8_t *blk = row + (uint64_t)b * 144u;
            const double xd = po_f16_to_f32(rd16(blk));
            const double xmin = po_f16_to_f32(rd16(blk + 2));
            for (uint32_t s = 0; s < 8; s++) { /* sub-block s: values 32s.. */
                int32_t sc, m;
                po_k4_scale_min(s, blk + 4, &sc, &m);
                for (uint32_t i = 0; i < 32; i++) {
                    const uint8_t byte = blk[16 + 32 * (s / 2) + i];
                    const int32_t q = (s & 1) ? (byte >> 4) : (byte & 0x0f);
                    v[32 * s + i] = xd * sc * q - xmin * m;
                }
            }
            break;
        }
        case PULSAR_QUANT_Q2_K: {
            const uint8_t *blk = row + (uint64_t)b * 84u;
            const double xd = po_f16_to_f32(rd16(blk + 80));
            const double xmin = po_f16_to_f32(rd16(blk + 82));
            for (uint32_t c = 0; c < 16; c++) { /* 16-value chunk c (cpu:852-872) */
                const uint32_t k = c / 8, js = (c % 8) / 2, half = c % 2;
                for (uint32_t i = 0; i < 16; i++) {
                    const int32_t q = (blk[16 + 32 * k + 16 * half + i] >> (2 * js)) & 3;
                    v[16 * c + i] = xd * (blk[c] & 0x0f) * q - xmin * (blk[c] >> 4);
                }
            }
            break;
        }
        case PULSAR_QUANT_Q6_K: {
            /* value 128h + 32q + i (h half, q quarter): low 4 bits from
             * ql[64h + 32(q&1) + i] nibble q>>1, high 2 from qh[32h + i]
             * bits 2q..2q+1, minus 32; scale sc[8h + (32q + i)/16] */
            const uint8_t *blk = row + (uint64_t)b * 210u;
            const double xd = po_f16_to_f32(rd16(blk + 208));
            const int8_t *sc = (const int8_t *)(blk + 192);
            for (uint32_t h = 0; h < 2; h++)
                for (uint32_t q = 0; q < 4; q++)
                    for (uint32_t i = 0; i < 32; i++) {
                        const uint8_t lb = blk[64 * h + 32 * (q & 1) + i];
                        const int32_t lo = (q >> 1) ? (lb >> 4) : (lb & 0x0f);
                        const int32_t hi = (blk[128 + 32 * h + i] >> (2 * q)) & 3;
                        const uint32_t vi = 32 * q + i;
                        v[128 * h + vi] = xd * sc[8 * h + vi / 16] * ((lo | (hi << 4)) - 32);
                    }
            break;
        }
        case PULSAR_QUANT_IQ2_XXS: {
            const uint8_t *blk = row + (uint64_t)b * 66u;
            const double xd = po_f16_to_f32(rd16(blk));
            for (uint32_t g = 0; g < 8; g++) {
                const uint32_t aux0 = rd32(blk + 2 + 8 * g);
                const uint32_t aux1 = rd32(blk + 6 + 8 * g);
                const double db = 0.125 * xd * (2.0 * (aux1 >> 28) + 1.0);
                for (uint32_t k = 0; k < 4; k++) {
                    const uint32_t sm = sign_mask((aux1 >> (7 * k)) & 127u);
                    for (uint32_t i = 0; i < 8; i++) {
                        const double mag = po_iq2xxs_mag((aux0 >> (8 * k)) & 0xffu, i);
                        v[32 * g + 8 * k + i] = ((sm >> i) & 1u) ? -db * mag : db * mag;
                    }
                }
            }
            break;
        }
        case PULSAR_QUANT_MXFP4: {
            /* textbook OCP MX: value = E2M1(code) * 2^(e - 127), E2M1
             * magnitudes {0, .5, 1, 1.5, 2, 3, 4, 6}, bit 3 = sign
             * (crates/gguf/src/lib.rs:73-76); the reference flushes e < 2 */
            static const double e2m1[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
            const uint32_t nv = valid32_in_sb(n, b);
            for (uint32_t k = 0; k < nv; k++) {
                const uint8_t *bp = row + (uint64_t)b * 136u + 17u * k;
                const double scale = bp[0] < 2 ? 0.0 : ldexp(1.0, (int)bp[0] - 127);
                for (uint32_t i = 0; i < 16; i++) {
                    const uint8_t lo = bp[1 + i] & 0x0f, hi = bp[1 + i] >> 4;
                    v[32 * k + i] = (lo & 8 ? -1.0 : 1.0) * e2m1[lo & 7] * scale;
                    v[32 * k + 16 + i] = (hi & 8 ? -1.0 : 1.0) * e2m1[hi & 7] * scale;
                }
            }
            break;
        }
        case PULSAR_QUANT_Q5_K: { /* 8 sub-blocks of 32: xd sc q5 - xmin m */
            const uint8_t *blk = row + (uint64_t)b * 176u;
            const double xd = po_f16_to_f32(rd16(blk)), xmin = po_f16_to_f32(rd16(blk + 2));
            for (uint32_t s = 0; s < 8; s++) {
                int32_t sc, m;
                po_k4_scale_min(s, blk + 4, &sc, &m);
                for (uint32_t i = 0; i < 32; i++) {
                    const uint8_t byte = blk[48 + 32 * (s / 2) + i];
                    const int32_t lo = (s & 1) ? (byte >> 4) : (byte & 0x0f);
                    const int32_t q = lo | (((blk[16 + i] >> s) & 1) << 4);
                    v[32 * s + i] = xd * sc * q - xmin * m;
                }
            }
            break;
        }
        case PULSAR_QUANT_Q3_K: { /* cpu:921-935: 16-value chunk c = 8k + 2js + half */
            const uint8_t *blk = row + (uint64_t)b * 110u;
            const double xd = po_f16_to_f32(rd16(blk + 108));
            int32_t sc[16];
            k3_scales(blk + 96, sc);
            for (uint32_t c = 0; c < 16; c++) {
                const uint32_t k = c / 8, js = (c % 8) / 2, half = c % 2;
                for (uint32_t i = 0; i < 16; i++) {
                    const uint32_t l = 16 * half + i;
                    int32_t q = (blk[32 + 32 * k + l] >> (2 * js)) & 3;
                    if ((blk[l] & (1u << (4 * k + js))) == 0) q -= 4;
                    v[16 * c + i] = xd * sc[c] * q;
                }
            }
            break;
        }
        case PULSAR_QUANT_IQ2_XS: { /* cpu:1008-1022 */
            const uint8_t *blk = row + (uint64_t)b * 74u;
            const double xd = po_f16_to_f32(rd16(blk));
            for (uint32_t g = 0; g < 8; g++)
                for (uint32_t j = 0; j < 4; j++) {
                    const uint32_t q = rd16(blk + 2 + 2 * (4 * g + j));
                    const uint32_t sm = sign_mask(q >> 9);
                    const double ls = j < 2 ? 2 * (blk[66 + g] & 0x0f) + 1 : 2 * (blk[66 + g] >> 4) + 1;
                    for (uint32_t i = 0; i < 8; i++)
                        v[32 * g + 8 * j + i] = 0.125 * xd * ls * iq2xs_mag(q & 511u, i) * ((sm >> i) & 1u ? -1.0 : 1.0);
                }
            break;
        }
        case PULSAR_QUANT_IQ3_XXS: { /* cpu:1050-1073 */
            const uint8_t *blk = row + (uint64_t)b * 98u;
            const double xd = po_f16_to_f32(rd16(blk));
            for (uint32_t g = 0; g < 8; g++) {
                const uint32_t aux = rd32(blk + 66 + 4 * g);
                const double db = xd * (0.5 + (aux >> 28)) * 0.5;
                for (uint32_t j = 0; j < 4; j++) {
                    const uint32_t sm = sign_mask((aux >> (7 * j)) & 127u);
                    for (uint32_t i = 0; i < 4; i++) {
                        v[32 * g + 8 * j + i] = db * iq3xxs_mag(blk[2 + 8 * g + 2 * j], i) * ((sm >> i) & 1u ? -1.0 : 1.0);
                        v[32 * g + 8 * j + 4 + i] =
                            db * iq3xxs_mag(blk[3 + 8 * g + 2 * j], i) * ((sm >> (4 + i)) & 1u ? -1.0 : 1.0);
                    }
                }
            }
            break;
        }
        case PULSAR_QUANT_IQ4_XS: { /* d (ls - 32) kvalues[q], ls 6-bit split low 4 / high 2 */
            const uint8_t *blk = row + (uint64_t)b * 136u;
            const double xd = po_f16_to_f32(rd16(blk));
            const uint32_t sh = rd16(blk + 2);
            for (uint32_t ib = 0; ib < 8; ib++) {
                const int32_t ls = (int32_t)(((blk[4 + ib / 2] >> (4 * (ib & 1))) & 0x0fu) | (((sh >> (2 * ib)) & 3u) << 4)) - 32;
                for (uint32_t j = 0; j < 16; j++) {
                    const uint8_t q = blk[8 + 16 * ib + j];
                    v[32 * ib + j] = xd * ls * k_iq4nl[q & 0x0f];
                    v[32 * ib + 16 + j] = xd * ls * k_iq4nl[q >> 4];
                }
            }
            break;
        }
        case PULSAR_QUANT_Q8_0:
        case PULSAR_QUANT_Q4_0:
        case PULSAR_QUANT_Q5_1:
        case PULSAR_QUANT_IQ4_NL: { /* 8 blocks of 32 values with an f16 scale each */
            const uint32_t bb = quant == PULSAR_QUANT_Q8_0 ? 34u : quant == PULSAR_QUANT_Q5_1 ? 24u : 18u;
            for (uint32_t k = 0; k < 8; k++) {
                const uint8_t *bp = row + (uint64_t)b * 8u * bb + (uint64_t)bb * k;
                const double d = po_f16_to_f32(rd16(bp));
                for (uint32_t i = 0; i < 32; i++) {
                    double val;
                    if (quant == PULSAR_QUANT_Q8_0) {
                        val = d * (int8_t)bp[2 + i];
                    } else {
                        const uint32_t off = quant == PULSAR_QUANT_Q5_1 ? 8u : 2u;
                        const int32_t nib = i < 16 ? (bp[off + i] & 0x0f) : (bp[off + i - 16] >> 4);
                        if (quant == PULSAR_QUANT_Q4_0)
                            val = d * (nib - 8);
                        else if (quant == PULSAR_QUANT_IQ4_NL)
                            val = d * k_iq4nl[nib];
                        else /* value i's fifth bit is bit i of qh */
                            val = d * (nib | (int32_t)(((rd32(bp + 4) >> i) & 1u) << 4)) + po_f16_to_f32(rd16(bp + 2));
                    }
                    v[32 * k + i] = val;
                }
            }
            break;
        }
        case PULSAR_QUANT_IQ3_S: { /* d (1 + 2 sc) +-grid, 9-bit indices, explicit sign bytes */
            const uint8_t *blk = row + (uint64_t)b * 110u;
            const double d = po_f16_to_f32(rd16(blk));
            for (uint32_t g = 0; g < 8; g++) {
                const int32_t sc = (g & 1) ? (blk[106 + g / 2] >> 4) : (blk[106 + g / 2] & 0x0f);
                for (uint32_t p = 0; p < 8; p++) { /* grid entry p of the group: values 4p .. 4p+3 */
                    const uint32_t idx = blk[2 + 8 * g + p] | ((((uint32_t)blk[66 + g] >> p) & 1u) << 8);
                    const uint32_t s = blk[74 + 4 * g + p / 2];
                    for (uint32_t j = 0; j < 4; j++) {
                        const uint32_t bit = 4 * (p & 1) + j;
                        v[32 * g + 4 * p + j] = d * (1 + 2 * sc) * iq3s_mag(idx, j) * ((s >> bit) & 1u ? -1.0 : 1.0);
                    }
                }
            }
            break;
        }
        case PULSAR_QUANT_IQ2_S: { /* d (0.5 + n) / 4 +-grid, 10-bit indices */
            const uint8_t *blk = row + (uint64_t)b * 82u;
            const double d = po_f16_to_f32(rd16(blk));
            for (uint32_t g = 0; g < 8; g++)
                for (uint32_t j = 0; j < 4; j++) {
                    const uint32_t idx = blk[2 + 4 * g + j] | ((((uint32_t)blk[66 + g] >> (2 * j)) & 3u) << 8);
                    const uint32_t s = blk[34 + 4 * g + j];
                    const int32_t n = j < 2 ? (blk[74 + g] & 0x0f) : (blk[74 + g] >> 4);
                    for (uint32_t k = 0; k < 8; k++)
                        v[32 * g + 8 * j + k] = d * (0.5 + n) * 0.25 * iq2s_mag(idx, k) * ((s >> k) & 1u ? -1.0 : 1.0);
                }
            break;
        }
        case PULSAR_QUANT_IQ1_S: { /* d (2 s + 1) (g +- 1/8), g ternary */
            const uint8_t *blk = row + (uint64_t)b * 50u;
            const double d = po_f16_to_f32(rd16(blk));
            for (uint32_t g = 0; g < 8; g++) {
                const uint32_t qh = rd16(blk + 34 + 2 * g);
                const double dl = d * (2 * ((qh >> 12) & 7u) + 1);
                const double delta = (qh & 0x8000u) ? -0.125 : 0.125;
                for (uint32_t j = 0; j < 4; j++) {
                    const uint32_t idx = blk[2 + 4 * g + j] | (((qh >> (3 * j)) & 7u) << 8);
                    for (uint32_t k = 0; k < 8; k++) v[32 * g + 8 * j + k] = dl * (iq1s_val(idx, k) + delta);
                }
            }
            break;
        }
        case PULSAR_QUANT_NVFP4: { /* OCP E2M1 times a UE4M3 scale per 16 values */
            static const double e2m1[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
            for (uint32_t k = 0; k < 4; k++) {
                const uint8_t *bp = row + (uint64_t)b * 144u + 36u * k;
                for (uint32_t sub = 0; sub < 4; sub++) {
                    const uint8_t e = bp[sub];
                    const int ex = (e >> 3) & 0xF, man = e & 7;
                    const double scale = (e == 0 || e == 0x7F) ? 0.0
                                         : ex == 0 ? ldexp((double)man, -9) : ldexp(1.0 + man / 8.0, ex - 7);
                    for (uint32_t i = 0; i < 8; i++) {
                        const uint8_t q = bp[4 + 8 * sub + i];
                        const uint8_t lo = q & 0x0f, hi = q >> 4;
                        v[64 * k + 16 * sub + i] = (lo & 8 ? -1.0 : 1.0) * e2m1[lo & 7] * scale;
                        v[64 * k + 16 * sub + 8 + i] = (hi & 8 ? -1.0 : 1.0) * e2m1[hi & 7] * scale;
                    }
                }
            }
            break;
        }
        default:
            break;
        }
        for (uint32_t i = 0; i < 256; i++) {
            const uint64_t c = (uint64_t)b * 256u + i;
            if (c < n) out[c] = v[i];
        }
    }
}

static int quant_ok(uint32_t quant) { return po_sb_bytes(quant) != 0; }

/* cu:4895-4906 argument contract; each output is the lane's row dot */
int po_matmul_kq(float *out, const uint8_t *w, const pulsar_block_q8_K *xq,
                 uint32_t in_dim, uint32_t out_dim, uint32_t n_tok,
                 uint64_t row_bytes, uint32_t quant) {
    quant &= ~PULSAR_QUANT_A4_OK;
    if (in_dim == 0 || in_dim % 256u != 0 || out_dim == 0 || n_tok == 0 || row_bytes == 0 ||
        quant == PULSAR_QUANT_MXFP4 || !quant_ok(quant))
        return 0;
    const uint32_t nb = in_dim / 256u;
    for (uint32_t t = 0; t < n_tok; t++)
        for (uint32_t r = 0; r < out_dim; r++)
            out[(uint64_t)t * out_dim + r] =
                po_vec_dot(quant, w + (uint64_t)r * row_bytes, xq + (uint64_t)t * nb, in_dim, NULL);
    return 1;
}

/* ---------------------------------------------------------------- glu -- */

/* cu:124-141 == elib:2131-2157 */
float po_glu(float g, float u, uint32_t op) {
    if (op == 2u) {
        g = fminf(g, 7.0f);
        u = fminf(fmaxf(u, -7.0f), 7.0f);
        return g / (1.0f + expf(-1.702f * g)) * (u + 1.0f);
    }
    return g / (1.0f + expf(-g)) * u;
}

/* ---------------------------------------------------------------- MoE -- */

/* cu:2566-2614 semantics with the lane's per-row sequential dots
 * (elib:2042-2050): NULL gate/up -> 0; bias added to the projection output
 * before the combine; router weight multiplies the combine. */
int po_moe_pair_swiglu(float *mid, const pulsar_expert_ptrs *ptrs, const float *weights,
                       const pulsar_block_q8_K *xq, uint32_t in_dim, uint32_t mid_dim,
                       uint32_t n_used, uint32_t n_tok, uint64_t row_bytes,
                       uint32_t quant, uint32_t act_op) {
    if (in_dim == 0 || mid_dim == 0 || n_used == 0 || n_tok == 0 || row_bytes == 0 ||
        !quant_ok(quant) || (act_op != 0u && act_op != 2u))
        return 0;
    const uint32_t nb = (in_dim + 255u) / 256u;
    for (uint32_t t = 0; t < n_tok; t++) {
        for (uint32_t s = 0; s < n_used; s++) {
            const uint64_t so = (uint64_t)t * n_used + s;
            const pulsar_expert_ptrs p = ptrs[so];
            float *m = mid + so * mid_dim;
            if (!p.gate || !p.up) {
                memset(m, 0, (size_t)mid_dim * 4u);
                continue;
            }
            for (uint32_t r = 0; r < mid_dim; r++) {
                float g = po_vec_dot(quant, (const uint8_t *)p.gate + (uint64_t)r * row_bytes,
                                     xq + (uint64_t)t * nb, in_dim, NULL);
                float u = po_vec_dot(quant, (const uint8_t *)p.up + (uint64_t)r * row_bytes,
                                     xq + (uint64_t)t * nb, in_dim, NULL);
                if (p.gate_b) g += p.gate_b[r];
                if (p.up_b) u += p.up_b[r];
                m[r] = po_glu(g, u, act_op) * weights[so];
            }
        }
    }
    return 1;
}

/* cu:2616-2647 semantics in the lane's form (elib:2086-2093): per output
 * row, the slots' full row dots summed in slot order; NULL down skipped. */
int po_moe_down(float *out, const pulsar_expert_ptrs *ptrs, const pulsar_block_q8_K *midq,
                uint32_t mid_dim, uint32_t out_dim, uint32_t n_used, uint32_t n_tok,
                uint64_t row_bytes, uint32_t quant) {
    if (mid_dim == 0 || out_dim == 0 || n_used == 0 || n_tok == 0 || row_bytes == 0 ||
        !quant_ok(quant))
        return 0;
    const uint32_t mb = (mid_dim + 255u) / 256u;
    for (uint32_t t = 0; t < n_tok; t++) {
        for (uint32_t r = 0; r < out_dim; r++) {
            float sum = 0.0f;
            for (uint32_t s = 0; s < n_used; s++) {
                const uint64_t so = (uint64_t)t * n_used + s;
                const pulsar_expert_ptrs p = ptrs[so];
                if (!p.down) continue;
                sum += po_vec_dot(quant, (const uint8_t *)p.down + (uint64_t)r * row_bytes,
                                  midq + so * mb, mid_dim, NULL);
            }
            out[(uint64_t)t * out_dim + r] = sum;
        }
    }
    return 1;
}

/* cu:3601-3619 */
int po_moe_down_bias(float *out, const pulsar_expert_ptrs *ptrs, const float *weights,
                     uint32_t out_dim, uint32_t n_used, uint32_t n_tok) {
    if (out_dim == 0 || n_used == 0 || n_tok == 0) return 0;
    for (uint32_t t = 0; t < n_tok; t++)
        for (uint32_t r = 0; r < out_dim; r++) {
            float b = 0.0f;
            for (uint32_t s = 0; s < n_used; s++) {
                const uint64_t so = (uint64_t)t * n_used + s;
                if (ptrs[so].down_b) b += weights[so] * ptrs[so].down_b[r];
            }
            if (b != 0.0f) out[(uint64_t)t * out_dim + r] += b;
        }
    return 1;
}

/* ------------------------------------------------------------- router -- */

/* cu:6504-6535 contract; the sum here is sequential in f64 (the kernel's
 * tree order differs; tests compare within a stated tolerance) */
int po_matmul_f32(float *out, const float *w, const float *x, uint32_t in_dim,
                  uint32_t out_dim, uint32_t n_tok) {
    if (in_dim == 0 || out_dim == 0 || n_tok == 0) return 0;
    for (uint32_t t = 0; t < n_tok; t++)
        for (uint32_t o = 0; o < out_dim; o++) {
            double s = 0.0;
            for (uint32_t i = 0; i < in_dim; i++)
                s += (double)w[(uint64_t)o * in_dim + i] * (double)x[(uint64_t)t * in_dim + i];
            out[(uint64_t)t * out_dim + o] = (float)s;
        }
    return 1;
}

/* cu:3621-3638 */
int po_add_bias_rows(float *x, const float *bias, uint32_t dim, uint32_t rows) {
    if (dim == 0 || rows == 0) return 0;
    for (uint64_t i = 0; i < (uint64_t)rows * dim; i++) x[i] += bias[i % dim];
    return 1;
}

/* cu:913-921 */
static float router_sigmoid(float x) {
    if (x >= 0.0f) {
        const float e = expf(-x);
        return 1.0f / (1.0f + e);
    }
    const float e = expf(x);
    return e / (1.0f + e);
}

/* cu:938-1050 (kernel semantics) with the contract of cu:1052-1064 */
int po_router_select(int32_t *selected, float *weights, const float *logits,
                     const float *bias, uint32_t n_expert, uint32_t k_used,
                     float weight_scale, uint32_t n_tok, uint32_t mode, uint32_t n_shexp) {
    if (n_expert == 0 || k_used == 0 || k_used > n_expert || n_tok == 0 ||
        (mode != 2u && n_shexp != 0) || n_expert + (mode == 2u ? n_shexp : 0u) > 1024u)
        return 0;
    const uint32_t sink = mode == 2u ? n_shexp : 0u;
    const uint32_t n_logit = n_expert + sink, n_slot = k_used + sink;
    float *prob = (float *)malloc(n_expert * sizeof(float));
    float *score = (float *)malloc(n_expert * sizeof(float));
    for (uint32_t t = 0; t < n_tok; t++) {
        const float *lg = logits + (uint64_t)t * n_logit;
        int32_t *sel = selected + (uint64_t)t * n_slot;
        float *w = weights + (uint64_t)t * n_slot;
        for (uint32_t e = 0; e < n_expert; e++) {
            const float raw = lg[e];
            const float p = mode == 1u ? raw : router_sigmoid(raw);
            prob[e] = mode == 2u ? raw : p;
            score[e] = p + (bias ? bias[e] : 0.0f);
        }
        float sum = 0.0f;
        for (uint32_t k = 0; k < k_used; k++) {
            /* cu:922-925 comparator: higher score wins, ties go to the
             * lower index, starting from (-inf, UINT32_MAX) */
            uint32_t best = UINT32_MAX;
            float best_score = -INFINITY;
            for (uint32_t e = 0; e < n_expert; e++) {
                if (score[e] > best_score || (score[e] == best_score && e < best)) {
                    best_score = score[e];
                    best = e;
                }
            }
            if (best == UINT32_MAX) {
                /* every score NaN: no expert compares better than the
                 * start, so the slot keeps (UINT32_MAX as int32 = -1,
                 * prob 0) (cu:979-1009) and routes nowhere. The reference
                 * kernel gives this only when its warp has no padding lane
                 * (n_expert == 32 J, cu:1068-1090); with one, the padding
                 * lane's -inf wins and the id is n_expert, outside the
                 * bank. Here it is -1 in both cases, as on the GPU path. */
                sel[k] = -1;
                w[k] = 0.0f;
                continue;
            }
            sel[k] = (int32_t)best;
            w[k] = prob[best];
            sum += prob[best];
            score[best] = -INFINITY;
        }
        if (mode == 2u) {
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
            float m = -INFINITY;
            for (uint32_t k = 0; k < k_used; k++) m = fmaxf(m, w[k]);
            float es = 0.0f;
            for (uint32_t k = 0; k < k_used; k++) {
                w[k] = expf(w[k] - m);
                es += w[k];
            }
            for (uint32_t k = 0; k < k_used; k++) w[k] = w[k] / es * weight_scale;
        } else {
            sum = fmaxf(sum, 6.103515625e-5f);
            for (uint32_t k = 0; k < k_used; k++) w[k] = w[k] / sum * weight_scale;
        }
    }
    free(prob);
    free(score);
    return 1;
}

/* --------------------------------------------------------------- LCG --- */

float po_lcg(uint64_t *state) {
    *state = *state * 6364136223846793005ull + 1442695040888963407ull;
    return ((float)(*state >> 33) / (float)(1ull << 31)) - 1.0f;
}

/* ------------------------------------------------------ threaded lane -- */

/* A persistent worker pool (the Lane's Pool, elib:1883-1930): jobs are
 * claimed from an atomic counter; the caller joins on completion. */
typedef void (*po_job_fn)(void *ctx, uint32_t job);

typedef struct {
    pthread_mutex_t mu;
    pthread_cond_t cv_start, cv_done;
    uint32_t n_threads;
    uint64_t generation;
    po_job_fn fn;
    void *ctx;
    uint32_t n_jobs;
    uint32_t next_job;
    uint32_t active;
    pthread_t *tids;
} po_pool;

static po_pool g_pool = {PTHREAD_MUTEX_INITIALIZER, PTHREAD_COND_INITIALIZER,
                         PTHREAD_COND_INITIALIZER, 0, 0, NULL, NULL, 0, 0, 0, NULL};

static void *pool_worker(void *arg) {
    (void)arg;
    uint64_t seen = 0;
    pthread_mutex_lock(&g_pool.mu);
    for (;;) {
        while (g_pool.generation == seen) pthread_cond_wait(&g_pool.cv_start, &g_pool.mu);
        seen = g_pool.generation;
        g_pool.active++;
        for (;;) {
            if (g_pool.next_job >= g_pool.n_jobs) break;
            const uint32_t j = g_pool.next_job++;
            po_job_fn fn = g_pool.fn;
            void *ctx = g_pool.ctx;
            pthread_mutex_unlock(&g_pool.mu);
            fn(ctx, j);
            pthread_mutex_lock(&g_pool.mu);
        }
        g_pool.active--;
        if (g_pool.active == 0) pthread_cond_broadcast(&g_pool.cv_done);
    }
    return NULL;
}

static void pool_run(uint32_t threads, po_job_fn fn, void *ctx, uint32_t n_jobs) {
    if (threads <= 1 || n_jobs <= 1) {
        for (uint32_t j = 0; j < n_jobs; j++) fn(ctx, j);
        return;
    }
    pthread_mutex_lock(&g_pool.mu);
    while (g_pool.n_threads < threads) {
        g_pool.tids = (pthread_t *)realloc(g_pool.tids, (g_pool.n_threads + 1) * sizeof(pthread_t));
        pthread_create(&g_pool.tids[g_pool.n_threads], NULL, pool_worker, NULL);
        pthread_detach(g_pool.tids[g_pool.n_threads]);
        g_pool.n_threads++;
    }
    g_pool.fn = fn;
    g_pool.ctx = ctx;
    g_pool.n_jobs = n_jobs;
    g_pool.next_job = 0;
    g_pool.generation++;
    pthread_cond_broadcast(&g_pool.cv_start);
    /* wait until every job is claimed and every worker that woke is idle */
    while (g_pool.next_job < g_pool.n_jobs || g_pool.active > 0)
        pthread_cond_wait(&g_pool.cv_done, &g_pool.mu);
    pthread_mutex_unlock(&g_pool.mu);
}

typedef struct {
    float *out;
    double *abs_sum;
    const uint8_t *w;
    const pulsar_block_q8_K *xq;
    uint32_t in_dim, out_dim, n_tok, quant;
    uint64_t row_bytes;
} mv_ctx;

static void mv_job(void *vctx, uint32_t job) {
    const mv_ctx *c = (const mv_ctx *)vctx;
    const uint32_t nb = (c->in_dim + 255u) / 256u;
    const uint32_t lo = job * 256u;
    const uint32_t hi = lo + 256u < c->out_dim ? lo + 256u : c->out_dim;
    for (uint32_t r = lo; r < hi; r++)
        for (uint32_t t = 0; t < c->n_tok; t++) {
            const uint64_t o = (uint64_t)t * c->out_dim + r;
            c->out[o] = po_vec_dot(c->quant, c->w + (uint64_t)r * c->row_bytes, c->xq + (uint64_t)t * nb,
                                   c->in_dim, c->abs_sum ? c->abs_sum + o : NULL);
        }
}

int po_rows_dot(float *out, const uint8_t *w, uint64_t row_bytes, uint32_t rows,
                const pulsar_block_q8_K *xq, uint32_t n, uint32_t n_tok, uint32_t quant,
                uint32_t threads, double *abs_sum) {
    if (n == 0 || rows == 0 || n_tok == 0 || row_bytes == 0 || !quant_ok(quant) ||
        (quant != PULSAR_QUANT_MXFP4 && n % 256u != 0) || (quant == PULSAR_QUANT_MXFP4 && n % 32u != 0))
        return 0;
    mv_ctx c = {out, abs_sum, w, xq, n, rows, n_tok, quant, row_bytes};
    pool_run(threads, mv_job, &c, (rows + 255u) / 256u);
    return 1;
}

int po_matmul_kq_mt(float *out, const uint8_t *w, const pulsar_block_q8_K *xq,
                    uint32_t in_dim, uint32_t out_dim, uint32_t n_tok,
                    uint64_t row_bytes, uint32_t quant, uint32_t threads, double *abs_sum) {
    quant &= ~PULSAR_QUANT_A4_OK;
    if (in_dim == 0 || in_dim % 256u != 0 || out_dim == 0 || n_tok == 0 || row_bytes == 0 ||
        !quant_ok(quant) || quant == PULSAR_QUANT_MXFP4)
        return 0;
    mv_ctx c = {out, abs_sum, w, xq, in_dim, out_dim, n_tok, quant, row_bytes};
    pool_run(threads, mv_job, &c, (out_dim + 255u) / 256u);
    return 1;
}

/* Lane stage A job: rows [lo, hi) of one (token, slot) pair's gate/up
 * (elib:2037-2053), stage B job: rows [lo, hi) of one token's down sum over
 * its slots (elib:2078-2096). */
typedef struct {
    const pulsar_expert_ptrs *ptrs;
    const float *weights;
    const pulsar_block_q8_K *xq, *midq;
    float *mid, *out;
    uint32_t in_dim, mid_dim, out_dim, n_used, n_tok, gq, dq, act_op;
    uint64_t grb, drb;
    uint32_t jobs_per_pair, jobs_per_tok;
} lane_ctx;

static void lane_a_job(void *vctx, uint32_t job) {
    const lane_ctx *c = (const lane_ctx *)vctx;
    const uint32_t so = job / c->jobs_per_pair;
    const uint32_t lo = (job % c->jobs_per_pair) * 256u;
    const uint32_t hi = lo + 256u < c->mid_dim ? lo + 256u : c->mid_dim;
    const uint32_t t = so / c->n_used;
    const uint32_t nb = (c->in_dim + 255u) / 256u;
    const pulsar_expert_ptrs p = c->ptrs[so];
    float *m = c->mid + (uint64_t)so * c->mid_dim;
    for (uint32_t r = lo; r < hi; r++) {
        if (!p.gate || !p.up) {
            m[r] = 0.0f;
            continue;
        }
        float g = po_vec_dot(c->gq, (const uint8_t *)p.gate + (uint64_t)r * c->grb,
                             c->xq + (uint64_t)t * nb, c->in_dim, NULL);
        float u = po_vec_dot(c->gq, (const uint8_t *)p.up + (uint64_t)r * c->grb,
                             c->xq + (uint64_t)t * nb, c->in_dim, NULL);
        if (p.gate_b) g += p.gate_b[r];
        if (p.up_b) u += p.up_b[r];
        m[r] = po_glu(g, u, c->act_op) * c->weights[so];
    }
}

static void lane_b_job(void *vctx, uint32_t job) {
    const lane_ctx *c = (const lane_ctx *)vctx;
    const uint32_t t = job / c->jobs_per_tok;
    const uint32_t lo = (job % c->jobs_per_tok) * 512u;
    const uint32_t hi = lo + 512u < c->out_dim ? lo + 512u : c->out_dim;
    const uint32_t mb = (c->mid_dim + 255u) / 256u;
    for (uint32_t r = lo; r < hi; r++) {
        float sum = 0.0f;
        for (uint32_t s = 0; s < c->n_used; s++) {
            const uint64_t so = (uint64_t)t * c->n_used + s;
            const pulsar_expert_ptrs p = c->ptrs[so];
            if (!p.down) continue;
            sum += po_vec_dot(c->dq, (const uint8_t *)p.down + (uint64_t)r * c->drb,
                              c->midq + so * mb, c->mid_dim, NULL);
        }
        c->out[(uint64_t)t * c->out_dim + r] = sum;
    }
}

int po_lane_moe(float *out, const pulsar_expert_ptrs *ptrs, const float *weights,
                const float *x, uint32_t in_dim, uint32_t mid_dim, uint32_t out_dim,
                uint32_t n_used, uint32_t n_tok, uint64_t gate_row_bytes,
                uint32_t gate_quant, uint64_t down_row_bytes, uint32_t down_quant,
                uint32_t act_op, uint32_t threads) {
    if (in_dim == 0 || mid_dim == 0 || out_dim == 0 || n_used == 0 || n_tok == 0 ||
        !quant_ok(gate_quant) || !quant_ok(down_quant))
        return 0;
    const uint32_t nb = (in_dim + 255u) / 256u, mb = (mid_dim + 255u) / 256u;
    pulsar_block_q8_K *xq = (pulsar_block_q8_K *)malloc((size_t)n_tok * nb * sizeof(pulsar_block_q8_K));
    pulsar_block_q8_K *midq =
            (pulsar_block_q8_K *)malloc((size_t)n_tok * n_used * mb * sizeof(pulsar_block_q8_K));
    float *mid = (float *)malloc((size_t)n_tok * n_used * mid_dim * sizeof(float));
    po_quantize_q8_K(xq, x, in_dim, n_tok);
    lane_ctx c = {ptrs, weights, xq, midq, mid, out, in_dim, mid_dim, out_dim, n_used, n_tok,
                  gate_quant, down_quant, act_op, gate_row_bytes, down_row_bytes,
                  (mid_dim + 255u) / 256u, (out_dim + 511u) / 512u};
    pool_run(threads, lane_a_job, &c, n_tok * n_used * c.jobs_per_pair);
    po_quantize_q8_K(midq, mid, mid_dim, n_tok * n_used);
    pool_run(threads, lane_b_job, &c, n_tok * c.jobs_per_tok);
    free(xq);
    free(midq);
    free(mid);
    return 1;
}
