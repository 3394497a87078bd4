/* lane_avx2.c - AVX2 row dots of the CPU expert lane's formats.
 *
 * TEST INFRASTRUCTURE ONLY (see pulsar_oracle.h): the vector twin of the
 * scalar dots in pulsar_oracle.c, used by po_vec_dot when AVX2 is enabled,
 * as the reference lane dispatches to its AVX2 paths
 * (crates/quant/src/cpu_dot.rs:76-86, 242-247, 721-726). Each super-block's
 * integer sums are exact int32 in any order, and the fp32 epilogue and the
 * sequential sum over super-blocks are the scalar ones, so every result is
 * bit-identical to the scalar path (the reference asserts the same,
 * cpu_dot.rs:902, 987, 1076).
 *
 * Vector scheme (restating cpu_dot.rs:398-714): unsigned codes times signed
 * q8 by vpmaddubsw (pair sums stay below 2^15: codes <= 43, |q8| <= 127),
 * widened by vpmaddwd against the per-group scales (or ones) and summed.
 */
#include <immintrin.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

#include "pulsar_oracle.h"

#define PO_AVX2 __attribute__((target("avx2")))

float po_f16_to_f32(uint16_t h);
void po_k4_scale_min(uint32_t j, const uint8_t *q, int32_t *sc, int32_t *m);
uint32_t po_iq2xxs_mag(uint32_t idx, uint32_t j);

static inline uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline uint32_t ld32(const uint8_t *p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}

PO_AVX2 static inline int32_t hsum8(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_unpackhi_epi64(s, s));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 1));
    return _mm_cvtsi128_si32(s);
}

/* IQ2_XXS tables: grid rows as 8 magnitude bytes, sign rows as 8 bytes of
 * +1 / -1 (0x01 / 0xff) for the parity-completed 7-bit sign index. */
static uint64_t g_iq2_grid64[256];
static uint64_t g_iq2_sign64[128];
static pthread_once_t g_tables_once = PTHREAD_ONCE_INIT;

static void build_tables(void) {
    for (uint32_t idx = 0; idx < 256; idx++) {
        uint64_t w = 0;
        for (uint32_t j = 0; j < 8; j++) w |= (uint64_t)po_iq2xxs_mag(idx, j) << (8 * j);
        g_iq2_grid64[idx] = w;
    }
    for (uint32_t s = 0; s < 128; s++) {
        const uint32_t full = s | ((uint32_t)(__builtin_popcount(s) & 1) << 7);
        uint64_t w = 0;
        for (uint32_t j = 0; j < 8; j++) w |= (uint64_t)(((full >> j) & 1u) ? 0xffu : 0x01u) << (8 * j);
        g_iq2_sign64[s] = w;
    }
}

/* Q4_K super-block: isum (scaled 32-value sums) and msum (mins x bsums). */
PO_AVX2 static void q4k_sums(const uint8_t *blk, const pulsar_block_q8_K *y, int32_t *isum, int32_t *msum) {
    const __m256i nib = _mm256_set1_epi8(0x0f), ones = _mm256_set1_epi16(1);
    __m256i acc = _mm256_setzero_si256();
    int32_t m = 0;
    for (uint32_t j = 0; j < 4; j++) {
        int32_t sc1, m1, sc2, m2;
        po_k4_scale_min(2 * j, blk + 4, &sc1, &m1);
        po_k4_scale_min(2 * j + 1, blk + 4, &sc2, &m2);
        const __m256i codes = _mm256_loadu_si256((const __m256i *)(blk + 16 + 32 * j));
        const __m256i lo = _mm256_and_si256(codes, nib);
        const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(codes, 4), nib);
        const __m256i xa = _mm256_loadu_si256((const __m256i *)(y->qs + 64 * j));
        const __m256i xb = _mm256_loadu_si256((const __m256i *)(y->qs + 64 * j + 32));
        const __m256i s1 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, xa), ones);
        const __m256i s2 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, xb), ones);
        acc = _mm256_add_epi32(acc, _mm256_mullo_epi32(s1, _mm256_set1_epi32(sc1)));
        acc = _mm256_add_epi32(acc, _mm256_mullo_epi32(s2, _mm256_set1_epi32(sc2)));
        m += m1 * (y->bsums[4 * j] + y->bsums[4 * j + 1]) + m2 * (y->bsums[4 * j + 2] + y->bsums[4 * j + 3]);
    }
    *isum = hsum8(acc);
    *msum = m;
}

/* Q2_K super-block: isum over the 16 scaled 16-value groups, summs = mins x bsums. */
PO_AVX2 static void q2k_sums(const uint8_t *blk, const pulsar_block_q8_K *y, int32_t *isum, int32_t *summs) {
    const __m256i two = _mm256_set1_epi8(3);
    int32_t m = 0;
    for (uint32_t j = 0; j < 16; j++) m += y->bsums[j] * (int32_t)(blk[j] >> 4);
    __m256i acc = _mm256_setzero_si256();
    for (uint32_t k = 0; k < 2; k++) {
        const __m256i codes = _mm256_loadu_si256((const __m256i *)(blk + 16 + 32 * k));
        for (uint32_t s = 0; s < 4; s++) {
            /* bytes 0-15: group 8k + 2s (half 0), bytes 16-31: group 8k + 2s + 1 */
            const __m256i q = _mm256_and_si256(_mm256_srl_epi16(codes, _mm_cvtsi32_si128((int)(2 * s))), two);
            const __m256i x = _mm256_loadu_si256((const __m256i *)(y->qs + 128 * k + 32 * s));
            const uint32_t g = 8 * k + 2 * s;
            const __m256i scl = _mm256_set_m128i(_mm_set1_epi16((int16_t)(blk[g + 1] & 0x0f)),
                                                 _mm_set1_epi16((int16_t)(blk[g] & 0x0f)));
            acc = _mm256_add_epi32(acc, _mm256_madd_epi16(_mm256_maddubs_epi16(q, x), scl));
        }
    }
    *isum = hsum8(acc);
    *summs = m;
}

/* IQ2_XXS super-block: bsum = sum over 32-groups of sumi * (2 * scale + 1). */
PO_AVX2 static int32_t iq2xxs_bsum(const uint8_t *blk, const pulsar_block_q8_K *y) {
    const __m256i ones = _mm256_set1_epi16(1);
    __m256i acc = _mm256_setzero_si256();
    for (uint32_t g = 0; g < 8; g++) {
        const uint32_t aux0 = ld32(blk + 2 + 8 * g), aux1 = ld32(blk + 6 + 8 * g);
        const __m256i mags = _mm256_set_epi64x((long long)g_iq2_grid64[aux0 >> 24],
                                               (long long)g_iq2_grid64[(aux0 >> 16) & 0xffu],
                                               (long long)g_iq2_grid64[(aux0 >> 8) & 0xffu],
                                               (long long)g_iq2_grid64[aux0 & 0xffu]);
        const __m256i sgn = _mm256_set_epi64x((long long)g_iq2_sign64[(aux1 >> 21) & 127u],
                                              (long long)g_iq2_sign64[(aux1 >> 14) & 127u],
                                              (long long)g_iq2_sign64[(aux1 >> 7) & 127u],
                                              (long long)g_iq2_sign64[aux1 & 127u]);
        const __m256i x = _mm256_sign_epi8(_mm256_loadu_si256((const __m256i *)(y->qs + 32 * g)), sgn);
        const __m256i s = _mm256_madd_epi16(_mm256_maddubs_epi16(mags, x), ones);
        acc = _mm256_add_epi32(acc, _mm256_mullo_epi32(s, _mm256_set1_epi32((int32_t)(2u * (aux1 >> 28) + 1u))));
    }
    return hsum8(acc);
}

int po_avx2_supported(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2");
}

int po_avx2_has_format(uint32_t quant) {
    return quant == PULSAR_QUANT_Q4_K || quant == PULSAR_QUANT_Q2_K || quant == PULSAR_QUANT_IQ2_XXS;
}

/* Row dot over n values (a multiple of 256) with the scalar epilogue of
 * each format (cpu:250-279, 732-767, 92-122) and the sequential fp32 sum. */
PO_AVX2 float po_avx2_vec_dot(uint32_t quant, const uint8_t *row, const pulsar_block_q8_K *xq, uint32_t n) {
    const uint32_t nb = n / 256u;
    float total = 0.0f;
    switch (quant) {
    case PULSAR_QUANT_Q4_K:
        for (uint32_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + (uint64_t)b * 144u;
            const float xd = po_f16_to_f32(ld16(blk)), xmin = po_f16_to_f32(ld16(blk + 2)), yd = xq[b].d;
            int32_t isum, msum;
            q4k_sums(blk, xq + b, &isum, &msum);
            total += xd * yd * (float)isum - xmin * yd * (float)msum;
        }
        break;
    case PULSAR_QUANT_Q2_K:
        for (uint32_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + (uint64_t)b * 84u;
            const float xd = po_f16_to_f32(ld16(blk + 80)), xmin = po_f16_to_f32(ld16(blk + 82)), yd = xq[b].d;
            int32_t isum, summs;
            q2k_sums(blk, xq + b, &isum, &summs);
            total += yd * xd * (float)isum - yd * xmin * (float)summs;
        }
        break;
    case PULSAR_QUANT_IQ2_XXS:
        pthread_once(&g_tables_once, build_tables);
        for (uint32_t b = 0; b < nb; b++) {
            const uint8_t *blk = row + (uint64_t)b * 66u;
            const float xd = po_f16_to_f32(ld16(blk)), yd = xq[b].d;
            total += 0.125f * xd * yd * (float)iq2xxs_bsum(blk, xq + b);
        }
        break;
    default:
        return 0.0f;
    }
    return total;
}
