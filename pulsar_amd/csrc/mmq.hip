// mmq.hip - int8 matrix-core (v_mfma_i32_16x16x32_i8) kernels:
//   mmq_gemm_kernel: the dense Q4_K / Q6_K matvec for token chunks and
//     prefill (5 or more tokens; 16- or 32-token tiles). A block computes
//     16 RT weight rows x 16 NT tokens; its waves split each K chunk's
//     super-blocks and the partials are added in wave order through LDS
//     (deterministic);
//   moe_grouped_mmq_kq_kernel: the grouped MoE stages (16 rows x up to 16
//     (token, slot) pairs of one expert per MFMA tile) for Q2_K, IQ2_XXS,
//     MXFP4, Q4_K, Q5_K and Q6_K experts.
// Every kernel produces exact int32 group sums with MFMA, applies the
// format's integer scales in int32 and accumulates super-blocks in order.
// mmq_gemm_kernel forms each super-block's fp32 value in the reference's
// operation order (two roundings per multiply-add); the grouped kernel's
// epilogues are fused multiply-adds (__builtin_fmaf, one rounding), which
// differ from the reference's sums by at most one rounding per step.
//
// Operand layout of v_mfma_i32_16x16x32_i8 (8 int8 per lane):
//   A[i][k]: lane i + 16 * kq, K slots of lane group kq
//   B[k][j]: lane j + 16 * kq, the same K slots
//   D[i][j]: lane j + 16 * (i / 4), element i % 4
// Which 8 slots a lane group holds does not matter: A and B hold the same
// ones, and every sum is over whole lane groups.
#include <type_traits>

#include "pk_rowdot.h"
#include "pk_route.h"

namespace pk {

typedef int32_t v4i __attribute__((ext_vector_type(4)));

PK_DEV v4i mfma16x16x32(uint2 a, uint2 b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a), __builtin_bit_cast(long, b), c, 0,
                                                 0, 0);
}
PK_DEV v4i mfma16x16x32(uint2 a, uint2 b) {
    const v4i z = {0, 0, 0, 0};
    return mfma16x16x32(a, b, z);
}

// LDS loads at aligned offsets
PK_DEV uint2 lds64(const uint8_t *p) { return *(const uint2 *)p; }
PK_DEV uint4 lds128(const uint8_t *p) { return *(const uint4 *)p; }
PK_DEV float4 lds_f4(const float *p) { return *(const float4 *)p; }

// ----------------------------------------------------------------- Q6_K --
// Step s = (h, q) of a super-block covers values 128h + 32q + [0, 32):
// group g0 = 8h + 2q (values 0..15: lane groups kq 0, 1) and g0 + 1 (lane
// groups 2, 3). Lane group kq holds values 8kq .. 8kq+7 of the step, for A
// (the tokens' q8 bytes 128h + 32q + 8kq) and B (the rows' codes: nibble
// q / 2 of ql[64h + 32 (q & 1) + 8kq], bits 2q..2q+1 of qh[32h + 8kq]).
// MFMA(A, B) sums both groups, MFMA(A, B with lane groups 2, 3 zeroed) the
// first, so sc0 D0 + sc1 D1 = (sc0 - sc1) D_lo + sc1 D_all, exact in int32.
struct MmaQ6K {
    static constexpr uint32_t kSbBytes = 210;
    static constexpr uint32_t kDOff = 208;  // f16 d within the block
    struct W {
        uint2 la[2], lb[2], qh[2];
        uint4 sc;
        uint32_t d;
    };
    // from an LDS copy of the super-block (8-byte aligned)
    PK_DEV static W load_lds(const uint8_t *blk, uint32_t kq, uint32_t d_off) {
        W w;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            w.la[h] = lds64(blk + 64 * h + 8 * kq);
            w.lb[h] = lds64(blk + 64 * h + 32 + 8 * kq);
            w.qh[h] = lds64(blk + 128 + 32 * h + 8 * kq);
        }
        w.sc = lds128(blk + 192);
        w.d = *(const uint16_t *)(blk + d_off);
        return w;
    }
    // signed code c - 32 of four values: the low nibble, plus the 2 high
    // bits h mapped through the byte table {0xE0, 0xF0, 0x00, 0x10} =
    // (h - 2) << 4 (v_perm_b32 picks table byte h for every byte)
    PK_DEV static uint32_t code(uint32_t l, uint32_t qh, uint32_t nsh, uint32_t hsh) {
        const uint32_t hf = (qh >> hsh) & 0x03030303u;
        const uint32_t hi = __builtin_amdgcn_perm(0u, 0x1000F0E0u, hf);
        return ((l >> nsh) & 0x0f0f0f0fu) | hi;
    }
    // B operand of step (h, q)
    PK_DEV static uint2 codes(const W &w, int h, int q) {
        const uint2 l = (q & 1) ? w.lb[h] : w.la[h];
        const uint32_t nsh = (q >> 1) ? 4u : 0u, hsh = 2u * q;
        return make_uint2(code(l.x, w.qh[h].x, nsh, hsh), code(l.y, w.qh[h].y, nsh, hsh));
    }
};

// --------------------------------------------- dense GEMM (chunks, prefill) --
// Q4_K for the MFMA kernels: K slice t (32 values) is sub-block t; lane
// group kq holds qs bytes 32 (t / 2) + 8 kq + [0, 8), nibble t % 2. Codes
// 0..15 are int8 as they are; the 6-bit scale multiplies each slice's D
// (24-bit products), and the min term sum_t m_t (bsums[2t] + bsums[2t+1])
// comes from two MFMAs on those sums split as 128 h + l (l in [0, 128),
// |h| <= 32). Super-block value xd yd isum - xmin yd msum (cpu_dot.rs:250-279).
struct MmaQ4K {
    static constexpr uint32_t kSbBytes = 144;
    struct W {
        uint2 q[4];  // qs bytes 32c + 8kq + [0, 8)
        uint4 hdr;   // d, dmin, scales[12]
    };
    PK_DEV static W load_lds(const uint8_t *blk, uint32_t kq) {
        W w;
#pragma unroll
        for (int c = 0; c < 4; c++) w.q[c] = lds64(blk + 16u + 32u * c + 8u * kq);
        w.hdr = lds128(blk);
        return w;
    }
    PK_DEV static uint2 codes(const W &w, int t) {
        const uint2 q = w.q[t >> 1];
        const uint32_t sh = 4u * (t & 1);
        return make_uint2((q.x >> sh) & 0x0f0f0f0fu, (q.y >> sh) & 0x0f0f0f0fu);
    }
};

// Q5_K (176 B: d, dmin, scales[12], qh[32] @16, qs[128] @48): Q4_K's codes
// of lane group kq plus the fifth bit of value 32t + 8kq + i, bit t of qh
// byte 8kq + i (pulsar_kernels.cu:5892-5918).
struct MmaQ5K {
    static constexpr uint32_t kSbBytes = 176;
    struct W {
        uint2 q[4];  // qs bytes 32c + 8kq + [0, 8)
        uint4 hdr;   // d, dmin, scales[12]
        uint2 qh;    // qh bytes 8kq + [0, 8)
    };
    PK_DEV static W load_lds(const uint8_t *blk, uint32_t kq) {
        W w;
#pragma unroll
        for (int c = 0; c < 4; c++) w.q[c] = lds64(blk + 48u + 32u * c + 8u * kq);
        w.hdr = lds128(blk);
        w.qh = lds64(blk + 16u + 8u * kq);
        return w;
    }
    PK_DEV static uint2 codes(const W &w, int t) {
        const uint2 q = w.q[t >> 1];
        const uint32_t sh = 4u * (t & 1);
        return make_uint2(((q.x >> sh) & 0x0f0f0f0fu) | (((w.qh.x >> t) & 0x01010101u) << 4),
                          ((q.y >> sh) & 0x0f0f0f0fu) | (((w.qh.y >> t) & 0x01010101u) << 4));
    }
};
// the scale/min K-quant decoders by format
template <uint32_t Q>
using MmaKq = typename std::conditional<Q == PULSAR_QUANT_Q5_K, MmaQ5K, MmaQ4K>::type;

// Per-format pieces of the dense GEMM: super-block bytes, 16-byte copies
// per row super-block (the last one may overlap the previous: it ends at
// the super-block's end), the LDS slot offset of f16 d, bsums needed.
template <uint32_t Q>
struct GemmFmt;
template <>
struct GemmFmt<PULSAR_QUANT_Q6_K> {
    static constexpr uint32_t kSb = 210, kChunks = 14, kDSlot = 16u * 13u + 208u - 194u;
    static constexpr bool kBsums = false;
};
template <>
struct GemmFmt<PULSAR_QUANT_Q4_K> {
    static constexpr uint32_t kSb = 144, kChunks = 9, kDSlot = 0;
    static constexpr bool kBsums = true;
};
template <>
struct GemmFmt<PULSAR_QUANT_Q5_K> {
    static constexpr uint32_t kSb = 176, kChunks = 11, kDSlot = 0;
    static constexpr bool kBsums = true;
};
// NVFP4: 4 blocks of 36 B (4 UE4M3 scale bytes, 4 x 8 code bytes)
template <>
struct GemmFmt<PULSAR_QUANT_NVFP4> {
    static constexpr uint32_t kSb = 144, kChunks = 9, kDSlot = 0;
    static constexpr bool kBsums = false;
};

// bsums b[2t] + b[2t + 1] for t = 4 (kq & 1) + [0, 4) of a token, split as
// 128 h + l: l bytes (kq < 2) or h bytes (kq >= 2)
PK_DEV uint32_t pair_sum_bytes(uint4 b, bool high) {
    const uint32_t w[4] = {b.x, b.y, b.z, b.w};
    uint32_t out = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int32_t s = (int32_t)(int16_t)(w[j] & 0xffffu) + (int32_t)(int16_t)(w[j] >> 16);
        const uint32_t v = high ? (uint32_t)(s >> 7) & 0xffu : (uint32_t)s & 0x7fu;
        out |= v << (8 * j);
    }
    return out;
}

// Block = 16 RT rows x 16 NT tokens, K in chunks of C super-blocks, NW =
// RT C waves. Per chunk the rows' super-blocks (row-contiguous 16-byte
// copies) and the tokens' q8 values (+ bsums for Q4_K, + d) are staged in
// LDS; wave (rt, sb) decodes row tile rt, super-block sb of the chunk once
// and multiplies it with all NT token tiles. The loads of D chunks are in
// flight at once, in D register buffers: chunks are taken in groups of D,
// and as buffer d is moved to LDS, the next group's chunk d is requested
// into it. Every thread issues every load (clamped, stored or not) in the
// same order in the first group and the loop, so each wait counts exactly
// the D - 1 chunks behind the one needed; only the last group's requests
// past the end of K (clamped to its last super-block) are wasted.
// The C partials of a row tile are added in wave order (deterministic).
template <uint32_t Q, uint32_t RT, uint32_t C, uint32_t NT, uint32_t D>
__global__ __launch_bounds__(64 * RT * C) void mmq_gemm_kernel(float *__restrict__ out, const uint8_t *__restrict__ w,
                                                               const pulsar_block_q8_K *__restrict__ xq, uint32_t nb,
                                                               uint32_t out_dim, uint32_t n_tok, uint64_t row_bytes) {
    using F = GemmFmt<Q>;
    constexpr uint32_t NW = RT * C, NTH = 64u * NW, TOK = 16u * NT, ROWS = 16u * RT;
    constexpr uint32_t kSlot = 16u * F::kChunks;
    constexpr uint32_t kRowPitch = C * kSlot + 16u;  // LDS bytes per row
    constexpr uint32_t kActPitch = 272u;             // LDS bytes per (super-block, token) q8 values
    constexpr uint32_t kAPer = F::kBsums ? 18u : 16u;  // 16-byte pieces per (token, super-block)
    constexpr uint32_t kWP = ROWS * C * F::kChunks, kWL = (kWP + NTH - 1u) / NTH;
    constexpr uint32_t kAP = TOK * C * kAPer, kAL = (kAP + NTH - 1u) / NTH;
    constexpr uint32_t kYL = (TOK * C + NTH - 1u) / NTH;
    constexpr uint32_t kWlBytes = ROWS * kRowPitch, kAlBytes = C * TOK * kActPitch;
    constexpr uint32_t kBlBytes = F::kBsums ? C * TOK * 32u : 0u;
    static_assert(NW * 16u * (TOK + 1u) * 4u <= kAlBytes, "partials alias the activation area");
    __shared__ __align__(16) uint8_t lds[kWlBytes + kAlBytes + kBlBytes + C * TOK * 4u];
    uint8_t *wl = lds, *al = lds + kWlBytes, *bl = al + kAlBytes;
    float *yl = (float *)(bl + kBlBytes);
    // the wave index through readfirstlane: known wave-uniform, so branches
    // on it stay scalar (a masked branch would let one side's loads be in
    // flight into registers the other side reuses, and force a full wait)
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t i = lane & 15u, kq = lane >> 4;
    const uint32_t t0 = blockIdx.x * TOK, r0 = blockIdx.y * ROWS;
    const uint8_t *xb = (const uint8_t *)xq;
    const uint64_t tok_bytes = (uint64_t)nb * 292u;
    const uint8_t *wsrc[kWL];
    uint32_t wsb[kWL], wdst[kWL];
#pragma unroll
    for (uint32_t m = 0; m < kWL; m++) {
        const uint32_t f = tid + NTH * m, ff = f < kWP ? f : kWP - 1u;
        const uint32_t c = ff % F::kChunks, rs = ff / F::kChunks, row = rs / C, sb = rs % C;
        const uint32_t gr = r0 + row < out_dim ? r0 + row : out_dim - 1u;
        wsrc[m] = w + (uint64_t)gr * row_bytes + (16u * c < F::kSb - 16u ? 16u * c : F::kSb - 16u);
        wsb[m] = sb;
        wdst[m] = f < kWP ? row * kRowPitch + sb * kSlot + 16u * c : UINT32_MAX;
    }
    const uint8_t *asrc[kAL];
    uint32_t asb[kAL], adst[kAL];
#pragma unroll
    for (uint32_t m = 0; m < kAL; m++) {
        const uint32_t f = tid + NTH * m, ff = f < kAP ? f : kAP - 1u;
        const uint32_t c = ff % kAPer, ts = ff / kAPer, t = ts / C, sb = ts % C;
        const uint32_t gt = t0 + t < n_tok ? t0 + t : n_tok - 1u;
        asrc[m] = xb + gt * tok_bytes + (c < 16u ? 4u + 16u * c : 260u + 16u * (c - 16u));
        asb[m] = sb;
        adst[m] = f >= kAP ? UINT32_MAX
                  : c < 16u ? kWlBytes + (sb * TOK + t) * kActPitch + 16u * c
                            : kWlBytes + kAlBytes + (sb * TOK + t) * 32u + 16u * (c - 16u);
    }
    const uint8_t *ysrc[kYL];
    uint32_t ysb[kYL], ydst[kYL];
#pragma unroll
    for (uint32_t m = 0; m < kYL; m++) {
        const uint32_t f = tid + NTH * m, ff = f < TOK * C ? f : TOK * C - 1u;
        const uint32_t t = ff / C, sb = ff % C;
        ysrc[m] = xb + (t0 + t < n_tok ? t0 + t : n_tok - 1u) * tok_bytes;
        ysb[m] = sb;
        ydst[m] = f < TOK * C ? sb * TOK + t : UINT32_MAX;
    }
    uint4 wreg[D][kWL], areg[D][kAL];
    uint32_t yreg[D][kYL];
    // load p of the chunk at kb into buffer d (p, d constants once the
    // callers' loops are unrolled): the weight pieces, then the q8 values,
    // then the d values
    constexpr uint32_t kNL = kWL + kAL + kYL;
    auto gload_one = [&](uint32_t kb, uint32_t d, uint32_t p) {
        if (p < kWL) {
            const uint32_t m = p;
            wreg[d][m] = ldw128(wsrc[m] + (uint64_t)(kb + wsb[m] < nb ? kb + wsb[m] : nb - 1u) * F::kSb);
        } else if (p < kWL + kAL) {
            const uint32_t m = p - kWL;
            areg[d][m] = ld128(asrc[m] + (uint64_t)(kb + asb[m] < nb ? kb + asb[m] : nb - 1u) * 292u);
        } else {
            const uint32_t m = p - kWL - kAL;
            yreg[d][m] = ld32(ysrc[m] + (uint64_t)(kb + ysb[m] < nb ? kb + ysb[m] : nb - 1u) * 292u);
        }
    };
    auto gload = [&](uint32_t kb, uint32_t d) {
#pragma unroll
        for (uint32_t p = 0; p < kNL; p++) gload_one(kb, d, p);
    };
    auto lstore = [&](uint32_t d) {
#pragma unroll
        for (uint32_t m = 0; m < kWL; m++)
            if ((m + 1u) * NTH <= kWP || wdst[m] != UINT32_MAX) *(uint4 *)(wl + wdst[m]) = wreg[d][m];
#pragma unroll
        for (uint32_t m = 0; m < kAL; m++)
            if ((m + 1u) * NTH <= kAP || adst[m] != UINT32_MAX) *(uint4 *)(lds + adst[m]) = areg[d][m];
#pragma unroll
        for (uint32_t m = 0; m < kYL; m++)
            if ((m + 1u) * NTH <= TOK * C || ydst[m] != UINT32_MAX)
                yl[ydst[m]] = __builtin_bit_cast(float, yreg[d][m]);
    };

    const uint32_t rt = wave / C, sbw = wave % C;
    float acc[NT][4];
#pragma unroll
    for (uint32_t n = 0; n < NT; n++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[n][r] = 0.0f;
    // decodes the chunk at kb; hook(st) runs at the start of each of the 8
    // steps. With one token tile (loads in the hook) a wave past the end of K
    // decodes its clamped copy too and adds nothing: a branch around the
    // decode would put the other side's loads on the decode's path, where
    // their registers force a full wait
    auto chunk = [&](uint32_t kb, auto hook) {
        const bool live = kb + sbw < nb;
        if (NT == 1u || live) {
            const uint8_t *wrow = wl + (rt * 16u + i) * kRowPitch + sbw * kSlot;
            const uint8_t *abase = al + (sbw * TOK + i) * kActPitch + 8u * kq;
            if constexpr (Q == PULSAR_QUANT_Q6_K) {
                const MmaQ6K::W wv = MmaQ6K::load_lds(wrow, kq, F::kDSlot);
                int32_t isum[NT][4];
#pragma unroll
                for (uint32_t n = 0; n < NT; n++)
#pragma unroll
                    for (int r = 0; r < 4; r++) isum[n][r] = 0;
#pragma unroll
                for (int st = 0; st < 8; st++) {
                    hook((uint32_t)st);
                    const int h = st >> 2, q = st & 3;
                    const uint2 c = MmaQ6K::codes(wv, h, q);
                    const uint2 c_lo = kq < 2 ? c : make_uint2(0u, 0u);
                    const int32_t s0 = (int32_t)(int8_t)byte_of(wv.sc, 8 * h + 2 * q);
                    const int32_t s1 = (int32_t)(int8_t)byte_of(wv.sc, 8 * h + 2 * q + 1);
#pragma unroll
                    for (uint32_t n = 0; n < NT; n++) {
                        const uint2 a = lds64(abase + 16u * n * kActPitch + 32u * st);
                        const v4i d_all = mfma16x16x32(a, c);
                        const v4i d_lo = mfma16x16x32(a, c_lo);
                        // |d| < 2^17, |s| < 2^8: 24-bit multiplies are exact
#pragma unroll
                        for (int r = 0; r < 4; r++) isum[n][r] += __mul24(s0 - s1, d_lo[r]) + __mul24(s1, d_all[r]);
                    }
                }
                const float xd = f16f((uint16_t)wv.d);
#pragma unroll
                for (uint32_t n = 0; n < NT; n++) {
                    const float4 yd4 = lds_f4(yl + sbw * TOK + 16u * n + 4u * kq);
                    const float yd[4] = {yd4.x, yd4.y, yd4.z, yd4.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[n][r] = live ? acc[n][r] + xd * yd[r] * (float)isum[n][r] : acc[n][r];
                }
            } else if constexpr (Q == PULSAR_QUANT_NVFP4) {
                // step t: block t / 2, 16-value sub-blocks s0 = 2 (t & 1) and
                // s0 + 1; lane group kq holds sub-block s0 + kq / 2, values
                // 8 (kq & 1) + [0, 8) (low / high nibbles of its 8 code bytes).
                // Two MFMAs split the step's sum by sub-block (all 32 values,
                // then the first sub-block alone); per sub-block the
                // reference's sumf += (ue4m3 / 2) * sumi in order
                // (pulsar_kernels.cu:5743-5771), then yd * sumf
                float f[NT][4];
#pragma unroll
                for (uint32_t n = 0; n < NT; n++)
#pragma unroll
                    for (int r = 0; r < 4; r++) f[n][r] = 0.0f;
                const uint32_t nsh = 4u * (kq & 1u);
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    hook((uint32_t)t);
                    const uint8_t *bp = wrow + 36u * (uint32_t)(t >> 1);
                    const uint8_t *sp = bp + 4u + 8u * (2u * (uint32_t)(t & 1) + (kq >> 1));
                    const uint2 c = make_uint2(mxfp4_kv4(*(const uint32_t *)sp >> nsh),
                                               mxfp4_kv4(*(const uint32_t *)(sp + 4) >> nsh));
                    const uint2 c_lo = kq < 2 ? c : make_uint2(0u, 0u);
                    const uint32_t e4 = *(const uint32_t *)bp;
                    const float d0 = ue4m3f(byte_of(e4, 2u * (uint32_t)(t & 1))) * 0.5f;
                    const float d1 = ue4m3f(byte_of(e4, 2u * (uint32_t)(t & 1) + 1u)) * 0.5f;
#pragma unroll
                    for (uint32_t n = 0; n < NT; n++) {
                        const uint2 a = lds64(abase + 16u * n * kActPitch + 32u * t);
                        const v4i d_all = mfma16x16x32(a, c);
                        const v4i d_lo = mfma16x16x32(a, c_lo);
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            f[n][r] += d0 * (float)d_lo[r];
                            f[n][r] += d1 * (float)(d_all[r] - d_lo[r]);
                        }
                    }
                }
#pragma unroll
                for (uint32_t n = 0; n < NT; n++) {
                    const float4 yd4 = lds_f4(yl + sbw * TOK + 16u * n + 4u * kq);
                    const float yd[4] = {yd4.x, yd4.y, yd4.z, yd4.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[n][r] = live ? acc[n][r] + yd[r] * f[n][r] : acc[n][r];
                }
            } else {  // Q4_K, Q5_K
                using M = MmaKq<Q>;
                const typename M::W wv = M::load_lds(wrow, kq);
                int32_t isum[NT][4];
#pragma unroll
                for (uint32_t n = 0; n < NT; n++)
#pragma unroll
                    for (int r = 0; r < 4; r++) isum[n][r] = 0;
                uint32_t mins[2] = {0u, 0u};
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    hook((uint32_t)t);
                    int32_t sc, mn;
                    Fmt<PULSAR_QUANT_Q4_K>::scale_min(wv.hdr, (uint32_t)t, sc, mn);
                    mins[t >> 2] |= (uint32_t)mn << (8 * (t & 3));
                    const uint2 b = M::codes(wv, t);
#pragma unroll
                    for (uint32_t n = 0; n < NT; n++) {
                        const v4i d = mfma16x16x32(lds64(abase + 16u * n * kActPitch + 32u * t), b);
                        // |d| < 2^17, sc < 64
#pragma unroll
                        for (int r = 0; r < 4; r++) isum[n][r] += __mul24(sc, d[r]);
                    }
                }
                // min term: K slots [l_0..3 | l_4..7 | h_0..3 | h_4..7] per lane group
                // against the mins in lane groups 0, 1 (D_l) and 2, 3 (D_h)
                const uint32_t mw = mins[kq & 1u];
                const uint2 bl_ = kq < 2u ? make_uint2(mw, 0u) : make_uint2(0u, 0u);
                const uint2 bh_ = kq < 2u ? make_uint2(0u, 0u) : make_uint2(mw, 0u);
                const uint32_t xh = wv.hdr.x;
                const float xd = f16f((uint16_t)xh), xmin = f16f((uint16_t)(xh >> 16));
#pragma unroll
                for (uint32_t n = 0; n < NT; n++) {
                    const uint4 bs = lds128(bl + (sbw * TOK + 16u * n + i) * 32u + 16u * (kq & 1u));
                    const uint2 alh = make_uint2(pair_sum_bytes(bs, kq >= 2u), 0u);
                    const v4i dl = mfma16x16x32(alh, bl_);
                    const v4i dh = mfma16x16x32(alh, bh_);
                    const float4 yd4 = lds_f4(yl + sbw * TOK + 16u * n + 4u * kq);
                    const float yd[4] = {yd4.x, yd4.y, yd4.z, yd4.w};
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int32_t msum = dl[r] + 128 * dh[r];
                        const float v = xd * yd[r] * (float)isum[n][r] - xmin * yd[r] * (float)msum;
                        acc[n][r] = live ? acc[n][r] + v : acc[n][r];
                    }
                }
            }
        }
    };
    const uint32_t n_grp = (nb + C * D - 1u) / (C * D);  // groups of D chunks
#pragma unroll
    for (uint32_t d = 0; d < D; d++) gload(d * C, d);
    uint32_t g = 0;
    for (; g + 1u < n_grp; g++) {
#pragma unroll
        for (uint32_t d = 0; d < D; d++) {
            const uint32_t kb = (g * D + d) * C;
            lstore(d);
            __syncthreads();
            // the chunk D ahead, in flight while this one and the next D - 1
            // are decoded. One token tile: its loads spread over the decode's
            // steps (issued at once, they stall the wave until the memory
            // pipeline drains); two tiles decode long enough to hide them,
            // and interleaving would cost them occupancy
            if constexpr (NT == 1) {
                chunk(kb, [&](uint32_t st) {
#pragma unroll
                    for (uint32_t p = 0; p < kNL; p++)
                        if (p * 8u / kNL == st) gload_one(kb + D * C, d, p);
                });
            } else {
                gload(kb + D * C, d);
                chunk(kb, [](uint32_t) {});
            }
            __syncthreads();
        }
    }
#pragma unroll
    for (uint32_t d = 0; d < D; d++) {  // the last group: nothing left to request
        const uint32_t kb = (g * D + d) * C;
        if (kb < nb) {
            lstore(d);
            __syncthreads();
            chunk(kb, [](uint32_t) {});
            __syncthreads();
        }
    }
    // partials [wave][row][token] over the activation area (all reads of it are done)
    float *part = (float *)al;
#pragma unroll
    for (uint32_t n = 0; n < NT; n++)
#pragma unroll
        for (int r = 0; r < 4; r++) part[(wave * 16u + i) * (TOK + 1u) + 16u * n + 4u * kq + r] = acc[n][r];
    __syncthreads();
    for (uint32_t e = tid; e < TOK * ROWS; e += NTH) {
        const uint32_t row = e % ROWS, tok = e / ROWS;
        if (r0 + row < out_dim && t0 + tok < n_tok) {
            const uint32_t prt = row / 16u;
            float v = part[((prt * C) * 16u + row % 16u) * (TOK + 1u) + tok];
#pragma unroll
            for (uint32_t k = 1; k < C; k++) v += part[((prt * C + k) * 16u + row % 16u) * (TOK + 1u) + tok];
            out[(uint64_t)(t0 + tok) * out_dim + r0 + row] = v;
        }
    }
}

// token-tile width by chunk size: 32-token tiles (measured on Q4_K / Q6_K
// 4096-wide rows at 64 and 256 tokens) beat 16-token tiles, which decode
// every weight twice as often, and 64-token tiles, which leave too few blocks
#ifndef PK_GEMM_NT2
#define PK_GEMM_NT2 32u
#endif
// chunks in flight (cold weights, 16 tokens): 32-row tiles over Q6_K 8192 x
// 4096 13.0 / 12.5 / 13.7 us at 1 / 2 / 4 (all requested at once, the last
// chunk's data comes with the first: the decodes then run back to back);
// 16-row tiles over Q4_K 4096 x 4096 7.7 / 7.8 / 9.3 us
#ifndef PK_GEMM_D_NT2
#define PK_GEMM_D_NT2 1u
#endif
#ifndef PK_GEMM_D_R16
#define PK_GEMM_D_R16 1u
#endif
#ifndef PK_GEMM_D_R32
#define PK_GEMM_D_R32 2u
#endif

template <uint32_t Q>
static int launch_gemm_q(float *out, const uint8_t *w, const pulsar_block_q8_K *xq, uint32_t nb, uint32_t out_dim,
                         uint32_t n_tok, uint64_t row_bytes) {
#define PK_GEMM(RT, C, NT, D)                                                                                \
    hipLaunchKernelGGL((mmq_gemm_kernel<Q, RT, C, NT, D>), dim3((n_tok + 16u * NT - 1u) / (16u * NT),         \
                                                                (out_dim + 16u * RT - 1u) / (16u * RT)),       \
                       dim3(64 * RT * C), 0, pk::stream(), out, w, xq, nb, out_dim, n_tok, row_bytes)
    // below 8192 rows a 32-row tile leaves CUs idle (4096 rows: 128 blocks);
    // 16-row tiles with 8 super-blocks per chunk measured fastest there
    // (Q4_K 4096 x 4096, 16 tokens: 8.7 -> 6.9 us), 32-row tiles with 4
    // above (Q6_K 8192 x 4096: 11.8 us; 16-row tiles 12.9-14.0 us). Q4_K
    // takes 32-row tiles with 8 super-blocks per chunk above: 16 waves per
    // block, 4 per SIMD within 128 VGPRs (cold weights, 16 tokens: 8192 x
    // 4096 11.1 -> 9.9 us, 14336 x 4096 19.2 -> 16.6 us; 5-31 tokens and
    // 14336-wide rows alike); Q6_K and NVFP4 spill at that cap (Q6_K 8192 x
    // 4096 12.8 -> 21.5 us)
    if (n_tok >= PK_GEMM_NT2)
        PK_GEMM(2, 2, 2, PK_GEMM_D_NT2);
    else if (out_dim < 8192u)
        PK_GEMM(1, 8, 1, PK_GEMM_D_R16);
    else if (Q == PULSAR_QUANT_Q4_K)
        PK_GEMM(2, 8, 1, 1);
    else
        PK_GEMM(2, 4, 1, PK_GEMM_D_R32);
#undef PK_GEMM
    return launch_ok("matmul_kq gemm launch");
}

// MFMA GEMM for token chunks / prefill (the reference's prefill GEMM formats,
// pulsar_kernels.cu:4914-4916: Q4_K, Q6_K, NVFP4, plus Q5_K, which the
// reference runs through its per-token matvec); -1 for other formats.
int launch_gemm(uint32_t quant, float *out, const uint8_t *w, const pulsar_block_q8_K *xq, uint32_t in_dim,
                uint32_t out_dim, uint32_t n_tok, uint64_t row_bytes) {
    const uint32_t nb = in_dim / 256u;
    if ((uint64_t)((out_dim + 31u) / 32u) > 65535u) return -1;  // grid y
    switch (quant) {
    case PULSAR_QUANT_Q6_K: return launch_gemm_q<PULSAR_QUANT_Q6_K>(out, w, xq, nb, out_dim, n_tok, row_bytes);
    case PULSAR_QUANT_Q4_K: return launch_gemm_q<PULSAR_QUANT_Q4_K>(out, w, xq, nb, out_dim, n_tok, row_bytes);
    case PULSAR_QUANT_NVFP4: return launch_gemm_q<PULSAR_QUANT_NVFP4>(out, w, xq, nb, out_dim, n_tok, row_bytes);
    case PULSAR_QUANT_Q5_K: return launch_gemm_q<PULSAR_QUANT_Q5_K>(out, w, xq, nb, out_dim, n_tok, row_bytes);
    default: return -1;
    }
}

// ------------------------------------ grouped Q2_K / IQ2_XXS / MXFP4 (MoE) --
// Block = 16 rows per wave (kGqWaves waves: 64 rows, MXFP4 192) x up to
// kGqPairs pairs of one expert group, the whole K per wave (no split). The pairs' q8_K rows are staged in LDS
// once per pair tile (load_act_lds layout); each wave streams its 16 rows
// super-block by super-block: a contiguous copy (consecutive lanes on
// consecutive bytes of a row) to registers, the next super-block's copy in
// flight while the current one, moved to the wave's LDS slot, is decoded.
// Lane group kq holds values 32t + 8kq + [0, 8) of K slice t (32 values);
// A = the pairs' q8 values (lanes of pairs past the tile read zeros),
// B = the rows' signed int8 weights; D lane (row i, kq) holds pairs 4kq + r.
//
// Q2_K (84 B: scales[16] @0, qs[64] @16, f16 d, dmin @80): value
// 32t + 8kq + i sits in qs byte 32(t / 4) + 16(kq / 2) + 8(kq % 2) + i at
// bits 2(t % 4), sub-block 2t + kq / 2. Codes are pre-scaled by their
// sub-block scale (3 x 15 fits int8; one v_pk_mul_lo_u16 scales four code
// bytes, two per 16-bit half, c sc <= 45 so no carry crosses a byte), so
// the 8 chained MFMAs of a super-block give
// isum = sum_c (sc_c & 15) sum q q8 exactly; summs = sum_c bsums_c
// (sc_c >> 4) comes from two MFMAs on bsums split as 128 h + l, l in
// [0, 128). Super-block value yd xd isum - yd xmin summs (cpu_dot.rs:732-767).
// IQ2_XXS (66 B: f16 d @0, 8 x {aux0, aux1} @2): lane group kq holds grid
// entry kq of each 32-group (8 values, signed through the LDS sign table);
// one MFMA per group gives sumi, bsum += sumi (2 (aux1 >> 28) + 1), super-
// block value 0.125 xd yd bsum (cpu_dot.rs:92-122).
// Per (row, pair) the super-block values are added in order; the row's
// value is then complete (no cross-wave sum). Formats with a min term (Q2_K,
// Q4_K, Q5_K) form each super-block value in the CPU lane's operation order,
// since its two products can cancel; the single-product formats (Q6_K,
// IQ2_XXS, MXFP4) fold the value into the sum with one fused multiply-add,
// within an ulp of the lane's value.
template <uint32_t Q>
struct GmmqFmt;
// Row super-block copies: kPieces 16-byte pieces (piece_off) to slot 16c,
// kTails small loads (tail_off, kTailBytes each) to kTailSlot + c. `lim`
// bounds the clamped unit (super-blocks, or 32-blocks for MXFP4; kLimPerSb
// of them per super-block); consecutive super-blocks are kSbBytes apart.
// Q2_K and Q6_K copy their f16 scales as one more 16-byte piece that starts
// at them (slot kTailSlot): a separate 2- or 4-byte load per (row, super-
// block) touches a new cache line in every lane. The piece of a row's last
// super-block is held inside the row, which puts the scales kTailLast bytes
// further into it. Measured: c4 Q2_K gate / up weight stream alone 86 ->
// 74 us (with the decode the stage 99.6 -> 98.1 us, the layer 164.9 ->
// 161.5 us), Q6_K down stages of 16- and 64-token Q4_K / Q6_K layers 3-6%
// faster. IQ2_XXS keeps its
// separate d load: a d piece (2-byte aligned, overlapping the first code
// piece) made its gate / up stage slower (110 -> 123 us).
template <>
struct GmmqFmt<PULSAR_QUANT_Q2_K> {
    static constexpr uint32_t kPieces = 6, kTails = 0, kTailBytes = 4;
    static constexpr uint32_t kSbBytes = 84, kLimPerSb = 1;
    static constexpr uint32_t kTailSlot = 80, kTailLast = 12;  // d, dmin
    static constexpr uint32_t kSlot = 96;                      // LDS bytes per row super-block
    PK_DEV static uint32_t piece_off(uint32_t sb, uint32_t c, uint32_t lim) {
        // scales, qs: bytes 0..79; piece 5 from d, dmin
        const uint32_t o = (sb < lim ? sb : lim - 1u) * 84u + 16u * c;
        return o < 84u * lim - 16u ? o : 84u * lim - 16u;
    }
    PK_DEV static uint32_t tail_off(uint32_t, uint32_t, uint32_t) { return 0u; }
};
template <>
struct GmmqFmt<PULSAR_QUANT_IQ2_XXS> {
    static constexpr uint32_t kPieces = 4, kTails = 1, kTailBytes = 4;
    static constexpr uint32_t kSbBytes = 66, kLimPerSb = 1;
    static constexpr uint32_t kTailSlot = 64, kTailLast = 0;  // d (the upper 2 bytes unused)
    static constexpr uint32_t kSlot = 80;
    PK_DEV static uint32_t piece_off(uint32_t sb, uint32_t c, uint32_t lim) {
        return (sb < lim ? sb : lim - 1u) * 66u + 2u + 16u * c;  // the 8 groups: bytes 2..65
    }
    PK_DEV static uint32_t tail_off(uint32_t sb, uint32_t, uint32_t lim) { return (sb < lim ? sb : lim - 1u) * 66u; }
};
template <>
struct GmmqFmt<PULSAR_QUANT_MXFP4> {
    // super-block = 8 blocks of 17 bytes; block c's qs to slot 16c, its e
    // to slot 128 + c
    static constexpr uint32_t kPieces = 8, kTails = 8, kTailBytes = 1;
    static constexpr uint32_t kSbBytes = 136, kLimPerSb = 8;  // lim counts 32-blocks
    static constexpr uint32_t kTailSlot = 128, kTailLast = 0;
    static constexpr uint32_t kSlot = 144;
    PK_DEV static uint32_t piece_off(uint32_t sb, uint32_t c, uint32_t lim) {
        const uint32_t b = 8u * sb + c;
        return 17u * (b < lim ? b : lim - 1u) + 1u;
    }
    PK_DEV static uint32_t tail_off(uint32_t sb, uint32_t c, uint32_t lim) {
        const uint32_t b = 8u * sb + c;
        return 17u * (b < lim ? b : lim - 1u);
    }
};
template <>
struct GmmqFmt<PULSAR_QUANT_Q4_K> {
    static constexpr uint32_t kPieces = 9, kTails = 0, kTailBytes = 4;  // the whole 144 bytes
    static constexpr uint32_t kSbBytes = 144, kLimPerSb = 1;
    static constexpr uint32_t kTailSlot = 0, kTailLast = 0;
    static constexpr uint32_t kSlot = 144;
    PK_DEV static uint32_t piece_off(uint32_t sb, uint32_t c, uint32_t lim) {
        return (sb < lim ? sb : lim - 1u) * 144u + 16u * c;
    }
    PK_DEV static uint32_t tail_off(uint32_t, uint32_t, uint32_t) { return 0u; }
};
template <>
struct GmmqFmt<PULSAR_QUANT_Q5_K> {
    static constexpr uint32_t kPieces = 11, kTails = 0, kTailBytes = 4;  // the whole 176 bytes
    static constexpr uint32_t kSbBytes = 176, kLimPerSb = 1;
    static constexpr uint32_t kTailSlot = 0, kTailLast = 0;
    static constexpr uint32_t kSlot = 176;
    PK_DEV static uint32_t piece_off(uint32_t sb, uint32_t c, uint32_t lim) {
        return (sb < lim ? sb : lim - 1u) * 176u + 16u * c;
    }
    PK_DEV static uint32_t tail_off(uint32_t, uint32_t, uint32_t) { return 0u; }
};
template <>
struct GmmqFmt<PULSAR_QUANT_Q6_K> {
    static constexpr uint32_t kPieces = 14, kTails = 0, kTailBytes = 2;  // bytes 0..207, piece 13 from d
    static constexpr uint32_t kSbBytes = 210, kLimPerSb = 1;
    static constexpr uint32_t kTailSlot = 208, kTailLast = 14;
    static constexpr uint32_t kSlot = 224;
    PK_DEV static uint32_t piece_off(uint32_t sb, uint32_t c, uint32_t lim) {
        const uint32_t o = (sb < lim ? sb : lim - 1u) * 210u + 16u * c;
        return o < 210u * lim - 16u ? o : 210u * lim - 16u;
    }
    PK_DEV static uint32_t tail_off(uint32_t, uint32_t, uint32_t) { return 0u; }
};
#ifndef PK_GQ_SBS
#define PK_GQ_SBS 2u
#endif
#ifndef PK_GQ_ACT_LDS
#define PK_GQ_ACT_LDS 16384u
#endif
constexpr uint32_t kGqSbs = PK_GQ_SBS;         // super-blocks per row per copy step
constexpr uint32_t kGqPairs = 16;              // pairs per tile (the MFMA's 16 columns)
constexpr uint32_t kGqActLds = PK_GQ_ACT_LDS;  // LDS bytes for a tile's staged q8_K rows
#ifndef PK_GQ_ACT_LDS_PAIR
#define PK_GQ_ACT_LDS_PAIR 24576u
#endif
constexpr uint32_t kGqActLdsPair = PK_GQ_ACT_LDS_PAIR;  // the same for gate / up stages (see the launch)
#ifndef PK_GQ_ACT_LDS_MX
#define PK_GQ_ACT_LDS_MX 61440u
#endif
constexpr uint32_t kGqActLdsMx = PK_GQ_ACT_LDS_MX;  // the same for MXFP4 experts

// Per 16-bit half: a * b (low 16 bits), one v_pk_mul_lo_u16
typedef unsigned short pk_ushort2 __attribute__((ext_vector_type(2)));
PK_DEV uint32_t pk_mul16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(pk_ushort2, a) * __builtin_bit_cast(pk_ushort2, b));
}


// Tiles of at most 4 pairs: the MFMA result of pairs 0..3 sits in the kq = 0
// lanes (lane i, element r = pair r); this moves element p of lane i to lane
// i + 16 p, so every lane holds one (row, pair) value and the fp32 epilogue
// runs once per lane instead of once per element (two permlane16 swaps,
// one permlane32 swap).
PK_DEV uint32_t gather_pairs(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3) {
    const auto a = __builtin_amdgcn_permlane16_swap(d0, d1, false, false);  // rows: d0.0 d1.0 ..
    const auto c = __builtin_amdgcn_permlane16_swap(d2, d3, false, false);  // rows: d2.0 d3.0 ..
    return __builtin_amdgcn_permlane32_swap(a[0], c[0], false, false)[0];    // d0.0 d1.0 d2.0 d3.0
}
PK_DEV int32_t gather_pairs(const v4i &d) {
    return (int32_t)gather_pairs((uint32_t)d[0], (uint32_t)d[1], (uint32_t)d[2], (uint32_t)d[3]);
}
PK_DEV float gather_pairs(const float (&f)[4]) {
    return __uint_as_float(gather_pairs(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
                                        __float_as_uint(f[3])));
}

// Waves per block, 16 rows each. MXFP4 blocks take 12: their pair tiles are
// large (16 pairs of 2880-value rows, ~58 KiB, one block per CU), and
// sharing one tile over more rows keeps more waves per CU resident (c5
// 64-token layer: 4 waves 215 us, 8 waves 196 us, 12 waves 185 us, 2880 rows
// in 15 whole blocks; 16 waves, 128 VGPRs and 12 blocks per group, 221 us);
// the K-quant layers measured slower with 8 (c4 Q2_K 183 -> 192 us).
template <uint32_t Q>
constexpr uint32_t kGqWaves = Q == PULSAR_QUANT_MXFP4 ? 12u : 4u;

// 16-row tiles per wave: a wave walks T consecutive row tiles of its expert
// with the weight pipeline running across the tile boundaries, so the
// block's group record, pair list and activation staging serve T times the
// rows. Measured (stage timings, alternating libraries): MXFP4 2 in both
// stages (c5 64 tokens: gate / up 112.3 -> 97.5 us, its 2880 rows in 8
// blocks of 384 so the 32 experts' blocks make one round of 256 blocks,
// one per CU; down 56.9 -> 51.9 us; 3 and 4 leave CUs idle in the down
// stage, 64 / 81 us); IQ2_XXS down 2 (c4 60.5 -> 57.0 us); Q2_K down 2
// with its first step requested before the staging (c4 44.8 -> 43.7 us;
// either change alone measured within noise or slower); 1 for the
// others: two tiles in the K-quant gate / up stages cost them occupancy or
// block count (c4 Q2_K 85.3 -> 92.0 us, IQ2_XXS 104.5 -> 150.2 us).
template <uint32_t Q, bool PAIR>
constexpr uint32_t kGqTiles = Q == PULSAR_QUANT_MXFP4 ? 2u : ((Q == PULSAR_QUANT_IQ2_XXS || Q == PULSAR_QUANT_Q2_K) && !PAIR) ? 2u : 1u;
template <uint32_t Q, bool PAIR>
constexpr uint32_t kGqBlockRows = 16u * kGqWaves<Q> * kGqTiles<Q, PAIR>;

// amdgpu_waves_per_eu(2): register allocation for at least two waves per
// SIMD. Left to itself the compiler spends more (Q2_K pair 164 VGPRs, Q4_K
// 240, Q5_K 286); with the bound, 152 / 161 / 231, no spills, and the c4
// layers run 2-4% faster (Q2_K 182 -> 178 us, IQ2_XXS 205 -> 198 us).
// G: where the block's group comes from (CsrGroups: the caller's CSR;
// ExpertGroups: one group per bank expert, its pair list collected into the
// dynamic LDS at byte lst_off, after the pair tile).
template <uint32_t Q, bool PAIR, typename G>
__global__ __launch_bounds__(64 * kGqWaves<Q>) __attribute__((amdgpu_waves_per_eu(2))) void moe_grouped_mmq_kq_kernel(
        float *__restrict__ out, const G src, const float *__restrict__ weights,
        const pulsar_block_q8_K *__restrict__ act, uint32_t k_blocks, uint32_t lim, uint32_t n_rows,
        uint32_t n_used, uint64_t row_bytes, uint32_t act_op, uint32_t pmax, uint32_t lst_off) {
    using F = GmmqFmt<Q>;
    constexpr uint32_t NM = PAIR ? 2 : 1;
    constexpr bool kIq2 = Q == PULSAR_QUANT_IQ2_XXS;
    constexpr bool kMx = Q == PULSAR_QUANT_MXFP4;
    // MXFP4, Q4_K and Q6_K super-block rows are 136-210 contiguous bytes already
    constexpr uint32_t S = (kMx || Q == PULSAR_QUANT_Q4_K || Q == PULSAR_QUANT_Q5_K || Q == PULSAR_QUANT_Q6_K) ? 1u : kGqSbs;
    // LDS bytes per row: S slots, padded by 16 bytes (the K-quants; without
    // the pad the c4 Q2_K gate / up stage went 81.9 -> 87.4 us, with 32
    // bytes 83.1 us) or not at all (MXFP4: c5 64-token gate / up 96.2 ->
    // 95.4 us, 32 bytes 95.1 us, 48 bytes 103 us)
    constexpr uint32_t kRowL = S * F::kSlot + (kMx ? 0u : 16u);
    constexpr uint32_t kWp = NM * 16u * S * F::kPieces;  // weight pieces per step
    constexpr uint32_t kWj = (kWp + 63u) / 64u;         // ... per lane
    constexpr uint32_t kTp = NM * 16u * S * F::kTails;  // tails per step
    constexpr uint32_t kTj = (kTp + 63u) / 64u;
    constexpr uint32_t kTjA = kTj > 0u ? kTj : 1u;  // array extent
    extern __shared__ __align__(16) uint8_t acts_lds[];
    __shared__ uint2 lut[kIq2 ? kIq2LutRows : 1];
    __shared__ __align__(16) uint8_t wl[kGqWaves<Q>][NM * 16u * kRowL];  // [wave][matrix][row][step slot]
    __shared__ uint32_t pr_l[kGqPairs];
    if (kIq2) {
        fill_iq2xxs_lut(lut);
        __syncthreads();
    }
    const uint32_t group = blockIdx.y;
    const typename G::Group grp = src.group(group);
    const pulsar_expert_ptrs &p = grp.p;
    const uint8_t *w0 = PAIR ? (const uint8_t *)p.gate : (const uint8_t *)p.down;
    const uint8_t *w1 = PAIR ? (const uint8_t *)p.up : nullptr;
    const bool nul = grp.is_null();  // block-uniform
    if (!nul && (!w0 || (PAIR && !w1))) return;
    uint32_t *lst = (uint32_t *)(acts_lds + lst_off);
    uint32_t s0, s1;
    src.range(grp, lst, s0, s1);
    if (s0 >= s1) return;
    if (nul) {  // unrouted slots: their rows of this block are 0
        const uint32_t nr = kGqBlockRows<Q, PAIR>, r0 = blockIdx.x * nr;
        for (uint32_t it = threadIdx.x; it < (s1 - s0) * nr; it += blockDim.x) {
            const uint32_t pr = src.pair(s0 + it / nr, lst), row = r0 + it % nr;
            if (row < n_rows) out[((uint64_t)(pr >> 4) * n_used + (pr & 15u)) * n_rows + row] = 0.0f;
        }
        return;
    }
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t i = lane & 15u, kq = lane >> 4;
    constexpr uint32_t T = kGqTiles<Q, PAIR>;
    const uint32_t rw0 = (blockIdx.x * kGqWaves<Q> + wave) * 16u * T;  // the wave's first row
    const bool active = rw0 < n_rows;                                  // wave-uniform
    const uint32_t n_steps = (k_blocks + S - 1u) / S;
    // the wave's row tiles that hold rows
    const uint32_t n_tiles = !active ? 0u : (n_rows - rw0 + 15u) / 16u < T ? (n_rows - rw0 + 15u) / 16u : T;
    auto row_src = [&](uint32_t mt, uint32_t r) {
        const uint32_t gr = rw0 + r < n_rows ? rw0 + r : n_rows - 1u;
        return as_global(PAIR && mt ? w1 : w0) + (uint64_t)gr * row_bytes;
    };
    // weight copy: piece q = lane + 64 j is piece q % kPieces of super-block
    // (q / kPieces) % S of row (q / (kPieces S)) % 16 of matrix q / (16 S
    // kPieces): consecutive lanes on consecutive bytes of a row's S super-
    // blocks. Lanes past the last piece load one too (never stored), so
    // every lane issues the same loads and the waits count them exactly.
    // wsrc: the piece's address in step 0 (super-block sl of its row,
    // clamped to the row's last unit), wlim: the offset from there to the
    // piece in the row's last unit
    const uint8_t *wsrc[kWj];
    uint32_t wlim[kWj], wdst[kWj];
    // the piece's step-0 address in row tile `tile` (rows past the matrix
    // clamped to its last row, whose pieces are loaded and never stored)
    auto wsrc_at = [&](uint32_t j, uint32_t tile) {
        const uint32_t q = lane + 64u * j, qq = q < kWp ? q : kWp - 1u;
        const uint32_t c = qq % F::kPieces, rs = qq / F::kPieces, sl = rs % S, rm = rs / S;
        return row_src(rm / 16u, 16u * tile + rm % 16u) + F::piece_off(sl, c, lim);
    };
#pragma unroll
    for (uint32_t j = 0; j < kWj; j++) {
        const uint32_t q = lane + 64u * j, qq = q < kWp ? q : kWp - 1u;
        const uint32_t c = qq % F::kPieces, rs = qq / F::kPieces, sl = rs % S, rm = rs / S;
        const uint32_t o0 = F::piece_off(sl, c, lim);
        wsrc[j] = wsrc_at(j, 0u);
        wlim[j] = F::piece_off(lim, c, lim) - o0;
        wdst[j] = q < kWp ? (rm * kRowL + sl * F::kSlot + 16u * c) : UINT32_MAX;
    }
    // tails (d / dmin, MXFP4 e): kTails per (matrix, row, super-block of the step)
    const uint8_t *tsrc[kTjA];
    uint32_t tlim[kTjA], tdst[kTjA];
    auto tsrc_at = [&](uint32_t j, uint32_t tile) {
        const uint32_t q = lane + 64u * j, qq = q < kTp ? q : kTp - 1u;
        const uint32_t c = qq % (F::kTails ? F::kTails : 1u), rs = qq / (F::kTails ? F::kTails : 1u);
        const uint32_t sl = rs % S, rm = rs / S;
        return row_src(rm / 16u, 16u * tile + rm % 16u) + F::tail_off(sl, c, lim);
    };
#pragma unroll
    for (uint32_t j = 0; j < kTj; j++) {
        const uint32_t q = lane + 64u * j, qq = q < kTp ? q : kTp - 1u;
        const uint32_t c = qq % (F::kTails ? F::kTails : 1u), rs = qq / (F::kTails ? F::kTails : 1u);
        const uint32_t sl = rs % S, rm = rs / S;
        const uint32_t o0 = F::tail_off(sl, c, lim);
        tsrc[j] = tsrc_at(j, 0u);
        tlim[j] = F::tail_off(lim, c, lim) - o0;
        tdst[j] = q < kTp ? (rm * kRowL + sl * F::kSlot + F::kTailSlot + c) : UINT32_MAX;
    }
    uint8_t *wl_w = &wl[wave][0];
    const uint32_t act_bytes = act_row_pitch(k_blocks);
    uint4 wv[kWj];
    uint32_t tv[kTjA];
    auto issue = [&](uint32_t tile, uint32_t step, bool adv) {
        // a new row tile: the pieces' step-0 addresses move 16 rows on
        // (the tile before it was whole), or are formed again with the
        // rows clamped when the tile ends past the matrix (wave-uniform
        // branches, no loads under them). adv = false: the walk's last
        // (tile, step) requested again past the end (one-step rows), whose
        // addresses are the current ones and must not move on
        if (T > 1u && adv && step == 0u && tile > 0u) {
            if (rw0 + 16u * tile + 16u <= n_rows) {
#pragma unroll
                for (uint32_t j = 0; j < kWj; j++) wsrc[j] += 16u * row_bytes;
#pragma unroll
                for (uint32_t j = 0; j < kTj; j++) tsrc[j] += 16u * row_bytes;
            } else {
#pragma unroll
                for (uint32_t j = 0; j < kWj; j++) wsrc[j] = wsrc_at(j, tile);
#pragma unroll
                for (uint32_t j = 0; j < kTj; j++) tsrc[j] = tsrc_at(j, tile);
            }
        }
        // the step-0 address plus the step's uniform offset, held at the
        // lane's last unit of the row (units past the row are loaded
        // from it, never used): one min and one 64-bit add per load
        const uint32_t so = step * S * F::kSbBytes;
#pragma unroll
        for (uint32_t j = 0; j < kWj; j++) wv[j] = ldw128(wsrc[j] + (so < wlim[j] ? so : wlim[j]));
#pragma unroll
        for (uint32_t j = 0; j < kTj; j++) {
            const uint8_t *tp = tsrc[j] + (so < tlim[j] ? so : tlim[j]);
            tv[j] = F::kTailBytes == 4u ? ldw32(tp) : F::kTailBytes == 2u ? (uint32_t)ldw16(tp) : ldw8(tp);
        }
    };
    // MXFP4 (both stages) and the IQ2_XXS and Q2_K down stages request
    // their first step of weights before the pair tile's activations are
    // staged, so the two round trips overlap (alternating libraries: c5
    // 64-token layer 162.4 -> 160.5 us, gate / up 94.9 -> 93.4, down 49.3 ->
    // 48.5; c4 IQ2_XXS down 53.9 -> 52.8 us; c4 Q2_K down, with two row
    // tiles per wave, 44.8 -> 43.7 us, though it then fetches ~9% more: the
    // lines its first two steps share leave the L2 while the staging runs).
    // The Q2_K gate / up stage fetched 5% more that way for no measurable
    // gain, and IQ2_XXS gate / up is unchanged.
    constexpr bool kEarly = kMx || ((kIq2 || Q == PULSAR_QUANT_Q2_K) && !PAIR);
    if (kEarly && active) issue(0u, 0u, true);
    for (uint32_t t0 = s0; t0 < s1; t0 += pmax) {
        const uint32_t m = s1 - t0 < pmax ? s1 - t0 : pmax;
        if (t0 != s0) __syncthreads();  // the previous tile's activations are consumed
        if (threadIdx.x < m) pr_l[threadIdx.x] = src.pair(t0 + threadIdx.x, lst);
        __syncthreads();
        stage_q8_rows<2, Q == PULSAR_QUANT_Q2_K>(acts_lds, m, k_blocks, act_bytes, [&](uint32_t j) {
            const uint32_t pr = pr_l[j];
            return act + (PAIR ? (uint64_t)(pr >> 4) : (uint64_t)(pr >> 4) * n_used + (pr & 15u)) * k_blocks;
        });
        __syncthreads();
        if (!active) continue;  // wave-uniform; the block's barriers above are reached
        // lane (pair i, kq): its pair's record (the last pair's past the tile)
        const uint8_t *ar = acts_lds + (i < m ? i : m - 1u) * act_bytes;
        // tiles of at most 4 pairs (wave-uniform): lane (row i, pair kq)
        // accumulates acs; larger tiles: lane (row i, kq) pairs 4 kq + r in
        // acc. Q4_K, Q5_K and Q6_K keep the one path: the second one costs
        // their pair stages occupancy (Q4_K 127 -> 169 VGPRs)
        constexpr bool kSmallPath = Q == PULSAR_QUANT_Q2_K || kIq2 || kMx;
        const bool small_rt = kSmallPath && m <= 4u;
        // tiles of one pair (most c4 groups): its values are element 0 of
        // the kq = 0 lanes, so no gather, and the IQ2_XXS gate / up stage
        // forms its per-element scale products for that element only (c4
        // 97.9 -> 96.4 us; in the down stage the second copy of the group
        // loop cost a wave per SIMD, 54.7 -> 55.4 us)
        const bool one_rt = (Q == PULSAR_QUANT_Q2_K || (kIq2 && PAIR)) && m == 1u;
        // The Q2_K gate / up stage and both IQ2_XXS stages walk their steps
        // in three copies, one per epilogue (one pair, tiles of at most 4,
        // larger), chosen once per pair tile: with the choice made per
        // super-block, the branches' merges cost every step register copies
        // (c4, alternating libraries: Q2_K gate / up 80.3 -> 77.7 us,
        // IQ2_XXS gate / up 97.4 -> 92.4 us, IQ2_XXS down 54.9 -> 53.7 us).
        // MODE 0: chosen at run time (the other stages: the MXFP4 gate / up
        // copies spill, the Q2_K down copies cost a wave per SIMD and time,
        // the MXFP4 down copies measured the same).
        constexpr bool kModes = (Q == PULSAR_QUANT_Q2_K && PAIR) || kIq2;
        using Mode0 = std::integral_constant<int, 0>;
        auto flags = [&](auto mode_c, bool &one, bool &small) {
            constexpr int MODE = decltype(mode_c)::value;
            one = MODE == 0 ? one_rt : MODE == 1;
            small = MODE == 0 ? small_rt : MODE != 3;
        };
        float acc[NM][4], acs[NM];
#pragma unroll
        for (uint32_t mt = 0; mt < NM; mt++) {
            acs[mt] = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; r++) acc[mt][r] = 0.0f;
        }
        // super-block sb from the wave's LDS slot ws (row i of matrix 0)
        auto sb_compute = [&](uint32_t sb, const uint8_t *ws, auto mode_c) {
            bool one, small;
            flags(mode_c, one, small);
            // the scales' slot offset (the row's last super-block: its copy is
            // held inside the row)
            const uint32_t tail_at = F::kTailSlot + (sb + 1u == lim ? F::kTailLast : 0u);
            const uint8_t *rec = ar + sb * kActLdsPitch;  // d @0, q8 values @16, bsums @272
            // pairs past the tile read the last pair's values: their MFMA
            // rows and sums are never stored
            float yd[4];
            if (!small) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t pi = 4u * kq + r < m ? 4u * kq + r : m - 1u;
                    yd[r] = *(const float *)(acts_lds + pi * act_bytes + sb * kActLdsPitch);
                }
            }
            const float yd1 = *(const float *)(acts_lds + (kq < m ? kq : m - 1u) * act_bytes + sb * kActLdsPitch);
            auto a_at = [&](uint32_t t) { return *(const uint2 *)(rec + 16u + 32u * t + 8u * kq); };
            if constexpr (kMx) {
                // lane group kq: values 8 kq + [0, 8) of a block, nibble kq >> 1
                // of qs bytes 8 (kq & 1) + [0, 8), so each half-wave reads 16
                // contiguous bytes of every pair's q8 values and of every row's
                // codes (with lane groups on values {0, 16, 8, 24}[kq] the pair
                // reads of a half-wave fell on half the banks twice: ~1.0M
                // conflict cycles per c5 64-token launch, now ~1K, the stage
                // time unchanged); per block the reference's sumf +=
                // scale_half(e) * sumi for sumi != 0 (an fma of a power of two
                // and an int < 2^24 is exact, and sumi = 0 adds +0 to a sum
                // that is never -0), then yd * sumf
                const uint32_t nsh = 4u * (kq >> 1), a_piece = kq, w_piece = kq & 1u;
                const uint32_t nb = lim - 8u * sb < 8u ? lim - 8u * sb : 8u;
                uint2 ev[NM];
                float f[NM][4];
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    ev[mt] = *(const uint2 *)(ws + mt * 16u * kRowL + F::kTailSlot);
#pragma unroll
                    for (int r = 0; r < 4; r++) f[mt][r] = 0.0f;
                }
#pragma unroll
                for (uint32_t bl = 0; bl < 8; bl++) {
                    if (bl >= nb) break;  // uniform: the row's last super-block may be short
                    const uint2 a = *(const uint2 *)(rec + 16u + 32u * bl + 8u * a_piece);
#pragma unroll
                    for (uint32_t mt = 0; mt < NM; mt++) {
                        const uint2 qq = *(const uint2 *)(ws + mt * 16u * kRowL + 16u * bl + 8u * w_piece);
                        const v4i d = mfma16x16x32(a, make_uint2(mxfp4_kv4(qq.x >> nsh), mxfp4_kv4(qq.y >> nsh)));
                        const float sc = mxfp4_scale_half(byte_of(ev[mt], bl));
                        for (int r = 0; r < 4; r++) f[mt][r] = __builtin_fmaf(sc, (float)d[r], f[mt][r]);
                    }
                }
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    if (small) {
                        acs[mt] = __builtin_fmaf(yd1, gather_pairs(f[mt]), acs[mt]);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[mt][r] = __builtin_fmaf(yd[r], f[mt][r], acc[mt][r]);
                    }
                }
            } else if constexpr (Q == PULSAR_QUANT_Q6_K) {
                // two MFMAs per 32-value step (both 16-value scale groups, then
                // the first alone): sc0 D0 + sc1 D1 = (sc0 - sc1) D_lo + sc1 D_all
                MmaQ6K::W wv[NM];
                int32_t isum[NM][4];
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    wv[mt] = MmaQ6K::load_lds(ws + mt * 16u * kRowL, kq, tail_at);
#pragma unroll
                    for (int r = 0; r < 4; r++) isum[mt][r] = 0;
                }
#pragma unroll
                for (int st = 0; st < 8; st++) {
                    const int h = st >> 2, q = st & 3;
                    const uint2 a = a_at((uint32_t)st);
#pragma unroll
                    for (uint32_t mt = 0; mt < NM; mt++) {
                        const uint2 c = MmaQ6K::codes(wv[mt], h, q);
                        const v4i d_all = mfma16x16x32(a, c);
                        const v4i d_lo = mfma16x16x32(a, kq < 2 ? c : make_uint2(0u, 0u));
                        const int32_t s0 = (int32_t)(int8_t)byte_of(wv[mt].sc, 8 * h + 2 * q);
                        const int32_t s1 = (int32_t)(int8_t)byte_of(wv[mt].sc, 8 * h + 2 * q + 1);
#pragma unroll
                        for (int r = 0; r < 4; r++) isum[mt][r] += __mul24(s0 - s1, d_lo[r]) + __mul24(s1, d_all[r]);
                    }
                }
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    const float xd = f16f((uint16_t)wv[mt].d);
                    if (small) {
                        const v4i is = {isum[mt][0], isum[mt][1], isum[mt][2], isum[mt][3]};
                        acs[mt] = __builtin_fmaf(xd * yd1, (float)gather_pairs(is), acs[mt]);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[mt][r] = __builtin_fmaf(xd * yd[r], (float)isum[mt][r], acc[mt][r]);
                    }
                }
            } else if constexpr (Q == PULSAR_QUANT_Q4_K || Q == PULSAR_QUANT_Q5_K) {
                // one MFMA per 32-value sub-block, its 6-bit scale on D; the
                // min term from two MFMAs on the bsum pair sums split 128 h + l
                using M = MmaKq<Q>;
                typename M::W wv[NM];
                int32_t isum[NM][4];
                uint32_t mins[NM][2];
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    wv[mt] = M::load_lds(ws + mt * 16u * kRowL, kq);
                    mins[mt][0] = mins[mt][1] = 0u;
#pragma unroll
                    for (int r = 0; r < 4; r++) isum[mt][r] = 0;
                }
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const uint2 a = a_at((uint32_t)t);
#pragma unroll
                    for (uint32_t mt = 0; mt < NM; mt++) {
                        int32_t sc, mn;
                        Fmt<PULSAR_QUANT_Q4_K>::scale_min(wv[mt].hdr, (uint32_t)t, sc, mn);
                        mins[mt][t >> 2] |= (uint32_t)mn << (8 * (t & 3));
                        const v4i d = mfma16x16x32(a, M::codes(wv[mt], t));
#pragma unroll
                        for (int r = 0; r < 4; r++) isum[mt][r] += __mul24(sc, d[r]);
                    }
                }
                const uint4 bs = *(const uint4 *)(rec + 272u + 16u * (kq & 1u));
                const uint2 alh = make_uint2(pair_sum_bytes(bs, kq >= 2u), 0u);
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    const uint32_t mw = mins[mt][kq & 1u];
                    const v4i dl = mfma16x16x32(alh, kq < 2u ? make_uint2(mw, 0u) : make_uint2(0u, 0u));
                    const v4i dh = mfma16x16x32(alh, kq < 2u ? make_uint2(0u, 0u) : make_uint2(mw, 0u));
                    const float xd = f16f((uint16_t)wv[mt].hdr.x), xmin = f16f((uint16_t)(wv[mt].hdr.x >> 16));
                    if (small) {
                        const v4i is = {isum[mt][0], isum[mt][1], isum[mt][2], isum[mt][3]};
                        const v4i ms = {dl[0] + 128 * dh[0], dl[1] + 128 * dh[1], dl[2] + 128 * dh[2], dl[3] + 128 * dh[3]};
                        acs[mt] += xd * yd1 * (float)gather_pairs(is) - xmin * yd1 * (float)gather_pairs(ms);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int32_t msum = dl[r] + 128 * dh[r];
                            acc[mt][r] += xd * yd[r] * (float)isum[mt][r] - xmin * yd[r] * (float)msum;
                        }
                    }
                }
            } else if constexpr (!kIq2) {
                uint4 sc[NM], scl[NM];
                uint2 qv[NM][2];
                v4i isum[NM];
                // v_perm selectors: scale byte 2 (t & 1) + kq / 2 of scale word
                // t / 2 into bytes 0 and 2, zeros into bytes 1 and 3
                const uint32_t sel_even = 0x0C000C00u + (kq >> 1) * 0x00010001u, sel_odd = sel_even + 0x00020002u;
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    const uint8_t *wm = ws + mt * 16u * kRowL;
                    sc[mt] = *(const uint4 *)wm;
                    // the 4-bit scales (low nibbles), masked once per super-block
                    scl[mt] = make_uint4(sc[mt].x & 0x0f0f0f0fu, sc[mt].y & 0x0f0f0f0fu, sc[mt].z & 0x0f0f0f0fu,
                                         sc[mt].w & 0x0f0f0f0fu);
#pragma unroll
                    for (uint32_t k = 0; k < 2; k++)
                        qv[mt][k] = *(const uint2 *)(wm + 16u + 32u * k + 16u * (kq >> 1) + 8u * (kq & 1u));
                    isum[mt] = v4i{0, 0, 0, 0};
                }
#pragma unroll
                for (uint32_t t = 0; t < 8; t++) {
                    const uint2 a = a_at(t);
                    const uint32_t sh = 2u * (t & 3u);
#pragma unroll
                    for (uint32_t mt = 0; mt < NM; mt++) {
                        // scales of sub-blocks 2t + kq / 2 (t even: byte kq / 2 of
                        // scale word t / 2, t odd: byte kq / 2 + 2), as both
                        // 16-bit halves of s2
                        const uint32_t scw[4] = {scl[mt].x, scl[mt].y, scl[mt].z, scl[mt].w};
                        const uint32_t s2 = __builtin_amdgcn_perm(0u, scw[t >> 1], (t & 1u) ? sel_odd : sel_even);
                        // codes (0..3 per byte) times the scale, per 16-bit half:
                        // c0 sc + 256 c1 sc with c sc <= 45, so no carry between bytes
                        const uint2 q = qv[mt][t >> 2];
                        const uint2 b = make_uint2(pk_mul16((q.x >> sh) & 0x03030303u, s2),
                                                   pk_mul16((q.y >> sh) & 0x03030303u, s2));
                        isum[mt] = mfma16x16x32(a, b, isum[mt]);
                    }
                }
                // lane (pair i, kq): the l (kq < 2) or h (kq >= 2) bytes of bsums
                // 8 (kq & 1) + [0, 8), split when the tile was staged; zeros in
                // the other lane groups of each operand
                const uint2 ab = *(const uint2 *)(rec + 272u + 16u * (kq & 1u) + 8u * (kq >> 1));
                const uint2 zero = make_uint2(0u, 0u);
                const uint2 al = kq < 2u ? ab : zero, ah = kq < 2u ? zero : ab;
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    // mins of sub-blocks 8 (kq & 1) + [0, 8)
                    const uint2 s8 = (kq & 1u) ? make_uint2(sc[mt].z, sc[mt].w) : make_uint2(sc[mt].x, sc[mt].y);
                    const uint2 mn = make_uint2((s8.x >> 4) & 0x0f0f0f0fu, (s8.y >> 4) & 0x0f0f0f0fu);
                    const v4i dl = mfma16x16x32(al, mn);
                    const v4i dh = mfma16x16x32(ah, mn);
                    const uint32_t dd = *(const uint32_t *)(ws + mt * 16u * kRowL + tail_at);
                    const float xd = f16f((uint16_t)dd), xmin = f16f((uint16_t)(dd >> 16));
                    if (one) {  // a single pair: its values are element 0 of the kq = 0 lanes already
                        acs[mt] += yd1 * xd * (float)isum[mt][0] - yd1 * xmin * (float)(dl[0] + 128 * dh[0]);
                    } else if (small) {
                        const v4i sm = {dl[0] + 128 * dh[0], dl[1] + 128 * dh[1], dl[2] + 128 * dh[2], dl[3] + 128 * dh[3]};
                        acs[mt] += yd1 * xd * (float)gather_pairs(isum[mt]) - yd1 * xmin * (float)gather_pairs(sm);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            const int32_t summs = dl[r] + 128 * dh[r];
                            acc[mt][r] += yd[r] * xd * (float)isum[mt][r] - yd[r] * xmin * (float)summs;
                        }
                    }
                }
            } else {
                int32_t bsum[NM][4];
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++)
#pragma unroll
                    for (int r = 0; r < 4; r++) bsum[mt][r] = 0;
// two groups unrolled: measured against 1, 4 and 8 (c4 IQ2_XXS layer 197 ->
// 185 us from 4)
#ifndef PK_GQ_IQ2_UNROLL
#define PK_GQ_IQ2_UNROLL 2
#endif
                // the group loop in two copies (a single-pair tile scales one
                // element), chosen once per super-block
                auto groups = [&](auto one_c) {
#pragma unroll PK_GQ_IQ2_UNROLL
                    for (uint32_t g = 0; g < 8; g++) {
                        const uint2 a = a_at(g);
#pragma unroll
                        for (uint32_t mt = 0; mt < NM; mt++) {
                            const uint2 aux = *(const uint2 *)(ws + mt * 16u * kRowL + 8u * g);
                            uint2 b;
                            iq2_signed8(lut, (aux.x >> (8u * kq)) & 0xffu, (aux.y >> (7u * kq)) & 127u, b.x, b.y);
                            const v4i d = mfma16x16x32(a, b);
                            const int32_t ls = (int32_t)(2u * (aux.y >> 28) + 1u);
                            if constexpr (decltype(one_c)::value) {
                                bsum[mt][0] += __mul24(d[0], ls);
                            } else {
#pragma unroll
                                for (int r = 0; r < 4; r++) bsum[mt][r] += __mul24(d[r], ls);
                            }
                        }
                    }
                };
                if constexpr (PAIR) {
                    if (one)
                        groups(std::true_type{});
                    else
                        groups(std::false_type{});
                } else {
                    groups(std::false_type{});
                }
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    const float xd8 = 0.125f * f16f(*(const uint16_t *)(ws + mt * 16u * kRowL + F::kTailSlot));
                    if (one) {
                        acs[mt] = __builtin_fmaf(xd8 * yd1, (float)bsum[mt][0], acs[mt]);
                    } else if (small) {
                        const v4i bs = {bsum[mt][0], bsum[mt][1], bsum[mt][2], bsum[mt][3]};
                        acs[mt] = __builtin_fmaf(xd8 * yd1, (float)gather_pairs(bs), acs[mt]);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[mt][r] = __builtin_fmaf(xd8 * yd[r], (float)bsum[mt][r], acc[mt][r]);
                    }
                }
            }
        };
        // lane (row i, kq) of row tile `tile`: pairs 4kq + r of the pair
        // tile (small tiles: pair kq); the accumulators restart at zero
        auto store_tile = [&](uint32_t tile, auto mode_c) {
            bool one, small;
            flags(mode_c, one, small);
            (void)one;
            const uint32_t orow = rw0 + 16u * tile + i;
            if (orow < n_rows) {
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const uint32_t pi = small ? kq : 4u * kq + r;
                    if (pi >= m || (small && r > 0)) break;
                    const uint32_t pr = pr_l[pi];
                    const uint64_t so = (uint64_t)(pr >> 4) * n_used + (pr & 15u);
                    if (PAIR) {
                        float g = small ? acs[0] : acc[0][r], u = small ? acs[NM - 1] : acc[NM - 1][r];
                        if (p.gate_b) g += ldwf(p.gate_b + orow);
                        if (p.up_b) u += ldwf(p.up_b + orow);
                        out[so * n_rows + orow] = glu(g, u, act_op) * weights[so];
                    } else {
                        out[so * n_rows + orow] = small ? acs[0] : acc[0][r];
                    }
                }
            }
#pragma unroll
            for (uint32_t mt = 0; mt < NM; mt++) {
                acs[mt] = 0.0f;
#pragma unroll
                for (int r = 0; r < 4; r++) acc[mt][r] = 0.0f;
            }
        };
        if (T > 1u && t0 != s0) {  // a later pair tile: back to the first row tile
#pragma unroll
            for (uint32_t j = 0; j < kWj; j++) wsrc[j] = wsrc_at(j, 0u);
#pragma unroll
            for (uint32_t j = 0; j < kTj; j++) tsrc[j] = tsrc_at(j, 0u);
        }
        if (!kEarly || t0 != s0) issue(0u, 0u, true);
        // (tile, step) in order; the next one's loads are in flight while
        // this one is decoded (past the last, the last again: never stored)
        const uint32_t tiles = T == 1u ? 1u : n_tiles;
        auto walk = [&](auto mode_c) {
        for (uint32_t tile = 0; tile < tiles; tile++) {
            for (uint32_t step = 0; step < n_steps; step++) {
    #pragma unroll
                for (uint32_t j = 0; j < kWj; j++)
                    if ((j + 1u) * 64u <= kWp || wdst[j] != UINT32_MAX) *(uint4 *)(wl_w + wdst[j]) = wv[j];
    #pragma unroll
                for (uint32_t j = 0; j < kTj; j++) {
                    if ((j + 1u) * 64u > kTp && tdst[j] == UINT32_MAX) continue;
                    if (F::kTailBytes == 4u)
                        *(uint32_t *)(wl_w + tdst[j]) = tv[j];
                    else if (F::kTailBytes == 2u)
                        *(uint16_t *)(wl_w + tdst[j]) = (uint16_t)tv[j];
                    else
                        wl_w[tdst[j]] = (uint8_t)tv[j];
                }
                // the wave's own LDS slots: visible to the wave's other lanes
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                uint32_t nt = tile, ns = step + 1u;
                const bool more = ns < n_steps || tile + 1u < tiles;
                if (ns == n_steps) {
                    ns = tile + 1u < tiles ? 0u : step;
                    nt = tile + 1u < tiles ? tile + 1u : tile;
                }
                issue(nt, ns, more);
#pragma unroll
                for (uint32_t sl = 0; sl < S; sl++)
                    if (step * S + sl < k_blocks)
                        sb_compute(step * S + sl, wl_w + i * kRowL + sl * F::kSlot, mode_c);
                // this step's LDS reads are consumed before the next copy
                __builtin_amdgcn_wave_barrier();
            }
            store_tile(tile, mode_c);
        }
        };
        if constexpr (kModes) {
            if (one_rt)
                walk(std::integral_constant<int, 1>{});
            else if (small_rt)
                walk(std::integral_constant<int, 2>{});
            else
                walk(std::integral_constant<int, 3>{});
        } else {  // the same walk, written out (as a lambda it compiled differently)
        for (uint32_t tile = 0; tile < tiles; tile++) {
            for (uint32_t step = 0; step < n_steps; step++) {
    #pragma unroll
                for (uint32_t j = 0; j < kWj; j++)
                    if ((j + 1u) * 64u <= kWp || wdst[j] != UINT32_MAX) *(uint4 *)(wl_w + wdst[j]) = wv[j];
    #pragma unroll
                for (uint32_t j = 0; j < kTj; j++) {
                    if ((j + 1u) * 64u > kTp && tdst[j] == UINT32_MAX) continue;
                    if (F::kTailBytes == 4u)
                        *(uint32_t *)(wl_w + tdst[j]) = tv[j];
                    else if (F::kTailBytes == 2u)
                        *(uint16_t *)(wl_w + tdst[j]) = (uint16_t)tv[j];
                    else
                        wl_w[tdst[j]] = (uint8_t)tv[j];
                }
                // the wave's own LDS slots: visible to the wave's other lanes
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                uint32_t nt = tile, ns = step + 1u;
                const bool more = ns < n_steps || tile + 1u < tiles;
                if (ns == n_steps) {
                    ns = tile + 1u < tiles ? 0u : step;
                    nt = tile + 1u < tiles ? tile + 1u : tile;
                }
                issue(nt, ns, more);
#pragma unroll
                for (uint32_t sl = 0; sl < S; sl++)
                    if (step * S + sl < k_blocks)
                        sb_compute(step * S + sl, wl_w + i * kRowL + sl * F::kSlot, Mode0{});
                // this step's LDS reads are consumed before the next copy
                __builtin_amdgcn_wave_barrier();
            }
            store_tile(tile, Mode0{});
        }
        }
    }
}

// Grouped MoE stages of Q2_K, IQ2_XXS, MXFP4, Q4_K, Q5_K and Q6_K experts
// on the matrix cores; -1 for the other formats (the caller then uses the
// lane kernels of moe.hip). `src` is the group source (CsrGroups or
// ExpertGroups), n_group the grid's group count; lst_bytes the LDS the
// source's pair list needs (0 for the caller's CSR).
template <typename G>
int launch_grouped_mmq_kq(bool pair, uint32_t quant, float *out, const G &src, const float *weights,
                          const pulsar_block_q8_K *act, uint32_t k_dim, uint32_t n_rows, uint32_t n_used,
                          uint32_t n_group, uint64_t row_bytes, uint32_t act_op, uint32_t lst_bytes) {
    if (quant != PULSAR_QUANT_Q2_K && quant != PULSAR_QUANT_IQ2_XXS && quant != PULSAR_QUANT_MXFP4 &&
        quant != PULSAR_QUANT_Q4_K && quant != PULSAR_QUANT_Q5_K && quant != PULSAR_QUANT_Q6_K)
        return -1;
    const uint32_t k_blocks = (k_dim + 255u) / 256u;
    const uint32_t lim = quant == PULSAR_QUANT_MXFP4 ? k_dim / 32u : k_blocks;
    const uint32_t per_pair = act_row_pitch(k_blocks);
    // MXFP4 layers route many pairs to each expert (gpt-oss: 64 tokens x 4 of
    // 32 experts), so their tiles take more pairs per weight pass
    // Gate / up tiles of 4096-value rows hold 5 pairs instead of 3 (4880 bytes
    // each), so an expert with 4 or 5 pairs takes one weight pass, not two;
    // their blocks keep 3 per CU (VGPRs allow no more; Q2_K: 26.7 KiB static
    // + 24.4 KiB tile + the pair list, x 3 < 160 KiB). Down stages keep 16 KiB:
    // their blocks are smaller and 5 fit per CU. Large pair lists (many
    // tokens) keep the smaller tile.
    const uint32_t budget = quant == PULSAR_QUANT_MXFP4          ? kGqActLdsMx
                            : pair && lst_bytes <= 1024u ? kGqActLdsPair
                                                         : kGqActLds;
    if (per_pair > budget) return -1;  // one pair's row does not fit: lane kernels
    uint32_t pmax = budget / per_pair;
    pmax = pmax < kGqPairs ? pmax : kGqPairs;
    const uint32_t lst_off = (pmax * per_pair + 15u) & ~15u;
    const size_t lds = (size_t)lst_off + lst_bytes;
#define PK_GQ(Q, P)                                                                                              \
    hipLaunchKernelGGL((moe_grouped_mmq_kq_kernel<Q, P, G>),                                                     \
                       dim3((n_rows + kGqBlockRows<Q, P> - 1u) / kGqBlockRows<Q, P>, n_group),                     \
                       dim3(64u * kGqWaves<Q>), lds, pk::stream(), out, src, weights, act, k_blocks, lim, n_rows, \
                       n_used, row_bytes, act_op, pmax, lst_off)
    if (quant == PULSAR_QUANT_Q2_K && pair)
        PK_GQ(PULSAR_QUANT_Q2_K, true);
    else if (quant == PULSAR_QUANT_Q2_K)
        PK_GQ(PULSAR_QUANT_Q2_K, false);
    else if (quant == PULSAR_QUANT_IQ2_XXS && pair)
        PK_GQ(PULSAR_QUANT_IQ2_XXS, true);
    else if (quant == PULSAR_QUANT_IQ2_XXS)
        PK_GQ(PULSAR_QUANT_IQ2_XXS, false);
    else if (quant == PULSAR_QUANT_Q4_K && pair)
        PK_GQ(PULSAR_QUANT_Q4_K, true);
    else if (quant == PULSAR_QUANT_Q4_K)
        PK_GQ(PULSAR_QUANT_Q4_K, false);
    else if (quant == PULSAR_QUANT_Q5_K && pair)
        PK_GQ(PULSAR_QUANT_Q5_K, true);
    else if (quant == PULSAR_QUANT_Q5_K)
        PK_GQ(PULSAR_QUANT_Q5_K, false);
    else if (quant == PULSAR_QUANT_Q6_K && pair)
        PK_GQ(PULSAR_QUANT_Q6_K, true);
    else if (quant == PULSAR_QUANT_Q6_K)
        PK_GQ(PULSAR_QUANT_Q6_K, false);
    else if (pair)
        PK_GQ(PULSAR_QUANT_MXFP4, true);
    else
        PK_GQ(PULSAR_QUANT_MXFP4, false);
#undef PK_GQ
    return launch_ok(pair ? "moe pair swiglu grouped (mfma) launch" : "moe down grouped (mfma) launch");
}
template int launch_grouped_mmq_kq<CsrGroups>(bool, uint32_t, float *, const CsrGroups &, const float *,
                                              const pulsar_block_q8_K *, uint32_t, uint32_t, uint32_t, uint32_t,
                                              uint64_t, uint32_t, uint32_t);
template int launch_grouped_mmq_kq<ExpertGroups>(bool, uint32_t, float *, const ExpertGroups &, const float *,
                                                 const pulsar_block_q8_K *, uint32_t, uint32_t, uint32_t, uint32_t,
                                                 uint64_t, uint32_t, uint32_t);

}  // namespace pk
