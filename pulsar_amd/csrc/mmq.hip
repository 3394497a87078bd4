// mmq.hip - dense matvec for token chunks (5..16 tokens per tile) on the
// int8 matrix cores: v_mfma_i32_16x16x64_i8.
//
// A block computes 16 RT weight rows x 16 tokens. Its NW waves split the
// row's super-blocks (split-K); every wave produces exact int32 group sums
// with MFMA, applies the format's integer scales in int32, forms the per-
// super-block fp32 value in the reference's operation order, accumulates its
// super-blocks in order, and the NW partials are added in wave order through
// LDS (deterministic).
//
// Operand layout of v_mfma_i32_16x16x64_i8 (16 int8 per lane):
//   A[i][k]: lane i + 16 * kq, K slots of lane group kq
//   B[k][j]: lane j + 16 * kq, the same K slots
//   D[i][j]: lane j + 16 * (i / 4), element i % 4
// Which 16 slots a lane group holds does not matter here: A and B hold the
// same ones, and every sum below is over whole lane groups.
#include "pk_rowdot.h"
#include "pk_route.h"

namespace pk {

typedef int32_t v4i __attribute__((ext_vector_type(4)));

PK_DEV v4i mfma16x16x32(uint2 a, uint2 b) {
    const v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, a), __builtin_bit_cast(long, b), z, 0,
                                                 0, 0);
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

#ifndef PK_MMQ_RT
#define PK_MMQ_RT 2u
#endif
#ifndef PK_MMQ_C
#define PK_MMQ_C 4u
#endif

// Tile of 16 RT rows x 16 tokens, K walked in chunks of C super-blocks.
// Each chunk's weights (16 RT rows x C super-blocks) and activations (16
// tokens x C super-blocks) are copied HBM -> LDS with row-contiguous
// 16-byte loads (a wave's load covers 4 consecutive super-blocks of one
// row), the next chunk's loads are issued before the current chunk's MFMAs,
// and wave (rt, sb) = (w / C, w % C) takes row tile rt, super-block sb of
// each chunk. LDS rows are padded so the 16 rows (tokens) an MFMA operand
// read touches fall in distinct banks.
template <uint32_t Q, uint32_t RT, uint32_t C>
struct MmqTile {
    static constexpr uint32_t NW = RT * C;                          // waves
    static constexpr uint32_t NT = 64u * NW;                        // threads
    static constexpr uint32_t kRows = 16u * RT;
    static constexpr uint32_t kSb = MmaQ6K::kSbBytes;               // bytes per row super-block
    static constexpr uint32_t kChunks = (kSb + 15u) / 16u;          // 16-byte loads per row super-block
    static constexpr uint32_t kSlot = 16u * kChunks;                // LDS bytes per row super-block
    // the last load of a super-block reads its final 16 bytes (kSb - 16 ..)
    // and is stored at slot offset 16 (kChunks - 1): d lands here
    static constexpr uint32_t kDSlot = 16u * (kChunks - 1u) + MmaQ6K::kDOff - (kSb - 16u);
    static constexpr uint32_t kRowPitch = C * kSlot + 16u;          // LDS bytes per row (padded)
    static constexpr uint32_t kActPitch = 256u + 16u;               // LDS bytes per (token, super-block)
    static constexpr uint32_t kWLoads = kRows * C * 16u / NT;       // weight loads per thread
    static constexpr uint32_t kALoads = 16u * C * 16u / NT;         // activation loads per thread
    static_assert(kRows * C * 16u % NT == 0 && 16u * C * 16u % NT == 0, "tile shape");
    static_assert(C * 16u <= NT, "one activation scale per thread");
};

template <uint32_t Q, uint32_t RT, uint32_t C>
__global__ __launch_bounds__(64 * RT * C) void mmq_kernel(float *__restrict__ out, const uint8_t *__restrict__ w,
                                                          const pulsar_block_q8_K *__restrict__ xq, uint32_t nb,
                                                          uint32_t out_dim, uint32_t n_tok, uint64_t row_bytes) {
    using T = MmqTile<Q, RT, C>;
    __shared__ __align__(16) uint8_t wl[T::kRows * T::kRowPitch];
    __shared__ __align__(16) uint8_t al[C * 16u * T::kActPitch];
    __shared__ __align__(16) float yl[C * 16u];
    __shared__ float part[T::NW][16][17];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t i = lane & 15u, kq = lane >> 4;
    const uint32_t r0 = blockIdx.x * T::kRows, t0 = blockIdx.y * 16u;
    const uint8_t *xb = (const uint8_t *)xq;
    const uint64_t tok_bytes = (uint64_t)nb * 292u;

    // ---- HBM -> registers -> LDS copy of one chunk (super-blocks kb ..).
    // Per-thread source pointers (chunk 0) and LDS offsets are fixed.
    const uint8_t *wsrc[T::kWLoads];
    uint32_t wsb[T::kWLoads], wdst[T::kWLoads];
    bool wact[T::kWLoads];
#pragma unroll
    for (uint32_t m = 0; m < T::kWLoads; m++) {
        const uint32_t f = tid + T::NT * m, c = f & 15u, rs = f >> 4;
        const uint32_t row = rs / C, sb = rs % C;
        const uint32_t gr = r0 + row < out_dim ? r0 + row : out_dim - 1u;
        const uint32_t off = 16u * c < T::kSb - 16u ? 16u * c : T::kSb - 16u;
        wsrc[m] = w + (uint64_t)gr * row_bytes + (uint64_t)sb * T::kSb + off;
        wsb[m] = sb;
        wdst[m] = row * T::kRowPitch + sb * T::kSlot + 16u * c;
        wact[m] = c < T::kChunks;
    }
    const uint8_t *asrc[T::kALoads];
    uint32_t asb[T::kALoads], adst[T::kALoads];
#pragma unroll
    for (uint32_t m = 0; m < T::kALoads; m++) {
        const uint32_t f = tid + T::NT * m, c = f & 15u, ts = f >> 4;
        const uint32_t t = ts / C, sb = ts % C;
        const uint32_t gt = t0 + t < n_tok ? t0 + t : n_tok - 1u;
        asrc[m] = xb + gt * tok_bytes + (uint64_t)sb * 292u + 4u + 16u * c;
        asb[m] = sb;
        adst[m] = (sb * 16u + t) * T::kActPitch + 16u * c;
    }
    const uint32_t ysb = tid % C, yt = tid / C;
    const uint8_t *ysrc = xb + (t0 + yt < n_tok ? t0 + yt : n_tok - 1u) * tok_bytes + (uint64_t)ysb * 292u;
    const bool yact = tid < C * 16u;

    uint4 wreg[T::kWLoads], areg[T::kALoads];
    uint32_t yreg = 0;
    auto gload = [&](uint32_t kb) {
#pragma unroll
        for (uint32_t m = 0; m < T::kWLoads; m++)
            if (wact[m] && kb + wsb[m] < nb) wreg[m] = ld128(wsrc[m] + (uint64_t)kb * T::kSb);
#pragma unroll
        for (uint32_t m = 0; m < T::kALoads; m++)
            if (kb + asb[m] < nb) areg[m] = ld128(asrc[m] + (uint64_t)kb * 292u);
        if (yact && kb + ysb < nb) yreg = ld32(ysrc + (uint64_t)kb * 292u);
    };
    auto lstore = [&]() {
#pragma unroll
        for (uint32_t m = 0; m < T::kWLoads; m++)
            if (wact[m]) *(uint4 *)(wl + wdst[m]) = wreg[m];
#pragma unroll
        for (uint32_t m = 0; m < T::kALoads; m++) *(uint4 *)(al + adst[m]) = areg[m];
        if (yact) yl[ysb * 16u + yt] = __builtin_bit_cast(float, yreg);
    };

    const uint32_t rt = wave / C, sbw = wave % C;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    gload(0);
    for (uint32_t kb = 0; kb < nb; kb += C) {
        lstore();
        __syncthreads();
        if (kb + C < nb) gload(kb + C);  // in flight during this chunk's MFMAs
        if (kb + sbw < nb) {
            uint2 a[8];
            const uint8_t *ab = al + (sbw * 16u + i) * T::kActPitch + 8u * kq;
#pragma unroll
            for (int st = 0; st < 8; st++) a[st] = lds64(ab + 32u * st);
            const float4 yd4 = lds_f4(yl + sbw * 16u + 4u * kq);
            const float yd[4] = {yd4.x, yd4.y, yd4.z, yd4.w};
            const MmaQ6K::W wv =
                MmaQ6K::load_lds(wl + (rt * 16u + i) * T::kRowPitch + sbw * T::kSlot, kq, T::kDSlot);
            int32_t isum[4] = {0, 0, 0, 0};
#pragma unroll
            for (int st = 0; st < 8; st++) {
                const int h = st >> 2, q = st & 3;
                const uint2 c = MmaQ6K::codes(wv, h, q);
                const uint2 c_lo = kq < 2 ? c : make_uint2(0u, 0u);
                const v4i d_all = mfma16x16x32(a[st], c);
                const v4i d_lo = mfma16x16x32(a[st], c_lo);
                const int32_t s0 = (int32_t)(int8_t)byte_of(wv.sc, 8 * h + 2 * q);
                const int32_t s1 = (int32_t)(int8_t)byte_of(wv.sc, 8 * h + 2 * q + 1);
#pragma unroll
                // |d| < 2^17, |s| < 2^8: 24-bit multiplies are exact
                for (int r = 0; r < 4; r++) isum[r] += __mul24(s0 - s1, d_lo[r]) + __mul24(s1, d_all[r]);
            }
            const float xd = f16f((uint16_t)wv.d);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[r] += xd * yd[r] * (float)isum[r];
        }
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 4; r++) part[wave][i][4 * kq + r] = acc[r];
    __syncthreads();
    for (uint32_t e = tid; e < 16u * T::kRows; e += T::NT) {
        const uint32_t row = e % T::kRows, tok = e / T::kRows;
        if (r0 + row < out_dim && t0 + tok < n_tok) {
            const uint32_t prt = row / 16u;
            float v = part[prt * C][row % 16u][tok];
#pragma unroll
            for (uint32_t k = 1; k < C; k++) v += part[prt * C + k][row % 16u][tok];
            out[(uint64_t)(t0 + tok) * out_dim + r0 + row] = v;
        }
    }
}

int launch_mmq(uint32_t quant, float *out, const uint8_t *w, const pulsar_block_q8_K *xq, uint32_t in_dim,
               uint32_t out_dim, uint32_t n_tok, uint64_t row_bytes) {
    constexpr uint32_t RT = PK_MMQ_RT, C = PK_MMQ_C;
    const uint32_t nb = in_dim / 256u;
    const dim3 grid((out_dim + 16u * RT - 1u) / (16u * RT), (n_tok + 15u) / 16u);
    switch (quant) {
    case PULSAR_QUANT_Q6_K:
        hipLaunchKernelGGL((mmq_kernel<PULSAR_QUANT_Q6_K, RT, C>), grid, dim3(64 * RT * C), 0, pk::stream(), out,
                           w, xq, nb, out_dim, n_tok, row_bytes);
        return launch_ok("matmul_kq mmq launch");
    default:
        return -1;  // no MFMA kernel for this format: caller falls back
    }
}

// ------------------------------------------------- grouped MXFP4 (MoE) --
// One block per (16-row tile, expert group); the group's (token, slot)
// pairs are taken 16 at a time. Per 32-value block one
// v_mfma_i32_16x16x32_i8 gives the exact block sums for 16 pairs x 16 rows:
// A = the pairs' q8 values, B = the rows' E2M1 codes doubled to int8. Lane
// group kq holds values {0, 16, 8, 24}[kq] + [0, 8) of the block: nibble
// kq & 1 of qs bytes 8 (kq >> 1) .. + 7. The 4 waves take contiguous ranges
// of the row's super-blocks. Per super-block a wave copies the 16 rows'
// blocks (one 17-byte block per lane: a wave-wide load covers 8 rows x 136
// contiguous bytes; qs to 16-byte aligned slots, e apart) and the 16 pairs'
// q8 values (a wave-wide load covers 4 pairs x 256 bytes) into its own LDS
// area, so every global load is contiguous and every MFMA operand is an
// aligned LDS read. Per (row, pair) and in block order the reference's
// sumf += scale_half(e) * sumi for sumi != 0, then row += yd * sumf per
// super-block (pulsar_kernels.cu:5715-5741) in the wave's range; the
// block adds the 4 ranges in order.
constexpr uint32_t kMmqPairs = 16;

template <bool PAIR>
__global__ __launch_bounds__(256) void moe_grouped_mmq_mxfp4_kernel(
        float *__restrict__ out, const pulsar_expert_ptrs *__restrict__ gptrs, const uint32_t *__restrict__ starts,
        const uint32_t *__restrict__ pairs, const float *__restrict__ weights,
        const pulsar_block_q8_K *__restrict__ act, uint32_t k_dim, uint32_t k_blocks, uint32_t n_rows,
        uint32_t n_used, uint64_t row_bytes, uint32_t act_op) {
    constexpr uint32_t NM = PAIR ? 2 : 1;
    // rows / pairs padded by 16 bytes: the 16 rows (pairs) an MFMA operand
    // read touches fall in distinct LDS banks
    __shared__ __align__(16) uint4 wq_l[4][NM][16][9];    // [wave][matrix][row][block] qs
    __shared__ __align__(8) uint8_t we_l[4][NM][16][8];   // e
    __shared__ __align__(16) uint4 aq_l[4][16][17];       // [wave][pair][16-byte piece] q8 values
    __shared__ float part[4][NM][16][17];                 // [wave][matrix][row][pair]
    __shared__ uint32_t pr_l[kMmqPairs];
    const uint32_t group = blockIdx.y;
    const pulsar_expert_ptrs p = gptrs[group];
    const uint8_t *w0 = PAIR ? (const uint8_t *)p.gate : (const uint8_t *)p.down;
    const uint8_t *w1 = PAIR ? (const uint8_t *)p.up : nullptr;
    if (!w0 || (PAIR && !w1)) return;
    const uint32_t s0 = starts[group], s1 = starts[group + 1];
    if (s0 >= s1) return;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const uint32_t i = lane & 15u, kq = lane >> 4;
    const uint32_t row0 = blockIdx.x * 16u;
    // weight copy lanes: block lane & 7 of rows lane >> 3 and 8 + (lane >> 3)
    const uint32_t cb = lane & 7u, cr = lane >> 3;
    const uint8_t *cp[NM][2];  // block b of the row: e at 17b, qs at 17b + 1
#pragma unroll
    for (uint32_t h = 0; h < 2; h++) {
        const uint32_t r = row0 + cr + 8u * h;
        const uint64_t ro = (uint64_t)(r < n_rows ? r : n_rows - 1u) * row_bytes;
        cp[0][h] = as_global(w0) + ro;
        if (PAIR) cp[NM - 1][h] = as_global(w1) + ro;
    }
    const uint32_t nsh = 4u * (kq & 1u);
    const uint32_t a_piece = (kq >> 1) + 2u * (kq & 1u);  // 8-byte piece of a 32-value block: 0, 2, 1, 3
    const uint32_t nblk32 = k_dim / 32u;
    const uint32_t per = (k_blocks + 3u) / 4u;
    const uint32_t sb_lo = wave * per, sb_hi = sb_lo + per < k_blocks ? sb_lo + per : k_blocks;
    for (uint32_t t0 = s0; t0 < s1; t0 += kMmqPairs) {
        const uint32_t m = s1 - t0 < kMmqPairs ? s1 - t0 : kMmqPairs;
        if (t0 != s0) __syncthreads();  // the previous tile's partials are consumed
        if (threadIdx.x < m) pr_l[threadIdx.x] = pairs[t0 + threadIdx.x];
        __syncthreads();
        // activation copy lanes: piece lane & 15 of pairs lane >> 4 + 4j
        const uint8_t *ap[4];
#pragma unroll
        for (uint32_t j = 0; j < 4; j++) {
            const uint32_t pi = (lane >> 4) + 4u * j;
            const uint32_t pr = pr_l[pi < m ? pi : 0u];
            ap[j] = (const uint8_t *)(act + (PAIR ? (uint64_t)(pr >> 4) : (uint64_t)(pr >> 4) * n_used + (pr & 15u)) *
                                                k_blocks) + 4u + 16u * (lane & 15u);
        }
        const uint8_t *drow[4];  // yd of pairs 4kq + r
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t pi = 4u * kq + r;
            const uint32_t pr = pr_l[pi < m ? pi : 0u];
            drow[r] = (const uint8_t *)(act + (PAIR ? (uint64_t)(pr >> 4) : (uint64_t)(pr >> 4) * n_used + (pr & 15u)) *
                                                  k_blocks);
        }
        float acc[NM][4];
#pragma unroll
        for (uint32_t mt = 0; mt < NM; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[mt][r] = 0.0f;
        for (uint32_t sb = sb_lo; sb < sb_hi; sb++) {
            const uint32_t b0 = sb * 8u, nb = nblk32 - b0 < 8u ? nblk32 - b0 : 8u;
            // copy the super-block's 16 rows (clamped: never past the row)
            const uint64_t co = 17ull * (b0 + (cb < nb ? cb : 0u));
            uint4 q[NM][2];
            uint32_t e[NM][2];
#pragma unroll
            for (uint32_t mt = 0; mt < NM; mt++)
#pragma unroll
                for (uint32_t h = 0; h < 2; h++) {
                    q[mt][h] = ldw128(cp[mt][h] + co + 1u);
                    e[mt][h] = ldw8(cp[mt][h] + co);
                }
            uint4 av[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) av[j] = ld128(ap[j] + (uint64_t)sb * 292u);
            float yd[4];
#pragma unroll
            for (int r = 0; r < 4; r++) yd[r] = __builtin_bit_cast(float, ld32(drow[r] + (uint64_t)sb * 292u));
#pragma unroll
            for (uint32_t mt = 0; mt < NM; mt++)
#pragma unroll
                for (uint32_t h = 0; h < 2; h++) {
                    wq_l[wave][mt][cr + 8u * h][cb] = q[mt][h];
                    we_l[wave][mt][cr + 8u * h][cb] = (uint8_t)e[mt][h];
                }
#pragma unroll
            for (uint32_t j = 0; j < 4; j++) {
                const uint32_t pi = (lane >> 4) + 4u * j;
                aq_l[wave][pi][lane & 15u] = pi < m ? av[j] : make_uint4(0u, 0u, 0u, 0u);
            }
            // the wave's own LDS area: visible to the wave's other lanes
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float f[NM][4];
#pragma unroll
            for (uint32_t mt = 0; mt < NM; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) f[mt][r] = 0.0f;
            uint2 ev[NM];
#pragma unroll
            for (uint32_t mt = 0; mt < NM; mt++) ev[mt] = *(const uint2 *)&we_l[wave][mt][i][0];
#pragma unroll
            for (uint32_t bl = 0; bl < 8; bl++) {
                if (bl >= nb) break;  // uniform
                const uint2 a = *((const uint2 *)&aq_l[wave][i][0] + 4u * bl + a_piece);
#pragma unroll
                for (uint32_t mt = 0; mt < NM; mt++) {
                    const uint2 qq = *((const uint2 *)&wq_l[wave][mt][i][bl] + (kq >> 1));
                    const uint2 c = make_uint2(mxfp4_kv4(qq.x >> nsh), mxfp4_kv4(qq.y >> nsh));
                    const v4i d = mfma16x16x32(a, c);
                    const float sc = mxfp4_scale_half(byte_of(ev[mt], bl));
                    // = the reference's `if (sumi != 0) sumf += sc * sumi`: sc
                    // is 0 or a power of two and |sumi| < 2^24, so sc * sumi is
                    // exact and one fma rounds like the multiply-add; a zero
                    // sumi adds +0, which leaves sumf (never -0) unchanged
#pragma unroll
                    for (int r = 0; r < 4; r++) f[mt][r] = __builtin_fmaf(sc, (float)d[r], f[mt][r]);
                }
            }
#pragma unroll
            for (uint32_t mt = 0; mt < NM; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) acc[mt][r] += yd[r] * f[mt][r];
        }
#pragma unroll
        for (uint32_t mt = 0; mt < NM; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) part[wave][mt][i][4u * kq + r] = acc[mt][r];
        __syncthreads();
        // one thread per (row, pair): the 4 ranges in order, then the epilogue
        const uint32_t ri = threadIdx.x & 15u, pi = threadIdx.x >> 4;
        if (pi < m && row0 + ri < n_rows) {
            const float g = ((part[0][0][ri][pi] + part[1][0][ri][pi]) + part[2][0][ri][pi]) + part[3][0][ri][pi];
            const uint32_t pr = pr_l[pi];
            const uint64_t so = (uint64_t)(pr >> 4) * n_used + (pr & 15u);
            const uint32_t orow = row0 + ri;
            if (PAIR) {
                float u = ((part[0][NM - 1][ri][pi] + part[1][NM - 1][ri][pi]) + part[2][NM - 1][ri][pi]) +
                          part[3][NM - 1][ri][pi];
                float gg = g;
                if (p.gate_b) gg += ldwf(p.gate_b + orow);
                if (p.up_b) u += ldwf(p.up_b + orow);
                out[so * n_rows + orow] = glu(gg, u, act_op) * weights[so];
            } else {
                out[so * n_rows + orow] = g;
            }
        }
    }
}

// Grouped MoE stages of MXFP4 experts on the matrix cores (pair: gate/up +
// combine into mid; down: per-pair partials). Returns the launch status.
int launch_grouped_mmq_mxfp4(bool pair, float *out, const void *gptrs, const void *starts, const void *pairs,
                             const float *weights, const pulsar_block_q8_K *act, uint32_t k_dim, uint32_t n_rows,
                             uint32_t n_used, uint32_t n_group, uint64_t row_bytes, uint32_t act_op) {
    const uint32_t k_blocks = (k_dim + 255u) / 256u;
    const dim3 grid((n_rows + 15u) / 16u, n_group);
    const size_t lds = 0;
    if (pair)
        hipLaunchKernelGGL(moe_grouped_mmq_mxfp4_kernel<true>, grid, dim3(256), lds, pk::stream(), out,
                           (const pulsar_expert_ptrs *)gptrs, (const uint32_t *)starts, (const uint32_t *)pairs,
                           weights, act, k_dim, k_blocks, n_rows, n_used, row_bytes, act_op);
    else
        hipLaunchKernelGGL(moe_grouped_mmq_mxfp4_kernel<false>, grid, dim3(256), lds, pk::stream(), out,
                           (const pulsar_expert_ptrs *)gptrs, (const uint32_t *)starts, (const uint32_t *)pairs,
                           weights, act, k_dim, k_blocks, n_rows, n_used, row_bytes, act_op);
    return launch_ok(pair ? "moe pair swiglu grouped (mfma) launch" : "moe down grouped (mfma) launch");
}

}  // namespace pk
