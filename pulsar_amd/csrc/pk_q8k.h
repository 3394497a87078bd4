// pk_q8k.h - the q8_K activation quantizer as a wave-level device function,
// shared by the quantize kernel and the kernels that quantize their own
// inputs (fused decode layer).
#pragma once

#include "pk_common.h"

namespace pk {

// One wave quantizes 256-value block b of row xr (lane l owns values
// 4l .. 4l+3) with the CPU lane's algorithm (crates/quant/src/cpu_dot.rs:26-50):
//   amax = max |x|; amax == 0 -> d = 0, all quants 0;
//   d = amax / 127, inv = 127 / amax (IEEE division, correctly rounded),
//   q = clamp(round_half_away(x * inv), -127, 127), bsums = sums of 16.
// Values past in_dim are 0 (pulsar_kernels.cu:1499-1501). Writes f32 d at
// ob, the 256 int8 quants at ob + QOFF and the 16 int16 bsums at ob + BOFF.
// This lane's 4 values of block b (0 past in_dim).
PK_DEV void load_block4(const float *xr, uint32_t in_dim, uint32_t b, float (&v)[4]) {
    const uint32_t c0 = b * 256u + 4u * (threadIdx.x & 63u);
    if (c0 + 4u <= in_dim) {
        const uint4 w = ld128((const uint8_t *)(xr + c0));
        v[0] = __uint_as_float(w.x);
        v[1] = __uint_as_float(w.y);
        v[2] = __uint_as_float(w.z);
        v[3] = __uint_as_float(w.w);
    } else {
#pragma unroll
        for (int j = 0; j < 4; j++) v[j] = c0 + j < in_dim ? xr[c0 + j] : 0.0f;
    }
}

// One lane's share of a block: its 4 quants packed, their sum, and the
// block's d. No branch on amax == 0: there inv = 127 / 0 = inf and every
// x * inv is 0 * inf = NaN, which the saturating conversion maps to 0, the
// quants of an all-zero block (so two blocks can share one instruction
// stream).
PK_DEV void quantize_lane(const float (&v)[4], float am, uint32_t &packed, int32_t &s4, float &d) {
    d = am / 127.0f;
    const float inv = 127.0f / am;
    packed = 0;
    s4 = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        float q = roundf(v[j] * inv);
        // Rust's saturating `as i8` maps NaN (0 * inf when 127/amax
        // overflows or amax is 0) to 0
        q = q != q ? 0.0f : fminf(fmaxf(q, -127.0f), 127.0f);
        const int32_t qi = (int32_t)q;
        s4 += qi;
        packed |= ((uint32_t)qi & 0xffu) << (8 * j);
    }
}

template <uint32_t QOFF, uint32_t BOFF>
PK_DEV void store_quant(uint8_t *ob, uint32_t packed, int32_t s4, float d) {
    const uint32_t lane = threadIdx.x & 63u;
    *(uint32_t *)(ob + QOFF + 4 * lane) = packed;
    if ((lane & 3u) == 0u) *(int16_t *)(ob + BOFF + 2 * (lane >> 2)) = (int16_t)s4;
    if (lane == 0) *(float *)ob = d;
}

template <uint32_t QOFF, uint32_t BOFF>
PK_DEV void quantize_vals_wave(const float (&v)[4], uint8_t *ob) {
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = wave_max(am);
    uint32_t packed;
    int32_t s4;
    float d;
    quantize_lane(v, am, packed, s4, d);
    s4 = group_sum<4>(s4);
    store_quant<QOFF, BOFF>(ob, packed, s4, d);
}

// Two blocks at once (the same arithmetic; their reductions interleave).
// The second block is stored only when has1.
template <uint32_t QOFF, uint32_t BOFF>
PK_DEV void quantize_vals_wave2(const float (&v0)[4], const float (&v1)[4], uint8_t *ob0, uint8_t *ob1, bool has1) {
    float a0 = fmaxf(fmaxf(fabsf(v0[0]), fabsf(v0[1])), fmaxf(fabsf(v0[2]), fabsf(v0[3])));
    float a1 = fmaxf(fmaxf(fabsf(v1[0]), fabsf(v1[1])), fmaxf(fabsf(v1[2]), fabsf(v1[3])));
    a0 = wave_max(a0);
    a1 = wave_max(a1);
    uint32_t p0, p1;
    int32_t s0, s1;
    float d0, d1;
    quantize_lane(v0, a0, p0, s0, d0);
    quantize_lane(v1, a1, p1, s1, d1);
    s0 = group_sum<4>(s0);
    s1 = group_sum<4>(s1);
    store_quant<QOFF, BOFF>(ob0, p0, s0, d0);
    if (has1) store_quant<QOFF, BOFF>(ob1, p1, s1, d1);
}

template <uint32_t QOFF, uint32_t BOFF>
PK_DEV void quantize_block_wave(const float *xr, uint32_t in_dim, uint32_t b, uint8_t *ob) {
    float v[4];
    load_block4(xr, in_dim, b, v);
    quantize_vals_wave<QOFF, BOFF>(v, ob);
}

}  // namespace pk
