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

template <uint32_t QOFF, uint32_t BOFF>
PK_DEV void quantize_vals_wave(const float (&v)[4], uint8_t *ob) {
    const uint32_t lane = threadIdx.x & 63u;
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = wave_max(am);
    uint32_t packed = 0;
    int32_t s4 = 0;
    float d = 0.0f;
    if (am != 0.0f) {
        d = am / 127.0f;
        const float inv = 127.0f / am;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float q = roundf(v[j] * inv);
            // Rust's saturating `as i8` maps NaN (0 * inf when 127/amax
            // overflows) to 0
            q = q != q ? 0.0f : fminf(fmaxf(q, -127.0f), 127.0f);
            const int32_t qi = (int32_t)q;
            s4 += qi;
            packed |= ((uint32_t)qi & 0xffu) << (8 * j);
        }
    }
    *(uint32_t *)(ob + QOFF + 4 * lane) = packed;
    s4 = group_sum<4>(s4);
    if ((lane & 3u) == 0u) *(int16_t *)(ob + BOFF + 2 * (lane >> 2)) = (int16_t)s4;
    if (lane == 0) *(float *)ob = d;
}

template <uint32_t QOFF, uint32_t BOFF>
PK_DEV void quantize_block_wave(const float *xr, uint32_t in_dim, uint32_t b, uint8_t *ob) {
    float v[4];
    load_block4(xr, in_dim, b, v);
    quantize_vals_wave<QOFF, BOFF>(v, ob);
}

}  // namespace pk
