// pk_common.h - device helpers shared by every kernel of libpulsar_moe.
//
// Target: gfx950 (CDNA4), wave64. Compiled with -ffp-contract=off so every
// fp32 expression rounds in source order, like the reference's CPU lane
// (crates/quant/src/cpu_dot.rs never fuses a*b+c).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/pulsar_moe.h"

#define PK_DEV __device__ __forceinline__

namespace pk {

constexpr uint32_t kWave = 64;

// Stream of every launch made by the calling thread: its per-thread
// default stream (hipStreamPerThread), as the reference's launches use
// cudaStreamPerThread, unless pulsar_set_stream selected another.
hipStream_t stream();

// Error reporting with the reference's message shape (pulsar_kernels.cu:25-29).
static inline int launch_ok(const char *what) {
    const hipError_t err = hipGetLastError();
    if (err == hipSuccess) return 1;
    fprintf(stderr, "pulsar-kernels: %s: %s\n", what, hipGetErrorString(err));
    return 0;
}

static inline int reject(const char *what) {
    fprintf(stderr, "pulsar-kernels: %s: invalid arguments\n", what);
    return 0;
}

// A pointer read from memory (expert tables) is generic to the compiler;
// this marks it as global memory so loads through it are global loads.
PK_DEV const uint8_t *as_global(const void *p) {
    return (const uint8_t *)(const __attribute__((address_space(1))) uint8_t *)p;
}
PK_DEV const float *as_global_f(const float *p) {
    return (const float *)(const __attribute__((address_space(1))) float *)p;
}

// Makes a register-resident value opaque to the optimiser at this point,
// so work derived from it is not hoisted out of the enclosing loop (keeps
// the register count of pair loops at one decode's worth).
template <typename T>
PK_DEV void opaque(T &v) {
    static_assert(sizeof(T) % 4 == 0, "word-sized members");
    uint32_t w[sizeof(T) / 4];
    __builtin_memcpy(w, &v, sizeof(T));
#pragma unroll
    for (uint32_t i = 0; i < sizeof(T) / 4; i++) asm volatile("" : "+v"(w[i]));
    __builtin_memcpy(&v, w, sizeof(T));
}

// ---------------------------------------------------------------- loads --
// Weight blocks sit at 1/2/4-byte alignment inside rows (MXFP4 17 B,
// Q6_K 210 B, IQ2_XXS 66 B, Q2_K 84 B); gfx950 global loads accept any
// byte alignment, so these compile to single global_load_dword[x2|x4].
PK_DEV uint32_t ld32(const uint8_t *p) {
    uint32_t v;
    __builtin_memcpy(&v, p, 4);
    return v;
}
PK_DEV uint2 ld64(const uint8_t *p) {
    uint2 v;
    __builtin_memcpy(&v, p, 8);
    return v;
}
PK_DEV uint4 ld128(const uint8_t *p) {
    uint4 v;
    __builtin_memcpy(&v, p, 16);
    return v;
}
typedef uint32_t u32x4_u __attribute__((ext_vector_type(4), aligned(1)));
typedef uint32_t u32x2_u __attribute__((ext_vector_type(2), aligned(1)));
typedef uint32_t u32_u __attribute__((aligned(1)));
typedef uint16_t u16_u __attribute__((aligned(1)));
#define PK_GLOBAL __attribute__((address_space(1)))
// Weight loads, any alignment, always from global memory. Expert weight
// pointers are read from pointer tables, so the compiler cannot infer their
// address space: a generic (flat) load would also count against the LDS
// wait counter and make LDS reads wait for HBM. The explicit global address
// space keeps them plain global loads.
PK_DEV uint4 ldw128(const uint8_t *p) {
    const u32x4_u v = *(const PK_GLOBAL u32x4_u *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
PK_DEV uint2 ldw64(const uint8_t *p) {
    const u32x2_u v = *(const PK_GLOBAL u32x2_u *)p;
    return make_uint2(v.x, v.y);
}
PK_DEV uint32_t ldw32(const uint8_t *p) { return *(const PK_GLOBAL u32_u *)p; }
PK_DEV uint16_t ldw16(const uint8_t *p) { return *(const PK_GLOBAL u16_u *)p; }
PK_DEV uint32_t ldw8(const uint8_t *p) { return *(const PK_GLOBAL uint8_t *)p; }
PK_DEV float ldwf(const float *p) { return *(const PK_GLOBAL float *)p; }
#define PK_LDS __attribute__((address_space(3)))
// 16 bytes from LDS at any byte offset: gfx950 DS reads accept unaligned
// addresses (one ds_read_b128).
PK_DEV uint4 lds128u(const uint8_t *p) {
    const u32x4_u v = *(const PK_LDS u32x4_u *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
PK_DEV uint32_t lds8(const uint8_t *p) { return *(const PK_LDS uint8_t *)p; }
PK_DEV uint16_t ld16(const uint8_t *p) {
    uint16_t v;
    __builtin_memcpy(&v, p, 2);
    return v;
}

// Exact f16 -> f32 (v_cvt_f32_f16 is exact for every finite f16).
PK_DEV float f16f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Signed 4 x int8 dot product accumulated into int32 (v_dot4_i32_i8).
PK_DEV int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// --------------------------------------------------------- cross-lane ----
// Partner value for the reduction step that doubles the group size from s
// to 2s lanes (aligned groups). Steps 1 and 2 are quad permutes, 4 and 8
// mirror the half-row / row (lane i <-> 7-i / 15-i: the partner lies in the
// other half of the 2s group, which is all a sum needs), 16 is a ds_swizzle
// xor and 32 a cross-half bpermute.
PK_DEV int32_t partner(int32_t v, uint32_t s) {
    switch (s) {
    case 1: return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);   // quad_perm 1,0,3,2
    case 2: return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);   // quad_perm 2,3,0,1
    case 4: return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);  // row_half_mirror
    case 8: return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);  // row_mirror
    case 16: return __builtin_amdgcn_ds_swizzle(v, 0x401F);                    // xor 16
    default: return __shfl_xor(v, 32, 64);                                     // xor 32
    }
}
PK_DEV float partner(float v, uint32_t s) {
    return __builtin_bit_cast(float, partner(__builtin_bit_cast(int32_t, v), s));
}

// Sum over aligned groups of G lanes (G a power of two <= 64); every lane
// of the group ends with the group total. Integer sums are exact in any
// order; float sums follow this fixed tree.
template <uint32_t G, typename T>
PK_DEV T group_sum(T v) {
#pragma unroll
    for (uint32_t s = 1; s < G; s <<= 1) v += partner(v, s);
    return v;
}

// Same with a run-time group size (uniform across the wave), starting after
// the groups of `from` lanes have already been summed.
template <typename T>
PK_DEV T group_sum_from(T v, uint32_t from, uint32_t g) {
    for (uint32_t s = from; s < g; s <<= 1) v += partner(v, s);
    return v;
}

// Accumulating DPP moves for reductions that end in the LAST lane of each
// group: row_shr:n reads lane i-n of the same 16-lane row (0 where that
// lane is outside the row), row_bcast:15 / :31 add lane 15 / 31 of the
// preceding row(s) into rows 1,3 / 2,3 (the other rows add 0).
template <int N>
PK_DEV float dpp_shr(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int32_t, v),
                                                                 0x110 + N, 0xF, 0xF, true));
}
template <int N>
PK_DEV int32_t dpp_shr(int32_t v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x110 + N, 0xF, 0xF, true);
}
PK_DEV float dpp_bcast15(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int32_t, v),
                                                                 0x142, 0xA, 0xF, false));
}
PK_DEV float dpp_bcast31(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int32_t, v),
                                                                 0x143, 0xC, 0xF, false));
}

PK_DEV int32_t lane_xor(int32_t v, uint32_t m) { return __shfl_xor(v, (int)m, 64); }
PK_DEV float lane_xor(float v, uint32_t m) { return __shfl_xor(v, (int)m, 64); }

PK_DEV float wave_max(float v) {
#pragma unroll
    for (uint32_t m = 1; m < 64; m <<= 1) v = fmaxf(v, lane_xor(v, m));
    return v;
}

// ------------------------------------------------------------ combine --
// Gated combine (pulsar_kernels.cu:124-141 == crates/engine/src/lib.rs:2131-2157):
// op 0 silu(g) * u; op 2 swiglu_oai (gate clamped above at 7, up to +-7,
// sigmoid sharpened by 1.702, up + 1). expf is the device libm's.
PK_DEV float glu(float g, float u, uint32_t op) {
    if (op == 2u) {
        g = fminf(g, 7.0f);
        u = fminf(fmaxf(u, -7.0f), 7.0f);
        return g / (1.0f + expf(-1.702f * g)) * (u + 1.0f);
    }
    return g / (1.0f + expf(-g)) * u;
}

}  // namespace pk
