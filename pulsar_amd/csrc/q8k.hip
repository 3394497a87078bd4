// q8k.hip - f32 -> q8_K activation quantizer and the streaming-read probe.
#include "pk_common.h"

namespace pk {

static thread_local hipStream_t g_stream = nullptr;
hipStream_t stream() { return g_stream; }

// One wave per 256-value block; lane l owns values 4l .. 4l+3.
// Algorithm of the CPU lane (crates/quant/src/cpu_dot.rs:26-50):
//   amax = max |x|; amax == 0 -> d = 0, all quants 0;
//   d = amax / 127, inv = 127 / amax (IEEE division, correctly rounded),
//   q = clamp(round_half_away(x * inv), -127, 127), bsums = sums of 16.
// Values past in_dim in the tail block are 0 (pulsar_kernels.cu:1499-1501).
__global__ __launch_bounds__(256) void quantize_q8k_kernel(pulsar_block_q8_K *__restrict__ out,
                                                           const float *__restrict__ x,
                                                           uint32_t in_dim, uint32_t nb,
                                                           uint64_t n_blocks) {
    const uint64_t gblk = (uint64_t)blockIdx.x * (blockDim.x / 64u) + threadIdx.x / 64u;
    if (gblk >= n_blocks) return;  // whole wave
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t row = gblk / nb;
    const uint32_t b = (uint32_t)(gblk - row * nb);
    const uint32_t c0 = b * 256u + 4u * lane;
    const float *xr = x + row * in_dim;
    float v[4];
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
    float am = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    am = wave_max(am);
    uint8_t *ob = (uint8_t *)(out + gblk);
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
    *(uint32_t *)(ob + 4 + 4 * lane) = packed;
    s4 = group_sum<4>(s4);
    if ((lane & 3u) == 0u) *(int16_t *)(ob + 260 + 2 * (lane >> 2)) = (int16_t)s4;
    if (lane == 0) *(float *)ob = d;
}

// Streaming read through the CUs (pulsar_kernels.cu:4875-4893): every
// lane folds 16-byte loads; the sink is written only if the fold hits an
// impossible value, which keeps the loads alive.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void bw_read_kernel(const u32x4 *__restrict__ p, uint64_t n16,
                                                      float *sink) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(&p[i]);
        acc ^= v.x + v.y + v.z + v.w;
    }
    if (acc == 0x9e3779b9u) sink[0] = (float)acc;  // practically never; the sink stays valid
}

}  // namespace pk

extern "C" int pulsar_quantize_q8_K(void *out, const void *x, uint32_t in_dim, uint32_t n_rows) {
    if (!out || !x || in_dim == 0 || n_rows == 0) return pk::reject("q8_K quantize");
    const uint32_t nb = (in_dim + 255u) / 256u;
    const uint64_t n_blocks = (uint64_t)nb * n_rows;
    const uint64_t grid = (n_blocks + 3u) / 4u;
    if (grid > 0x7fffffffull) return pk::reject("q8_K quantize");
    hipLaunchKernelGGL(pk::quantize_q8k_kernel, dim3((uint32_t)grid), dim3(256), 0, pk::stream(),
                       (pulsar_block_q8_K *)out, (const float *)x, in_dim, nb, n_blocks);
    return pk::launch_ok("q8_K quantize launch");
}

extern "C" int pulsar_bw_read(void *buf, uint64_t bytes, void *sink) {
    if (!buf || !sink || bytes < 16) return pk::reject("bw_read");
    hipLaunchKernelGGL(pk::bw_read_kernel, dim3(4096), dim3(256), 0, pk::stream(), (const pk::u32x4 *)buf,
                       bytes / 16u, (float *)sink);
    return pk::launch_ok("bw_read launch");
}

extern "C" int pulsar_set_stream(void *stream) {
    pk::g_stream = (hipStream_t)stream;
    return 1;
}
