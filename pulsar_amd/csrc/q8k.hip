// q8k.hip - f32 -> q8_K activation quantizer and the streaming-read probe.
#include "pk_q8k.h"

namespace pk {

// The calling thread's per-thread default stream unless pulsar_set_stream
// chose another: the reference builds with --default-stream=per-thread
// (crates/kernels/build.rs:42-48), so its launches land on
// cudaStreamPerThread, where Graph::capture records them
// (crates/kernels/src/lib.rs:755-790).
static thread_local hipStream_t g_stream = hipStreamPerThread;
hipStream_t stream() { return g_stream; }

// One wave per 256-value block (quantize_block_wave).
__global__ __launch_bounds__(256) void quantize_q8k_kernel(pulsar_block_q8_K *__restrict__ out,
                                                           const float *__restrict__ x,
                                                           uint32_t in_dim, uint32_t nb,
                                                           uint64_t n_blocks) {
    const uint64_t gblk = (uint64_t)blockIdx.x * (blockDim.x / 64u) + threadIdx.x / 64u;
    if (gblk >= n_blocks) return;  // whole wave
    const uint64_t row = gblk / nb;
    const uint32_t b = (uint32_t)(gblk - row * nb);
    quantize_block_wave<4u, 260u>(x + row * in_dim, in_dim, b, (uint8_t *)(out + gblk));
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
    pk::g_stream = stream ? (hipStream_t)stream : hipStreamPerThread;
    return 1;
}
