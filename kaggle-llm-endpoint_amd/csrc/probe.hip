// Streaming-read probe (measurement only; no counterpart in the reference): the practical HBM read rate of this part
// for a plain stream, the ceiling the weight-streaming kernels are compared against.  Every thread reads 16-byte
// pieces in a grid-stride loop (one wavefront instruction = 1 KB contiguous), four loads in flight per thread, and
// folds them with XOR; one word per wavefront is written so that no load is dead.
//
// Built into its own library, libmi355probe.so, which only the benchmark and its test load: it is not part of the
// operator's C ABI (include/mi355moe.h), whose status codes it shares.
#include <hip/hip_runtime.h>

#include "mi355moe.h"

// Reads `bytes` (a multiple of 16) from src with 16-byte loads in a grid-stride loop of `workgroups` 256-thread
// workgroups and writes one XOR word per wavefront to sink (workgroups * 4 u32).
extern "C" int mi_read_probe(const void *src, size_t bytes, uint32_t *sink, int32_t workgroups, void *stream);

namespace mi {

__device__ __forceinline__ uint32_t fold(uint4 v) { return v.x ^ v.y ^ v.z ^ v.w; }

__global__ void __launch_bounds__(256) read_probe_kernel(const uint4 *__restrict__ src, size_t n16,
                                                         uint32_t *__restrict__ sink) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
        acc ^= fold(a) ^ fold(b) ^ fold(c) ^ fold(d);
    }
    for (; i < n16; i += stride) acc ^= fold(src[i]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc ^= __shfl_xor(acc, o, 64);
    if ((threadIdx.x & 63) == 0) sink[blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64] = acc;
}

}  // namespace mi

extern "C" int mi_read_probe(const void *src, size_t bytes, uint32_t *sink, int32_t workgroups, void *stream) {
    if (!src || !sink) return MI_ERR_NULL;
    if (bytes == 0 || bytes % 16 || (uintptr_t)src % 16 || workgroups <= 0 || workgroups > (1 << 20)) return MI_ERR_ARG;
    hipLaunchKernelGGL(mi::read_probe_kernel, dim3(workgroups), dim3(256), 0, (hipStream_t)stream,
                       (const uint4 *)src, bytes / 16, sink);
    return hipGetLastError() == hipSuccess ? MI_OK : MI_ERR_LAUNCH;
}
