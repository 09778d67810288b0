// Streaming-read reference for measurements: reads every 16-byte word of a
// device buffer once (grid-stride, all loads independent) and folds them into
// one word per workgroup, so the compiler keeps every load. bench.py times it
// over buffers of a decode's byte count to give the read floor the decode
// kernels are compared with. Not part of the attention path: linked only
// into the bench build of the library.
#include <hip/hip_runtime.h>
#include <cstdint>

#include "../../include/bonsai_pot_hip_bench.h"

namespace {

__global__ __launch_bounds__(256) void read_floor_kernel(const uint4* src, uint64_t n16, uint32_t* sink) {
    uint32_t acc = 0;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    // Four loads in flight per thread per step.
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
        acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
    }
    for (; i < n16; i += stride) {
        const uint4 a = src[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    __shared__ uint32_t red[256];
    red[threadIdx.x] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int k = 0; k < 256; k++) t ^= red[k];
        sink[blockIdx.x] = t;
    }
}

}  // namespace

extern "C" bp_status bp_debug_read_floor(const void* src, uint64_t bytes, void* sink, uint32_t n_workgroups,
                                         void* stream) {
    if (!src || !sink || n_workgroups == 0 || (reinterpret_cast<uintptr_t>(src) & 15u))
        return BP_ERR_INVALID_ARG;
    hipLaunchKernelGGL(read_floor_kernel, dim3(n_workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(src), bytes / 16, static_cast<uint32_t*>(sink));
    return hipGetLastError() == hipSuccess ? BP_OK : BP_ERR_HIP;
}
