// Measurement references, linked only into the bench build of the library
// (not part of the attention path):
//  * read_floor_kernel: reads every 16-byte word of a device buffer once
//    (grid-stride, all loads independent) and folds them into one word per
//    workgroup, so the compiler keeps every load. bench.py times it over
//    buffers of a decode's byte count to give the read floor the decode
//    kernels are compared with.
//  * mfma_rate_kernel: back-to-back v_mfma_f32_32x32x16_f16 on random f16
//    operands, four independent accumulators per wave. bench.py times it as
//    the f16 matrix rate the chip sustains on real data (random operands draw
//    more power than constant ones and run at a lower clock), beside the
//    nominal peak the prefill roofline is priced against.
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

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfma_rate_kernel(float* sink, uint32_t iters, uint32_t seed) {
    // Per-lane xorshift: operands uniform in [-2, 2), different in every lane.
    uint32_t x = (blockIdx.x * 256u + threadIdx.x) * 2654435761u + seed * 40503u + 1u;
    f16x8 a, b;
    for (int e = 0; e < 8; e++) {
        x ^= x << 13; x ^= x >> 17; x ^= x << 5;
        a[e] = static_cast<_Float16>(static_cast<float>(static_cast<int>(x & 0xFFFFu) - 32768) * (1.0f / 16384.0f));
        x ^= x << 13; x ^= x >> 17; x ^= x << 5;
        b[e] = static_cast<_Float16>(static_cast<float>(static_cast<int>(x & 0xFFFFu) - 32768) * (1.0f / 16384.0f));
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (uint32_t it = 0; it < iters; it++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(b, b, c3, 0, 0, 0);
    }
    float t = 0.0f;
    for (int i = 0; i < 16; i++) t += (c0[i] + c1[i]) + (c2[i] + c3[i]);
    sink[blockIdx.x * 256u + threadIdx.x] = t;
}

}  // namespace

extern "C" bp_status bp_debug_mfma_rate(void* sink, uint32_t iters, uint32_t n_workgroups, uint32_t seed,
                                        void* stream) {
    if (!sink || n_workgroups == 0 || iters == 0) return BP_ERR_INVALID_ARG;
    hipLaunchKernelGGL(mfma_rate_kernel, dim3(n_workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<float*>(sink), iters, seed);
    return hipGetLastError() == hipSuccess ? BP_OK : BP_ERR_HIP;
}

extern "C" bp_status bp_debug_read_floor(const void* src, uint64_t bytes, void* sink, uint32_t n_workgroups,
                                         void* stream) {
    if (!src || !sink || n_workgroups == 0 || (reinterpret_cast<uintptr_t>(src) & 15u))
        return BP_ERR_INVALID_ARG;
    hipLaunchKernelGGL(read_floor_kernel, dim3(n_workgroups), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4*>(src), bytes / 16, static_cast<uint32_t*>(sink));
    return hipGetLastError() == hipSuccess ? BP_OK : BP_ERR_HIP;
}
