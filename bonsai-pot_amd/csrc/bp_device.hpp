// Device helpers shared by the gfx950 kernels.
//
// The library is compiled with -ffp-contract=off: every `a * b + c` below is
// two IEEE-rounded operations unless written as __builtin_fmaf. The norm,
// RoPE and quantization stages rely on that to be bit-exact with the CPU
// oracle; the attention kernels ask for FMA explicitly where they want it.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace bp {

__device__ __forceinline__ float h2f(uint16_t x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
}
__device__ __forceinline__ uint16_t f2h(float x) {  // v_cvt_f16_f32: round to nearest even
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Sign-extend byte `i` of a packed word to float (exact).
__device__ __forceinline__ float i8f(uint32_t w, int i) {
    return static_cast<float>(static_cast<int32_t>(w << (24 - 8 * i)) >> 24);
}

}  // namespace bp
