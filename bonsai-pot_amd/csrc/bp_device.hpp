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


// Lane exchanges across 16- and 32-lane rows without LDS: v_permlane16_swap /
// v_permlane32_swap of a register with itself leave, in every lane, the pair
// {v[l], v[l ^ 16]} (resp. {v[l], v[l ^ 32]}) in the two results, in an order
// that depends on the row; max and sum of the pair do not depend on it.
// (The results are copied to scalars before the bit casts: a bit cast of a
// vector element directly is miscompiled to element 0.)
struct LanePair { float a, b; };
__device__ __forceinline__ LanePair xchg16(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return {__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1)};
}
__device__ __forceinline__ LanePair xchg32(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return {__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1)};
}
// IEEE-754-2019 maximum (NaN-propagating): lowers to v_maximum(3)_f32 with no
// input canonicalization, where fmaxf (maxNum) first quiets each operand with
// an extra v_max_f32 x, x, x when the compiler cannot prove it canonical (an
// MFMA result or a lane exchange). Differs from fmaxf only for NaN inputs.
__device__ __forceinline__ float fmax_p(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max_xor16(float v) { const LanePair p = xchg16(v); return fmax_p(p.a, p.b); }
__device__ __forceinline__ float max_xor32(float v) { const LanePair p = xchg32(v); return fmax_p(p.a, p.b); }
__device__ __forceinline__ float sum_xor16(float v) { const LanePair p = xchg16(v); return p.a + p.b; }
__device__ __forceinline__ float sum_xor32(float v) { const LanePair p = xchg32(v); return p.a + p.b; }

// Value of lane (lane ^ S) for S = 1, 2, 4, 8 by DPP lane moves (quad
// permutes; half-row mirror + quad permute; row rotation by 8), by a lane
// permute through the LDS crossbar otherwise. Pure data movement, so
// reductions keep their exact pairing order.
template <int S>
__device__ __forceinline__ uint32_t lane_xor(uint32_t v) {
    const int x = static_cast<int>(v);
    if constexpr (S == 1) return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false));
    else if constexpr (S == 2) return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false));
    else if constexpr (S == 4) {
        const int m = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);   // lane ^ 7 (half-row mirror)
        return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, m, 0x1B, 0xF, 0xF, false));   // then ^ 3
    } else if constexpr (S == 8) return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, false));
    else return static_cast<uint32_t>(__shfl_xor(x, S));
}
template <int S>
__device__ __forceinline__ float lane_xor(float v) {
    return __builtin_bit_cast(float, lane_xor<S>(__builtin_bit_cast(uint32_t, v)));
}

// Butterfly reductions over the wave (partners lane ^ 32, ^ 16, .., ^ 1, so
// every lane ends with the same value): row exchanges by v_permlane32/16_swap
// and DPP lane moves, no LDS round trip per step.
__device__ __forceinline__ float wave_max(float v) {
    LanePair p = xchg32(v);
    v = fmaxf(p.a, p.b);
    p = xchg16(v);
    v = fmaxf(p.a, p.b);
    v = fmaxf(v, lane_xor<8>(v));
    v = fmaxf(v, lane_xor<4>(v));
    v = fmaxf(v, lane_xor<2>(v));
    return fmaxf(v, lane_xor<1>(v));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = sum_xor16(sum_xor32(v));
    v += lane_xor<8>(v);
    v += lane_xor<4>(v);
    v += lane_xor<2>(v);
    return v + lane_xor<1>(v);
}
// Value of lane 4 (lane / 4) + K (a quad broadcast).
template <int K>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), K | (K << 2) | (K << 4) | (K << 6),
                                                             0xF, 0xF, false));
}

// Sign-extend byte `i` of a packed word to float (exact).
__device__ __forceinline__ float i8f(uint32_t w, int i) {
    return static_cast<float>(static_cast<int32_t>(w << (24 - 8 * i)) >> 24);
}

}  // namespace bp
