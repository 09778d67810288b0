// Per-head RMSNorm * weight + NEOX RoPE and the Q8_0 quantizer in the
// one-wave-per-head form used by the fused decode step. The standalone
// q_norm_rope / kv_writeback kernels (norm_rope_writeback.hip) run 8 lanes per
// head with the same pairing tree, so every path produces the same bits.
//
// Layout: one 64-lane wavefront per 128-wide head, lane j holding the RoPE
// pair (x[j], x[j+64]); the lane exchanges of strides 1-8 are DPP moves. Every f32 operation is one IEEE-rounded op in the
// order of the reference shaders (src/shaders/q_norm_rope_fused.wgsl,
// src/shaders/kv_writeback_fused.wgsl in the reference repository): the
// library is built with -ffp-contract=off, sqrt and divide are correctly
// rounded, and the RMSNorm sum uses the fixed butterfly
//   s_j = x_j*x_j + x_{j+64}*x_{j+64};  s += shfl_xor(s, 32, 16, 8, 4, 2, 1).
#pragma once

#include "bp_device.hpp"

namespace bp {

// RMSNorm(x) * w followed by NEOX RoPE, for the pair (x0 = x[j], x1 = x[j+64]).
// q_norm_rope_fused.wgsl:53-93 / kv_writeback_fused.wgsl:69-108.
__device__ __forceinline__ void norm_rope_pair(float x0, float x1, float w0, float w1, float c,
                                               float s, float eps, float& o0, float& o1) {
    float sq = x0 * x0 + x1 * x1;
    sq = sq + lane_xor<32>(sq);
    sq = sq + lane_xor<16>(sq);
    sq = sq + lane_xor<8>(sq);
    sq = sq + lane_xor<4>(sq);
    sq = sq + lane_xor<2>(sq);
    sq = sq + lane_xor<1>(sq);
    float inv_h = 1.0f / sqrtf(sq / 128.0f + eps);
    float n0 = x0 * inv_h * w0;
    float n1 = x1 * inv_h * w1;
    o0 = n0 * c - n1 * s;   // kv_writeback_fused.wgsl:102
    o1 = n0 * s + n1 * c;   // kv_writeback_fused.wgsl:107
}

// Q8_0-quantize the pair and store it; lanes 0-31 own blocks 0 and 2, lanes
// 32-63 blocks 1 and 3 (kv_writeback_fused.wgsl:118-200).
__device__ __forceinline__ void quantize_store_pair(float x0, float x1, int lane, float* d_row,
                                                    int8_t* qs_row) {
    float a0 = fabsf(x0), a1 = fabsf(x1);
    a0 = fmaxf(a0, lane_xor<1>(a0)); a1 = fmaxf(a1, lane_xor<1>(a1));
    a0 = fmaxf(a0, lane_xor<2>(a0)); a1 = fmaxf(a1, lane_xor<2>(a1));
    a0 = fmaxf(a0, lane_xor<4>(a0)); a1 = fmaxf(a1, lane_xor<4>(a1));
    a0 = fmaxf(a0, lane_xor<8>(a0)); a1 = fmaxf(a1, lane_xor<8>(a1));
    a0 = fmaxf(a0, lane_xor<16>(a0)); a1 = fmaxf(a1, lane_xor<16>(a1));
    float d0 = a0 / 127.0f, d1 = a1 / 127.0f;
    float i0 = d0 > 0.0f ? 1.0f / d0 : 0.0f;
    float i1 = d1 > 0.0f ? 1.0f / d1 : 0.0f;
    int q0 = static_cast<int>(fminf(fmaxf(rintf(x0 * i0), -127.0f), 127.0f));
    int q1 = static_cast<int>(fminf(fmaxf(rintf(x1 * i1), -127.0f), 127.0f));
    // Gather 4 consecutive lanes' bytes into one little-endian word.
    uint32_t p = (static_cast<uint32_t>(q0) & 0xffu) | ((static_cast<uint32_t>(q1) & 0xffu) << 8);
    const uint32_t p0 = quad_bcast<0>(p), p1 = quad_bcast<1>(p), p2 = quad_bcast<2>(p), p3 = quad_bcast<3>(p);
    if ((lane & 3) == 0) {
        uint32_t lo = (p0 & 0xffu) | ((p1 & 0xffu) << 8) | ((p2 & 0xffu) << 16) | ((p3 & 0xffu) << 24);
        uint32_t hi = (p0 >> 8) | ((p1 >> 8) << 8) | ((p2 >> 8) << 16) | ((p3 >> 8) << 24);
        *reinterpret_cast<uint32_t*>(qs_row + lane) = lo;
        *reinterpret_cast<uint32_t*>(qs_row + 64 + lane) = hi;
    }
    if ((lane & 31) == 0) {
        int blk = lane >> 5;          // 0 or 1
        d_row[blk] = d0;              // elements [32*blk, 32*blk+32)
        d_row[blk + 2] = d1;          // elements [64+32*blk, ...)
    }
}

}  // namespace bp
