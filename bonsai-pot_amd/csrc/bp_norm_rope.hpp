// Per-head RMSNorm * weight + NEOX RoPE and the Q8_0 quantizer in two forms
// with the same pairing tree, so every path produces the same bits: one
// wavefront per 128-wide head (the fused decode step), and 8 lanes per head
// (the standalone q_norm_rope / kv_writeback kernels and the fused prefill
// step's preparation pass), further down.
//
// Wavefront form: one 64-lane wavefront per 128-wide head, lane j holding the RoPE
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

// Standalone kernels: 8 lanes per (token, head) item, 8 items per wave, 4 waves
// per workgroup. Lane L of an item holds dims 8L .. 8L+7 and their RoPE
// partners 64 + 8L .. 64 + 8L+7, so loads and stores are 16-byte vectors and
// the per-item scalar work (sqrt, the Q8_0 divides) is shared by 8 lanes
// instead of 64. The RMSNorm sum reproduces the pairing tree of the 64-lane
// butterfly exactly: partner j ^ 32 / 16 / 8 is lane L ^ 4 / 2 / 1 at the same
// slot i, partner j ^ 4 / 2 / 1 is slot i ^ 4 / 2 / 1 of the same lane. Each
// Q8_0 block is 4 lanes (block L / 4 for dims 8L.., 2 + L / 4 for 64 + 8L..).
constexpr int kItemLanes = 8;

template <bool kVec>
__device__ __forceinline__ void load8(const uint16_t* p, float* out) {
    if constexpr (kVec) {
        const uint4 w = *reinterpret_cast<const uint4*>(p);
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            out[2 * i] = h2f(static_cast<uint16_t>(u[i]));
            out[2 * i + 1] = h2f(static_cast<uint16_t>(u[i] >> 16));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) out[i] = h2f(p[i]);
    }
}

template <bool kVec>
__device__ __forceinline__ void store8(uint16_t* p, const float* v) {
    if constexpr (kVec) {
        uint32_t u[4];
#pragma unroll
        for (int i = 0; i < 4; i++) u[i] = static_cast<uint32_t>(f2h(v[2 * i])) | (static_cast<uint32_t>(f2h(v[2 * i + 1])) << 16);
        *reinterpret_cast<uint4*>(p) = make_uint4(u[0], u[1], u[2], u[3]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) p[i] = f2h(v[i]);
    }
}

// RMSNorm * w + NEOX RoPE of one item in the 8-lane layout (same operations
// as norm_rope_pair, per slot i): x0 = dims 8L + i, x1 = dims 64 + 8L + i;
// w0 / w1 the weights of those dims, c0 / c1 the 16 f16 (cos, sin) of pairs
// 8L .. 8L+7 (the table row's elements 16L .. 16L+15).
__device__ __forceinline__ void norm_rope8_vals(float* x0, float* x1, const float* w0, const float* w1, uint4 c0,
                                                uint4 c1, float eps) {
    float s[8];
#pragma unroll
    for (int i = 0; i < 8; i++) s[i] = x0[i] * x0[i] + x1[i] * x1[i];
#pragma unroll
    for (int i = 0; i < 8; i++) s[i] = s[i] + lane_xor<4>(s[i]);   // j ^ 32
#pragma unroll
    for (int i = 0; i < 8; i++) s[i] = s[i] + lane_xor<2>(s[i]);   // j ^ 16
#pragma unroll
    for (int i = 0; i < 8; i++) s[i] = s[i] + lane_xor<1>(s[i]);   // j ^ 8
    const float t0 = s[0] + s[4], t1 = s[1] + s[5], t2 = s[2] + s[6], t3 = s[3] + s[7];   // j ^ 4
    const float sq = (t0 + t2) + (t1 + t3);                                                 // j ^ 2, j ^ 1
    const float inv_h = 1.0f / sqrtf(sq / 128.0f + eps);
    const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float c = h2f(static_cast<uint16_t>(cw[i])), sn = h2f(static_cast<uint16_t>(cw[i] >> 16));
        const float n0 = x0[i] * inv_h * w0[i];
        const float n1 = x1[i] * inv_h * w1[i];
        x0[i] = n0 * c - n1 * sn;   // kv_writeback_fused.wgsl:102
        x1[i] = n0 * sn + n1 * c;   // kv_writeback_fused.wgsl:107
    }
}

// The same with the weights and the table row loaded here.
template <bool kVec>
__device__ __forceinline__ void norm_rope8(float* x0, float* x1, const uint16_t* w, const uint16_t* cs_row,
                                           int L, float eps) {
    float w0[8], w1[8];
    load8<kVec>(w + 8 * L, w0);
    load8<kVec>(w + 64 + 8 * L, w1);
    // cos/sin of pairs 8L .. 8L+7: 16 consecutive f16 of the table row.
    const uint4 c0 = *reinterpret_cast<const uint4*>(cs_row + 16 * L);
    const uint4 c1 = *reinterpret_cast<const uint4*>(cs_row + 16 * L + 8);
    norm_rope8_vals(x0, x1, w0, w1, c0, c1, eps);
}

// Eight f16 (one 16-byte word) -> f32.
__device__ __forceinline__ void unpack8(uint4 w, float* out) {
    const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        out[2 * i] = h2f(static_cast<uint16_t>(u[i]));
        out[2 * i + 1] = h2f(static_cast<uint16_t>(u[i] >> 16));
    }
}

// Q8_0 of the 8 values of one lane and its block (kv_writeback_fused.wgsl:118-200).
__device__ __forceinline__ float quantize8(const float* x, uint2& packed) {
    float a = fabsf(x[0]);
#pragma unroll
    for (int i = 1; i < 8; i++) a = fmaxf(a, fabsf(x[i]));
    a = fmaxf(a, lane_xor<1>(a));
    a = fmaxf(a, lane_xor<2>(a));
    const float d = a / 127.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
        b[i] = static_cast<uint32_t>(static_cast<int>(fminf(fmaxf(rintf(x[i] * inv), -127.0f), 127.0f))) & 0xffu;
    packed.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    packed.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    return d;
}

}  // namespace bp
