// Q-side norm+RoPE and K/V writeback into the Q8_0 cache, for gfx950.
//
// Restates src/shaders/q_norm_rope_fused.wgsl and
// src/shaders/kv_writeback_fused.wgsl (reference repository). Layout: 8 lanes
// per (token, head) item, 8 items per wavefront (kItemLanes, bp_norm_rope.hpp); the
// fused decode step keeps the one-wave-per-item form of bp_norm_rope.hpp.
//
// Bit-exactness. Every f32 operation is one IEEE-rounded op in the order of
// the reference shader (no contraction, correctly rounded sqrt and divide),
// and the RMSNorm reduction uses the fixed pairing tree
//   s_j = x_j*x_j + x_{j+64}*x_{j+64};  s += partner j ^ 32, 16, 8, 4, 2, 1
// (the 64-lane xor butterfly of bp_norm_rope.hpp), so cache bytes and f16
// outputs match the CPU oracle, and the fused decode path, bit for bit.
#include "bp_kernels.hpp"
#include "bp_norm_rope.hpp"

namespace bp {
namespace {

__device__ __forceinline__ void quantize_store8(const float* x0, const float* x1, int L, float* d_row, int8_t* qs_row) {
    uint2 p0, p1;
    const float d0 = quantize8(x0, p0), d1 = quantize8(x1, p1);
    *reinterpret_cast<uint2*>(qs_row + 8 * L) = p0;
    *reinterpret_cast<uint2*>(qs_row + 64 + 8 * L) = p1;
    if ((L & 3) == 0) {
        d_row[L >> 2] = d0;        // elements [32 (L / 4), +32)
        d_row[2 + (L >> 2)] = d1;  // elements [64 + 32 (L / 4), +32)
    }
}

// (token, head) of item i: shift and mask when the head count is a power of
// two (a uniform branch), else an integer division.
__device__ __forceinline__ void divmod_heads(uint32_t i, uint32_t n, uint32_t shift, uint32_t& tok, uint32_t& head) {
    if (shift < 32) {
        tok = i >> shift;
        head = i & (n - 1);
    } else {
        tok = i / n;
        head = i % n;
    }
}
static uint32_t head_shift_of(uint32_t n) {
    return n != 0 && (n & (n - 1)) == 0 ? static_cast<uint32_t>(__builtin_ctz(n)) : 32u;
}

// Item it = 8 (4 blockIdx.x + wave) + lane / 8 of the m_tokens x n_head
// (token-major) grid. Items past the end compute on a clamped item and store
// nothing (the lane exchanges need every lane of the 8-lane group).
template <bool kVec>
__global__ __launch_bounds__(256) void q_norm_rope_kernel(QNormRopeArgs a) {
    const int lane = threadIdx.x & 63, L = lane & (kItemLanes - 1);
    const uint32_t it_raw = kItemLanes * (4 * blockIdx.x + (threadIdx.x >> 6)) + (lane >> 3);
    const bool live = it_raw < a.n_items;
    const uint32_t it = live ? it_raw : a.n_items - 1;
    uint32_t head, tok;
    divmod_heads(it, a.n_head, a.head_shift, tok, head);
    uint16_t* q = a.act + a.q_off + static_cast<uint64_t>(tok) * a.q_dim + head * kHeadDim;
    float x0[8], x1[8];
    load8<kVec>(q + 8 * L, x0);
    load8<kVec>(q + 64 + 8 * L, x1);
    norm_rope8<kVec>(x0, x1, a.w_norms + a.w_off, a.rope_cs + static_cast<uint64_t>(a.pos_base + tok) * kHeadDim, L,
                     a.eps);
    if (live) {
        store8<kVec>(q + 8 * L, x0);   // q_norm_rope_fused.wgsl:95
        store8<kVec>(q + 64 + 8 * L, x1);
    }
}

// Item = (token, KV head) pair, same numbering as above: K gets norm + RoPE +
// Q8_0, V Q8_0 only.
template <bool kVec>
__global__ __launch_bounds__(256) void kv_writeback_kernel(KvWritebackArgs a) {
    const int lane = threadIdx.x & 63, L = lane & (kItemLanes - 1);
    const uint32_t pr_raw = kItemLanes * (4 * blockIdx.x + (threadIdx.x >> 6)) + (lane >> 3);
    const bool live = pr_raw < a.n_pairs;
    const uint32_t pr = live ? pr_raw : a.n_pairs - 1;
    uint32_t head, tok;
    divmod_heads(pr, a.n_kv_head, a.head_shift, tok, head);
    const uint64_t tok_off = static_cast<uint64_t>(tok) * a.kv_dim + head * kHeadDim;
    const uint16_t* k = a.act + a.k_cur_off + tok_off;
    const uint16_t* v = a.act + a.v_cur_off + tok_off;
    const uint64_t row = static_cast<uint64_t>(a.pos_base) + tok;
    float k0[8], k1[8], v0[8], v1[8];
    load8<kVec>(k + 8 * L, k0);
    load8<kVec>(k + 64 + 8 * L, k1);
    load8<kVec>(v + 8 * L, v0);
    load8<kVec>(v + 64 + 8 * L, v1);
    norm_rope8<kVec>(k0, k1, a.w_norms + a.w_off, a.rope_cs + row * kHeadDim, L, a.eps);
    const uint64_t nb_row = a.kv_dim / kBlock;
    const uint64_t d_idx = row * nb_row + head * (kHeadDim / kBlock);
    const uint64_t qs_idx = row * a.kv_dim + head * kHeadDim;
    uint2 pk0, pk1, pv0, pv1;
    const float dk0 = quantize8(k0, pk0), dk1 = quantize8(k1, pk1);
    const float dv0 = quantize8(v0, pv0), dv1 = quantize8(v1, pv1);
    if (live) {
        *reinterpret_cast<uint2*>(a.k_qs + qs_idx + 8 * L) = pk0;
        *reinterpret_cast<uint2*>(a.k_qs + qs_idx + 64 + 8 * L) = pk1;
        *reinterpret_cast<uint2*>(a.v_qs + qs_idx + 8 * L) = pv0;
        *reinterpret_cast<uint2*>(a.v_qs + qs_idx + 64 + 8 * L) = pv1;
        if ((L & 3) == 0) {
            a.k_d[d_idx + (L >> 2)] = dk0;
            a.k_d[d_idx + 2 + (L >> 2)] = dk1;
            a.v_d[d_idx + (L >> 2)] = dv0;
            a.v_d[d_idx + 2 + (L >> 2)] = dv1;
        }
    }
}

}  // namespace

hipError_t launch_q_norm_rope(const QNormRopeArgs& a, uint32_t n_head, uint32_t m_tokens,
                              hipStream_t s) {
    QNormRopeArgs b = a;
    b.n_head = n_head;
    b.n_items = n_head * m_tokens;
    b.head_shift = head_shift_of(n_head);
    const dim3 grid((b.n_items + 4 * kItemLanes - 1) / (4 * kItemLanes));
    // 16-byte vectors when the caller's offsets allow them.
    if ((b.q_off | b.w_off | b.q_dim) % 8 == 0 && reinterpret_cast<uintptr_t>(b.act) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(b.w_norms) % 16 == 0)
        hipLaunchKernelGGL(q_norm_rope_kernel<true>, grid, dim3(256), 0, s, b);
    else
        hipLaunchKernelGGL(q_norm_rope_kernel<false>, grid, dim3(256), 0, s, b);
    return hipGetLastError();
}

hipError_t launch_kv_writeback(const KvWritebackArgs& a, uint32_t n_kv_head, uint32_t m_tokens,
                               hipStream_t s) {
    KvWritebackArgs b = a;
    b.n_kv_head = n_kv_head;
    b.n_pairs = n_kv_head * m_tokens;
    b.head_shift = head_shift_of(n_kv_head);
    const dim3 grid((b.n_pairs + 4 * kItemLanes - 1) / (4 * kItemLanes));
    if ((b.k_cur_off | b.v_cur_off | b.w_off) % 8 == 0 && reinterpret_cast<uintptr_t>(b.act) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(b.w_norms) % 16 == 0)
        hipLaunchKernelGGL(kv_writeback_kernel<true>, grid, dim3(256), 0, s, b);
    else
        hipLaunchKernelGGL(kv_writeback_kernel<false>, grid, dim3(256), 0, s, b);
    return hipGetLastError();
}

}  // namespace bp
