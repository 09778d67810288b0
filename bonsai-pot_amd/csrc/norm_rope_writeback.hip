// Q-side norm+RoPE and K/V writeback into the Q8_0 cache, for gfx950.
//
// Restates src/shaders/q_norm_rope_fused.wgsl and
// src/shaders/kv_writeback_fused.wgsl (reference repository) with a
// wave64-native layout: ONE wavefront per (head, token), 4 per workgroup,
// lane j holding the RoPE pair (x[j], x[j+64]). The pair partner therefore lives in the same
// lane (no LDS round trip), the 128-element sum of squares is a 6-step xor
// butterfly, and each 32-element Q8_0 block is one 32-lane half of the wave
// (blocks 0/2 in lanes 0-31, blocks 1/3 in lanes 32-63).
//
// Bit-exactness. Every f32 operation is one IEEE-rounded op in the order of
// the reference shader (no contraction, correctly rounded sqrt and divide),
// and the RMSNorm reduction uses the fixed butterfly order
//   s_j = x_j*x_j + x_{j+64}*x_{j+64};  s += shfl_xor(s, 32, 16, 8, 4, 2, 1)
// so cache bytes and f16 outputs match the CPU oracle bit for bit.
#include "bp_kernels.hpp"
#include "bp_norm_rope.hpp"

namespace bp {
namespace {

// 4 waves per workgroup: wave w takes item 4 blockIdx.x + w of the
// m_tokens x n_head (token-major) grid.
__global__ __launch_bounds__(256) void q_norm_rope_kernel(QNormRopeArgs a) {
    const int j = threadIdx.x & 63;
    const uint32_t it = 4 * blockIdx.x + (threadIdx.x >> 6);
    if (it >= a.n_items) return;
    const uint32_t head = it % a.n_head, tok = it / a.n_head;
    uint16_t* q = a.act + a.q_off + static_cast<uint64_t>(tok) * a.q_dim + head * kHeadDim;
    const uint16_t* cs = a.rope_cs + static_cast<uint64_t>(a.pos_base + tok) * kHeadDim + 2 * j;
    float o0, o1;
    norm_rope_pair(h2f(q[j]), h2f(q[j + 64]), h2f(a.w_norms[a.w_off + j]),
                   h2f(a.w_norms[a.w_off + j + 64]), h2f(cs[0]), h2f(cs[1]), a.eps, o0, o1);
    q[j] = f2h(o0);          // q_norm_rope_fused.wgsl:95
    q[j + 64] = f2h(o1);
}

// 4 waves per workgroup: wave w takes (token, KV head) pair 4 blockIdx.x + w
// (token-major).
__global__ __launch_bounds__(256) void kv_writeback_kernel(KvWritebackArgs a) {
    const int j = threadIdx.x & 63;
    const uint32_t pr = 4 * blockIdx.x + (threadIdx.x >> 6);
    if (pr >= a.n_pairs) return;
    const uint32_t head = pr % a.n_kv_head, tok = pr / a.n_kv_head;
    const uint64_t tok_off = static_cast<uint64_t>(tok) * a.kv_dim + head * kHeadDim;
    const uint16_t* k = a.act + a.k_cur_off + tok_off;
    const uint16_t* v = a.act + a.v_cur_off + tok_off;
    const uint64_t row = static_cast<uint64_t>(a.pos_base) + tok;
    const uint16_t* cs = a.rope_cs + row * kHeadDim + 2 * j;
    float k0, k1;
    norm_rope_pair(h2f(k[j]), h2f(k[j + 64]), h2f(a.w_norms[a.w_off + j]),
                   h2f(a.w_norms[a.w_off + j + 64]), h2f(cs[0]), h2f(cs[1]), a.eps, k0, k1);
    const uint64_t nb_row = a.kv_dim / kBlock;
    const uint64_t d_idx = row * nb_row + head * (kHeadDim / kBlock);
    const uint64_t qs_idx = row * a.kv_dim + head * kHeadDim;
    quantize_store_pair(k0, k1, j, a.k_d + d_idx, a.k_qs + qs_idx);
    quantize_store_pair(h2f(v[j]), h2f(v[j + 64]), j, a.v_d + d_idx, a.v_qs + qs_idx);
}

}  // namespace

hipError_t launch_q_norm_rope(const QNormRopeArgs& a, uint32_t n_head, uint32_t m_tokens,
                              hipStream_t s) {
    QNormRopeArgs b = a;
    b.n_head = n_head;
    b.n_items = n_head * m_tokens;
    hipLaunchKernelGGL(q_norm_rope_kernel, dim3((b.n_items + 3) / 4), dim3(256), 0, s, b);
    return hipGetLastError();
}

hipError_t launch_kv_writeback(const KvWritebackArgs& a, uint32_t n_kv_head, uint32_t m_tokens,
                               hipStream_t s) {
    KvWritebackArgs b = a;
    b.n_kv_head = n_kv_head;
    b.n_pairs = n_kv_head * m_tokens;
    hipLaunchKernelGGL(kv_writeback_kernel, dim3((b.n_pairs + 3) / 4), dim3(256), 0, s, b);
    return hipGetLastError();
}

}  // namespace bp
