// Q1_0 decode matvecs (gfx950): y = W x with 1-bit weights, one f16 scale per
// 128-weight block. Same results as src/shaders/matvec_q1_0.wgsl,
// matvec_q1_0_silu.wgsl and matvec_q1_0_fused_normed.wgsl (reference
// repository), bit for bit wherever the reference fixes the arithmetic:
//
//  * Weight tensor layout (byte offsets into the weight buffer): d[n][nb] f16
//    at d_offset, qs[n][nb][16] at qs_offset (4-byte aligned); bit e of a
//    block's 128-bit little-endian qs selects +x[e] (1) or -x[e] (0).
//  * Per (row, block): four f16 accumulators (component c = e mod 4, elements
//    in increasing order), block sum ((c0 + c1) + c2) + c3 in f16, then in f32
//    acc_t = acc_t + d * sum for the row's lane t = block mod 8 (blocks in
//    increasing order), and the 8 lane sums combined by the xor 1, 2, 4
//    butterfly (matvec_q1_0.wgsl:93-123).
//
// Layout here: one wave = 8 rows x 8 block-lanes, a 256-thread workgroup 32
// rows. x (the staged activation: plain, silu(gate) * up, or RMS-normed) sits
// in LDS as f16, each 128-element block padded by 8 halves so that the 8
// block-lanes of a wave read 8 different bank groups.
//
// Inner loop: a sign bit becomes the f16 multiplier +-1 with one v_perm_b32
// per two elements, from 8 pre-shifted copies of the inverted qs word whose
// bytes are 0x3C | (sign << 7); then one v_pk_fma_f16 adds +-x to two
// accumulators. (fma(+-1, x, c) rounds once, exactly as c + (+-x) does.)
#include "bp_device.hpp"
#include "bp_kernels.hpp"

namespace bp {
namespace {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));

constexpr int kMvThreads = 256;
constexpr int kMvRowsPerWg = 32;
constexpr int kQ1Block = 128;
constexpr int kXBlockHalves = kQ1Block + 8;   // padded block in LDS

__device__ __forceinline__ float mv_f16_sum4(h2v c01, h2v c23) {
    const _Float16 s = ((c01.x + c01.y) + c23.x) + c23.y;   // f16 adds, in this order
    return static_cast<float>(s);
}

// One (row, block) of the inner loop: the f32 block sum of +-x.
__device__ __forceinline__ float q1_block(const uint32_t q[4], const uint16_t* xb) {
    h2v c01 = {static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f)}, c23 = c01;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t nq = ~q[w];
        uint32_t sp[8];   // bytes 0x3C | (inverted bit (8k + p) << 7)
#pragma unroll
        for (int p = 0; p < 8; p++) sp[p] = ((nq << (7 - p)) & 0x80808080u) | 0x3C3C3C3Cu;
#pragma unroll
        for (int j = 0; j < 4; j++) {   // 8 elements 32w + 8j .. +7
            const h8v x8 = *reinterpret_cast<const h8v*>(xb + 32 * w + 8 * j);
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {   // nibble i = 2j + hh: elements 4i .. 4i+3
                const int k = j;               // byte of the word holding bits 4i .. 4i+3
                const int p = 4 * hh;
                // bytes: 0x00, byte k of sp[p], 0x00, byte k of sp[p + 1] (selector 12 = 0x00)
                const uint32_t sel = 0x000C000Cu | (static_cast<uint32_t>(4 + k) << 24) | (static_cast<uint32_t>(k) << 8);
                const h2v s01 = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(sp[p + 1], sp[p], sel));
                const h2v s23 = __builtin_bit_cast(h2v, __builtin_amdgcn_perm(sp[p + 3], sp[p + 2], sel));
                const h2v x01 = {x8[4 * hh], x8[4 * hh + 1]};
                const h2v x23 = {x8[4 * hh + 2], x8[4 * hh + 3]};
                c01 = __builtin_elementwise_fma(s01, x01, c01);
                c23 = __builtin_elementwise_fma(s23, x23, c23);
            }
        }
    }
    return mv_f16_sum4(c01, c23);
}

// kMode: 0 plain (x = act), 1 silu (x = f16(silu(gate)) * up), 2 normed
// (x = act * w_norm, scale d * inv_rms, up to 3 row ranges).
template <int kMode>
__global__ __launch_bounds__(kMvThreads) void matvec_q1_0_kernel(MatvecArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t x_sh[];
    __shared__ float red_sh[kMvThreads / 64];
    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const uint32_t k = a.k, nb = k / kQ1Block;

    // ---- stage x (f16) into LDS, 8 halves at a time ----------------------------
    float ssq = 0.0f;
    for (uint32_t v = t; v < k / 8; v += kMvThreads) {
        const uint32_t e = 8 * v;
        uint16_t* dst = x_sh + (e / kQ1Block) * kXBlockHalves + (e % kQ1Block);
        if constexpr (kMode == 0) {
            *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(a.act + a.input_offset + e);
        } else if constexpr (kMode == 1) {
            // matvec_q1_0_silu.wgsl:86-102: silu in f32, then f16(silu) * up in f16.
            const h8v g = *reinterpret_cast<const h8v*>(a.act + a.gate_offset + e);
            const h8v u = *reinterpret_cast<const h8v*>(a.act + a.up_offset + e);
            h8v r;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float gf = static_cast<float>(g[i]);
                const float s = gf / (1.0f + expf(-gf));
                r[i] = static_cast<_Float16>(s) * u[i];
            }
            *reinterpret_cast<h8v*>(dst) = r;
        } else {
            // matvec_q1_0_fused_normed.wgsl:102-121: x * w_norm in f16; sum of x^2
            // in f32, 4 elements at a time in order.
            const h8v x = *reinterpret_cast<const h8v*>(a.act + a.input_offset + e);
            const h8v w = *reinterpret_cast<const h8v*>(a.w_norms + a.w_norm_off + e);
            h8v r;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float xf = static_cast<float>(x[i]);
                ssq = ssq + xf * xf;
                r[i] = x[i] * w[i];
            }
            *reinterpret_cast<h8v*>(dst) = r;
        }
    }
    float inv_rms = 1.0f;
    if constexpr (kMode == 2) {
        // Workgroup sum: xor butterfly in each wave, then the waves in order.
        ssq = wave_sum(ssq);
        if (lane == 0) red_sh[wave] = ssq;
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < kMvThreads / 64; w++) total += red_sh[w];
        inv_rms = 1.0f / sqrtf(total / static_cast<float>(k) + a.eps);
    } else {
        __syncthreads();
    }

    // ---- rows: lane = (row slot 8 x lane >> 3, block lane bt = lane & 7) --------
    const int bt = lane & 7;
    const uint32_t grow = blockIdx.x * kMvRowsPerWg + 8 * wave + (lane >> 3);
    const bool valid = grow < a.n_total;
    // Row range (normed: up to 3 tensors; ranges are multiples of 32 rows).
    uint32_t d_off = a.range[0].d_offset, qs_off = a.range[0].qs_offset, out_off = a.range[0].output_offset;
    uint32_t row = grow;
    if constexpr (kMode == 2) {
        if (grow >= a.range[0].n) {
            row = grow - a.range[0].n;
            d_off = a.range[1].d_offset; qs_off = a.range[1].qs_offset; out_off = a.range[1].output_offset;
            if (row >= a.range[1].n) {
                row -= a.range[1].n;
                d_off = a.range[2].d_offset; qs_off = a.range[2].qs_offset; out_off = a.range[2].output_offset;
            }
        }
    }
    const uint32_t rc = valid ? row : 0u;
    const uint8_t* dptr = a.weights + d_off + static_cast<uint64_t>(rc) * nb * 2;
    const uint8_t* qptr = a.weights + qs_off + static_cast<uint64_t>(rc) * nb * 16;

    float acc = 0.0f;
    for (uint32_t b = bt; b < nb; b += 8) {
        const uint32_t* qw = reinterpret_cast<const uint32_t*>(qptr + 16 * b);
        const uint32_t q[4] = {qw[0], qw[1], qw[2], qw[3]};
        float d = static_cast<float>(__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(dptr + 2 * b)));
        if constexpr (kMode == 2) d = d * inv_rms;
        const float sum = q1_block(q, x_sh + b * kXBlockHalves);
        acc = acc + d * sum;
    }
    // lanes bt, bt ^ 1, bt ^ 2, bt ^ 4 of the row
    acc = acc + __shfl_xor(acc, 1);
    acc = acc + __shfl_xor(acc, 2);
    acc = acc + __shfl_xor(acc, 4);
    if (bt == 0 && valid) {
        uint16_t* y = a.act + out_off + row;
        if (kMode != 2 && a.accumulate) *y = f2h(h2f(*y) + acc);
        else *y = f2h(acc);
    }
}

}  // namespace

hipError_t launch_matvec_q1_0(const MatvecArgs& a, int mode, hipStream_t s) {
    const uint32_t n_wg = (a.n_total + kMvRowsPerWg - 1) / kMvRowsPerWg;
    const size_t lds = static_cast<size_t>(a.k / kQ1Block) * kXBlockHalves * 2;
    if (mode == 0)
        hipLaunchKernelGGL(matvec_q1_0_kernel<0>, dim3(n_wg), dim3(kMvThreads), lds, s, a);
    else if (mode == 1)
        hipLaunchKernelGGL(matvec_q1_0_kernel<1>, dim3(n_wg), dim3(kMvThreads), lds, s, a);
    else
        hipLaunchKernelGGL(matvec_q1_0_kernel<2>, dim3(n_wg), dim3(kMvThreads), lds, s, a);
    return hipGetLastError();
}

uint32_t matvec_max_k() { return 16384; }

}  // namespace bp
