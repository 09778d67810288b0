// Prefill projections (gfx950): activations quantized to Q8_0, then
// y = W x for m tokens at once with Q1_0 weights. Same results as
// src/shaders/quantize_q8_0.wgsl and src/shaders/matmul_q1_0_q8_0.wgsl
// (reference repository), bit for bit:
//
//  * quantize: per 32 elements of a row, d = amax / 127 (f32), q =
//    clamp(rne(v * (1 / d)), -127, 127) (0 when d = 0); d (f32) at d_offset +
//    4 (row * k/32 + block), qs at qs_offset + row * k + 32 block (bytes).
//  * matmul: for each (token, weight row), over 128-blocks b and then their
//    four 32-blocks s, acc = acc + (a_d * w_d) * f32(sumi) in f32, with sumi
//    the exact integer sum of +-q over the 32 elements (bit e of the row's
//    block selects +q[e]); then f16(acc), or f16(f32(y) + acc) to accumulate.
//
// Matmul on the i8 matrix cores: one v_mfma_i32_16x16x32_i8 per (16 tokens x
// 16 weight rows, 32-block) gives every sumi exactly; the f32 scaling and the
// running sums then follow the reference's order in registers.
//  * Workgroup: 64 tokens x 64 weight rows, 4 waves; wave w owns weight rows
//    16w .. 16w + 15 for all 64 tokens (4 MFMA tiles share one B operand).
//  * The token tile (64 rows x 128 qs bytes + their 4 d's per 128-block) is
//    staged in LDS, double-buffered, one barrier per 128-block; rows are padded
//    to 136 bytes so that the 16 rows one A read touches hit distinct banks.
//  * B operand (8 sign bits -> 8 bytes of +-1): one lookup in a 256-entry LDS
//    table built at kernel start. Each lane loads its weight row's 16 qs bytes
//    and its d for the next 128-block while the current one is computed.
#include "bp_device.hpp"
#include "bp_kernels.hpp"

namespace bp {
namespace {

typedef int i4v __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- quantize
// 256 threads = 8 blocks of 32 elements; grid over m * k/32 blocks.
__global__ __launch_bounds__(256) void quantize_act_q8_0_kernel(QuantArgs a) {
    const uint32_t nb = a.k / 32;
    const uint32_t blk = blockIdx.x * 8 + (threadIdx.x >> 5);   // row * nb + b
    const uint32_t e = threadIdx.x & 31;
    if (blk >= a.m * nb) return;   // whole 32-lane groups leave together
    const uint32_t row = blk / nb, b = blk % nb;
    const float v = h2f(a.act[a.input_offset + static_cast<uint64_t>(row) * a.k + 32 * b + e]);
    float amax = fabsf(v);
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    amax = fmaxf(amax, __shfl_xor(amax, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    const float d = amax / 127.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    const float r = fminf(fmaxf(rintf(v * inv), -127.0f), 127.0f);
    // 4 lanes -> one little-endian word
    const uint32_t byte = static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xFFu;
    const uint32_t b1 = __shfl_down(byte, 1), b2 = __shfl_down(byte, 2), b3 = __shfl_down(byte, 3);
    if ((e & 3) == 0) {
        uint32_t* qs = reinterpret_cast<uint32_t*>(a.out + a.qs_offset + static_cast<uint64_t>(row) * a.k + 32 * b);
        qs[e / 4] = byte | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
    if (e == 0) *reinterpret_cast<float*>(a.out + a.d_offset + 4 * static_cast<uint64_t>(blk)) = d;
}

// ---------------------------------------------------------------- matmul
constexpr int kMmTokens = 64, kMmRows = 64, kMmThreads = 256;
constexpr int kRowStride = 136;   // bytes per token row of the staged qs (128 + 8)

struct MmStage {   // LDS image of one 128-block of the token tile
    uint8_t qs[kMmTokens * kRowStride];
    float d[kMmTokens * 4];   // [token][s]
};

__global__ __launch_bounds__(kMmThreads) void matmul_q1_0_q8_0_kernel(MatmulArgs a) {
    __shared__ __attribute__((aligned(16))) MmStage st[2];
    __shared__ uint2 lut[256];   // sign byte -> 8 bytes of +-1 (bit e set: +1)
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nb1 = a.k / 128, nb8 = a.k / 32;
    const uint32_t n0 = blockIdx.x * kMmRows, m0 = blockIdx.y * kMmTokens;
    const uint32_t g = lane >> 4, c = lane & 15;

    {   // table: byte v -> bytes (bit j ? 0x01 : 0xFF), j = 0..7
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            lo |= (((t >> j) & 1) ? 0x01u : 0xFFu) << (8 * j);
            hi |= (((t >> (j + 4)) & 1) ? 0x01u : 0xFFu) << (8 * j);
        }
        lut[t] = make_uint2(lo, hi);
    }

    // token tile loads: thread t -> token t / 4, 32 qs bytes at 32 (t % 4); and
    // d of (token t / 4, s = t % 4)
    const uint32_t lt = t >> 2, lq = t & 3;
    const bool tok_ok = m0 + lt < a.m;
    auto load_tok = [&](uint32_t b, uint4& q0, uint4& q1, float& dv) {
        q0 = make_uint4(0u, 0u, 0u, 0u);
        q1 = q0;
        dv = 0.0f;
        if (tok_ok && b < nb1) {
            const uint8_t* src = a.acts + a.a_qs_offset + static_cast<uint64_t>(m0 + lt) * a.k + 128 * b + 32 * lq;
            q0 = *reinterpret_cast<const uint4*>(src);
            q1 = *reinterpret_cast<const uint4*>(src + 16);
            dv = *reinterpret_cast<const float*>(a.acts + a.a_d_offset +
                                                 4 * (static_cast<uint64_t>(m0 + lt) * nb8 + 4 * b + lq));
        }
    };
    auto store_tok = [&](int buf, const uint4& q0, const uint4& q1, float dv) {
        uint8_t* dst = st[buf].qs + lt * kRowStride + 32 * lq;
        *reinterpret_cast<uint2*>(dst) = make_uint2(q0.x, q0.y);   // 8-byte aligned rows
        *reinterpret_cast<uint2*>(dst + 8) = make_uint2(q0.z, q0.w);
        *reinterpret_cast<uint2*>(dst + 16) = make_uint2(q1.x, q1.y);
        *reinterpret_cast<uint2*>(dst + 24) = make_uint2(q1.z, q1.w);
        st[buf].d[lt * 4 + lq] = dv;
    };
    // this lane's weight row (B column c of the wave's 16)
    const uint32_t wn = n0 + 16 * wave + c;
    const bool w_ok = wn < a.n;
    auto load_w = [&](uint32_t b, uint4& q, uint16_t& d) {
        q = make_uint4(0u, 0u, 0u, 0u);
        d = 0;
        if (w_ok && b < nb1) {
            const uint64_t rb = static_cast<uint64_t>(wn) * nb1 + b;
            q = *reinterpret_cast<const uint4*>(a.weights + a.w_qs_offset + 16 * rb);
            d = *reinterpret_cast<const uint16_t*>(a.weights + a.w_d_offset + 2 * rb);
        }
    };

    uint4 tq0, tq1, wq;
    float tdv;
    uint16_t wd16;
    load_tok(0, tq0, tq1, tdv);
    load_w(0, wq, wd16);
    store_tok(0, tq0, tq1, tdv);
    __syncthreads();

    float acc[4][4] = {};   // [token tile][j]: token 16 i + 4g + j, weight row wn
    for (uint32_t b = 0; b < nb1; b++) {
        const int cur = b & 1;
        // next 128-block in flight
        uint4 nq0, nq1, nwq;
        float ndv;
        uint16_t nwd;
        load_tok(b + 1, nq0, nq1, ndv);
        load_w(b + 1, nwq, nwd);

        const float wd = h2f(wd16);
        const uint32_t wbits[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
        for (int s = 0; s < 4; s++) {
            // B: elements 32 s + 8 g .. + 7 of the weight row, as +-1 bytes
            const uint2 bw = lut[(wbits[s] >> (8 * g)) & 0xFFu];
            const long bv = static_cast<long>((static_cast<uint64_t>(bw.y) << 32) | bw.x);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                // A: tokens 16 i + c, the same 8 elements
                const uint2 av2 = *reinterpret_cast<const uint2*>(st[cur].qs + (16 * i + c) * kRowStride + 32 * s + 8 * g);
                const long av = static_cast<long>((static_cast<uint64_t>(av2.y) << 32) | av2.x);
                const i4v z = {0, 0, 0, 0};
                const i4v sumi = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv, z, 0, 0, 0);
                // D[token 16 i + 4g + j][row c]
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float ad = st[cur].d[(16 * i + 4 * g + j) * 4 + s];
                    const float scale = ad * wd;
                    const float v = scale * static_cast<float>(sumi[j]);
                    acc[i][j] = acc[i][j] + v;
                }
            }
        }
        store_tok(cur ^ 1, nq0, nq1, ndv);
        wq = nwq;
        wd16 = nwd;
        __syncthreads();
    }

    // output: y[out + token * n + row]
    if (w_ok) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t tok = m0 + 16 * i + 4 * g + j;
                if (tok < a.m) {
                    uint16_t* y = a.y + a.out_offset + static_cast<uint64_t>(tok) * a.n + wn;
                    if (a.accumulate) *y = f2h(h2f(*y) + acc[i][j]);
                    else *y = f2h(acc[i][j]);
                }
            }
    }
}

}  // namespace

hipError_t launch_quantize_act_q8_0(const QuantArgs& a, hipStream_t s) {
    const uint32_t blocks = a.m * (a.k / 32);
    hipLaunchKernelGGL(quantize_act_q8_0_kernel, dim3((blocks + 7) / 8), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_matmul_q1_0_q8_0(const MatmulArgs& a, hipStream_t s) {
    const dim3 grid((a.n + kMmRows - 1) / kMmRows, (a.m + kMmTokens - 1) / kMmTokens);
    hipLaunchKernelGGL(matmul_q1_0_q8_0_kernel, grid, dim3(kMmThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace bp
