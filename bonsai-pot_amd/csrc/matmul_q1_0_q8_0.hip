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
//  * Workgroup: 64 (or, for narrow outputs, 32) tokens x 64 weight rows, 4
//    waves; wave w owns weight rows 16w .. 16w + 15 for all the tokens (the
//    MFMA token tiles share one B operand); a lane reads the a_d of its four
//    tokens for all four 32-blocks as one 16-byte LDS load each.
//  * The token tile (tokens x 128 qs bytes + their 4 d's per 128-block) is
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
// One thread per 32-element block: 64 bytes in (four 16-byte loads), the
// block max in registers, 32 quantized bytes + one f32 d out. Per element the
// operations are the reference's (|x| max, one IEEE divide for d, one for
// 1/d, rne(x * inv), clamp), so the bytes are identical.
__global__ __launch_bounds__(256) void quantize_act_q8_0_kernel(QuantArgs a) {
    const uint32_t nb = a.k / 32;
    const uint32_t blk = blockIdx.x * 256 + threadIdx.x;   // row * nb + b
    if (blk >= a.m * nb) return;
    const uint32_t row = blk / nb, b = blk % nb;
    const uint16_t* src = a.act + a.input_offset + static_cast<uint64_t>(row) * a.k + 32 * b;
    uint32_t w[16];
    if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 q = reinterpret_cast<const uint4*>(src)[i];
            w[4 * i] = q.x; w[4 * i + 1] = q.y; w[4 * i + 2] = q.z; w[4 * i + 3] = q.w;
        }
    } else {   // input_offset not a multiple of 8 elements: element loads
#pragma unroll
        for (int i = 0; i < 16; i++) w[i] = static_cast<uint32_t>(src[2 * i]) | (static_cast<uint32_t>(src[2 * i + 1]) << 16);
    }
    float v[32];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        v[2 * i] = h2f(static_cast<uint16_t>(w[i] & 0xFFFFu));
        v[2 * i + 1] = h2f(static_cast<uint16_t>(w[i] >> 16));
        amax = fmaxf(amax, fmaxf(fabsf(v[2 * i]), fabsf(v[2 * i + 1])));
    }
    const float d = amax / 127.0f;
    const float inv = d > 0.0f ? 1.0f / d : 0.0f;
    uint32_t out[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float r = fminf(fmaxf(rintf(v[4 * i + e] * inv), -127.0f), 127.0f);
            word |= (static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xFFu) << (8 * e);
        }
        out[i] = word;
    }
    uint4* qs = reinterpret_cast<uint4*>(a.out + a.qs_offset + static_cast<uint64_t>(row) * a.k + 32 * b);
    if ((reinterpret_cast<uintptr_t>(qs) & 15u) == 0) {
        qs[0] = make_uint4(out[0], out[1], out[2], out[3]);
        qs[1] = make_uint4(out[4], out[5], out[6], out[7]);
    } else {   // qs_offset a multiple of 4 only
#pragma unroll
        for (int i = 0; i < 8; i++) reinterpret_cast<uint32_t*>(qs)[i] = out[i];
    }
    *reinterpret_cast<float*>(a.out + a.d_offset + 4 * static_cast<uint64_t>(blk)) = d;
}

// ---------------------------------------------------------------- matmul
constexpr int kMmRows = 64, kMmThreads = 256;
constexpr int kRowStride = 136;   // bytes per token row of the staged qs (128 + 8)

template <int kTok> struct MmStage {   // LDS image of one 128-block of the token tile
    uint8_t qs[kTok * kRowStride];
    float d[kTok * 4];   // [token][s]
};

// kTok tokens x 64 weight rows per workgroup (kTok = 64, or 32 for narrow
// outputs so that the grid still fills the chip).
template <int kTok>
__global__ __launch_bounds__(kMmThreads) void matmul_q1_0_q8_0_kernel(MatmulArgs a) {
    constexpr int kTiles = kTok / 16;          // MFMA token tiles per wave
    constexpr int kTpt = kMmThreads / kTok;    // staging threads per token
    constexpr int kQpt = kTok / 32;            // 16-byte pieces per staging thread
    __shared__ __attribute__((aligned(16))) MmStage<kTok> st[2];
    __shared__ uint2 lut[256];   // sign byte -> 8 bytes of +-1 (bit e set: +1)
    const int t = threadIdx.x, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const uint32_t nb1 = a.k / 128, nb8 = a.k / 32;
    const uint32_t n0 = blockIdx.x * kMmRows, m0 = blockIdx.y * kTok;
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

    // token tile loads: thread t -> token t / kTpt, kQpt 16-byte pieces at
    // 16 kQpt (t % kTpt); threads with t % kTpt < 4 also load d of s = t % kTpt
    const uint32_t lt = t / kTpt, lq = t % kTpt;
    const bool tok_ok = m0 + lt < a.m;
    auto load_tok = [&](uint32_t b, uint4 (&q)[kQpt], float& dv) {
#pragma unroll
        for (int i = 0; i < kQpt; i++) q[i] = make_uint4(0u, 0u, 0u, 0u);
        dv = 0.0f;
        if (tok_ok && b < nb1) {
            const uint8_t* src = a.acts + a.a_qs_offset + static_cast<uint64_t>(m0 + lt) * a.k + 128 * b + 16 * kQpt * lq;
#pragma unroll
            for (int i = 0; i < kQpt; i++) q[i] = *reinterpret_cast<const uint4*>(src + 16 * i);
            if (lq < 4)
                dv = *reinterpret_cast<const float*>(a.acts + a.a_d_offset +
                                                     4 * (static_cast<uint64_t>(m0 + lt) * nb8 + 4 * b + lq));
        }
    };
    auto store_tok = [&](int buf, const uint4 (&q)[kQpt], float dv) {
        uint8_t* dst = st[buf].qs + lt * kRowStride + 16 * kQpt * lq;
#pragma unroll
        for (int i = 0; i < kQpt; i++) {
            *reinterpret_cast<uint2*>(dst + 16 * i) = make_uint2(q[i].x, q[i].y);   // 8-byte aligned rows
            *reinterpret_cast<uint2*>(dst + 16 * i + 8) = make_uint2(q[i].z, q[i].w);
        }
        if (lq < 4) st[buf].d[lt * 4 + lq] = dv;
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

    uint4 tq[kQpt], wq;
    float tdv;
    uint16_t wd16;
    load_tok(0, tq, tdv);
    load_w(0, wq, wd16);
    store_tok(0, tq, tdv);
    __syncthreads();

    float acc[kTiles][4] = {};   // [token tile][j]: token 16 i + 4g + j, weight row wn
    for (uint32_t b = 0; b < nb1; b++) {
        const int cur = b & 1;
        // next 128-block in flight
        uint4 nq[kQpt], nwq;
        float ndv;
        uint16_t nwd;
        load_tok(b + 1, nq, ndv);
        load_w(b + 1, nwq, nwd);

        const float wd = h2f(wd16);
        const uint32_t wbits[4] = {wq.x, wq.y, wq.z, wq.w};
        long bv[4];   // B for the four 32-blocks: elements 32 s + 8 g .. + 7 of the row, as +-1 bytes
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
            const uint2 bw = lut[(wbits[s4] >> (8 * g)) & 0xFFu];
            bv[s4] = static_cast<long>((static_cast<uint64_t>(bw.y) << 32) | bw.x);
        }
#pragma unroll
        for (int i = 0; i < kTiles; i++) {
            // a_d of this lane's 4 tokens, all four 32-blocks at once
            float4 ad[4];
#pragma unroll
            for (int j = 0; j < 4; j++) ad[j] = *reinterpret_cast<const float4*>(&st[cur].d[(16 * i + 4 * g + j) * 4]);
#pragma unroll
            for (int s4 = 0; s4 < 4; s4++) {
                // A: tokens 16 i + c, the same 8 elements
                const uint2 av2 = *reinterpret_cast<const uint2*>(st[cur].qs + (16 * i + c) * kRowStride + 32 * s4 + 8 * g);
                const long av = static_cast<long>((static_cast<uint64_t>(av2.y) << 32) | av2.x);
                const i4v z = {0, 0, 0, 0};
                const i4v sumi = __builtin_amdgcn_mfma_i32_16x16x32_i8(av, bv[s4], z, 0, 0, 0);
                // D[token 16 i + 4g + j][row c]; acc = acc + (a_d * w_d) * f32(sumi), blocks in order
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const float adv = s4 == 0 ? ad[j].x : s4 == 1 ? ad[j].y : s4 == 2 ? ad[j].z : ad[j].w;
                    const float scale = adv * wd;
                    const float v = scale * static_cast<float>(sumi[j]);
                    acc[i][j] = acc[i][j] + v;
                }
            }
        }
        store_tok(cur ^ 1, nq, ndv);
        wq = nwq;
        wd16 = nwd;
        __syncthreads();
    }

    // output: y[out + token * n + row]
    if (w_ok) {
#pragma unroll
        for (int i = 0; i < kTiles; i++)
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
    hipLaunchKernelGGL(quantize_act_q8_0_kernel, dim3((blocks + 255) / 256), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_matmul_q1_0_q8_0(const MatmulArgs& a, hipStream_t s) {
    // 64-token tiles unless that leaves fewer than ~3 workgroups per CU
    const uint32_t nx = (a.n + kMmRows - 1) / kMmRows;
    const uint32_t wg64 = nx * ((a.m + 63) / 64);
    if (wg64 >= 768 || a.m <= 32) {
        hipLaunchKernelGGL(matmul_q1_0_q8_0_kernel<64>, dim3(nx, (a.m + 63) / 64), dim3(kMmThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL(matmul_q1_0_q8_0_kernel<32>, dim3(nx, (a.m + 31) / 32), dim3(kMmThreads), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace bp
