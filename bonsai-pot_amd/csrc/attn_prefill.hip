// Causal (chunked) prefill attention over the Q8_0 KV cache on f16 MFMA (gfx950).
//
// Same result as src/shaders/attention.wgsl (reference repository) — token m
// attends rows [0, cur) with cur = causal ? pos + m + 1 : pos, f32 softmax,
// f16 output — computed as a flash-attention over LDS tiles:
//
//  * grid = (n_tiles, n_kv_head); a 512-thread workgroup owns one KV head and
//    64 query tokens. Wave w owns tokens [16 (w & 3), +16) of the tile for the
//    GQA head pair w >> 2 (heads 2(w>>2), +1), so every K/V chunk staged in LDS
//    serves 4 x 64 query rows, and 2 waves per SIMD let one wave's softmax
//    overlap the other's MFMAs. Tiles are issued heaviest first.
//  * K/V are consumed in chunks of 32 rows. Staging dequantizes Q8_0 to f16
//    (d * q, one rounding) into double-buffered LDS — K row-major, V
//    transposed (dim-major) so both MFMA operands are single 16-byte reads —
//    with a register prefetch distance of two chunks.
//  * S^T = K Q^T with v_mfma_f32_16x16x32_f16 (K = 32 dims per step): the
//    output fragment of lane l holds 8 keys of token (l % 16). With the keys
//    of a chunk stored in V^T in the matching permuted order, that fragment
//    is directly the B operand of O^T = V^T P^T — no shuffles, no LDS trip.
//  * Online softmax in the exp2 domain (scale * log2 e folded into one
//    multiply), row max across the 4 lane groups by swizzle/permute, and a
//    lazy running max (moved only by more than kLazy log2 units), so the O
//    accumulators are almost never touched by VALU.
//
// MFMA fragment layout used (v_mfma_f32_16x16x32_f16, lane l, g = l / 16):
//   A[i][k]: lane holds A[l % 16][8g .. 8g+7]
//   B[k][j]: lane holds B[8g .. 8g+7][l % 16]
//   D[i][j]: lane holds D[4g .. 4g+3][l % 16]
#include "bp_device.hpp"
#include "bp_kernels.hpp"

namespace bp {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 512;
constexpr int kHeadsPerWave = 2;
constexpr int kTileTok = 64;             // query tokens per workgroup
constexpr int kChunk = 32;               // cache rows per LDS chunk
constexpr int kKStride = kHeadDim + 8;   // halves per K row in LDS (pad vs bank conflicts)
constexpr int kVStride = kChunk + 8;     // halves per V^T row in LDS
constexpr float kLazy = 8.0f;            // lazy-rescale threshold (log2 units)

struct alignas(16) U4 { uint32_t w[4]; };

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Position of chunk row `key` (0..31) along the MFMA k axis of the PV step:
// lane group g holds S^T rows {4g..4g+3} (sub-tile 0) and {16+4g..16+4g+3}
// (sub-tile 1), which become its k slots 8g..8g+3 and 8g+4..8g+7.
__device__ __forceinline__ int v_slot(int key) {
    return key < 16 ? 8 * (key >> 2) + (key & 3) : 8 * ((key - 16) >> 2) + 4 + (key & 3);
}

// Reductions across the 4 lane groups of a token column (lanes l, l^16,
// l^32, l^48): xor 16 by ds_swizzle (bit mode), xor 32 by ds_bpermute.
__device__ __forceinline__ float swz_xor16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
}
__device__ __forceinline__ float group_max(float v) {
    v = fmaxf(v, swz_xor16(v));
    return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float group_sum(float v) {
    v += swz_xor16(v);
    return v + __shfl_xor(v, 32);
}

__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return static_cast<uint32_t>(f2h(a)) | (static_cast<uint32_t>(f2h(b)) << 16);
}

__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t k_lds[2][kChunk * kKStride];
    __shared__ __attribute__((aligned(16))) uint16_t v_lds[2][kHeadDim * kVStride];

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int lr = lane & 15, lg = lane >> 4;
    const uint32_t g = blockIdx.y;
    const uint32_t tile = a.n_tiles - 1 - blockIdx.x;        // heaviest first
    const uint32_t tile0 = tile * kTileTok;
    const uint32_t wtok0 = tile0 + 16 * (wave & 3);           // first token of this wave
    const uint32_t h0 = g * kGroup + kHeadsPerWave * (wave >> 2);   // first query head of this wave
    const uint32_t my_tok = wtok0 + lr;                       // token of this lane's column
    const uint32_t last_tok = min(tile0 + kTileTok, a.m_tokens) - 1;
    const uint32_t kend = a.causal ? a.pos + last_tok + 1 : a.pos;   // rows the tile needs
    const uint32_t n_chunks = (kend + kChunk - 1) / kChunk;
    // Rows this wave's tokens can see: [0, wave_kend).
    const uint32_t wave_last = min(wtok0 + 15, a.m_tokens - 1);
    const uint32_t wave_kend = a.causal ? a.pos + wave_last + 1 : a.pos;
    const bool wave_live = wtok0 < a.m_tokens;
    const uint32_t my_kend = a.causal ? a.pos + my_tok + 1 : a.pos;

    // ---- Q^T fragments (B operand of S^T = K Q^T), 2 heads x 4 k-steps ----
    f16x8 qb[kHeadsPerWave][4];
#pragma unroll
    for (int h = 0; h < kHeadsPerWave; h++) {
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            U4 raw = {{0, 0, 0, 0}};
            if (my_tok < a.m_tokens) {
                raw = *reinterpret_cast<const U4*>(a.q + static_cast<uint64_t>(my_tok) * a.q_stride +
                                                   (h0 + h) * kHeadDim + 32 * kk + 8 * lg);
            }
            qb[h][kk] = __builtin_bit_cast(f16x8, raw);
        }
    }

    f32x4 o[kHeadsPerWave][8];
#pragma unroll
    for (int h = 0; h < kHeadsPerWave; h++)
#pragma unroll
        for (int dt = 0; dt < 8; dt++) o[h][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run[kHeadsPerWave], l_run[kHeadsPerWave];
#pragma unroll
    for (int h = 0; h < kHeadsPerWave; h++) { m_run[h] = -INFINITY; l_run[h] = 0.0f; }
    const float c2 = a.scale * 1.4426950408889634f;   // scores in log2 units

    // ---- staging ------------------------------------------------------------
    // Threads 0..255 stage K: thread owns chunk row (t >> 3), dims
    //   [16 (t & 7), +16) -> row-major LDS writes of 2 x 16 bytes.
    // Threads 256..511 stage V: thread owns chunk row (t & 31), dims
    //   [16 ((t >> 5) & 7), +16) -> 16 transposed 2-byte writes into one V^T
    //   column; the 32 rows of a wave fill 32 consecutive columns.
    // Loads are unconditional from a clamped row (a predicated load becomes a
    // branch that drains all outstanding loads); rows past kend are zeroed
    // through their scale. Two register stages give a prefetch distance of 2
    // chunks: chunk c+2 is loaded while chunk c is computed and c+1 is staged.
    const bool stage_k = t < 256;
    const int srow = stage_k ? (t >> 3) : (t & 31);
    const int sseg = stage_k ? (t & 7) : ((t >> 5) & 7);
    const int8_t* sqs = stage_k ? a.k.qs : a.v.qs;
    const float* sd = stage_k ? a.k.d : a.v.d;
    const uint64_t kv_dim = a.kv_dim;
    const uint32_t nb_row = a.kv_dim / kBlock;
    const uint32_t scol = g * kHeadDim + 16 * sseg, sdcol = g * (kHeadDim / kBlock) + (sseg >> 1);
    struct Stage { U4 q; float d; };
    auto load_chunk = [&](Stage& S, uint32_t c) {
        const uint32_t r = c * kChunk + srow;
        const uint64_t rc = min(r, kend - 1);
        S.q = *reinterpret_cast<const U4*>(sqs + rc * kv_dim + scol);
        S.d = sd[rc * nb_row + sdcol];
        if (r >= kend) S.d = 0.0f;
    };
    auto store_chunk = [&](const Stage& S, int buf) {
        if (stage_k) {
            U4 lo, hi;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo.w[i] = pack2(S.d * i8f(S.q.w[i >> 1], 2 * (i & 1)), S.d * i8f(S.q.w[i >> 1], 2 * (i & 1) + 1));
                hi.w[i] = pack2(S.d * i8f(S.q.w[2 + (i >> 1)], 2 * (i & 1)),
                                S.d * i8f(S.q.w[2 + (i >> 1)], 2 * (i & 1) + 1));
            }
            uint16_t* kr = &k_lds[buf][srow * kKStride + 16 * sseg];
            *reinterpret_cast<U4*>(kr) = lo;
            *reinterpret_cast<U4*>(kr + 8) = hi;
        } else {
            uint16_t* vc = &v_lds[buf][(16 * sseg) * kVStride + v_slot(srow)];
#pragma unroll
            for (int i = 0; i < 16; i++) vc[i * kVStride] = f2h(S.d * i8f(S.q.w[i >> 2], i & 3));
        }
    };

    Stage S0, S1;
    load_chunk(S0, 0);
    if (n_chunks > 1) load_chunk(S1, 1);
    store_chunk(S0, 0);
    __syncthreads();

    // One chunk: prefetch chunk c+2 into `ld` (free: its chunk c was staged
    // last iteration), compute chunk c from LDS, stage chunk c+1 from `st`.
    auto step = [&](Stage& ld, const Stage& st, uint32_t c) {
        const int buf = c & 1;
        if (c + 2 < n_chunks) load_chunk(ld, c + 2);
        const uint32_t key0 = c * kChunk;
        if (wave_live && key0 < wave_kend) {
            const uint16_t* kb = k_lds[buf];
            const uint16_t* vb = v_lds[buf];
            // ---- S^T = K Q^T: 2 key sub-tiles x 2 heads --------------------
            f32x4 s[kHeadsPerWave][2];
#pragma unroll
            for (int st2 = 0; st2 < 2; st2++) {
                f16x8 ka[4];
#pragma unroll
                for (int kk = 0; kk < 4; kk++)
                    ka[kk] = *reinterpret_cast<const f16x8*>(kb + (16 * st2 + lr) * kKStride + 32 * kk + 8 * lg);
#pragma unroll
                for (int h = 0; h < kHeadsPerWave; h++) {
                    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int kk = 0; kk < 4; kk++) acc = mfma16(ka[kk], qb[h][kk], acc);
                    s[h][st2] = acc;
                }
            }
            // ---- mask (only chunks that reach past the earliest visible row)
            const bool need_mask = key0 + kChunk > (a.causal ? a.pos + wtok0 + 1 : a.pos);
#pragma unroll
            for (int h = 0; h < kHeadsPerWave; h++)
#pragma unroll
                for (int st2 = 0; st2 < 2; st2++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        float v = s[h][st2][j] * c2;
                        if (need_mask && key0 + 16 * st2 + 4 * lg + j >= my_kend) v = -INFINITY;
                        s[h][st2][j] = v;
                    }
            // ---- online softmax + P^T fragments ------------------------------
            f16x8 pb[kHeadsPerWave];
#pragma unroll
            for (int h = 0; h < kHeadsPerWave; h++) {
                float cm = fmaxf(fmaxf(fmaxf(s[h][0][0], s[h][0][1]), fmaxf(s[h][0][2], s[h][0][3])),
                                 fmaxf(fmaxf(s[h][1][0], s[h][1][1]), fmaxf(s[h][1][2], s[h][1][3])));
                cm = group_max(cm);
                // Lazy rescale: the running max of a row moves only when the chunk
                // max exceeds it by more than kLazy; p then stays below 2^kLazy,
                // which f16 P and the f32 accumulators hold as well as p <= 1.
                const bool up = cm > m_run[h] + kLazy;
                if (__any(up)) {
                    const float m_new = up ? cm : m_run[h];
                    const float alpha = __builtin_amdgcn_exp2f(m_run[h] - m_new);   // 0 from -inf
                    m_run[h] = m_new;
                    l_run[h] *= alpha;
#pragma unroll
                    for (int dt = 0; dt < 8; dt++) o[h][dt] *= alpha;
                }
                float p[8];
                float ps = 0.0f;
#pragma unroll
                for (int st2 = 0; st2 < 2; st2++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        p[4 * st2 + j] = __builtin_amdgcn_exp2f(s[h][st2][j] - m_run[h]);
                        ps += p[4 * st2 + j];
                    }
                l_run[h] += ps;
                U4 pk;
#pragma unroll
                for (int i = 0; i < 4; i++) pk.w[i] = pack2(p[2 * i], p[2 * i + 1]);
                pb[h] = __builtin_bit_cast(f16x8, pk);
            }
            // ---- O^T += V^T P^T ------------------------------------------------
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const f16x8 va = *reinterpret_cast<const f16x8*>(vb + (16 * dt + lr) * kVStride + 8 * lg);
#pragma unroll
                for (int h = 0; h < kHeadsPerWave; h++) o[h][dt] = mfma16(va, pb[h], o[h][dt]);
            }
        }
        if (c + 1 < n_chunks) store_chunk(st, buf ^ 1);
        __syncthreads();
    };
    for (uint32_t c = 0; c < n_chunks; c += 2) {
        step(S0, S1, c);
        if (c + 1 < n_chunks) step(S1, S0, c + 1);
    }

    if (!wave_live || my_tok >= a.m_tokens) return;
    // ---- normalize and write O (lane: token my_tok, dims 16dt + 4lg + j) ----
#pragma unroll
    for (int h = 0; h < kHeadsPerWave; h++) {
        const float inv_l = 1.0f / group_sum(l_run[h]);
        uint16_t* out = a.out + static_cast<uint64_t>(my_tok) * a.q_stride + (h0 + h) * kHeadDim;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            uint2 w;
            w.x = pack2(o[h][dt][0] * inv_l, o[h][dt][1] * inv_l);
            w.y = pack2(o[h][dt][2] * inv_l, o[h][dt][3] * inv_l);
            *reinterpret_cast<uint2*>(out + 16 * dt + 4 * lg) = w;
        }
    }
}

}  // namespace

hipError_t launch_prefill(const PrefillArgs& a, uint32_t n_kv_head, hipStream_t s) {
    hipLaunchKernelGGL(prefill_kernel, dim3(a.n_tiles, n_kv_head), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace bp
