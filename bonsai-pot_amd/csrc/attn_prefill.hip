// Causal (chunked) prefill attention over the Q8_0 KV cache on f16 MFMA (gfx950).
//
// Same result as src/shaders/attention.wgsl (reference repository) — token m
// attends rows [0, cur) with cur = causal ? pos + m + 1 : pos, f32 softmax,
// f16 output — computed as a flash-attention over LDS tiles:
//
//  * Query tokens form tiles of 32. A 512-thread workgroup owns one KV head
//    and a zig-zag PAIR of tiles (p, n_tiles-1-p): waves 0-3 take tile p,
//    waves 4-7 tile n_tiles-1-p, each wave 16 tokens x 2 GQA heads. Under the
//    causal mask the two tiles' work sums to the same amount for every pair,
//    so the 256 CUs finish together, and each SIMD holds one wave of each tile
//    (one's softmax overlaps the other's MFMAs). Both tiles read the same cache
//    rows (the light tile's range is a prefix of the heavy one's), so every
//    chunk is staged once.
//  * K/V are consumed in chunks of 64 rows. Every thread stages 16 bytes of K
//    and 2 x 8 bytes of V per chunk (register prefetch distance of two
//    chunks), dequantizing Q8_0 to f16 (d * q, one rounding) into
//    double-buffered LDS: K row-major, V transposed (dim-major, 16-byte groups
//    XOR-swizzled by row to spread the transposed writes over the banks), so
//    both MFMA operands are single 16-byte LDS reads.
//  * S^T = K Q^T with v_mfma_f32_16x16x32_f16 (K = 32 dims per step): the
//    output fragment of lane l holds 8 keys of token (l % 16) per 32 keys. With
//    the keys stored in V^T in the matching permuted order, those fragments are
//    directly the B operand of O^T = V^T P^T — no shuffles, no LDS trip.
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
constexpr int kChunk = 64;               // cache rows per LDS chunk
constexpr int kSub = kChunk / 16;        // 16-row S^T sub-tiles per chunk
constexpr int kKStride = kHeadDim + 8;   // halves per K row in LDS (pad vs bank conflicts)
constexpr int kVStride = kChunk + 8;     // halves per V^T row in LDS
constexpr float kLazy = 8.0f;            // lazy-rescale threshold (log2 units)

struct alignas(16) U4 { uint32_t w[4]; };

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Position of chunk row `key` (0..63) along the MFMA k axis of the PV step:
// per 32 keys, lane group g holds S^T rows {4g..4g+3} (first sub-tile) and
// {16+4g..16+4g+3} (second), which become its k slots 8g..8g+3, 8g+4..8g+7.
__device__ __forceinline__ int v_slot(int key) {
    const int k = key & 31;
    const int s = k < 16 ? 8 * (k >> 2) + (k & 3) : 8 * ((k - 16) >> 2) + 4 + (k & 3);
    return (key & 32) + s;
}
// Half-word offset of (V^T row, slot) in LDS: 16-byte group (slot >> 3) is
// XOR-swizzled with (row >> 3) & 7.
__device__ __forceinline__ int v_addr(int row, int slot) {
    return row * kVStride + 8 * ((slot >> 3) ^ ((row >> 3) & 7)) + (slot & 7);
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
    const uint32_t tile_a = blockIdx.x, tile_b = a.n_tiles - 1 - blockIdx.x;   // tile_b >= tile_a
    const uint32_t tile = (wave & 4) ? tile_b : tile_a;
    const bool wave_live = !((wave & 4) && tile_b == tile_a) &&
                           tile * kPrefillTileTok + 16 * (wave & 1) < a.m_tokens;
    const uint32_t wtok0 = tile * kPrefillTileTok + 16 * (wave & 1);   // first token of this wave
    const uint32_t h0 = g * kGroup + kHeadsPerWave * ((wave >> 1) & 1); // first query head
    const uint32_t my_tok = wtok0 + lr;                                   // this lane's column
    const uint32_t last_b = min(tile_b * kPrefillTileTok + kPrefillTileTok, a.m_tokens) - 1;
    const uint32_t kend = a.causal ? a.pos + last_b + 1 : a.pos;         // rows the pair needs
    const uint32_t n_chunks = (kend + kChunk - 1) / kChunk;
    // Rows this wave's tokens can see: [0, wave_kend).
    const uint32_t wave_last = min(wtok0 + 15, a.m_tokens - 1);
    const uint32_t wave_kend = a.causal ? a.pos + wave_last + 1 : a.pos;
    const uint32_t my_kend = a.causal ? a.pos + my_tok + 1 : a.pos;

    // ---- Q^T fragments (B operand of S^T = K Q^T), 2 heads x 4 k-steps ----
    f16x8 qb[kHeadsPerWave][4];
#pragma unroll
    for (int h = 0; h < kHeadsPerWave; h++) {
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            U4 raw = {{0, 0, 0, 0}};
            if (wave_live && my_tok < a.m_tokens) {
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
    // K: thread owns chunk row (t >> 3), dims [16 (t & 7), +16).
    // V: thread owns chunk rows 2u, 2u+1 (u = t >> 4), dims [8 (t & 15), +8);
    //    it writes each dim's two values as one 4-byte word of V^T (the rows
    //    of a key pair are adjacent slots).
    // Loads are unconditional from a clamped row (a predicated load becomes a
    // branch that drains all outstanding loads); rows past kend are zeroed
    // through their scale.
    const int krow = t >> 3, kseg = t & 7;
    const int vu = t >> 4, vdq = t & 15;
    const uint64_t kv_dim = a.kv_dim;
    const uint32_t nb_row = a.kv_dim / kBlock;
    const uint32_t kcol = g * kHeadDim + 16 * kseg, kdcol = g * (kHeadDim / kBlock) + (kseg >> 1);
    const uint32_t vcol = g * kHeadDim + 8 * vdq, vdcol = g * (kHeadDim / kBlock) + (vdq >> 2);
    struct Stage { U4 kq; uint2 v0, v1; float kd, vd0, vd1; };
    auto load_chunk = [&](Stage& S, uint32_t c) {
        const uint32_t kr = c * kChunk + krow, vr = c * kChunk + 2 * vu;
        const uint64_t krc = min(kr, kend - 1), vr0 = min(vr, kend - 1), vr1 = min(vr + 1, kend - 1);
        S.kq = *reinterpret_cast<const U4*>(a.k.qs + krc * kv_dim + kcol);
        S.v0 = *reinterpret_cast<const uint2*>(a.v.qs + vr0 * kv_dim + vcol);
        S.v1 = *reinterpret_cast<const uint2*>(a.v.qs + vr1 * kv_dim + vcol);
        S.kd = a.k.d[krc * nb_row + kdcol];
        S.vd0 = a.v.d[vr0 * nb_row + vdcol];
        S.vd1 = a.v.d[vr1 * nb_row + vdcol];
        if (kr >= kend) S.kd = 0.0f;
        if (vr >= kend) S.vd0 = 0.0f;
        if (vr + 1 >= kend) S.vd1 = 0.0f;
    };
    auto store_chunk = [&](const Stage& S, int buf) {
        U4 lo, hi;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo.w[i] = pack2(S.kd * i8f(S.kq.w[i >> 1], 2 * (i & 1)), S.kd * i8f(S.kq.w[i >> 1], 2 * (i & 1) + 1));
            hi.w[i] = pack2(S.kd * i8f(S.kq.w[2 + (i >> 1)], 2 * (i & 1)),
                            S.kd * i8f(S.kq.w[2 + (i >> 1)], 2 * (i & 1) + 1));
        }
        uint16_t* kr = &k_lds[buf][krow * kKStride + 16 * kseg];
        *reinterpret_cast<U4*>(kr) = lo;
        *reinterpret_cast<U4*>(kr + 8) = hi;
        const int slot = v_slot(2 * vu);   // even; 2u + 1 sits in slot + 1
        const uint32_t w0[2] = {S.v0.x, S.v0.y}, w1[2] = {S.v1.x, S.v1.y};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int row = 8 * vdq + i;
            *reinterpret_cast<uint32_t*>(&v_lds[buf][v_addr(row, slot)]) =
                pack2(S.vd0 * i8f(w0[i >> 2], i & 3), S.vd1 * i8f(w1[i >> 2], i & 3));
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
            // ---- S^T = K Q^T: 4 key sub-tiles x 2 heads --------------------
            f32x4 s[kHeadsPerWave][kSub];
#pragma unroll
            for (int st2 = 0; st2 < kSub; st2++) {
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
                for (int st2 = 0; st2 < kSub; st2++)
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        float v = s[h][st2][j] * c2;
                        if (need_mask && key0 + 16 * st2 + 4 * lg + j >= my_kend) v = -INFINITY;
                        s[h][st2][j] = v;
                    }
            // ---- online softmax + P^T fragments ------------------------------
            f16x8 pb[kHeadsPerWave][kSub / 2];
#pragma unroll
            for (int h = 0; h < kHeadsPerWave; h++) {
                float cm = -INFINITY;
#pragma unroll
                for (int st2 = 0; st2 < kSub; st2++)
                    cm = fmaxf(cm, fmaxf(fmaxf(s[h][st2][0], s[h][st2][1]), fmaxf(s[h][st2][2], s[h][st2][3])));
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
                float ps = 0.0f;
#pragma unroll
                for (int kc = 0; kc < kSub / 2; kc++) {
                    float p[8];
#pragma unroll
                    for (int half = 0; half < 2; half++)
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            p[4 * half + j] = __builtin_amdgcn_exp2f(s[h][2 * kc + half][j] - m_run[h]);
                            ps += p[4 * half + j];
                        }
                    U4 pk;
#pragma unroll
                    for (int i = 0; i < 4; i++) pk.w[i] = pack2(p[2 * i], p[2 * i + 1]);
                    pb[h][kc] = __builtin_bit_cast(f16x8, pk);
                }
                l_run[h] += ps;
            }
            // ---- O^T += V^T P^T ------------------------------------------------
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const int row = 16 * dt + lr;
#pragma unroll
                for (int kc = 0; kc < kSub / 2; kc++) {
                    const f16x8 va = *reinterpret_cast<const f16x8*>(vb + v_addr(row, 32 * kc + 8 * lg));
#pragma unroll
                    for (int h = 0; h < kHeadsPerWave; h++) o[h][dt] = mfma16(va, pb[h][kc], o[h][dt]);
                }
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
    const uint32_t n_pairs = (a.n_tiles + 1) / 2;
    hipLaunchKernelGGL(prefill_kernel, dim3(n_pairs, n_kv_head), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace bp
