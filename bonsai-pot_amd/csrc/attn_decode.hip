// Single-token decode attention over the Q8_0 KV cache (gfx950).
//
// Same result as src/shaders/attention_split.wgsl + attention_merge.wgsl
// (reference repository): scores s_t = (q . k_t) / sqrt(128) over the cache
// rows, softmax in f32, o = sum p_t v_t, f16 output. Two passes:
//
// Split pass (decode_split_kernel) — one workgroup per (group of KV heads,
// range of `split_len` rows), the grid ordered XCD-aware. Each wave owns
// one KV head (its 4 query heads) and streams 16-row batches with no
// workgroup barrier in the main loop, the next batch loaded before the
// current one is consumed (register double buffering). Loads are never
// predicated: rows past the range are clamped onto its last row and masked
// by their score. Two layouts (SplitShape): 4 waves on one KV head at short
// context; 4 KV heads x 2 row sets per 8-wave workgroup at long context, so
// that the heads of a row are read together.
//  * Both products run on the matrix core in f16 with f32 accumulation, on
//    exact f16 images of the int8 values: byte (x xor 0x80) under exponent
//    byte 0x64 is the f16 value 1152 + x (one v_perm_b32 per byte pair), and
//    the 1152 bias is removed algebraically.
//  * q.k (16x16x32): A = the batch's K rows (m = row), B = q of the 4 heads
//    with the k-slots of each Q8_0 block routed to its own column (h, b), so
//    D holds per-block partial dots and the FP32 block scales are applied
//    after the MFMA: s = sum_b d_b (D_b - 1152 sum_b q).
//  * Online softmax in the exp2 domain, per lane (row group, head); O is
//    rescaled only when some max moved (a wave ballot).
//  * p.v (16x16x16): O^T = W^T V with W = p d_v, split into two f16 terms
//    (hi + lo, so the weights keep f32-like precision), V bytes transposed
//    into the B layout with v_perm_b32.
//  * The row sets of a KV head are merged through LDS (log-sum-exp) into one
//    partial (o[128], m, l) per query head; with a single split the output is
//    written directly and the merge pass is skipped.
//
// Merge pass (decode_merge_kernel) — one 64-lane workgroup per (query head,
// 32-dim chunk): log-sum-exp over the splits (attention_merge.wgsl:85-129),
// every partial load issued up front, wave reductions by row swaps and DPP.
// Its leading arguments are scalar kernel parameters, preloaded into SGPRs
// at wave launch (this file is built with kernarg preloading).
//
// Fused step (launch_decode_step): the split pass also runs q_norm_rope on
// the 4 query heads of its KV head (same code as the standalone kernel, so the
// same bits) and, in the last split's workgroup, the kv_writeback of the new
// row `pos`; it streams rows [0, pos). The merge pass then adds row `pos`
// (whose bytes are in the cache by then) and writes the normalized q into
// act. One decode step is two launches instead of four.
#include "bp_kernels.hpp"
#include "bp_norm_rope.hpp"

namespace bp {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Split-pass layouts, by KV heads per workgroup (kH):
//  kH = 1: 4 waves, all on one KV head, each streaming every 4th 16-row batch;
//  kH = 4: 8 waves, wave w on KV head 4 hg + (w & 3) and row set w >> 2, so the
//          4 heads read the same rows together (512 contiguous bytes per row).
template <int kH> struct SplitShape {
    static constexpr int kWaves = kH == 1 ? 4 : 8;
    static constexpr int kThreads = 64 * kWaves;
    static constexpr int kRowSets = kWaves / kH;
    static constexpr int kWgPerCu = 8 / kWaves;   // at 2 waves per SIMD
};
// Split-K partials of one launch (n_head query heads, ns splits): the o rows
// first, [n_head][ns][128] f32 (512-byte rows, so a 32-dim piece is one whole
// 128-byte line), then the (m, l) pairs, [n_head][ns][2] f32.
constexpr int kPartStride = kHeadDim + 2;  // floats per (head, split) partial
__device__ __forceinline__ float* part_o(float* base, uint32_t h, uint32_t ns, uint32_t s) {
    return base + (static_cast<uint64_t>(h) * ns + s) * kHeadDim;
}
__device__ __forceinline__ float* part_ml(float* base, uint32_t n_head, uint32_t h, uint32_t ns, uint32_t s) {
    return base + static_cast<uint64_t>(n_head) * ns * kHeadDim + (static_cast<uint64_t>(h) * ns + s) * 2;
}
constexpr int kMaxSplits = 128;          // the merge pass holds (m, l) of splits lane, lane + 64
constexpr uint32_t kExp64 = 0x64646464u;
constexpr float kLog2e = 1.4426950408889634f;

struct alignas(16) Q16 { uint32_t w[4]; };

struct Batch {
    Q16 kq[2];        // q.k: the 32 bytes of block lg of row lr
    f32x4 kd, vd;     // scales of block (lr & 3) of rows 4 lg + j
    u32x2 vv[4];      // p.v: dims 8 lr .. +8 of rows 4 lg + j
};

__device__ __forceinline__ f32x4 mfma32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma16(f16x4 a, f16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}
// Pick element i (0..3) of a 4-vector with a non-uniform i: three selects on
// the bits of i (a chain of ternaries on i compiles to branches).
__device__ __forceinline__ float pick4(f32x4 v, int i) {
    const bool b0 = (i & 1) != 0, b1 = (i & 2) != 0;
    const float v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
    const float lo = b0 ? v1 : v0, hi = b0 ? v3 : v2;
    return b1 ? hi : lo;
}

template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, true));
}
// Sum over lanes l, l^8, l^16, l^32.
__device__ __forceinline__ float sum_slots(float v) {
    return sum_xor32(sum_xor16(v + dpp_f<0x128>(v)));   // row_ror:8 == xor 8 within 16 lanes
}

template <bool kFused, int kH>
__global__ __launch_bounds__(SplitShape<kH>::kThreads, SplitShape<kH>::kWgPerCu) void decode_split_kernel(DecodeArgs a) {
    constexpr int kWaves = SplitShape<kH>::kWaves, kRowSets = SplitShape<kH>::kRowSets;
    constexpr int kQPerWave = kH * kGroup / kWaves;   // query heads normalized per wave (fused)
    __shared__ __attribute__((aligned(16))) float o_red[kWaves][kGroup][kHeadDim + 4];   // per-wave O
    __shared__ float ml_sh[kWaves][kGroup][2];
    __shared__ __attribute__((aligned(16))) uint16_t qn_sh[kH][kGroup][kHeadDim];

    const int t = threadIdx.x;
    const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);   // uniform: scalar registers
    // Lane roles, all from (lr, lg) = (lane & 15, lane >> 4):
    //  q.k   A = K rows (m = row lr), B = q masked per block (n = lr = 4 h + b),
    //        so D lane holds the block-b partial dot of head h for rows 4 lg + j;
    //  p.v   A = W^T (m = lr = (h, b), rows 4 lg + j), B = V (n = dims, rows 4 lg + j),
    //        D lane holds O^T rows (head lg, block j) at dims (tile, lr).
    const int lr = lane & 15, lg = lane >> 4;
    const int hq = lr >> 2, bq = lr & 3;   // the (head, block) column of this lane
    // Wave w streams KV head kH hg + (w % kH), row set w / kH (see SplitShape).
    // XCD-aware order: workgroups are dealt to the 8 XCDs round-robin by
    // linear id (x fastest, then y, then z), so the grid is (split % 8, hg,
    // split / 8) — the head groups of one split share an XCD and hence its L2
    // copy of the rows' FP32 scale lines (one 128-byte line holds the scales of
    // all heads of a row). Three grid dimensions instead of a 1-D id keep two
    // integer divisions out of the kernel's start.
    const int hw = wave % kH, rs = wave / kH;
    const uint32_t hg = blockIdx.y;
    const uint32_t g = hg * kH + hw;
    const uint32_t split = blockIdx.z * 8 + blockIdx.x;
    // All arguments the first loads need are requested in one batch of scalar
    // loads (otherwise the idle-workgroup test below waits for n_splits first
    // and the rest is fetched in a second round trip).
    asm volatile("" ::"s"(a.n_rows), "s"(a.split_len), "s"(a.kv_dim), "s"(a.k.qs), "s"(a.k.d), "s"(a.v.qs),
                 "s"(a.v.d), "s"(a.q));
    if constexpr (kFused)
        asm volatile("" ::"s"(a.w_norms), "s"(a.rope_cs), "s"(a.pos), "s"(a.w_q_off), "s"(a.w_k_off),
                     "s"(a.k_cur), "s"(a.v_cur));
    if (split >= a.n_splits) return;
    const uint32_t row0 = min(split * a.split_len, a.n_rows);
    const uint32_t row_end = min(row0 + a.split_len, a.n_rows);
    // Last row a load may touch: row 0 when the range is empty (the fused step
    // at pos 0 streams no rows but still issues its unconditional first batch;
    // row 0 of the layer always exists since max_seq >= 1).
    const uint32_t row_last = row_end > 0 ? row_end - 1 : 0u;
    const float c2 = a.scale * kLog2e;   // scores in log2 units

    const uint32_t kv_dim = a.kv_dim;
    const uint32_t nb_row = a.kv_dim / kBlock;
    // 32-bit offsets from the layer bases (a layer's section is < 4 GiB).
    const uint32_t kcol = g * kHeadDim + 32 * lg;          // q.k: block lg
    const uint32_t vcol = g * kHeadDim + 8 * lr;           // p.v: dims 8 lr .. +8
    const uint32_t dcol = g * (kHeadDim / kBlock) + bq;    // scale of block bq
    auto load = [&](Batch& B, uint32_t b) {
        // row r0 + y, clamped to row_last, as base + min(y, lim) with a uniform
        // base and limit: the per-lane products are 24-bit (y < 16)
        const uint32_t r0 = row0 + 16u * (kRowSets * b + rs);
        const uint32_t base = min(r0, row_last), lim = row_last - base;
        const uint32_t qs_base = base * kv_dim, d_base = base * nb_row;
        const uint32_t kk = qs_base + __umul24(min(static_cast<uint32_t>(lr), lim), kv_dim) + kcol;
        B.kq[0] = *reinterpret_cast<const Q16*>(a.k.qs + kk);
        B.kq[1] = *reinterpret_cast<const Q16*>(a.k.qs + (kk + 16));
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t y = min(4u * lg + j, lim);
            // byte offsets in 32 bits: base (SGPRs) + one VGPR offset per load
            const uint32_t doff = (d_base + __umul24(y, nb_row) + dcol) * 4u;
            B.kd[j] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(a.k.d) + doff);
            B.vd[j] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(a.v.d) + doff);
            B.vv[j] = *reinterpret_cast<const u32x2*>(a.v.qs + (qs_base + __umul24(y, kv_dim) + vcol));
        }
    };
    const uint32_t n_rows = row_end - row0;
    const uint32_t n_batches =
        n_rows > 16u * rs ? (n_rows - 16u * rs + 16u * kRowSets - 1) / (16u * kRowSets) : 0u;
    // ---- query-side loads first (unconditional): waiting for them below then
    // leaves the first batch of rows in flight (loads retire in order). -----------
    const uint16_t* cs = a.rope_cs + static_cast<uint64_t>(a.pos) * kHeadDim + 2 * lane;
    // (kept as raw f16 bits until the first batch is requested: a conversion
    // here would wait for these loads before the batch's loads are issued)
    uint16_t qxr[kQPerWave][2] = {}, w0r = 0, w1r = 0, x0r = 0, x1r = 0, kw0r = 0, kw1r = 0;
    uint32_t csr = 0;
    Q16 qraw[4];   // q of head hq, dims 32 lg + 8 i .. +8
    // Fused step: wave w normalizes the workgroup's query heads kQPerWave w ..,
    // and waves w < 2 kH write row `pos` of KV head kH hg + (w % kH): K for
    // w < kH, V otherwise.
    const uint32_t qh0 = hg * kH * kGroup + kQPerWave * wave;
    const uint32_t g_wb = hg * kH + wave % kH;
    if constexpr (kFused) {
        const uint16_t* qr = a.q + static_cast<uint64_t>(qh0) * kHeadDim;
#pragma unroll
        for (int i = 0; i < kQPerWave; i++) {
            qxr[i][0] = qr[i * kHeadDim + lane];
            qxr[i][1] = qr[i * kHeadDim + lane + 64];
        }
        w0r = a.w_norms[a.w_q_off + lane];
        w1r = a.w_norms[a.w_q_off + lane + 64];
        csr = *reinterpret_cast<const uint32_t*>(cs);
        const uint16_t* src = (wave < kH ? a.k_cur : a.v_cur) + g_wb * kHeadDim;   // writeback input
        x0r = src[lane];
        x1r = src[lane + 64];
        kw0r = a.w_norms[a.w_k_off + lane];
        kw1r = a.w_norms[a.w_k_off + lane + 64];
    } else {
        const uint16_t* qp = a.q + (static_cast<uint64_t>(g) * kGroup + hq) * kHeadDim + 32 * lg;
#pragma unroll
        for (int i = 0; i < 4; i++) qraw[i] = *reinterpret_cast<const Q16*>(qp + 8 * i);
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t last_b = n_batches > 0 ? n_batches - 1 : 0u;
    Batch A, Bb;
    load(A, 0);   // unconditional (clamped rows) so that every path has the same loads pending
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (kFused) {
        float qx[kQPerWave][2];
#pragma unroll
        for (int i = 0; i < kQPerWave; i++) { qx[i][0] = h2f(qxr[i][0]); qx[i][1] = h2f(qxr[i][1]); }
        const float w0 = h2f(w0r), w1 = h2f(w1r), c0 = h2f(static_cast<uint16_t>(csr)),
                    s0 = h2f(static_cast<uint16_t>(csr >> 16));
        float x0 = h2f(x0r), x1 = h2f(x1r);
        const float kw0 = h2f(kw0r), kw1 = h2f(kw1r);
        // q_norm_rope (q_norm_rope_fused.wgsl:38-96), into LDS.
        uint16_t* qn = &qn_sh[0][0][0] + kQPerWave * wave * kHeadDim;
        uint16_t* qg = a.q_norm + static_cast<uint64_t>(qh0) * kHeadDim;
#pragma unroll
        for (int i = 0; i < kQPerWave; i++) {
            float o0, o1;
            norm_rope_pair(qx[i][0], qx[i][1], w0, w1, c0, s0, a.eps, o0, o1);
            qn[i * kHeadDim + lane] = f2h(o0);
            qn[i * kHeadDim + lane + 64] = f2h(o1);
            if (split == 0) {
                qg[i * kHeadDim + lane] = f2h(o0);
                qg[i * kHeadDim + lane + 64] = f2h(o1);
            }
        }
        if (split == a.n_splits - 1 && wave < 2 * kH) {
            // kv_writeback of row `pos` for KV head g_wb (kv_writeback_fused.wgsl):
            // K (norm + RoPE + Q8_0) or V (Q8_0).
            const uint64_t d_idx = static_cast<uint64_t>(a.pos) * nb_row + g_wb * (kHeadDim / kBlock);
            const uint64_t qs_idx = static_cast<uint64_t>(a.pos) * kv_dim + g_wb * kHeadDim;
            if (wave < kH) {
                norm_rope_pair(x0, x1, kw0, kw1, c0, s0, a.eps, x0, x1);
                quantize_store_pair(x0, x1, lane, const_cast<float*>(a.k.d) + d_idx,
                                    const_cast<int8_t*>(a.k.qs) + qs_idx);
            } else {
                quantize_store_pair(x0, x1, lane, const_cast<float*>(a.v.d) + d_idx,
                                    const_cast<int8_t*>(a.v.qs) + qs_idx);
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; i++) qraw[i] = *reinterpret_cast<const Q16*>(&qn_sh[hw][hq][32 * lg + 8 * i]);
    }
    // ---- B operand of q.k: q of head hq on block bq's k slots, zero elsewhere;
    // and the bias 1152 * sum(q over block bq) of the exact-f16 K trick. -----------
    f16x8 qop[4];
    float qsum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const f16x8 v = __builtin_bit_cast(f16x8, qraw[i]);
#pragma unroll
        for (int e = 0; e < 8; e++) qsum += static_cast<float>(v[e]);
        qop[i] = lg == bq ? v : f16x8{};
    }
    const float qb = 1152.0f * __shfl(qsum, lr + 16 * bq);   // from the lane holding block bq

    float lsum = 0.0f, m_run = -INFINITY;   // of head hq, unscaled score units
    f32x4 oacc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float bsum = 0.0f;   // column (hq, bq) sum of W, for the 1152 bias of V
    const h2 ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};

    // Scores of one batch (head hq, rows 4 lg + j), -inf past row_end.
    auto scores = [&](const Batch& B, uint32_t b, bool tail, float (&s)[4]) {
        // q.k on the matrix core: 4 MFMAs over the 32 bytes of block lg of row lr.
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t x = B.kq[i >> 1].w[2 * (i & 1)] ^ 0x80808080u;
            const uint32_t y = B.kq[i >> 1].w[2 * (i & 1) + 1] ^ 0x80808080u;
            const u32x4 kw = {__builtin_amdgcn_perm(kExp64, x, 0x04010400u), __builtin_amdgcn_perm(kExp64, x, 0x04030402u),
                              __builtin_amdgcn_perm(kExp64, y, 0x04010400u), __builtin_amdgcn_perm(kExp64, y, 0x04030402u)};
            d = mfma32(__builtin_bit_cast(f16x8, kw), qop[i], d);
        }
        // s(row 4 lg + j, head hq) = sum over the 4 blocks (the lane quad) of d_b * (D - bias).
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float v = B.kd[j] * (d[j] - qb);
            v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
            v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
            s[j] = v;
        }
        if (tail) {
            const uint32_t r0 = row0 + 16u * (kRowSets * b + rs) + 4u * lg;
#pragma unroll
            for (int j = 0; j < 4; j++) s[j] = r0 + j < row_end ? s[j] : -INFINITY;
        }
    };
    // Running max of head hq over the rows seen so far (exact), with the
    // rescale of O and the sums when it moves.
    auto update_max = [&](float bl) {
        const float bm = max_xor32(max_xor16(bl));
        const float m_new = fmaxf(m_run, bm);
        if (__builtin_amdgcn_ballot_w64(m_new != m_run) != 0) {
            const float alpha = __builtin_amdgcn_exp2f((m_run - m_new) * c2);   // 0 on the first batch
            lsum *= alpha;
            bsum *= alpha;
            // alpha of head lg: every lane of head h's quads holds it; lane
            // 20 h (lr = 4 h, row h) is read into a scalar register per head
            const float a0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), 0));
            const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), 20));
            const float a2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), 40));
            const float a3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), 60));
            const float ao = pick4(f32x4{a0, a1, a2, a3}, lg);   // head lg
#pragma unroll
            for (int i = 0; i < 8; i++) oacc[i] *= ao;
            m_run = m_new;
        }
    };
    // p = exp2 of the scores and O^T += W^T V for one batch.
    auto pv = [&](const Batch& B, const float (&s)[4]) {
        const float mc = m_run * c2;
        float w[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j], c2, -mc));
            lsum += p;
            w[j] = p * B.vd[j];
        }
        // A operand (W^T row (hq, bq), rows 4 lg + j) as two f16 terms.
        f16x4 whi, wlo;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            whi[j] = static_cast<_Float16>(w[j]);
            wlo[j] = static_cast<_Float16>(w[j] - static_cast<float>(whi[j]));
        }
        bsum = __builtin_amdgcn_fdot2(h2{whi[0], whi[1]}, ones, bsum, false);
        bsum = __builtin_amdgcn_fdot2(h2{whi[2], whi[3]}, ones, bsum, false);
        bsum = __builtin_amdgcn_fdot2(h2{wlo[0], wlo[1]}, ones, bsum, false);
        bsum = __builtin_amdgcn_fdot2(h2{wlo[2], wlo[3]}, ones, bsum, false);
        // B operand per output tile tt (dim 8 lr + tt): the 4 rows' bytes of
        // that dim, byte-transposed, as exact f16 values 1152 + v.
        uint32_t rw[4][2];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            rw[j][0] = B.vv[j].x ^ 0x80808080u;
            rw[j][1] = B.vv[j].y ^ 0x80808080u;
        }
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            const uint32_t t01l = __builtin_amdgcn_perm(rw[1][hf], rw[0][hf], 0x05010400u);   // r0b0 r1b0 r0b1 r1b1
            const uint32_t t01h = __builtin_amdgcn_perm(rw[1][hf], rw[0][hf], 0x07030602u);   // r0b2 r1b2 r0b3 r1b3
            const uint32_t t23l = __builtin_amdgcn_perm(rw[3][hf], rw[2][hf], 0x05010400u);
            const uint32_t t23h = __builtin_amdgcn_perm(rw[3][hf], rw[2][hf], 0x07030602u);
            const uint32_t src01[4] = {t01l, t01l, t01h, t01h};
            const uint32_t src23[4] = {t23l, t23l, t23h, t23h};
#pragma unroll
            for (int dd = 0; dd < 4; dd++) {
                const uint32_t sel = (dd & 1) ? 0x04030402u : 0x04010400u;
                const u32x2 bv = {__builtin_amdgcn_perm(kExp64, src01[dd], sel), __builtin_amdgcn_perm(kExp64, src23[dd], sel)};
                const f16x4 bop = __builtin_bit_cast(f16x4, bv);
                const int tt = 4 * hf + dd;
                oacc[tt] = mfma16(whi, bop, oacc[tt]);
                oacc[tt] = mfma16(wlo, bop, oacc[tt]);
            }
        }
    };

    auto consume = [&](const Batch& B, uint32_t b, bool tail) {
        float s[4];
        scores(B, b, tail, s);
        update_max(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
        pv(B, s);
    };
    // Two batches as one: both batches' scores first (independent MFMA and
    // VALU chains), one max update, then both P.V steps.
    auto consume2 = [&](const Batch& B0, uint32_t b0, const Batch& B1, uint32_t b1, bool tail) {
        float s0[4], s1[4];
        scores(B0, b0, false, s0);
        scores(B1, b1, tail, s1);
        update_max(fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])), fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3]))));
        pv(B0, s0);
        pv(B1, s1);
    };

    // Loads are unconditional (an index past the end re-reads the last batch,
    // an L2 hit) so that each wait leaves the next batch in flight.
    if (n_batches == 2) {
        // the two batches are already both in flight: consume them together
        load(Bb, 1);
        __builtin_amdgcn_sched_barrier(0);
        consume2(A, 0, Bb, 1, true);
    } else if (n_batches > 0) {
        uint32_t b = 0;
        while (true) {
            load(Bb, min(b + 1, last_b));
            __builtin_amdgcn_sched_barrier(0);
            if (b == last_b) { consume(A, b, true); break; }
            consume(A, b, false);
            ++b;
            load(A, min(b + 1, last_b));
            __builtin_amdgcn_sched_barrier(0);
            if (b == last_b) { consume(Bb, b, true); break; }
            consume(Bb, b, false);
            ++b;
        }
    }

    // ---- per-wave totals: l and the W column sums over the 4 row groups; O of
    // head lg, dims 8 lr .. +8 minus the 1152 bias of V -----------------------
    lsum = sum_xor32(sum_xor16(lsum));
    const float bs = sum_xor32(sum_xor16(bsum));
    const float bias = 1152.0f * __shfl(bs, 4 * lg + (lr >> 2));
    {
        float ov[8];
#pragma unroll
        for (int tt = 0; tt < 8; tt++) ov[tt] = pick4(oacc[tt], lr >> 2) - bias;
        float* dst = &o_red[wave][lg][8 * lr];
        *reinterpret_cast<float4*>(dst) = make_float4(ov[0], ov[1], ov[2], ov[3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(ov[4], ov[5], ov[6], ov[7]);
    }
    if (lg == 0 && bq == 0) {   // lane 4 h: head h's (m, l), m in log2 units
        ml_sh[wave][hq][0] = m_run * c2;
        ml_sh[wave][hq][1] = lsum;
    }
    __syncthreads();

    // ---- merge the row sets: thread t -> query head t / (128 / kE) of the
    // workgroup's 4 kH (KV head fw, its head fh), dims kE (t % (128 / kE)) .. ----
    constexpr int kE = kH * kGroup * kHeadDim / (64 * kWaves);   // 2 or 4 dims per thread
    constexpr int kTpH = kHeadDim / kE;                           // threads per query head
    const int fq = t / kTpH, fw = fq >> 2, fh = fq & 3, fd = kE * (t % kTpH);
    float M = -INFINITY;
#pragma unroll
    for (int r = 0; r < kRowSets; r++) M = fmaxf(M, ml_sh[fw + kH * r][fh][0]);
    float L = 0.0f;
    float o[kE] = {};
#pragma unroll
    for (int r = 0; r < kRowSets; r++) {
        const int w = fw + kH * r;
        const float mw = ml_sh[w][fh][0];
        const float e = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);   // row sets without rows
        L = __builtin_fmaf(e, ml_sh[w][fh][1], L);
#pragma unroll
        for (int k = 0; k < kE; k++) o[k] = __builtin_fmaf(e, o_red[w][fh][fd + k], o[k]);
    }
    const uint32_t qhd = (hg * kH + fw) * kGroup + fh;
    if (!kFused && a.n_splits == 1) {
        const float inv_l = 1.0f / L;
#pragma unroll
        for (int k = 0; k < kE; k += 2)
            *reinterpret_cast<uint32_t*>(a.out + static_cast<uint64_t>(qhd) * kHeadDim + fd + k) =
                static_cast<uint32_t>(f2h(o[k] * inv_l)) | (static_cast<uint32_t>(f2h(o[k + 1] * inv_l)) << 16);
        return;
    }
    float* part = part_o(a.partials, qhd, a.n_splits, split);
#pragma unroll
    for (int k = 0; k < kE; k += 2) *reinterpret_cast<float2*>(part + fd + k) = make_float2(o[k], o[k + 1]);
    if (t % kTpH == 0)
        *reinterpret_cast<float2*>(part_ml(a.partials, a.kv_dim / kHeadDim * kGroup, qhd, a.n_splits, split)) =
            make_float2(M, L);
}

// One wave per (query head, 32-dim chunk); kLoads = 8 (up to 64 splits) or
// 16 (up to 128) partial loads per lane.
template <bool kFused, int kLoads>
__global__ __launch_bounds__(64) void decode_merge_kernel(
    float* partials_, uint32_t n_splits_, uint32_t kv_dim_, const uint16_t* q_norm_, const float* kd_row_,
    const int8_t* kq_row_, const float* vd_row_, const int8_t* vq_row_, DecodeArgs a) {
    const int lane = threadIdx.x;
    const uint32_t h = blockIdx.x >> 2, c = blockIdx.x & 3;
    const uint32_t g = h / kGroup;
    const uint32_t ns = n_splits_;
    const float* ph = part_o(partials_, h, ns, 0);
    const float* pml = part_ml(partials_, kv_dim_ / kHeadDim * kGroup, h, ns, 0);
    const float c2 = a.scale * kLog2e;

    // O chunk loads: lane -> splits (lane >> 3) + 8i, dims 32c + 4 (lane & 7) .. +3.
    const int f4 = lane & 7;
    float4 ov[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; i++) {
        const uint32_t s = min(static_cast<uint32_t>((lane >> 3) + 8 * i), ns - 1);
        ov[i] = *reinterpret_cast<const float4*>(ph + static_cast<uint64_t>(s) * kHeadDim + 32 * c + 4 * f4);
    }
    // (m, l): with kLoads = 8 (up to 64 splits) of the same splits as this
    // lane's O loads, (lane >> 3) + 8 i, so that the weights are computed
    // in-lane; with 16, of splits lane and lane + 64 (two loads; the weights
    // are then exchanged between lanes, which measured faster there).
    constexpr bool kInLane = kLoads <= 8;
    float2 mlv[kLoads];
    float m_s0 = -INFINITY, m_s1 = -INFINITY;
    float2 ml0 = make_float2(-INFINITY, 0.0f), ml1 = make_float2(-INFINITY, 0.0f);
    if constexpr (kInLane) {
#pragma unroll
        for (int i = 0; i < kLoads; i++) {
            const uint32_t s = min(static_cast<uint32_t>((lane >> 3) + 8 * i), ns - 1);
            mlv[i] = *reinterpret_cast<const float2*>(pml + 2 * s);
        }
    } else {
        const uint32_t ls0 = min(static_cast<uint32_t>(lane), ns - 1), ls1 = min(static_cast<uint32_t>(lane) + 64u, ns - 1);
        ml0 = *reinterpret_cast<const float2*>(pml + 2 * ls0);
        ml1 = *reinterpret_cast<const float2*>(pml + 2 * ls1);
        m_s0 = static_cast<uint32_t>(lane) < ns ? ml0.x : -INFINITY;
        m_s1 = static_cast<uint32_t>(lane) + 64u < ns ? ml1.x : -INFINITY;
    }

    float s_new = -INFINITY;   // log2-domain score of the new row (fused step)
    // Row `pos` of V for dims d0 .. d0 + 3 (lanes 0-7 use it), loaded up front with
    // everything else so that the pass has a single memory round trip.
    const uint32_t d0 = 32 * c + 4 * f4;
    float vd_new = 0.0f;
    uint32_t vq_new = 0;
    if constexpr (kFused) {
        const uint16_t* qn = q_norm_ + static_cast<uint64_t>(h) * kHeadDim;
        const float* kd = kd_row_ + g * (kHeadDim / kBlock);
        const int8_t* kq = kq_row_ + g * kHeadDim;
        vd_new = vd_row_[g * (kHeadDim / kBlock) + (d0 >> 5)];
        vq_new = *reinterpret_cast<const uint32_t*>(vq_row_ + g * kHeadDim + d0);
        const uint16_t qa = qn[lane], qb = qn[lane + 64];
        const float q0 = h2f(qa), q1 = h2f(qb);
        const float k0 = kd[lane >> 5] * static_cast<float>(kq[lane]);
        const float k1 = kd[2 + (lane >> 5)] * static_cast<float>(kq[lane + 64]);
        s_new = wave_sum(q0 * k0 + q1 * k1) * c2;
        // q_norm_rope output: element 32 c + lane, already in a register of this wave.
        const uint16_t qv = static_cast<uint16_t>(__shfl(static_cast<int>(c < 2 ? qa : qb), static_cast<int>((32 * c + lane) & 63)));
        if (lane < 32) a.q_act[h * kHeadDim + 32 * c + lane] = qv;
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    float M, L, w_new;
    if constexpr (kInLane) {
        float mloc = -INFINITY;
#pragma unroll
        for (int i = 0; i < kLoads; i++) {
            if (static_cast<uint32_t>((lane >> 3) + 8 * i) >= ns) mlv[i].x = -INFINITY;   // clamped re-reads
            mloc = fmaxf(mloc, mlv[i].x);
        }
        M = fmaxf(wave_max(mloc), s_new);
        w_new = kFused ? __builtin_amdgcn_exp2f(s_new - M) : 0.0f;
        float lloc = 0.0f;
#pragma unroll
        for (int i = 0; i < kLoads; i++) {
            // 0 for splits >= ns and for splits without rows (m = -inf)
            const float wi = mlv[i].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mlv[i].x - M);
            lloc = __builtin_fmaf(wi, mlv[i].x == -INFINITY ? 0.0f : mlv[i].y, lloc);
            acc.x = __builtin_fmaf(wi, ov[i].x, acc.x);
            acc.y = __builtin_fmaf(wi, ov[i].y, acc.y);
            acc.z = __builtin_fmaf(wi, ov[i].z, acc.z);
            acc.w = __builtin_fmaf(wi, ov[i].w, acc.w);
        }
        // the 8 lane groups (lane >> 3) hold disjoint split sets: sum over them
        L = sum_slots(lloc) + w_new;
    } else {
        M = fmaxf(wave_max(fmaxf(m_s0, m_s1)), s_new);
        const float w0 = m_s0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_s0 - M);   // 0 for splits >= ns
        const float w1 = m_s1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_s1 - M);
        w_new = kFused ? __builtin_amdgcn_exp2f(s_new - M) : 0.0f;
        L = wave_sum(w0 * (m_s0 == -INFINITY ? 0.0f : ml0.y) + w1 * (m_s1 == -INFINITY ? 0.0f : ml1.y)) + w_new;
#pragma unroll
        for (int i = 0; i < kLoads; i++) {
            const float wi = __shfl(i < 8 ? w0 : w1, (lane >> 3) + 8 * (i & 7));
            acc.x = __builtin_fmaf(wi, ov[i].x, acc.x);
            acc.y = __builtin_fmaf(wi, ov[i].y, acc.y);
            acc.z = __builtin_fmaf(wi, ov[i].z, acc.z);
            acc.w = __builtin_fmaf(wi, ov[i].w, acc.w);
        }
    }
    acc.x = sum_slots(acc.x);
    acc.y = sum_slots(acc.y);
    acc.z = sum_slots(acc.z);
    acc.w = sum_slots(acc.w);
    if (lane < 8) {
        if constexpr (kFused) {
            const float vd = vd_new;
            acc.x = __builtin_fmaf(w_new, vd * static_cast<float>(static_cast<int8_t>(vq_new)), acc.x);
            acc.y = __builtin_fmaf(w_new, vd * static_cast<float>(static_cast<int8_t>(vq_new >> 8)), acc.y);
            acc.z = __builtin_fmaf(w_new, vd * static_cast<float>(static_cast<int8_t>(vq_new >> 16)), acc.z);
            acc.w = __builtin_fmaf(w_new, vd * static_cast<float>(static_cast<int8_t>(vq_new >> 24)), acc.w);
        }
        const float inv_l = 1.0f / L;
        uint2 o;
        o.x = static_cast<uint32_t>(f2h(acc.x * inv_l)) | (static_cast<uint32_t>(f2h(acc.y * inv_l)) << 16);
        o.y = static_cast<uint32_t>(f2h(acc.z * inv_l)) | (static_cast<uint32_t>(f2h(acc.w * inv_l)) << 16);
        *reinterpret_cast<uint2*>(a.out + static_cast<uint64_t>(h) * kHeadDim + d0) = o;
    }
}

}  // namespace

void decode_plan(uint32_t n_rows, uint32_t n_kv_head, int cu_count, uint32_t min_split_rows,
                 uint32_t wide_min_rows, uint32_t* split_len, uint32_t* n_splits, uint32_t* heads_per_wg) {
    // Layout: 4 KV heads per workgroup from wide_min_rows rows on (long
    // contexts: rows are read whole), else 1 (short contexts: 4 waves per head
    // keep each wave's chain short). Then enough workgroups to fill every CU
    // at 2 waves per SIMD, but at least min_split_rows rows each (fewer
    // partials at short context) and at most kMaxSplits splits; rows per split
    // are a multiple of one batch of all row sets.
    const uint32_t h = n_rows >= wide_min_rows && n_kv_head % 4 == 0 ? 4 : 1;
    const uint32_t wg_per_cu = h == 1 ? SplitShape<1>::kWgPerCu : SplitShape<4>::kWgPerCu;
    const uint32_t batch_rows = 16u * (h == 1 ? SplitShape<1>::kRowSets : SplitShape<4>::kRowSets);
    const uint32_t target = static_cast<uint32_t>(cu_count > 0 ? cu_count : 256) * wg_per_cu;
    const uint32_t groups = n_kv_head / h;
    uint32_t want = (target + groups - 1) / groups;
    if (want < 1) want = 1;
    if (want > kMaxSplits) want = kMaxSplits;
    uint32_t len = (n_rows + want - 1) / want;
    if (len < min_split_rows) len = min_split_rows;
    len = (len + batch_rows - 1) / batch_rows * batch_rows;
    *split_len = len;
    *n_splits = n_rows == 0 ? 1 : (n_rows + len - 1) / len;
    *heads_per_wg = h;
}

uint32_t decode_max_splits() { return kMaxSplits; }
uint32_t decode_partial_stride() { return kPartStride; }

template <bool kFused>
static void launch_split(const DecodeArgs& a, uint32_t n_kv_head, hipStream_t s) {
    const uint32_t z = (a.n_splits + 7) / 8;
    if (a.heads_per_wg == 4)
        hipLaunchKernelGGL((decode_split_kernel<kFused, 4>), dim3(8, n_kv_head / 4, z),
                           dim3(SplitShape<4>::kThreads), 0, s, a);
    else
        hipLaunchKernelGGL((decode_split_kernel<kFused, 1>), dim3(8, n_kv_head, z),
                           dim3(SplitShape<1>::kThreads), 0, s, a);
}

// The arguments of the merge pass's first loads go first and as scalars, so
// that they are preloaded into SGPRs at wave launch (this file is compiled with
// kernarg preloading) instead of fetched by the wave's first scalar loads; the
// fused step's row `pos` is passed as row pointers for the same reason.
template <bool kFused>
static void launch_merge(const DecodeArgs& a, uint32_t n_kv_head, hipStream_t s) {
    const uint64_t row = a.pos;
    const uint32_t nb_row = a.kv_dim / kBlock;
    const float* kd_row = kFused ? a.k.d + row * nb_row : nullptr;
    const int8_t* kq_row = kFused ? a.k.qs + row * a.kv_dim : nullptr;
    const float* vd_row = kFused ? a.v.d + row * nb_row : nullptr;
    const int8_t* vq_row = kFused ? a.v.qs + row * a.kv_dim : nullptr;
    if (a.n_splits > 64)
        hipLaunchKernelGGL((decode_merge_kernel<kFused, 16>), dim3(n_kv_head * kGroup * 4), dim3(64), 0, s,
                           a.partials, a.n_splits, a.kv_dim, a.q_norm, kd_row, kq_row, vd_row, vq_row, a);
    else
        hipLaunchKernelGGL((decode_merge_kernel<kFused, 8>), dim3(n_kv_head * kGroup * 4), dim3(64), 0, s,
                           a.partials, a.n_splits, a.kv_dim, a.q_norm, kd_row, kq_row, vd_row, vq_row, a);
}

hipError_t launch_decode(const DecodeArgs& a, uint32_t n_kv_head, hipStream_t s) {
    launch_split<false>(a, n_kv_head, s);
    if (a.n_splits > 1)
        launch_merge<false>(a, n_kv_head, s);
    return hipGetLastError();
}

hipError_t launch_decode_step(const DecodeArgs& a, uint32_t n_kv_head, hipStream_t s) {
    launch_split<true>(a, n_kv_head, s);
    launch_merge<true>(a, n_kv_head, s);
    return hipGetLastError();
}

}  // namespace bp
