// Causal (chunked) prefill attention over the Q8_0 KV cache on f16 MFMA (gfx950).
//
// Same result as src/shaders/attention.wgsl (reference repository) — token m
// attends rows [0, cur) with cur = causal ? pos + m + 1 : pos, f32 softmax,
// f16 output. Three forms, chosen by the host from the shapes:
//
// 1. Image pass + prefill32_kernel (long prompts): kv_dequant_kernel (or the
//    fused step's prefill_prep_kernel) writes the layer's K and V for rows
//    [0, cur of the last token) as an f16 image (f16(d * q) per value, plus a
//    K residual below), per KV head and 64-row chunk laid out as its LDS
//    image, so that a chunk is one linear copy; prefill32_kernel runs on
//    v_mfma_f32_32x32x16_f16 with 4 query heads x 32 tokens per role and the
//    two waves of each SIMD one phase apart (its own comment below).
// 2. Image pass + prefill_kernel<1, 8> / <1, 4> (shorter prompts): one query
//    head per wave on v_mfma_f32_16x16x32_f16, two or four workgroups per
//    (KV head, tile pair), so that small grids still fill the CUs.
// 3. prefill_split_kernel + prefill_merge_kernel (few tokens over a long
//    cache): the keys split over workgroups that read the cache's Q8_0 rows
//    themselves (no image), partials merged by their log-sum-exp weights.
//
// prefill_kernel, a flash-attention over LDS tiles of the image:
//  * Query tokens form tiles of 32; a "unit" is 16 tokens x 1 GQA head (one
//    wave's MFMA columns). A workgroup owns one KV head and a zig-zag PAIR of
//    tiles: light tile A = p, heavy tile B = n_tiles-1-p (grid KV head
//    fastest: one head per XCD). Two 8-wave workgroups split the 4 query
//    heads of a (KV head, pair), or four 4-wave workgroups (one query head
//    each, wave w on unit w & 1 of tile A if w < 2, of tile B otherwise).
//  * Work balance (split-K inside the workgroup): with n_A / n_B the 64-row
//    chunks tiles A / B attend and mid = ceil((n_A + n_B) / 2), the B waves
//    take B's chunks [0, mid) while the A waves take A's chunks [0, n_A) and
//    then B's chunks [mid, n_B); the two halves of B are merged through LDS at
//    the end (log-sum-exp). Every pair then runs ~(n_A + n_B) / 2 iterations
//    with two busy waves per SIMD, so the 256 CUs finish together. (A middle
//    tile paired with itself is simply split between its two waves.)
//  * Chunks are staged from two streams — stream 1 serves chunk i (A waves
//    while i < n_A, B waves), stream 2 serves B's chunk mid + i - n_A — copied
//    from the image straight into double-buffered LDS by global_load_lds (no
//    registers), so both MFMA operands are single 16-byte LDS reads. The
//    copies for iteration i+1 are issued during iteration i's q.k MFMAs.
//  * S^T = K Q^T with v_mfma_f32_16x16x32_f16 (K = 32 dims per step): the
//    output fragment of lane l holds 8 keys of token (l % 16) per 32 keys. With
//    the keys stored in V^T in the matching permuted order, those fragments are
//    directly the B operand of O^T = V^T P^T — no shuffles, no LDS trip.
//  * Online softmax in the exp2 domain (p = exp2(s * scale * log2 e - m) is
//    one FMA and one exp), row max across the 4 lane groups by lane-row
//    swaps (v_permlane16/32_swap), and a lazy running max (moved only by more than kLazy
//    log2 units), so the O accumulators are almost never touched by VALU.
//
// MFMA fragment layout used (v_mfma_f32_16x16x32_f16, lane l, g = l / 16):
//   A[i][k]: lane holds A[l % 16][8g .. 8g+7]
//   B[k][j]: lane holds B[8g .. 8g+7][l % 16]
//   D[i][j]: lane holds D[4g .. 4g+3][l % 16]
#include "bp_device.hpp"
#include "bp_kernels.hpp"
#include "bp_norm_rope.hpp"

namespace bp {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;               // cache rows per LDS chunk
constexpr int kSub = kChunk / 16;        // 16-row S^T sub-tiles per chunk
constexpr int kKHalves = kChunk * kHeadDim;   // K rows, 256 B each
constexpr int kVHalves = kHeadDim * kChunk;   // V^T rows (dims), 128 B each
constexpr int kLBytes = kChunk * kHeadDim;    // K residual rows, 128 B each
constexpr int kBufHalves = kKHalves + kVHalves + kLBytes / 2;   // one staged chunk (40 KB)
// The K residual is 2^11 (k - f16(k)) in fp6 (e2m3) with one power-of-two
// scale per 32-element block; the q.k correction MFMA applies that scale
// times 2^-11 through its E8M0 operand.
constexpr int kResidShift = 11;
constexpr int kE8M0Bias = 127;
constexpr float kLazy = 8.0f;            // lazy-rescale threshold (log2 units)
constexpr int kSplitStride = kHeadDim + 4;   // floats per key-split partial: O, m, l, 2 pad (16-byte rows)

struct alignas(16) U4 { uint32_t w[4]; };
typedef int i32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// c + (a . b) over 128 k of fp6 (e2m3) operands, each lane's 32 values
// scaled by 2^(sa - 127) (A) and 2^(sb - 127) (B): the q.k correction by the
// K residual. Lane l holds 32 k-values of row / column l % 16 in each
// operand, packed in the same element order for A and B (both by
// pack32_fp6), so the product pairs them whatever order the hardware walks k
// in. Elements 6, 7 of a and b are unused (fp6 operands are 6 registers).
__device__ __forceinline__ f32x4 mfma_resid(i32x8 a, i32x8 b, f32x4 c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 2, 2, 0, sa, 0, sb);
}
// Exponent e of the power-of-two block scale for fp6 e2m3 (largest finite
// 7.5): the smallest e with amax / 2^e <= 7.5, at least e_min, 0 for an
// all-zero block. From the bits of amax: amax = 1.f * 2^E, amax / 2^(E-2) =
// 4 * 1.f lies in [4, 8) and exceeds 7.5 exactly when f > 0.875.
__device__ __forceinline__ int fp6_scale_exp(float amax, int e_min) {
    const uint32_t b = __builtin_bit_cast(uint32_t, amax);
    if ((b & 0x7F800000u) == 0) return amax > 0.0f ? e_min : 0;   // zero or subnormal
    int e = static_cast<int>((b >> 23) & 0xFFu) - 127 - 2;
    if ((b & 0x007FFFFFu) > 0x00700000u) ++e;
    return e < e_min ? e_min : e;
}
// 32 floats / 2^e -> 32 fp6 e2m3 values (round to nearest even, saturating at
// +-7.5) packed 6 bits each into 6 words. The hardware conversion takes two
// 16-value halves and interleaves them: element 2j is v[j], 2j + 1 is v[16 + j].
// Issued as inline asm with an early-clobber result: the compiler's builtin
// may give the result registers that overlap the sources, and the instruction
// then returns wrong values (measured on the box with dense inputs: every
// element of a 32x32x64 product off; zero errors with disjoint registers).
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x6 __attribute__((ext_vector_type(6)));
__device__ __forceinline__ i32x6 cvt_fp6x32(const f32x16& lo, const f32x16& hi, float scale) {
    i32x6 r;
    asm volatile("v_cvt_scalef32_2xpk16_fp6_f32 %0, %1, %2, %3" : "=&v"(r) : "v"(lo), "v"(hi), "v"(scale));
    return r;
}
__device__ __forceinline__ i32x6 pack32_fp6(const float (&v)[32], int e) {
    f32x16 lo, hi;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        lo[i] = v[i];
        hi[i] = v[16 + i];
    }
    return cvt_fp6x32(lo, hi, __builtin_bit_cast(float, static_cast<uint32_t>(e + 127) << 23));
}

// Position of chunk row `key` (0..63) along the MFMA k axis of the PV step:
// per 32 keys, lane group g holds S^T rows {4g..4g+3} (first sub-tile) and
// {16+4g..16+4g+3} (second), which become its k slots 8g..8g+3, 8g+4..8g+7.
__device__ __forceinline__ int v_slot(int key) {
    const int k = key & 31;
    const int s = k < 16 ? 8 * (k >> 2) + (k & 3) : 8 * ((k - 16) >> 2) + 4 + (k & 3);
    return (key & 32) + s;
}
// The same for the 32x32x16 layout of prefill32_kernel: the S^T fragment of
// lane (c, g) holds keys 8j + 4g + i (acc 4j + i) of a 32-key tile, and the
// P^T operand of a 16-key step takes acc 8h .. 8h + 7 as its k slots
// 8g .. 8g + 7, so slot 8g + e holds key 16h + 4g + (e & 3) + 8 (e >> 2):
// within each 16 keys, bits 2 and 3 of the key index swapped.
__device__ __forceinline__ int v_slot32(int key) { return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1); }
// Bank-conflict swizzles of the staged chunk (no padding, so that the image
// in global memory is the LDS image and a chunk is one linear copy):
// 16-byte group j of K row r sits at group j ^ (r & 15); group j of V^T row
// (dim) d at group j ^ (d & 7).
__device__ __forceinline__ int k_addr(int row, int group) {
    return row * kHeadDim + 8 * (group ^ (row & 15));
}
__device__ __forceinline__ int v_addr(int dim, int group) {
    return dim * kChunk + 8 * (group ^ (dim & 7));
}
// Byte address of 16-byte group j of K-residual row r: j ^ (r & 7).
__device__ __forceinline__ int l_addr(int row, int group) {
    return row * kHeadDim + 16 * (group ^ (row & 7));
}
// The image of prefill32_kernel stores each section group-major instead:
// 16-byte group j of every row (dim) together, rows consecutive, so that the
// 32 lanes of a fragment read 512 contiguous bytes (no bank conflicts, no
// swizzle) and a lane's address for another group or row tile differs by a
// constant (an instruction offset, not a register per fragment).
__device__ __forceinline__ int k_addr32(int row, int group) { return (group * kChunk + row) * 8; }        // halves
__device__ __forceinline__ int l_addr32(int row, int group) { return (group * kChunk + row) * 16; }       // bytes
__device__ __forceinline__ int v_addr32(int dim, int group) { return (group * kHeadDim + dim) * 8; }     // halves

// Maximum across the 4 lane groups of a token column (lanes l, l^16, l^32,
// l^48), by lane-row swaps (no LDS round trip).
__device__ __forceinline__ float group_max(float v) { return max_xor32(max_xor16(v)); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// Two floats -> f16 pair with one packed round-to-nearest-even conversion.
__device__ __forceinline__ uint32_t pack2_rne(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, f16x2));
}
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return static_cast<uint32_t>(f2h(a)) | (static_cast<uint32_t>(f2h(b)) << 16);
}

// Image of one 64-row chunk (chunk c of KV head g) from its Q8_0 values, in
// three parts, each run by 256 threads (index t):
//  emit_k_rows: thread t -> row t >> 2, Q8_0 block t & 3 (kq0, kq1 its 32
//     bytes, kd its scale); writes 64 bytes of f16 and 32 bytes of residual;
//  emit_v_lds: thread t -> rows 4 (t >> 4) .. +3, dims 8 (t & 15) .. +7 (vq[i]
//     the 8 bytes of row 4 (t >> 4) + i, vd[i] its scale); each dim's 4 values
//     are 4 consecutive V^T slots, one 8-byte write into the LDS tile vt;
//  emit_v_rows (after a barrier): thread t -> V^T dim t >> 1, slots 32 (t & 1)
//     .. +32 from vt to the image.
// Each value is the reference's f32 d * q; K keeps f16(k) plus 2^11 (k -
// f16(k)) in fp6 e2m3 with one power-of-two scale per 32-element block (the
// residual of a block: 6 words of fp6, its E8M0 scale exponent less 11 in
// word 6, word 7 zero), V keeps f16(v).
typedef uint16_t VTile[kHeadDim][kChunk + 8];
// (The *_at forms write a chunk image at the given base: global memory or LDS.)
__device__ __forceinline__ void emit_k_rows_at(uint16_t* kdst, uint8_t* ldst, uint32_t vt_order, int t, const U4& kq0,
                                               const U4& kq1, float kd) {
    const int kr = t >> 2, kb = t & 3;
    uint32_t w[16];
    float r[32];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t x = i < 4 ? kq0.w[i] : kq1.w[i - 4];
        float k[4];
        _Float16 h[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            k[e] = kd * static_cast<float>(static_cast<int8_t>(x >> (8 * e)));
            h[e] = static_cast<_Float16>(k[e]);
            r[4 * i + e] = (k[e] - static_cast<float>(h[e])) * static_cast<float>(1 << kResidShift);
            amax = fmaxf(amax, fabsf(r[4 * i + e]));
        }
        w[2 * i] = __builtin_bit_cast(uint32_t, f16x2{h[0], h[1]});
        w[2 * i + 1] = __builtin_bit_cast(uint32_t, f16x2{h[2], h[3]});
    }
    if (vt_order) {
        // prefill32_kernel's residual blocks follow its q.k fragments: block
        // (m, h) = 2 m + h of a row holds dims 64 m + 16 j + 8 h + e (j, e <
        // 4, 8), i.e. dims 8 h .. +7 and 16 + 8 h .. +7 of Q8_0 blocks 2 m and
        // 2 m + 1 (this thread, kb, and its neighbour kb ^ 1, lanes t and
        // t ^ 1). Thread kb builds block kb: it sends the neighbour the half
        // of its values that the neighbour's block holds.
        const bool odd = kb & 1;
        float sent[16], got[16];
#pragma unroll
        for (int e2 = 0; e2 < 8; e2++) {
            sent[e2] = r[(odd ? 0 : 8) + e2];
            sent[8 + e2] = r[(odd ? 16 : 24) + e2];
        }
#pragma unroll
        for (int i = 0; i < 16; i++) got[i] = lane_xor<1>(sent[i]);
        float v[32];
        amax = 0.0f;
#pragma unroll
        for (int e2 = 0; e2 < 8; e2++) {
            v[e2] = odd ? got[e2] : r[e2];                  // j = 0: block 2m, dims 8h + e
            v[8 + e2] = odd ? got[8 + e2] : r[16 + e2];     // j = 1: block 2m, dims 16 + 8h + e
            v[16 + e2] = odd ? r[8 + e2] : got[e2];         // j = 2: block 2m+1, dims 8h + e
            v[24 + e2] = odd ? r[24 + e2] : got[8 + e2];    // j = 3: block 2m+1, dims 16 + 8h + e
        }
#pragma unroll
        for (int i = 0; i < 32; i++) {
            r[i] = v[i];
            amax = fmaxf(amax, fabsf(v[i]));
        }
    }
    // block scale 2^e, applied by the MFMA as E8M0 e + 127 - 11 (>= 0)
    const int e = fp6_scale_exp(amax, kResidShift - kE8M0Bias);
    const i32x6 p6 = pack32_fp6(r, e);
    const uint32_t lo[8] = {static_cast<uint32_t>(p6[0]), static_cast<uint32_t>(p6[1]), static_cast<uint32_t>(p6[2]),
                            static_cast<uint32_t>(p6[3]), static_cast<uint32_t>(p6[4]), static_cast<uint32_t>(p6[5]),
                            static_cast<uint32_t>(e + kE8M0Bias - kResidShift), 0u};
#pragma unroll
    for (int i = 0; i < 4; i++)
        *reinterpret_cast<U4*>(kdst + (vt_order ? k_addr32(kr, 4 * kb + i) : k_addr(kr, 4 * kb + i))) =
            U4{{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]}};
#pragma unroll
    for (int i = 0; i < 2; i++)
        *reinterpret_cast<U4*>(ldst + (vt_order ? l_addr32(kr, 2 * kb + i) : l_addr(kr, 2 * kb + i))) =
            U4{{lo[4 * i], lo[4 * i + 1], lo[4 * i + 2], lo[4 * i + 3]}};
}
__device__ __forceinline__ void emit_k_rows(const PrefillArgs& a, uint32_t g, uint32_t c, int t, const U4& kq0,
                                            const U4& kq1, float kd) {
    emit_k_rows_at(a.k16 + (static_cast<uint64_t>(g) * a.ws_chunks + c) * kKHalves,
                   a.kl8 + (static_cast<uint64_t>(g) * a.ws_chunks + c) * kLBytes, a.vt_order, t, kq0, kq1, kd);
}
__device__ __forceinline__ void emit_v_lds(int t, const uint2 (&vq)[4], const float (&vd)[4], VTile& vt, bool o32) {
    const int vq4 = t >> 4, vdg = t & 15;
    const int slot = o32 ? v_slot32(4 * vq4) : v_slot(4 * vq4);   // rows 4 vq4 .. +3 -> slots slot .. slot + 3
#pragma unroll
    for (int e = 0; e < 8; e++) {   // dim 8 vdg + e
        uint16_t hv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t word = e < 4 ? vq[i].x : vq[i].y;
            const float v = vd[i] * static_cast<float>(static_cast<int8_t>(word >> (8 * (e & 3))));
            hv[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
        }
        *reinterpret_cast<uint2*>(&vt[8 * vdg + e][slot]) =
            make_uint2(hv[0] | (static_cast<uint32_t>(hv[1]) << 16), hv[2] | (static_cast<uint32_t>(hv[3]) << 16));
    }
}
__device__ __forceinline__ void emit_v_rows_at(uint16_t* vdst, uint32_t vt_order, int t, const VTile& vt) {
    const int dim = t >> 1, s0 = 32 * (t & 1);
#pragma unroll
    for (int i = 0; i < 4; i++)
        *reinterpret_cast<U4*>(vdst + (vt_order ? v_addr32(dim, (s0 >> 3) + i) : v_addr(dim, (s0 >> 3) + i))) =
            *reinterpret_cast<const U4*>(&vt[dim][s0 + 8 * i]);
}
__device__ __forceinline__ void emit_v_rows(const PrefillArgs& a, uint32_t g, uint32_t c, int t, const VTile& vt) {
    emit_v_rows_at(a.vt16 + (static_cast<uint64_t>(g) * a.ws_chunks + c) * kVHalves, a.vt_order, t, vt);
}

// The Q8_0 inputs of emit_k_rows / emit_v_lds from the cache, for chunk c of
// KV head g and thread t (0..255): unconditional loads of clamped rows; rows
// past n_rows get d = 0.
__device__ __forceinline__ void load_k_q8(const PrefillArgs& a, uint32_t g, uint32_t c, int t, U4& kq0, U4& kq1,
                                          float& kd) {
    const uint32_t nb_row = a.kv_dim / kBlock;
    const uint32_t last = a.n_rows - 1;
    const int kr = t >> 2, kb = t & 3;
    const uint32_t krow = c * kChunk + kr, krc = min(krow, last);
    const uint8_t* kqp = reinterpret_cast<const uint8_t*>(a.k.qs) + static_cast<uint64_t>(krc) * a.kv_dim + g * kHeadDim + 32 * kb;
    kq0 = *reinterpret_cast<const U4*>(kqp);
    kq1 = *reinterpret_cast<const U4*>(kqp + 16);
    kd = a.k.d[static_cast<uint64_t>(krc) * nb_row + g * (kHeadDim / kBlock) + kb];
    if (krow > last) kd = 0.0f;
}
__device__ __forceinline__ void load_v_q8(const PrefillArgs& a, uint32_t g, uint32_t c, int t, uint2 (&vq)[4],
                                          float (&vd)[4]) {
    const uint32_t nb_row = a.kv_dim / kBlock;
    const uint32_t last = a.n_rows - 1;
    const int vq4 = t >> 4, vdg = t & 15;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t row = c * kChunk + 4 * vq4 + i, rc = min(row, last);
        vq[i] = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(a.v.qs) +
                                                static_cast<uint64_t>(rc) * a.kv_dim + g * kHeadDim + 8 * vdg);
        vd[i] = a.v.d[static_cast<uint64_t>(rc) * nb_row + g * (kHeadDim / kBlock) + (vdg >> 2)];
        if (row > last) vd[i] = 0.0f;
    }
}

// Dequantization pass: one 256-thread workgroup per (64-row chunk, KV head)
// writes the chunk's image from the cache, zeros past n_rows.
__global__ __launch_bounds__(256) void kv_dequant_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) VTile vt;
    const int t = threadIdx.x;
    // Grid (KV head, chunk), KV head fastest (as in prefill_kernel): head g's
    // chunks are written on the XCD whose L2 serves head g in the attention pass.
    const uint32_t g = blockIdx.x, c = blockIdx.y;
    U4 kq0, kq1;
    float kd, vd[4];
    uint2 vq[4];
    load_k_q8(a, g, c, t, kq0, kq1, kd);
    load_v_q8(a, g, c, t, vq, vd);
    emit_k_rows(a, g, c, t, kq0, kq1, kd);
    emit_v_lds(t, vq, vd, vt, a.vt_order != 0);
    __syncthreads();
    emit_v_rows(a, g, c, t, vt);
}

// Preparation pass of the fused prefill step (m_tokens new tokens at cache
// rows [pos, pos + m_tokens)), in place of the dequantization pass. Work comes
// in halves of 64-row chunks (32 rows). Grid (KV head g, part y), 256 threads:
// y < n_halves (both halves of every chunk the image covers, so that it is
// zero past n_rows) is part z = 0 of half y, then parts z = 1 .. 4 of each
// half that holds new rows:
//  z = 0: kv_writeback (kv_writeback_fused.wgsl) of the half's new rows of KV
//     head g into the cache, their Q8_0 bytes and scales also kept in LDS
//     (the half's other rows are read from the cache, rows < pos, or are zero,
//     rows past the last new row); then the half's image from those Q8_0
//     values, K rows by threads 0-127 while threads 128-255 transpose V.
//     Halves with no new row take their Q8_0 values from the cache directly.
//  z = 1 .. 4: q_norm_rope (q_norm_rope_fused.wgsl) of query head 4 g + z - 1
//     for the half's new tokens, in place.
// Both use the 8-lane item form of the standalone kernels (bp_norm_rope.hpp),
// one item per 8 lanes (32 items: every new row or token of the half at
// once), so q, the cache bytes and the image are bit for bit those of
// q_norm_rope + kv_writeback + the dequantization pass. Every offset is
// 8-element aligned (the host checks it), so all item loads and stores are 16
// bytes. The image helpers take thread indices of a whole-chunk workgroup
// (0..255): half h's K rows are those of threads 128 h .. +127, its V rows
// those of emit_v_lds threads 128 h .. +127, and its V^T slots those of
// emit_v_rows threads 2 d + h.
constexpr int kPrepThreads = 256;
constexpr int kHalf = kChunk / 2;
__global__ __launch_bounds__(kPrepThreads, 4) void prefill_prep_kernel(PrefillArgs a, PrefillStepArgs w) {
    __shared__ __attribute__((aligned(16))) VTile vt;
    __shared__ __attribute__((aligned(16))) uint8_t sq[2][kHalf][kHeadDim];   // K, V bytes of the half
    __shared__ float sd[2][kHalf][kHeadDim / kBlock];                        // their scales
    const int t = threadIdx.x;
    const int lane = t & 63, L = lane & (kItemLanes - 1);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    // part-0 halves: every half of the image (whole chunks: the image is zero
    // past n_rows), or with no image (direct) those holding new rows
    const uint32_t half0 = a.direct ? a.pos / kHalf : 0u;
    const uint32_t n_halves = a.direct ? (a.n_rows + kHalf - 1) / kHalf - half0 : 2 * ((a.n_rows + kChunk - 1) / kChunk);
    const uint32_t g = blockIdx.x;
    const uint32_t qi = blockIdx.y - n_halves;   // wraps (large) for part 0
    const bool q_part = blockIdx.y >= n_halves;
    const uint32_t hc = q_part ? a.pos / kHalf + (qi >> 2) : half0 + blockIdx.y;   // half index
    const uint32_t part = q_part ? 1 + (qi & 3) : 0u;
    const uint32_t c = hc >> 1, half = hc & 1;   // chunk, and which half of it
    const uint32_t row0 = hc * kHalf;
    const uint32_t new_lo = max(row0, a.pos), new_hi = min(row0 + kHalf, a.pos + a.m_tokens);
    const bool k_side = wave < 2;                 // threads 0-127: K rows; 128-255: V
    const int tq = t & 127;                       // thread index within the side
    const int tk = tq + 128 * half;               // emit_k_rows / emit_v_lds thread of this half
    U4 kq0, kq1;
    float kd, vd[4];
    uint2 vq[4];
    if (new_lo >= new_hi) {   // rows before pos only (q parts are launched for halves with new rows)
        if (k_side) {
            load_k_q8(a, g, c, tk, kq0, kq1, kd);
            emit_k_rows(a, g, c, tk, kq0, kq1, kd);
        } else {
            load_v_q8(a, g, c, tk, vq, vd);
            emit_v_lds(tk, vq, vd, vt, a.vt_order != 0);
        }
        __syncthreads();
        if (!k_side) emit_v_rows(a, g, c, 2 * tq + half, vt);
        return;
    }
    const uint32_t n_new = new_hi - new_lo, tok0 = new_lo - a.pos;
    const uint32_t item_raw = 8 * wave + (lane >> 3);   // this lane's item (0..31)
    const bool live = item_raw < n_new;
    const uint32_t item = live ? item_raw : n_new - 1;  // dead items compute on a clamped one
    if (part > 0) {
        // ---- q_norm_rope of query head 4 g + z - 1, token tok0 + item ----
        const uint32_t tok = tok0 + item;
        uint16_t* q = w.q_act + static_cast<uint64_t>(tok) * a.q_stride + (g * kGroup + part - 1) * kHeadDim;
        const uint4 qx0 = *reinterpret_cast<const uint4*>(q + 8 * L);
        const uint4 qx1 = *reinterpret_cast<const uint4*>(q + 64 + 8 * L);
        const uint16_t* cs = w.rope_cs + static_cast<uint64_t>(a.pos + tok) * kHeadDim + 16 * L;
        const uint4 c0 = *reinterpret_cast<const uint4*>(cs), c1 = *reinterpret_cast<const uint4*>(cs + 8);
        float wq0[8], wq1[8], x0[8], x1[8];
        load8<true>(w.w_norms + w.w_q_off + 8 * L, wq0);
        load8<true>(w.w_norms + w.w_q_off + 64 + 8 * L, wq1);
        unpack8(qx0, x0);
        unpack8(qx1, x1);
        norm_rope8_vals(x0, x1, wq0, wq1, c0, c1, w.eps);
        if (live) {
            store8<true>(q + 8 * L, x0);   // q_norm_rope_fused.wgsl:95
            store8<true>(q + 64 + 8 * L, x1);
        }
        return;
    }
    const uint32_t nb_row = a.kv_dim / kBlock;
    // ---- loads first: the half's other rows (thread -> K or V, row tq >> 2,
    // block tq & 3), then the new row of this lane's item ----
    const uint32_t orr = tq >> 2, okb = tq & 3, orow = row0 + orr;
    const bool other = orow < new_lo || orow >= new_hi;
    uint4 o0 = make_uint4(0, 0, 0, 0), o1 = o0;
    float od = 0.0f;
    if (other && orow < a.pos && !a.direct) {
        const int8_t* qs = k_side ? a.k.qs : a.v.qs;
        const float* dd = k_side ? a.k.d : a.v.d;
        const uint64_t qo = static_cast<uint64_t>(orow) * a.kv_dim + g * kHeadDim + 32 * okb;
        o0 = *reinterpret_cast<const uint4*>(qs + qo);
        o1 = *reinterpret_cast<const uint4*>(qs + qo + 16);
        od = dd[static_cast<uint64_t>(orow) * nb_row + g * (kHeadDim / kBlock) + okb];
    }
    const uint32_t row = new_lo + item, tok = row - a.pos;
    const uint64_t tok_off = static_cast<uint64_t>(tok) * a.kv_dim + g * kHeadDim;
    const uint4 kx0 = *reinterpret_cast<const uint4*>(w.k_cur + tok_off + 8 * L);
    const uint4 kx1 = *reinterpret_cast<const uint4*>(w.k_cur + tok_off + 64 + 8 * L);
    const uint4 vx0 = *reinterpret_cast<const uint4*>(w.v_cur + tok_off + 8 * L);
    const uint4 vx1 = *reinterpret_cast<const uint4*>(w.v_cur + tok_off + 64 + 8 * L);
    const uint16_t* cs = w.rope_cs + static_cast<uint64_t>(row) * kHeadDim + 16 * L;
    const uint4 c0 = *reinterpret_cast<const uint4*>(cs), c1 = *reinterpret_cast<const uint4*>(cs + 8);
    float wk0[8], wk1[8];
    load8<true>(w.w_norms + w.w_k_off + 8 * L, wk0);
    load8<true>(w.w_norms + w.w_k_off + 64 + 8 * L, wk1);
    // ---- kv_writeback of the new rows: cache and LDS ----
    {
        float k0[8], k1[8], v0[8], v1[8];
        unpack8(kx0, k0);
        unpack8(kx1, k1);
        unpack8(vx0, v0);
        unpack8(vx1, v1);
        norm_rope8_vals(k0, k1, wk0, wk1, c0, c1, w.eps);
        uint2 pk0, pk1, pv0, pv1;
        const float dk0 = quantize8(k0, pk0), dk1 = quantize8(k1, pk1);
        const float dv0 = quantize8(v0, pv0), dv1 = quantize8(v1, pv1);
        if (live) {
            const uint32_t rr = row - row0;
            const uint64_t qs_idx = static_cast<uint64_t>(row) * a.kv_dim + g * kHeadDim;
            const uint64_t d_idx = static_cast<uint64_t>(row) * nb_row + g * (kHeadDim / kBlock);
            *reinterpret_cast<uint2*>(w.k_qs + qs_idx + 8 * L) = pk0;
            *reinterpret_cast<uint2*>(w.k_qs + qs_idx + 64 + 8 * L) = pk1;
            *reinterpret_cast<uint2*>(w.v_qs + qs_idx + 8 * L) = pv0;
            *reinterpret_cast<uint2*>(w.v_qs + qs_idx + 64 + 8 * L) = pv1;
            *reinterpret_cast<uint2*>(&sq[0][rr][8 * L]) = pk0;
            *reinterpret_cast<uint2*>(&sq[0][rr][64 + 8 * L]) = pk1;
            *reinterpret_cast<uint2*>(&sq[1][rr][8 * L]) = pv0;
            *reinterpret_cast<uint2*>(&sq[1][rr][64 + 8 * L]) = pv1;
            if ((L & 3) == 0) {
                w.k_d[d_idx + (L >> 2)] = dk0;
                w.k_d[d_idx + 2 + (L >> 2)] = dk1;
                w.v_d[d_idx + (L >> 2)] = dv0;
                w.v_d[d_idx + 2 + (L >> 2)] = dv1;
                sd[0][rr][L >> 2] = dk0;
                sd[0][rr][2 + (L >> 2)] = dk1;
                sd[1][rr][L >> 2] = dv0;
                sd[1][rr][2 + (L >> 2)] = dv1;
            }
        }
    }
    if (a.direct) return;   // no image
    // ---- the half's other rows into LDS (zero past the new rows) ----
    if (other) {
        const int kv = k_side ? 0 : 1;
        *reinterpret_cast<uint4*>(&sq[kv][orr][32 * okb]) = o0;
        *reinterpret_cast<uint4*>(&sq[kv][orr][32 * okb + 16]) = o1;
        sd[kv][orr][okb] = od;
    }
    __syncthreads();
    // ---- the image, from the half's Q8_0 values in LDS ----
    if (k_side) {
        const int kr = tq >> 2, kb = tq & 3;
        kq0 = *reinterpret_cast<const U4*>(&sq[0][kr][32 * kb]);
        kq1 = *reinterpret_cast<const U4*>(&sq[0][kr][32 * kb + 16]);
        kd = sd[0][kr][kb];
        emit_k_rows(a, g, c, tk, kq0, kq1, kd);
    } else {
        const int vq4 = tq >> 4, vdg = tq & 15;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            vq[i] = *reinterpret_cast<const uint2*>(&sq[1][4 * vq4 + i][8 * vdg]);
            vd[i] = sd[1][4 * vq4 + i][vdg >> 2];
        }
        emit_v_lds(tk, vq, vd, vt, a.vt_order != 0);
    }
    __syncthreads();
    if (!k_side) emit_v_rows(a, g, c, 2 * tq + half, vt);
}

// Layouts (kHpw query heads per wave, kWaves waves per workgroup):
//  <1, 8>: short prompts: two workgroups (head sets) share a (KV head, tile
//      pair) and every wave does half the work, so that twice the workgroups run;
//  <1, 4>: shorter prompts: four workgroups of 4 waves (one query head each)
//      per (KV head, tile pair), one wave per SIMD.
template <int kHpw, int kWaves>
__global__ __launch_bounds__(64 * kWaves) void prefill_kernel(PrefillArgs a) {
    constexpr int kHeadsPerWave = kHpw;
    constexpr int kUnits = kWaves / 2;     // units per tile: (token half, head group)
    static_assert(kHpw == 1 && (kWaves == 8 || kWaves == 4), "layout");
    // lds[stream][buf]: staged chunk (K rows, V^T rows, K residual rows), 2
    // streams x 2 buffers (160 KB, all of the CU's LDS).
    __shared__ __attribute__((aligned(16))) uint16_t lds[2][2][kBufHalves];

    const int t = threadIdx.x;
    const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);   // uniform: scalar registers
    const int lr = lane & 15, lg = lane >> 4;
    const bool is_b = (wave & kUnits) != 0;          // B wave (heavy tile) or A wave
    // Grid (KV head, head set, tile pair), KV head fastest: workgroups are
    // dealt to the 8 XCDs round-robin by linear id (x fastest), so with 8 KV
    // heads each XCD serves one head and its L2 holds that head's K/V for all
    // the head's tile pairs. (Grid dimensions instead of a 1-D id: no integer
    // divisions at the kernel's start.)
    const uint32_t g = blockIdx.x, pair = blockIdx.z;
    const uint32_t hs = blockIdx.y;   // head set
    const uint32_t tile_a = pair, tile_b = a.n_tiles - 1 - pair;   // tile_b >= tile_a
    const uint32_t h0 = kWaves == 4 ? g * kGroup + hs   // first query head
                                    : g * kGroup + 2 * hs + kHeadsPerWave * ((wave >> 1) & 1);
    const uint32_t utok = 16 * (wave & 1);            // unit's first token within its tile
    const float c2 = a.scale * 1.4426950408889634f;   // scores in log2 units

    // Rows [0, kend) that tile x attends, and its chunk count.
    auto tile_kend = [&](uint32_t tile) {
        const uint32_t last = min(tile * kPrefillTileTok + kPrefillTileTok, a.m_tokens) - 1;
        return a.causal ? a.pos + last + 1 : a.pos;
    };
    const uint32_t kend_b = tile_kend(tile_b);
    const uint32_t n_tot = (kend_b + kChunk - 1) / kChunk;   // chunks tile B attends
    constexpr uint32_t c_lo = 0;
    const uint32_t n_b = n_tot;
    const uint32_t n_a = tile_b == tile_a ? 0u : (tile_kend(tile_a) + kChunk - 1) / kChunk;
    const uint32_t mid = (n_a + n_b + 1) / 2;        // B waves: [0, mid); A waves: [mid, n_b) of B
    const uint32_t n_iter = mid;                     // >= n_a + (n_b - mid)

    // ---- per-wave unit state -------------------------------------------------
    uint32_t wtok0 = 0, my_tok = 0, my_kend = 0, wave_kend = 0;
    bool unit_live = false;
    f16x8 qb[kHeadsPerWave][4];
    i32x8 q6[kHeadsPerWave];   // q of token my_tok, dims 32 lg .. +32, as fp6 (residual MFMA)
    int q6s[kHeadsPerWave];    // its E8M0 block scale
    f32x4 o[kHeadsPerWave][8];
    float m_run[kHeadsPerWave], l_run[kHeadsPerWave];
    f32x4 l_acc[kHeadsPerWave];   // row sums of P (every element holds the token's sum)
    const f16x8 ones8 = {1, 1, 1, 1, 1, 1, 1, 1};
    auto start_unit = [&](uint32_t tile) {
        wtok0 = tile * kPrefillTileTok + utok;
        my_tok = wtok0 + lr;
        unit_live = wtok0 < a.m_tokens;
        const uint32_t wave_last = min(wtok0 + 15, a.m_tokens - 1);
        wave_kend = unit_live ? (a.causal ? a.pos + wave_last + 1 : a.pos) : 0u;
        my_kend = a.causal ? a.pos + my_tok + 1 : a.pos;
#pragma unroll
        for (int h = 0; h < kHeadsPerWave; h++) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
                U4 raw = {{0, 0, 0, 0}};
                if (unit_live && my_tok < a.m_tokens)
                    raw = *reinterpret_cast<const U4*>(a.q + static_cast<uint64_t>(my_tok) * a.q_stride +
                                                       (h0 + h) * kHeadDim + 32 * kk + 8 * lg);
                qb[h][kk] = __builtin_bit_cast(f16x8, raw);
            }
            {
                U4 raw[4] = {};
                if (unit_live && my_tok < a.m_tokens) {
                    const uint16_t* qp = a.q + static_cast<uint64_t>(my_tok) * a.q_stride + (h0 + h) * kHeadDim + 32 * lg;
#pragma unroll
                    for (int i = 0; i < 4; i++) raw[i] = *reinterpret_cast<const U4*>(qp + 8 * i);
                }
                float qf[32];
                float amax = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const f16x8 v = __builtin_bit_cast(f16x8, raw[i]);
#pragma unroll
                    for (int j = 0; j < 8; j++) {
                        qf[8 * i + j] = static_cast<float>(v[j]);
                        amax = fmaxf(amax, fabsf(qf[8 * i + j]));
                    }
                }
                const int e = fp6_scale_exp(amax, -126);
                const i32x6 p6 = pack32_fp6(qf, e);
                q6[h] = i32x8{p6[0], p6[1], p6[2], p6[3], p6[4], p6[5], 0, 0};
                q6s[h] = e + kE8M0Bias;
            }
#pragma unroll
            for (int dt = 0; dt < 8; dt++) o[h][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
            m_run[h] = -INFINITY;
            l_run[h] = 0.0f;
            l_acc[h] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    // Normalize and store O (lane: token my_tok, dims 16dt + 4lg + j) by l_run,
    // the token's row sum.
    auto write_unit = [&]() {
        if (!unit_live || my_tok >= a.m_tokens) return;
#pragma unroll
        for (int h = 0; h < kHeadsPerWave; h++) {
            const float inv_l = 1.0f / l_run[h];
            uint16_t* out = a.out + static_cast<uint64_t>(my_tok) * a.q_stride + (h0 + h) * kHeadDim;
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                uint2 w;
                w.x = pack2(o[h][dt][0] * inv_l, o[h][dt][1] * inv_l);
                w.y = pack2(o[h][dt][2] * inv_l, o[h][dt][3] * inv_l);
                *reinterpret_cast<uint2*>(out + 16 * dt + 4 * lg) = w;
            }
        }
    };
    // A waves start on tile A (or, for a self-paired middle tile, directly on
    // the second half of it); B waves on tile B.
    start_unit(is_b || n_a == 0 ? tile_b : tile_a);

    // ---- staging: a chunk's K rows, V^T and K residual (40 KB, already
    // swizzled in the image) copied straight into LDS by global_load_lds (no
    // registers): each copy of a wave moves 1 KB, 16-byte pieces 64 (kWaves k +
    // w) + lane of K (1024 pieces), V^T (1024) and the residual (512). ---------
    const uint16_t* k16 = a.k16 + static_cast<uint64_t>(g) * a.ws_chunks * kKHalves;
    const uint16_t* vt16 = a.vt16 + static_cast<uint64_t>(g) * a.ws_chunks * kVHalves;
    const uint8_t* kl8 = a.kl8 + static_cast<uint64_t>(g) * a.ws_chunks * kLBytes;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    auto load_chunk = [&](uint16_t* buf, uint32_t c) {
        const uint16_t* ks = k16 + static_cast<uint64_t>(c) * kKHalves;
        const uint16_t* vs = vt16 + static_cast<uint64_t>(c) * kVHalves;
        const uint16_t* ls = reinterpret_cast<const uint16_t*>(kl8 + static_cast<uint64_t>(c) * kLBytes);
        constexpr int kKv = 16 / kWaves, kRes = 8 / kWaves;   // copies per wave: K (and V^T), residual
#pragma unroll
        for (int k = 0; k < 2 * kKv + kRes; k++) {
            const int sec = k < kKv ? 0 : k < 2 * kKv ? 1 : 2;   // K, V^T, residual
            const int kk = sec == 0 ? k : sec == 1 ? k - kKv : k - 2 * kKv;
            const int piece = 64 * (kWaves * kk + wv);           // 16-byte pieces within the section
            const uint16_t* src = (sec == 0 ? ks : sec == 1 ? vs : ls) + 8 * (piece + lane);
            uint16_t* dst = buf + (sec == 0 ? 0 : sec == 1 ? kKHalves : kKHalves + kVHalves) + 8 * piece;
            __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)src,
                                             (void __attribute__((address_space(3)))*)dst, 16, 0, 0);
        }
    };

    // ---- one chunk of attention for the current unit --------------------------
    // `issue` starts the copies of the next chunks; it runs once per call, in
    // the shadow of the q.k MFMAs (a copy's issue waits on the memory pipeline).
    auto compute = [&](const uint16_t* buf, uint32_t key0, auto&& issue) {
        if (!unit_live || key0 >= wave_kend) { issue(); return; }
        const uint16_t* kb = buf;
        const uint16_t* vb = buf + kKHalves;
        const uint8_t* lb = reinterpret_cast<const uint8_t*>(buf + kKHalves + kVHalves);
        // S^T = K Q^T, k-step outer: each step issues 8 independent MFMAs.
        f32x4 s[kHeadsPerWave][kSub];
#pragma unroll
        for (int h = 0; h < kHeadsPerWave; h++)
#pragma unroll
            for (int st2 = 0; st2 < kSub; st2++) s[h][st2] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
            f16x8 ka[kSub];
#pragma unroll
            for (int st2 = 0; st2 < kSub; st2++)
                ka[st2] = *reinterpret_cast<const f16x8*>(kb + k_addr(16 * st2 + lr, 4 * kk + lg));
#pragma unroll
            for (int st2 = 0; st2 < kSub; st2++)
#pragma unroll
                for (int h = 0; h < kHeadsPerWave; h++) s[h][st2] = mfma16(ka[st2], qb[h][kk], s[h][st2]);
        }
        // Residual correction: s += K residual . q on the fp6 matrix path, one
        // 128-deep MFMA per sub-tile and head; the lane's 32 bytes are its 32
        // residual values (6 words) and their E8M0 scale (word 6).
#pragma unroll
        for (int st2 = 0; st2 < kSub; st2++) {
            const int row = 16 * st2 + lr;
            const U4 r0 = *reinterpret_cast<const U4*>(lb + l_addr(row, 2 * lg));
            const U4 r1 = *reinterpret_cast<const U4*>(lb + l_addr(row, 2 * lg + 1));
            const i32x8 ra = {static_cast<int>(r0.w[0]), static_cast<int>(r0.w[1]), static_cast<int>(r0.w[2]),
                              static_cast<int>(r0.w[3]), static_cast<int>(r1.w[0]), static_cast<int>(r1.w[1]), 0, 0};
            const int sa = static_cast<int>(r1.w[2]);
#pragma unroll
            for (int h = 0; h < kHeadsPerWave; h++) s[h][st2] = mfma_resid(ra, q6[h], s[h][st2], sa, q6s[h]);
        }
        issue();
        // Mask (only chunks that reach past the unit's earliest visible row);
        // raw scores, the scale is applied inside the exponent.
        const bool need_mask = key0 + kChunk > (a.causal ? a.pos + wtok0 + 1 : a.pos);
        if (need_mask) {
#pragma unroll
            for (int h = 0; h < kHeadsPerWave; h++)
#pragma unroll
                for (int st2 = 0; st2 < kSub; st2++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        if (key0 + 16 * st2 + 4 * lg + j >= my_kend) s[h][st2][j] = -INFINITY;
        }
        // Online softmax (m_run in log2 units). Both heads' chunk maxima and the
        // (rare) rescale come first, so that the exponentials, P^T packing and
        // the P.V / row-sum MFMAs below form one block the scheduler can interleave.
        // Lazy rescale: the running max of a row moves only when the chunk max
        // exceeds it by more than kLazy; p then stays below 2^kLazy, which f16
        // P and the f32 accumulators hold as well as p <= 1. The test is made
        // first on each lane's own maximum and voted over the wave; only when
        // some lane passes it are the rows' maxima taken across their 4 lane
        // groups (scaling by c2 > 0 commutes with max, so this is the same test
        // and the same new max as on the row maxima).
        float lm[kHeadsPerWave];
        bool lane_up = false;
#pragma unroll
        for (int h = 0; h < kHeadsPerWave; h++) {
            float v = -INFINITY;
#pragma unroll
            for (int st2 = 0; st2 < kSub; st2++)
                v = fmax_p(v, fmax_p(fmax_p(s[h][st2][0], s[h][st2][1]), fmax_p(s[h][st2][2], s[h][st2][3])));
            lm[h] = v * c2;
            lane_up = lane_up || lm[h] > m_run[h] + kLazy;
        }
        if (__any(lane_up)) {
#pragma unroll
            for (int h = 0; h < kHeadsPerWave; h++) {
                const float cm = group_max(lm[h]);
                const bool up = cm > m_run[h] + kLazy;
                const float m_new = up ? cm : m_run[h];
                // 0 from -inf, 1 if kept (also for a row whose max is still
                // -inf, where the difference would be NaN)
                const float alpha = up ? __builtin_amdgcn_exp2f(m_run[h] - m_new) : 1.0f;
                m_run[h] = m_new;
                l_acc[h][0] *= alpha;   // only element 0 is read
#pragma unroll
                for (int dt = 0; dt < 8; dt++) o[h][dt] *= alpha;
            }
        }
        // P^T fragments, row sums (ones x P^T on the matrix core, so they use the
        // same f16-rounded P as O) and O^T += V^T P^T, per 32 keys.
#pragma unroll
        for (int kc = 0; kc < kSub / 2; kc++) {
            f16x8 pb[kHeadsPerWave];
#pragma unroll
            for (int h = 0; h < kHeadsPerWave; h++) {
                // m_run is still -inf only if every score of the token so far
                // is masked (a second-half unit whose first chunk lies past
                // the token's last row): then p = exp2(-inf) = 0, not NaN.
                const float neg_m = m_run[h] == -INFINITY ? 0.0f : -m_run[h];
                float p[8];
#pragma unroll
                for (int half = 0; half < 2; half++)
#pragma unroll
                    for (int j = 0; j < 4; j++)
                        p[4 * half + j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[h][2 * kc + half][j], c2, neg_m));
                U4 pk;
#pragma unroll
                for (int i = 0; i < 4; i++) pk.w[i] = pack2_rne(p[2 * i], p[2 * i + 1]);
                pb[h] = __builtin_bit_cast(f16x8, pk);
                l_acc[h] = mfma16(ones8, pb[h], l_acc[h]);
            }
#pragma unroll
            for (int dt = 0; dt < 8; dt++) {
                const f16x8 va = *reinterpret_cast<const f16x8*>(vb + v_addr(16 * dt + lr, 4 * kc + lg));
#pragma unroll
                for (int h = 0; h < kHeadsPerWave; h++) o[h][dt] = mfma16(va, pb[h], o[h][dt]);
            }
        }
    };

    // ---- main loop: iteration i computes stream-1 chunk i and (i >= n_a)
    // stream-2 chunk mid + i - n_a; loads for i+1 are issued first -----------
    auto c1_of = [&](uint32_t i) { return c_lo + i; };               // valid while i < mid
    auto has2 = [&](uint32_t i) { return i >= n_a && mid + (i - n_a) < n_b; };
    auto c2_of = [&](uint32_t i) { return c_lo + mid + (i - n_a); };
    // A copy into LDS completes when the issuing wave's vmcnt drains; the
    // barrier after that wait publishes it to the workgroup. (A key split
    // past the tile's last chunk has no iterations and copies nothing.)
    if (n_iter > 0) {
        load_chunk(lds[0][0], c1_of(0));
        if (has2(0)) load_chunk(lds[1][0], c2_of(0));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    for (uint32_t i = 0; i < n_iter; i++) {
        const int buf = i & 1;
        const bool next = i + 1 < n_iter, next2 = next && has2(i + 1);
        auto issue = [&]() {
            if (next) load_chunk(lds[0][buf ^ 1], c1_of(i + 1));
            if (next2) load_chunk(lds[1][buf ^ 1], c2_of(i + 1));
        };
        // One call site: a wave computes stream 1 (B waves; A waves while on
        // tile A) or stream 2 (A waves once on B's second half).
        const bool on1 = is_b || i < n_a;
        if (on1 || has2(i)) compute(lds[on1 ? 0 : 1][buf], (on1 ? c1_of(i) : c2_of(i)) * kChunk, issue);
        else issue();
        if (!is_b && i + 1 == n_a) {   // tile A done: store it, move to B's second half
#pragma unroll
            for (int h = 0; h < kHeadsPerWave; h++) l_run[h] = l_acc[h][0];
            write_unit();
            start_unit(tile_b);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    }

    // ---- merge the two halves of tile B: A waves hand (O, m, l) to B waves --
    // (the staging buffers are free: every wave is past the last barrier).
    float* xo = reinterpret_cast<float*>(&lds[0][0][0]);        // [kUnits][h][8 dt][4][64 lanes]
    float* xml = xo + kUnits * kHeadsPerWave * 8 * 4 * 64;      // [kUnits][h][2][64 lanes]
    const int unit = wave & (kUnits - 1);
    if (!is_b) {
#pragma unroll
        for (int h = 0; h < kHeadsPerWave; h++) {
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
#pragma unroll
                for (int j = 0; j < 4; j++) xo[(((unit * kHeadsPerWave + h) * 8 + dt) * 4 + j) * 64 + lane] = o[h][dt][j];
            xml[((unit * kHeadsPerWave + h) * 2 + 0) * 64 + lane] = m_run[h];
            xml[((unit * kHeadsPerWave + h) * 2 + 1) * 64 + lane] = l_acc[h][0];
        }
    }
    __syncthreads();
    if (!is_b) return;
    const bool split = mid < n_b;   // the A waves computed B's chunks [mid, n_b)
    float m_fin[kHeadsPerWave];
#pragma unroll
    for (int h = 0; h < kHeadsPerWave; h++) {
        float mb = m_run[h], lb = l_acc[h][0];
        m_fin[h] = mb;
        if (split) {
            const float ma = xml[((unit * kHeadsPerWave + h) * 2 + 0) * 64 + lane];
            const float la = xml[((unit * kHeadsPerWave + h) * 2 + 1) * 64 + lane];
            const float mm = fmaxf(mb, ma);
            const float eb = mb == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mb - mm);
            const float ea = ma == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ma - mm);
#pragma unroll
            for (int dt = 0; dt < 8; dt++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    o[h][dt][j] = o[h][dt][j] * eb + xo[(((unit * kHeadsPerWave + h) * 8 + dt) * 4 + j) * 64 + lane] * ea;
            lb = lb * eb + la * ea;
            m_fin[h] = mm;
        }
        l_run[h] = lb;
    }
    write_unit();
}

// Key-split merge: one wave per (token, query head) combines the n_ksplit
// (<= 64) partials by their log-sum-exp weights (as the decode merge,
// attention_merge.wgsl:85-129) and stores f16(O / L). Lane l reads dims
// 4 (l & 31) .. +3 of splits 2 k + (l >> 5), k < kLoads, all loads issued at
// once (past n_ksplit: the last split again, weight 0); lane s < n_ksplit
// holds split s's (m, l), its weight is fetched by a lane permute.
template <int kLoads>
__global__ __launch_bounds__(64) void prefill_merge_kernel(PrefillArgs a) {
    const int lane = threadIdx.x;
    const uint32_t tok = blockIdx.x, h = blockIdx.y;
    const uint32_t n_head = a.q_stride / kHeadDim, ns = a.n_ksplit;
    const float* pp = a.kpart + (static_cast<uint64_t>(tok) * n_head + h) * ns * kSplitStride;
    const int half = lane >> 5, d4 = 4 * (lane & 31);
    f32x4 ov[kLoads];
#pragma unroll
    for (int k = 0; k < kLoads; k++) {
        const uint32_t sp = min(static_cast<uint32_t>(2 * k + half), ns - 1);
        ov[k] = *reinterpret_cast<const f32x4*>(pp + sp * kSplitStride + d4);
    }
    float2 ml = make_float2(-INFINITY, 0.0f);
    if (static_cast<uint32_t>(lane) < ns) ml = *reinterpret_cast<const float2*>(pp + lane * kSplitStride + kHeadDim);
    const float M = wave_max(ml.x);
    const float w = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - M);   // 0 for splits without rows
    const float L = wave_sum(w * ml.y);
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < kLoads; k++) {
        const float wk = __shfl(w, 2 * k + half);   // lanes >= ns hold weight 0
        acc += wk * ov[k];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] += __shfl_xor(acc[i], 32);
    if (half == 0) {
        const float inv_l = 1.0f / L;
        uint2 o;
        o.x = pack2(acc[0] * inv_l, acc[1] * inv_l);
        o.y = pack2(acc[2] * inv_l, acc[3] * inv_l);
        *reinterpret_cast<uint2*>(a.out + static_cast<uint64_t>(tok) * a.q_stride + h * kHeadDim + d4) = o;
    }
}

// ============================================================================
// prefill32_kernel: the same attention (same image, same arithmetic: f16 K
// plus its fp6 residual, f16 V and P, f32 accumulation, exp2-domain online
// softmax with the lazy max) on v_mfma_f32_32x32x16_f16, with the two waves
// of each SIMD half an iteration apart so that one's softmax runs while the
// other's MFMAs do.
//
//  * Workgroup: 8 waves, one KV head g and a zig-zag pair of 32-token tiles
//    (light A = p, heavy B = n_tiles - 1 - p), processed one after the other,
//    so every pair runs about (n_A + n_B) / 2 iterations. Wave w owns query
//    head 4 g + (w & 3) for the tile's 32 tokens; "Y" waves (w >= 4) take the
//    first half of the tile's key chunks, "X" waves (w < 4) the second half,
//    and the halves are merged through LDS (log-sum-exp) at the end of the
//    tile. Waves w and w + 4 share a SIMD.
//  * Per 64-key chunk a wave runs an MFMA phase M(i) = S^T(i) = K Q^T (16
//    32x32x16 MFMAs + 4 fp6 residual MFMAs) and O^T += V^T P^T(i-1) (16
//    MFMAs), and a VALU phase V(i) = softmax of S^T(i) into P^T(i). Steps
//    alternate: in step 2i the X waves run M(i) while the Y waves run
//    V(i-1); in step 2i+1 the X waves run V(i) while the Y waves run M(i).
//    A barrier (no memory fence) ends each step.
//  * LDS: per stream (1: the Y waves' chunks, 2: the X waves') two K stages
//    (K rows + residual, 24 KB) and two V^T stages (16 KB), each a separate
//    object. A wave issues the copies of K(i+1) and V(i) of its own stream
//    at the start of its VALU phase V(i) and waits for them at the barrier
//    that ends it; they are first read in M(i+1).
//  * Fragments (lane l, c = l % 32, g = l / 32): S^T / O^T acc 4j + i holds
//    key (dim) 8j + 4g + i of token c; K / V^T operands hold row c, k slots
//    8g .. 8g + 7 of the 16-wide step; the P^T operand of 16-key step
//    h of a 32-key tile is acc 8h .. 8h + 7 (keys stored in V^T in v_slot32
//    order). The residual MFMA m (k = 64) pairs lane (c, g)'s 32 values of
//    residual block 2m + g of key c, dims 64m + 16j + 8g + e (the dims of its
//    q.k fragments in k-steps 4m .. 4m + 3), with q of token c at the same
//    dims, i.e. qb itself converted to fp6.
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32_resid(i32x8 a, i32x8 b, f32x16 c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 2, 2, 0, sa, 0, sb);
}
// Workgroup barriers without a memory fence (a workgroup-scope fence would
// also wait for the copies still in flight). Before the first, this wave's
// LDS reads are complete; before the second, also its copies into LDS.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void barrier_copies() {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

constexpr int kKStage = kKHalves + kLBytes / 2;   // K rows then residual rows (24 KB)
// x, as a value the compiler cannot see through (nor hoist what depends on it).
__device__ __forceinline__ uint32_t opaque(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}

__global__ __launch_bounds__(512) void prefill32_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t k1a[kKStage], k1b[kKStage], k2a[kKStage], k2b[kKStage];
    __shared__ __attribute__((aligned(16))) uint16_t v1a[kVHalves], v1b[kVHalves], v2a[kVHalves], v2b[kVHalves];

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int c = lane & 31, g8 = lane >> 5;   // token column, k-slot group
    const bool is_x = wave < 4;
    const uint32_t g = blockIdx.x, pair = blockIdx.z;
    const uint32_t head = g * kGroup + (wave & 3);
    const float c2 = a.scale * 1.4426950408889634f;

    // ---- per-tile state -------------------------------------------------------
    uint32_t n_ch = 0, mid = 0;   // the tile's key chunks; Y: [0, mid), X: [mid, n_ch)
    uint32_t wtok0 = 0, my_tok = 0, my_kend = 0, wave_kend = 0;
    bool unit_live = false;
    f16x8 qb[8];        // q of token my_tok, dims 16 ks + 8 g8 .. +7
    i32x8 q6[2];        // qb[4 m .. 4 m + 3] as fp6 (residual block 2 m + g8), for the residual MFMAs
    int q6s[2];         // their E8M0 scales
    f32x16 o[4];        // O^T, dims 32 dt + 8 j + 4 g8 + i
    f32x16 s[2];        // S^T of the current chunk, keys 32 kt + 8 j + 4 g8 + i
    f16x8 pb[4];        // P^T of the last softmax, 16-key steps
    float m_run = -INFINITY, l_run = 0.0f;   // l_run: this lane's keys only
    bool have_p = false;

    // Keys [0, kend) the tile attends, its 64-key chunks and the Y / X split.
    auto tile_geom = [&](uint32_t tile, uint32_t& kend, uint32_t& n, uint32_t& md) __attribute__((always_inline)) {
        const uint32_t last = min(tile * kPrefillTileTok + kPrefillTileTok, a.m_tokens) - 1;
        kend = a.causal ? a.pos + last + 1 : a.pos;
        n = (kend + kChunk - 1) / kChunk;
        md = (n + 1) / 2;
    };
    // Loads of a tile's q into qb (waited for where they are used).
    // Lanes of tokens past m_tokens load token 0's q: their scores are
    // computed and never stored.
    auto issue_q = [&](uint32_t tile) __attribute__((always_inline)) {
        const uint32_t tok = tile * kPrefillTileTok + c;
        const uint16_t* qp = a.q + static_cast<uint64_t>(tok < a.m_tokens ? tok : 0u) * a.q_stride + head * kHeadDim;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) qb[ks] = *reinterpret_cast<const f16x8*>(qp + 16 * ks + 8 * g8);
    };
    // Makes `tile` current: its token state, q as fp6 for the residual MFMAs,
    // fresh accumulators.
    auto enter_tile = [&](uint32_t tile) __attribute__((always_inline)) {
        tile_geom(tile, wave_kend, n_ch, mid);
        wtok0 = tile * kPrefillTileTok;
        my_tok = wtok0 + c;
        unit_live = wtok0 < a.m_tokens;
        my_kend = a.causal ? a.pos + my_tok + 1 : a.pos;
#pragma unroll
        for (int m = 0; m < 2; m++) {
            float qf[32];
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {   // the lane's q.k dims of k-steps 4 m .. 4 m + 3
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    qf[8 * i + j] = static_cast<float>(qb[4 * m + i][j]);
                    amax = fmaxf(amax, fabsf(qf[8 * i + j]));
                }
            }
            const int e = fp6_scale_exp(amax, -126);
            const i32x6 p6 = pack32_fp6(qf, e);
            q6[m] = i32x8{p6[0], p6[1], p6[2], p6[3], p6[4], p6[5], 0, 0};
            q6s[m] = e + kE8M0Bias;
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++) o[dt] = f32x16{};
        m_run = -INFINITY;
        l_run = 0.0f;
        have_p = false;
    };
    // f16(O / l) of this lane's token (l summed over the lane pair by the caller).
    auto write_out = [&](float l_tot) __attribute__((always_inline)) {
        if (!unit_live || my_tok >= a.m_tokens) return;
        const float inv_l = 1.0f / l_tot;
        uint16_t* out = a.out + static_cast<uint64_t>(my_tok) * a.q_stride + head * kHeadDim;
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint2 w;
                w.x = pack2(o[dt][4 * j] * inv_l, o[dt][4 * j + 1] * inv_l);
                w.y = pack2(o[dt][4 * j + 2] * inv_l, o[dt][4 * j + 3] * inv_l);
                *reinterpret_cast<uint2*>(out + 32 * dt + 8 * j + 4 * g8) = w;
            }
    };

    // ---- copies: 16-byte pieces, 1 KB per wave and instruction -------------
    const uint16_t* k16 = a.k16 + static_cast<uint64_t>(g) * a.ws_chunks * kKHalves;
    const uint16_t* vt16 = a.vt16 + static_cast<uint64_t>(g) * a.ws_chunks * kVHalves;
    const uint8_t* kl8 = a.kl8 + static_cast<uint64_t>(g) * a.ws_chunks * kLBytes;
    // Each copy moves the 1 KB at src (a uniform address) to LDS at dst,
    // lane l's 16 bytes from src + 16 l. Issued as inline asm, so that the
    // compiler neither tracks it nor waits for it before unrelated LDS reads:
    // the waits are barrier_copies' (this wave's copies of the step).
    const uint32_t lane16 = 16u * lane;
    auto lds_copy = [&](const void* src, void* dst) __attribute__((always_inline)) {
        const uint32_t lds = static_cast<uint32_t>(
            reinterpret_cast<uintptr_t>((void __attribute__((address_space(3)))*)dst));
        // (one wait state between the M0 write and the LDS DMA that reads it)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(lane16), "s"(src), "s"(lds)
                     : "m0");
    };
    // The 4 waves of a role copy their role's chunks: wave (w & 3) moves the
    // 1 KB pieces w & 3, +4, +8, ... of each section.
    const int rw = wave & 3;
    auto copy_k4 = [&](uint16_t* dst, uint32_t ch) __attribute__((always_inline)) {
        const uint16_t* ks = k16 + static_cast<uint64_t>(ch) * kKHalves;
        const uint8_t* ls = kl8 + static_cast<uint64_t>(ch) * kLBytes;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int piece = 64 * (4 * r + rw);
            lds_copy(ks + 8 * piece, dst + 8 * piece);
        }
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int piece = 64 * (4 * r + rw);
            lds_copy(ls + 16 * piece, reinterpret_cast<uint8_t*>(dst + kKHalves) + 16 * piece);
        }
    };

    // ---- MFMA phase pieces --------------------------------------------------
    // Both MFMA blocks keep four LDS fragment reads in flight ahead of the
    // MFMAs (sched_group_barrier: DS read = 0x100, MFMA = 0x008), so that
    // the LDS latency hides behind the previous MFMAs. The lane parts of the
    // fragment addresses (bytes) are made opaque at each use, so that the
    // compiler forms each stage's addresses where it reads them instead of
    // keeping a register per stage and fragment live across the loop.
    const uint32_t lane_k = 2 * k_addr32(c, g8), lane_rv = l_addr32(c, 2 * g8);   // = 2 v_addr32(c, g8)
    auto qk = [&](const uint16_t* kb) __attribute__((always_inline)) {
        const uint8_t* kp = reinterpret_cast<const uint8_t*>(kb) + opaque(lane_k);
        const uint8_t* lp = reinterpret_cast<const uint8_t*>(kb + kKHalves) + opaque(lane_rv);
        f16x8 ka[16];   // fragment n: k-step n >> 1, key tile n & 1
#pragma unroll
        for (int n = 0; n < 16; n++)
            ka[n] = *reinterpret_cast<const f16x8*>(kp + 2 * k_addr32(32 * (n & 1), 2 * (n >> 1)));
        U4 r0[4], r1[4];   // residual of key tile n & 1, k block 2 (n >> 1) + g8
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const int row = 32 * (n & 1), blk = 2 * (n >> 1);
            r0[n] = *reinterpret_cast<const U4*>(lp + l_addr32(row, 2 * blk));
            r1[n] = *reinterpret_cast<const U4*>(lp + l_addr32(row, 2 * blk + 1));
        }
#pragma unroll
        for (int kt = 0; kt < 2; kt++) s[kt] = f32x16{};
#pragma unroll
        for (int n = 0; n < 16; n++) s[n & 1] = mfma32(ka[n], qb[n >> 1], s[n & 1]);
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const i32x8 ra = {static_cast<int>(r0[n].w[0]), static_cast<int>(r0[n].w[1]), static_cast<int>(r0[n].w[2]),
                              static_cast<int>(r0[n].w[3]), static_cast<int>(r1[n].w[0]), static_cast<int>(r1[n].w[1]), 0, 0};
            s[n & 1] = mfma32_resid(ra, q6[n >> 1], s[n & 1], static_cast<int>(r1[n].w[2]), q6s[n >> 1]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int n = 0; n < 12; n++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
#pragma unroll
        for (int n = 0; n < 4; n++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };
    auto pv = [&](const uint16_t* vb) __attribute__((always_inline)) {
        const uint8_t* vp = reinterpret_cast<const uint8_t*>(vb) + opaque(lane_rv);
        f16x8 va[16];   // fragment n: 16-key step n >> 2, dim tile n & 3
#pragma unroll
        for (int n = 0; n < 16; n++)
            va[n] = *reinterpret_cast<const f16x8*>(vp + 2 * v_addr32(32 * (n & 3), 2 * (n >> 2)));
#pragma unroll
        for (int n = 0; n < 16; n++) o[n & 3] = mfma32(va[n], pb[n >> 2], o[n & 3]);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int n = 0; n < 12; n++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };
    // ---- VALU phase: mask, lazy running max, exponentials, P^T, row sums -----
    // `hook(k)`, k = 0 .. 4, is called at five points spread over the VALU
    // work (each issues two of the phase's copies: their issue then waits for
    // the shared address unit between VALU instructions, not all at once).
    auto softmax = [&](uint32_t key0, auto&& hook) __attribute__((always_inline)) {
        hook(0);
        const bool need_mask = key0 + kChunk > (a.causal ? a.pos + wtok0 + 1 : a.pos);
        if (need_mask) {
            // key 32 kt + 8 j + 4 g8 + i of the chunk is visible while below
            // my_kend - key0 (as integers); a masked score becomes -inf by a
            // bit select on the sign of (my_kend - key0 - 1 - key): no compare
            // masks (scalar registers) per element.
            const int nv1 = static_cast<int>(my_kend - key0) - 1 - 4 * g8;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t dead = static_cast<uint32_t>((nv1 - (32 * kt + 8 * (r >> 2) + (r & 3))) >> 31);
                    const float x = s[kt][r];   // (a bit cast of a vector element directly is miscompiled)
                    s[kt][r] = __builtin_bit_cast(float, (dead & 0xFF800000u) | (~dead & __builtin_bit_cast(uint32_t, x)));
                }
        }
        // (independent chains throughout: four partial maxima, the exponent
        // arguments in place, then the exponentials, then packing, four
        // partial row sums, so that no VALU result is waited for at once)
        float pm[4];
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const int kt = q4 >> 1, r0 = 8 * (q4 & 1);
            pm[q4] = fmax_p(fmax_p(fmax_p(s[kt][r0], s[kt][r0 + 1]), fmax_p(s[kt][r0 + 2], s[kt][r0 + 3])),
                            fmax_p(fmax_p(s[kt][r0 + 4], s[kt][r0 + 5]), fmax_p(s[kt][r0 + 6], s[kt][r0 + 7])));
        }
        const float lm = fmax_p(fmax_p(pm[0], pm[1]), fmax_p(pm[2], pm[3])) * c2;
        hook(1);
        if (__any(lm > m_run + kLazy)) {
            const float cm = max_xor32(lm);   // the token's max over both lane groups
            const bool up = cm > m_run + kLazy;
            const float m_new = up ? cm : m_run;
            const float alpha = up ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; dt++) o[dt] *= alpha;
        }
        // m_run is still -inf only if every score of the token so far is
        // masked (the X waves' chunks can all lie past an early token's last
        // row): then p = exp2(-inf) = 0, not NaN.
        const float neg_m = m_run == -INFINITY ? 0.0f : -m_run;
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int r = 0; r < 16; r++) s[kt][r] = __builtin_fmaf(s[kt][r], c2, neg_m);
        hook(2);
#pragma unroll
        for (int r = 0; r < 16; r++) s[0][r] = __builtin_amdgcn_exp2f(s[0][r]);
        hook(3);
#pragma unroll
        for (int r = 0; r < 16; r++) s[1][r] = __builtin_amdgcn_exp2f(s[1][r]);
        hook(4);
        float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const int kt = st >> 1, r0 = 8 * (st & 1);
            U4 pk;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pk.w[i] = pack2_rne(s[kt][r0 + 2 * i], s[kt][r0 + 2 * i + 1]);
                ls[i] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk.w[i]), f16x2{1, 1}, ls[i], false);
            }
            pb[st] = __builtin_bit_cast(f16x8, pk);
        }
        l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };

    // ---- one tile ---------------------------------------------------------------
    // The Y waves work on chunks [0, mid) from stream 1, the X waves on
    // [mid, n_ch) from stream 2, and each role copies its own stream. Both run
    // the same loop, iteration i = [copies of K(i+1) and V(i); M(i): P.V of
    // i-1, then q.k of i; barrier; V(i): softmax of i; barrier], iterations
    // 0 .. mid (the last only finishes the P.V of mid - 1); the Y waves run it
    // one barrier later than the X waves, so that X's M phase meets Y's V
    // phase and the other way round. Copies issued in an iteration's VALU
    // phase are waited for at its end (K(i+1) and V(i) are first read in the
    // next iteration's M phase).
    // K(0) of this role's stream for `tile` (into stage 0) and its q loads:
    // issued before the previous tile's merge, so that their latency hides
    // behind it.
    auto issue_tile = [&](uint32_t tile) __attribute__((always_inline)) {
        uint32_t kend, n, md;
        tile_geom(tile, kend, n, md);
        const uint32_t ch0 = is_x ? md : 0u, cnt = is_x ? n - md : md;
        if (cnt > 0) copy_k4(is_x ? k2a : k1a, ch0);
        issue_q(tile);
    };
    auto process = [&]() __attribute__((always_inline)) {
        const uint32_t ch0 = is_x ? mid : 0u;                // this role's first chunk
        const uint32_t cnt = is_x ? n_ch - mid : mid;        // and its chunk count
        uint16_t* const kst0 = is_x ? k2a : k1a;             // this role's stages
        uint16_t* const kst1 = is_x ? k2b : k1b;
        uint16_t* const vst0 = is_x ? v2a : v1a;
        uint16_t* const vst1 = is_x ? v2b : v1b;
        barrier_copies();              // K(0) (issue_tile) has landed
        if (!is_x) barrier_copies();   // Y: one step behind
        auto iter = [&](auto parc, uint32_t i) __attribute__((always_inline)) {
            constexpr int par = decltype(parc)::value;
            const bool live = unit_live && i < cnt && (ch0 + i) * kChunk < wave_kend;
            if (have_p) {
                pv(par ? vst0 : vst1);   // V(i-1)
                have_p = false;
            }
            if (live) qk(par ? kst1 : kst0);
            barrier_lds();
            // K(i+1) and V(i) are copied during the VALU phase (their issue
            // would delay the MFMAs; here the other wave's MFMA phase covers
            // it): 10 copies of 1 KB, two at each softmax hook.
            const bool k_on = i + 1 < cnt, v_on = i < cnt;
            uint16_t* const kd = par ? kst0 : kst1;
            uint16_t* const vd = par ? vst1 : vst0;
            const uint16_t* const ks = k16 + static_cast<uint64_t>(ch0 + i + 1) * kKHalves;
            const uint8_t* const ls = kl8 + static_cast<uint64_t>(ch0 + i + 1) * kLBytes;
            const uint16_t* const vs = vt16 + static_cast<uint64_t>(ch0 + i) * kVHalves;
            auto hook = [&](int k) __attribute__((always_inline)) {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int n = 2 * k + j;   // 0-3: K rows, 4-5: K residual, 6-9: V^T
                    const int piece = 64 * (4 * (n < 4 ? n : n < 6 ? n - 4 : n - 6) + rw);
                    if (n < 4 && k_on) lds_copy(ks + 8 * piece, kd + 8 * piece);
                    else if (n < 6 && k_on) lds_copy(ls + 16 * piece, reinterpret_cast<uint8_t*>(kd + kKHalves) + 16 * piece);
                    else if (n >= 6 && v_on) lds_copy(vs + 8 * piece, vd + 8 * piece);
                }
                __builtin_amdgcn_sched_barrier(0);
            };
            if (live) {
                softmax((ch0 + i) * kChunk, hook);
                have_p = true;
            } else {
#pragma unroll
                for (int k = 0; k < 5; k++) hook(k);
            }
            barrier_copies();
        };
        uint32_t i = 0;
        for (; i + 1 <= mid; i += 2) {
            iter(std::integral_constant<int, 0>{}, i);
            iter(std::integral_constant<int, 1>{}, i + 1);
        }
        if (i <= mid) iter(std::integral_constant<int, 0>{}, i);
        if (is_x) barrier_copies();   // X: the step Y is behind
    };
    // Merge: X hands (O, m, l) to Y through LDS (the V stages and K stage 1:
    // K stage 0 may already receive the next tile's K(0)); Y stores f16(O / l).
    auto merge = [&]() __attribute__((always_inline)) {
        const float l_tot = sum_xor32(l_run);
        float* xo = reinterpret_cast<float*>((wave & 3) == 0 ? v1a : (wave & 3) == 1 ? v1b : (wave & 3) == 2 ? v2a : v2b);
        float* xml = reinterpret_cast<float*>(k1b) + (wave & 3) * 128;
        if (is_x) {
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) xo[(dt * 16 + r) * 64 + lane] = o[dt][r];
            if (lane < 32) {
                xml[lane] = m_run;
                xml[64 + lane] = l_tot;
            }
        }
        barrier_lds();
        if (!is_x) {
            const float mx = xml[c], lx = xml[64 + c];
            const float mm = fmaxf(m_run, mx);
            const float ey = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - mm);
            const float ex = mx == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mx - mm);
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[dt][r] = o[dt][r] * ey + xo[(dt * 16 + r) * 64 + lane] * ex;
            write_out(l_tot * ey + lx * ex);
        }
        barrier_lds();   // the merge area is the next tile's stages
    };

    const uint32_t tile_a = pair, tile_b = a.n_tiles - 1 - pair;   // tile_b >= tile_a
    issue_tile(tile_a);
    enter_tile(tile_a);
    for (uint32_t tile = tile_a;; tile = tile_b) {   // (one code instance for both tiles)
        process();
        const bool more = tile != tile_b;
        if (more) issue_tile(tile_b);
        merge();
        if (!more) break;
        enter_tile(tile_b);
    }
}

// ============================================================================
// prefill_split_kernel: short chunks over long caches (few query tiles, many
// cache rows), split over the keys. Same arithmetic as prefill32_kernel (f16
// K plus its fp6 residual, f16 V and P, f32 accumulation, exp2-domain online
// softmax with the lazy max, the same 32x32x16 fragments), but the workgroup
// reads the layer's Q8_0 rows from the cache itself instead of a prepared
// image, so a call touches each cache row once instead of re-imaging the
// whole layer:
//  * Grid (KV head g, key split s, tile pair z); 8 waves. Wave w owns query
//    head 4 g + (w & 3) for the 32 tokens of tile 2 z + (w >> 2), so the
//    workgroup's 8 waves share one stream of chunks: rows of split s, i.e.
//    64-row chunks [s * split_chunks, +split_chunks) of those the pair's last
//    token attends.
//  * Per chunk: its Q8_0 bytes and scales (18 KB) are copied into LDS by
//    global_load_lds (18 copies of 1 KB spread over the waves), issued two
//    chunks ahead; waves 0-3 convert the K rows (emit_k_rows: f16 rows and
//    the fp6 residual) and waves 4-7 transpose V (emit_v_lds, then
//    emit_v_rows after a barrier) into the compute stage of the next chunk
//    while every wave computes on the current one (S^T = K Q^T, softmax, O^T
//    += V^T P^T), double-buffered.
//  * Each wave writes its partial (O unnormalized, m in log2 units, l) per
//    token to kpart; prefill_merge_kernel combines the splits.
__global__ __launch_bounds__(512) void prefill_split_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t stk[2][kKStage];    // K rows + residual, per stage
    __shared__ __attribute__((aligned(16))) uint16_t stv[2][kVHalves];   // V^T, per stage
    __shared__ __attribute__((aligned(16))) uint8_t rq[2][2][kChunk][kHeadDim];          // [buf][K, V][row]: Q8_0 bytes
    __shared__ __attribute__((aligned(16))) float rd[2][2][kChunk][kHeadDim / kBlock];   // and scales

    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int c = lane & 31, g8 = lane >> 5;
    const uint32_t g = blockIdx.x, split = blockIdx.y, tpair = blockIdx.z;
    const uint32_t tile = 2 * tpair + (wave >> 2);
    const uint32_t head = g * kGroup + (wave & 3);
    const uint32_t wtok0 = tile * kPrefillTileTok;
    const bool unit_live = wtok0 < a.m_tokens;
    const uint32_t my_tok = wtok0 + c;
    const uint32_t my_kend = a.pos + my_tok + 1;   // causal: token m attends rows [0, pos + m]
    const uint32_t wave_kend = unit_live ? a.pos + min(wtok0 + kPrefillTileTok, a.m_tokens) : 0u;
    const uint32_t pair_kend = a.pos + min(2 * kPrefillTileTok * (tpair + 1), a.m_tokens);
    const uint32_t n_ch = (pair_kend + kChunk - 1) / kChunk;
    const uint32_t c0 = min(split * a.split_chunks, n_ch), cnt = min(c0 + a.split_chunks, n_ch) - c0;

    // ---- q of this lane's token (tokens past m_tokens load token 0's) ----------
    f16x8 qb[8];
    {
        const uint16_t* qp = a.q + static_cast<uint64_t>(my_tok < a.m_tokens ? my_tok : 0u) * a.q_stride +
                             head * kHeadDim;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) qb[ks] = *reinterpret_cast<const f16x8*>(qp + 16 * ks + 8 * g8);
    }

    // ---- copies of a chunk's Q8_0 rows into raw buffer b: copy n (0..17) by
    // wave n % 8: n < 8 K bytes of rows 8 n .. +7, 8..15 V bytes, 16 / 17 the
    // K / V scales of the 64 rows (rows past n_rows: the last row again) ----
    const uint32_t nb_row = a.kv_dim / kBlock;
    const uint32_t last_row = a.n_rows - 1;
    auto dma = [&](uint32_t ch, int b) __attribute__((always_inline)) {
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const int n = wave + 8 * k;
            if (n >= 18) break;
            const bool is_v = (n >= 8 && n < 16) || n == 17;
            const char* base;
            uint32_t off;
            uint32_t lds;
            if (n < 16) {
                const uint32_t row = min(ch * kChunk + 8 * (n & 7) + (lane >> 3), last_row);
                off = row * a.kv_dim + 16 * (lane & 7);
                base = reinterpret_cast<const char*>(is_v ? a.v.qs : a.k.qs) + g * kHeadDim;
                lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
                    (void __attribute__((address_space(3)))*)&rq[b][is_v][8 * (n & 7)][0]));
            } else {
                const uint32_t row = min(ch * kChunk + lane, last_row);
                off = row * nb_row * 4;
                base = reinterpret_cast<const char*>(is_v ? a.v.d : a.k.d) + g * (kHeadDim / kBlock) * 4;
                lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
                    (void __attribute__((address_space(3)))*)&rd[b][is_v][0][0]));
            }
            // (one wait state between the M0 write and the LDS DMA that reads it)
            lds = __builtin_amdgcn_readfirstlane(lds);   // uniform (the compiler cannot tell)
            asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                         : "m0");
        }
    };
    // ---- the chunk in raw buffer b into compute stage st: K rows by waves
    // 0-3 (emit_k_rows), V^T by waves 4-7: thread (dims 4 dq .. +3, 16-byte
    // group j of V^T, i.e. slots 8 j .. +7 holding keys v_slot32(slot)) reads
    // the 4 bytes of those dims of the 8 keys, writes 4 groups ----
    auto emit = [&](int b, int st) __attribute__((always_inline)) {
        if (t < 256) {
            const int kr = t >> 2, kb = t & 3;
            const U4 kq0 = *reinterpret_cast<const U4*>(&rq[b][0][kr][32 * kb]);
            const U4 kq1 = *reinterpret_cast<const U4*>(&rq[b][0][kr][32 * kb + 16]);
            emit_k_rows_at(stk[st], reinterpret_cast<uint8_t*>(stk[st] + kKHalves), 1u, t, kq0, kq1, rd[b][0][kr][kb]);
        } else {
            const int tv = t - 256, dq = tv & 31, j = tv >> 5;
            uint32_t x[8];
            float d[8];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int key = v_slot32(8 * j + e);   // (v_slot32 is its own inverse)
                x[e] = *reinterpret_cast<const uint32_t*>(&rq[b][1][key][4 * dq]);
                d[e] = rd[b][1][key][dq >> 3];
            }
            __builtin_amdgcn_sched_barrier(0);   // all 16 reads in flight before the first wait
#pragma unroll
            for (int n = 0; n < 4; n++) {
                const int dd = (n + dq + (dq >> 2)) & 3;   // rotated: fewer bank conflicts between lanes
                U4 grp;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const float v0 = d[e] * static_cast<float>(static_cast<int8_t>(x[e] >> (8 * dd)));
                    const float v1 = d[e + 1] * static_cast<float>(static_cast<int8_t>(x[e + 1] >> (8 * dd)));
                    grp.w[e >> 1] = pack2_rne(v0, v1);
                }
                *reinterpret_cast<U4*>(stv[st] + v_addr32(4 * dq + dd, j)) = grp;
            }
        }
    };

    // ---- q as fp6 for the residual MFMAs (as prefill32_kernel's enter_tile) ----
    i32x8 q6[2];
    int q6s[2];
#pragma unroll
    for (int m = 0; m < 2; m++) {
        float qf[32];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                qf[8 * i + j] = static_cast<float>(qb[4 * m + i][j]);
                amax = fmaxf(amax, fabsf(qf[8 * i + j]));
            }
        const int e = fp6_scale_exp(amax, -126);
        const i32x6 p6 = pack32_fp6(qf, e);
        q6[m] = i32x8{p6[0], p6[1], p6[2], p6[3], p6[4], p6[5], 0, 0};
        q6s[m] = e + kE8M0Bias;
    }
    f32x16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) o[dt] = f32x16{};
    f32x16 s[2];
    f16x8 pb[4];
    float m_run = -INFINITY, l_run = 0.0f;
    const float c2 = a.scale * 1.4426950408889634f;

    // ---- compute on a stage (the fragments of prefill32_kernel) ----
    const uint32_t lane_k = 2 * k_addr32(c, g8), lane_rv = l_addr32(c, 2 * g8);
    auto qk = [&](const uint16_t* kb) __attribute__((always_inline)) {
        const uint8_t* kp = reinterpret_cast<const uint8_t*>(kb) + opaque(lane_k);
        const uint8_t* lp = reinterpret_cast<const uint8_t*>(kb + kKHalves) + opaque(lane_rv);
        f16x8 ka[16];
#pragma unroll
        for (int n = 0; n < 16; n++)
            ka[n] = *reinterpret_cast<const f16x8*>(kp + 2 * k_addr32(32 * (n & 1), 2 * (n >> 1)));
        U4 r0[4], r1[4];
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const int row = 32 * (n & 1), blk = 2 * (n >> 1);
            r0[n] = *reinterpret_cast<const U4*>(lp + l_addr32(row, 2 * blk));
            r1[n] = *reinterpret_cast<const U4*>(lp + l_addr32(row, 2 * blk + 1));
        }
#pragma unroll
        for (int kt = 0; kt < 2; kt++) s[kt] = f32x16{};
#pragma unroll
        for (int n = 0; n < 16; n++) s[n & 1] = mfma32(ka[n], qb[n >> 1], s[n & 1]);
#pragma unroll
        for (int n = 0; n < 4; n++) {
            const i32x8 ra = {static_cast<int>(r0[n].w[0]), static_cast<int>(r0[n].w[1]), static_cast<int>(r0[n].w[2]),
                              static_cast<int>(r0[n].w[3]), static_cast<int>(r1[n].w[0]), static_cast<int>(r1[n].w[1]), 0, 0};
            s[n & 1] = mfma32_resid(ra, q6[n >> 1], s[n & 1], static_cast<int>(r1[n].w[2]), q6s[n >> 1]);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int n = 0; n < 12; n++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
#pragma unroll
        for (int n = 0; n < 4; n++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };
    auto pv = [&](const uint16_t* vb) __attribute__((always_inline)) {
        const uint8_t* vp = reinterpret_cast<const uint8_t*>(vb) + opaque(lane_rv);
        f16x8 va[16];
#pragma unroll
        for (int n = 0; n < 16; n++)
            va[n] = *reinterpret_cast<const f16x8*>(vp + 2 * v_addr32(32 * (n & 3), 2 * (n >> 2)));
#pragma unroll
        for (int n = 0; n < 16; n++) o[n & 3] = mfma32(va[n], pb[n >> 2], o[n & 3]);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int n = 0; n < 12; n++) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    };
    auto softmax = [&](uint32_t key0) __attribute__((always_inline)) {
        if (key0 + kChunk > a.pos + wtok0 + 1) {   // some key past the wave's first token's last row
            const int nv1 = static_cast<int>(my_kend - key0) - 1 - 4 * g8;
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const uint32_t dead = static_cast<uint32_t>((nv1 - (32 * kt + 8 * (r >> 2) + (r & 3))) >> 31);
                    const float x = s[kt][r];   // (a bit cast of a vector element directly is miscompiled)
                    s[kt][r] = __builtin_bit_cast(float, (dead & 0xFF800000u) | (~dead & __builtin_bit_cast(uint32_t, x)));
                }
        }
        float pm[4];
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const int kt = q4 >> 1, r0 = 8 * (q4 & 1);
            pm[q4] = fmax_p(fmax_p(fmax_p(s[kt][r0], s[kt][r0 + 1]), fmax_p(s[kt][r0 + 2], s[kt][r0 + 3])),
                            fmax_p(fmax_p(s[kt][r0 + 4], s[kt][r0 + 5]), fmax_p(s[kt][r0 + 6], s[kt][r0 + 7])));
        }
        const float lm = fmax_p(fmax_p(pm[0], pm[1]), fmax_p(pm[2], pm[3])) * c2;
        if (__any(lm > m_run + kLazy)) {
            const float cm = max_xor32(lm);
            const bool up = cm > m_run + kLazy;
            const float m_new = up ? cm : m_run;
            const float alpha = up ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < 4; dt++) o[dt] *= alpha;
        }
        const float neg_m = m_run == -INFINITY ? 0.0f : -m_run;
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int r = 0; r < 16; r++) s[kt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][r], c2, neg_m));
        float ls[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int st = 0; st < 4; st++) {
            const int kt = st >> 1, r0 = 8 * (st & 1);
            U4 pk;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pk.w[i] = pack2_rne(s[kt][r0 + 2 * i], s[kt][r0 + 2 * i + 1]);
                ls[i] = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pk.w[i]), f16x2{1, 1}, ls[i], false);
            }
            pb[st] = __builtin_bit_cast(f16x8, pk);
        }
        l_run += (ls[0] + ls[1]) + (ls[2] + ls[3]);
    };

    // ---- the chunk loop: iteration i computes chunk c0 + i from stage i & 1,
    // converts chunk c0 + i + 1 into the other stage and copies chunk c0 + i + 2
    // into the raw buffer chunk c0 + i held ----
    if (cnt > 0) dma(c0, 0);
    if (cnt > 1) dma(c0 + 1, 1);
    barrier_copies();
    if (cnt > 0) emit(0, 0);
    for (uint32_t i = 0; i < cnt; i++) {
        const int st = static_cast<int>(i & 1);
        barrier_copies();   // stage st complete; raw chunk i + 1 landed
        if (i + 2 < cnt) dma(c0 + i + 2, st);
        if (i + 1 < cnt) emit(1 - st, 1 - st);
        const uint32_t key0 = (c0 + i) * kChunk;
        if (unit_live && key0 < wave_kend) {
            qk(stk[st]);
            softmax(key0);
            pv(stv[st]);
        }
    }

    // ---- partial of this split: O (unnormalized), m (log2 units), l ----
    const float l_tot = sum_xor32(l_run);
    if (!unit_live || my_tok >= a.m_tokens) return;
    const uint32_t n_head = a.q_stride / kHeadDim;
    float* pp = a.kpart + ((static_cast<uint64_t>(my_tok) * n_head + head) * a.n_ksplit + split) * kSplitStride;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            *reinterpret_cast<f32x4*>(pp + 32 * dt + 8 * j + 4 * g8) =
                f32x4{o[dt][4 * j], o[dt][4 * j + 1], o[dt][4 * j + 2], o[dt][4 * j + 3]};
    if (g8 == 0) *reinterpret_cast<float2*>(pp + kHeadDim) = make_float2(m_run, l_tot);
}

}  // namespace

static void launch_prefill_merge(const PrefillArgs& a, uint32_t n_kv_head, hipStream_t s) {
    const dim3 grid(a.m_tokens, n_kv_head * kGroup);
    if (a.n_ksplit <= 8)
        hipLaunchKernelGGL(prefill_merge_kernel<4>, grid, dim3(64), 0, s, a);
    else if (a.n_ksplit <= 16)
        hipLaunchKernelGGL(prefill_merge_kernel<8>, grid, dim3(64), 0, s, a);
    else if (a.n_ksplit <= 32)
        hipLaunchKernelGGL(prefill_merge_kernel<16>, grid, dim3(64), 0, s, a);
    else
        hipLaunchKernelGGL(prefill_merge_kernel<32>, grid, dim3(64), 0, s, a);
}

static void launch_attention(const PrefillArgs& a, uint32_t n_kv_head, hipStream_t s) {
    const uint32_t n_pairs = (a.n_tiles + 1) / 2;
    if (a.direct) {
        hipLaunchKernelGGL(prefill_split_kernel, dim3(n_kv_head, a.n_ksplit, n_pairs), dim3(512), 0, s, a);
        launch_prefill_merge(a, n_kv_head, s);
    } else if (a.heads_per_wave == 2)
        hipLaunchKernelGGL(prefill32_kernel, dim3(n_kv_head, 1, n_pairs), dim3(512), 0, s, a);
    else if (a.wg_waves == 4)
        hipLaunchKernelGGL((prefill_kernel<1, 4>), dim3(n_kv_head, 4, n_pairs), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL((prefill_kernel<1, 8>), dim3(n_kv_head, 2, n_pairs), dim3(512), 0, s, a);
}

// HIP's grid limit in y and z.
constexpr uint64_t kGridYZMax = 65535;
static uint64_t attention_grid_z(const PrefillArgs& a) {
    return (a.n_tiles + 1) / 2;
}
// Preparation pass, grid y: the image's halves (or with no image, the halves
// holding new rows), then kGroup q parts per half holding new rows.
static uint64_t prep_grid_y(const PrefillArgs& a) {
    const uint64_t new_halves = (static_cast<uint64_t>(a.n_rows) + kHalf - 1) / kHalf - a.pos / kHalf;
    const uint64_t n_halves = a.direct ? new_halves : 2 * ((static_cast<uint64_t>(a.n_rows) + kChunk - 1) / kChunk);
    return n_halves + kGroup * new_halves;
}

bool prefill_grid_fits(const PrefillArgs& a, bool step) {
    const uint64_t y = step ? prep_grid_y(a) : a.direct ? 0 : (static_cast<uint64_t>(a.n_rows) + kChunk - 1) / kChunk;
    return y <= kGridYZMax && attention_grid_z(a) <= kGridYZMax;
}

hipError_t launch_prefill(const PrefillArgs& a, uint32_t n_kv_head, hipStream_t s) {
    if (!a.direct)
        hipLaunchKernelGGL(kv_dequant_kernel, dim3(n_kv_head, (a.n_rows + kChunk - 1) / kChunk), dim3(256), 0, s, a);
    launch_attention(a, n_kv_head, s);
    return hipGetLastError();
}

hipError_t launch_prefill_step(const PrefillArgs& a, const PrefillStepArgs& w, uint32_t n_kv_head, hipStream_t s,
                               bool prep_only) {
    // grid y: the image's chunks (two halves each), then kGroup q parts per
    // half holding rows [pos, pos + m)
    hipLaunchKernelGGL(prefill_prep_kernel, dim3(n_kv_head, static_cast<uint32_t>(prep_grid_y(a))), dim3(kPrepThreads),
                       0, s, a, w);
    if (!prep_only) launch_attention(a, n_kv_head, s);
    return hipGetLastError();
}

}  // namespace bp
