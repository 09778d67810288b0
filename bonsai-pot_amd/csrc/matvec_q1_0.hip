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
// x (the staged activation: plain, silu(gate) * up, or RMS-normed) sits in LDS
// as f16, each 128-element block split into two half-blocks: half 0 holds the
// pairs (x[4i], x[4i+1]) and half 1 the pairs (x[4i+2], x[4i+3]), i = 0..31, so
// that one lane runs the accumulators of components 0, 1 and its neighbour
// those of 2, 3 (two independent packed f16 chains; the order of every chain
// is unchanged). Half-blocks are 144 bytes apart, so the 8 half-blocks that a
// wave reads at once fall in 8 different bank groups.
//
// Inner loop: a sign bit becomes the f16 multiplier +-1 with one v_perm_b32
// per two elements, from pre-shifted copies of the inverted qs word whose
// bytes are 0x3C | (sign << 7); then one v_pk_fma_f16 adds +-x to the lane's
// two accumulators. (fma(+-1, x, c) rounds once, exactly as c + (+-x) does.)
#include "bp_device.hpp"
#include "bp_kernels.hpp"

namespace bp {
namespace {

typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef _Float16 h8v __attribute__((ext_vector_type(8)));

constexpr int kMvMaxThreads = 1024;
constexpr int kQ1Block = 128;
constexpr int kHalfStride = 72;               // halves from one half-block to the next (64 + 8 pad)
constexpr int kBlockHalves = 2 * kHalfStride; // one 128-element block in LDS

// One lane's half of a (row, block): components 2h and 2h + 1, i.e. the
// elements 4i + 2h and 4i + 2h + 1 for i = 0..31 in order, as one packed pair
// of f16 accumulators. xh: the half-block of x.
__device__ __forceinline__ h2v q1_half(const uint32_t q[4], const uint16_t* xh, uint32_t h) {
    h2v c = {static_cast<_Float16>(0.0f), static_cast<_Float16>(0.0f)};
    const uint32_t sh = 2 * h;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t nq = ~q[w];
        // byte k of s[m] = 0x3C | (inverted bit 8k + p << 7), p = 2h + {0, 1, 4, 5}
        const uint32_t s0 = __builtin_amdgcn_bitop3_b32(nq << (7 - sh), 0x80808080u, 0x3C3C3C3Cu, 0xEA);
        const uint32_t s1 = __builtin_amdgcn_bitop3_b32(nq << (6 - sh), 0x80808080u, 0x3C3C3C3Cu, 0xEA);
        const uint32_t s4 = __builtin_amdgcn_bitop3_b32(nq << (3 - sh), 0x80808080u, 0x3C3C3C3Cu, 0xEA);
        const uint32_t s5 = __builtin_amdgcn_bitop3_b32(nq << (2 - sh), 0x80808080u, 0x3C3C3C3Cu, 0xEA);
        const h8v xa = *reinterpret_cast<const h8v*>(xh + 16 * w);       // pairs i = 8w .. 8w + 3
        const h8v xb = *reinterpret_cast<const h8v*>(xh + 16 * w + 8);   // pairs i = 8w + 4 .. 8w + 7
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // bytes: 0x00, byte k of the low word, 0x00, byte k of the high word
            const uint32_t sel = 0x000C000Cu | (static_cast<uint32_t>(4 + k) << 24) | (static_cast<uint32_t>(k) << 8);
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {   // pair m = 2k + hh of the word: bits 8k + 4hh + 2h + {0, 1}
                const int m = 2 * k + hh;
                const h2v sg = __builtin_bit_cast(h2v, hh == 0 ? __builtin_amdgcn_perm(s1, s0, sel)
                                                                : __builtin_amdgcn_perm(s5, s4, sel));
                const h2v xp = m < 4 ? h2v{xa[2 * m], xa[2 * m + 1]} : h2v{xb[2 * m - 8], xb[2 * m - 7]};
                c = __builtin_elementwise_fma(sg, xp, c);
            }
        }
    }
    return c;
}

// Weights of one lane's (row, block) in a tile: 16 qs bytes and the f16 scale.
struct WTile {
    uint4 q;
    uint16_t d;
    bool ok;
};

// Tile t of a workgroup: rows 8 (t / tcols) .. + 7, blocks 4 (t % tcols) .. + 3;
// lane = (row slot lane >> 3, block (lane >> 1) & 3, half lane & 1). A wave
// walks tiles wave, wave + n_wave, ...; it keeps the tile's (row group, block
// group) in scalar registers and steps them without a division.
struct TilePos {
    uint32_t tile, rq, col;   // wave-uniform
};
__device__ __forceinline__ void tile_step(TilePos& p, uint32_t n_wave, uint32_t tcols) {
    p.tile += n_wave;
    p.col += n_wave;
    while (p.col >= tcols) {
        p.col -= tcols;
        ++p.rq;
    }
}

// Weights of one lane's (row, block) in a tile. Loads are unconditional (the
// row and block clamped into range), so no lane branches around them; `ok`
// says whether the lane's (row, block) exists.
__device__ __forceinline__ WTile load_tile(const MatvecArgs& a, const TilePos& p, uint32_t n_tiles, uint32_t nb,
                                           uint32_t n_here, uint32_t rbase, uint32_t d_off, uint32_t qs_off, int lane) {
    WTile w;
    const uint32_t r = p.rq * 8 + (lane >> 3), b = p.col * 4 + ((lane >> 1) & 3);
    w.ok = p.tile < n_tiles && r < n_here && b < nb;
    const uint32_t rc = min(r, n_here - 1), bc = min(b, nb - 1);
    const uint32_t rb = (rbase + rc) * nb + bc;
    w.q = *reinterpret_cast<const uint4*>(a.weights + qs_off + 16 * rb);
    w.d = *reinterpret_cast<const uint16_t*>(a.weights + d_off + 2 * rb);
    return w;
}

// Stores 8 consecutive x values (elements e .. e + 7, e a multiple of 8) into
// the two half-blocks.
__device__ __forceinline__ void stage8(uint16_t* x_sh, uint32_t e, h8v r) {
    uint16_t* blk = x_sh + (e / kQ1Block) * kBlockHalves + (e % kQ1Block) / 2;
    typedef _Float16 h4v __attribute__((ext_vector_type(4)));
    *reinterpret_cast<h4v*>(blk) = h4v{r[0], r[1], r[4], r[5]};
    *reinterpret_cast<h4v*>(blk + kHalfStride) = h4v{r[2], r[3], r[6], r[7]};
}

// kMode: 0 plain (x = act), 1 silu (x = f16(silu(gate)) * up), 2 normed
// (x = act * w_norm, scale d * inv_rms, up to 3 row ranges).
//
// A workgroup owns rows_per_wg rows (its first weight loads are issued before
// anything else). Pass 1 stages x. Pass 2: its waves share the tiles of those
// rows (8 rows x 4 blocks x 2 halves each) and put each block's f32 term
// d * sum in LDS. Pass 3: thread (row, t) adds its terms t, t + 8, ... in order
// and the 8 row lanes combine by the xor 1, 2, 4 butterfly.
template <int kMode>
__global__ __launch_bounds__(kMvMaxThreads) void matvec_q1_0_kernel(MatvecArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t x_sh[];
    __shared__ float red_sh[4];
    const int t = threadIdx.x, n_thr = blockDim.x;
    const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), n_wave = n_thr >> 6;
    const uint32_t k = a.k, nb = k / kQ1Block;
    const uint32_t rows = a.rows_per_wg;
    float* terms = reinterpret_cast<float*>(x_sh + nb * kBlockHalves);   // [rows][nb]

    // This workgroup's rows lie in one range (ranges are multiples of 16 rows
    // and rows_per_wg divides 16).
    const uint32_t row0 = blockIdx.x * rows;
    uint32_t d_off = a.range[0].d_offset, qs_off = a.range[0].qs_offset, out_off = a.range[0].output_offset;
    uint32_t rbase = row0;                       // first row of the workgroup within its range
    if constexpr (kMode == 2) {
        if (rbase >= a.range[0].n) {
            rbase -= a.range[0].n;
            d_off = a.range[1].d_offset; qs_off = a.range[1].qs_offset; out_off = a.range[1].output_offset;
            if (rbase >= a.range[1].n) {
                rbase -= a.range[1].n;
                d_off = a.range[2].d_offset; qs_off = a.range[2].qs_offset; out_off = a.range[2].output_offset;
            }
        }
    }
    const uint32_t n_here = min(rows, a.n_total - row0);   // rows of this workgroup that exist

    const uint32_t tcols = (nb + 3) / 4;
    const uint32_t n_tiles = (rows / 8) * tcols;
    TilePos pos = {static_cast<uint32_t>(wave), 0u, static_cast<uint32_t>(wave)};   // (rq, col) = divmod(wave, tcols)
    while (pos.col >= tcols) {   // no division: wave < 16, usually < tcols
        pos.col -= tcols;
        ++pos.rq;
    }
    WTile cur = load_tile(a, pos, n_tiles, nb, n_here, rbase, d_off, qs_off, lane);   // in flight during pass 1

    // ---- pass 1: stage x (f16) into LDS, 8 elements at a time --------------------
    float ssq = 0.0f;
    if constexpr (kMode == 0) {
        for (uint32_t v = t; v < k / 8; v += n_thr)
            stage8(x_sh, 8 * v, *reinterpret_cast<const h8v*>(a.act + a.input_offset + 8 * v));
    } else if constexpr (kMode == 1) {
        // matvec_q1_0_silu.wgsl:86-102: silu in f32, then f16(silu) * up in f16.
        for (uint32_t v = t; v < k / 8; v += n_thr) {
            const h8v g = *reinterpret_cast<const h8v*>(a.act + a.gate_offset + 8 * v);
            const h8v u = *reinterpret_cast<const h8v*>(a.act + a.up_offset + 8 * v);
            h8v r;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float gf = static_cast<float>(g[i]);
                const float sl = gf / (1.0f + expf(-gf));
                r[i] = static_cast<_Float16>(sl) * u[i];
            }
            stage8(x_sh, 8 * v, r);
        }
    } else {
        // matvec_q1_0_fused_normed.wgsl:102-121: x * w_norm in f16; the sum of
        // x^2 in f32 by 256 threads (element groups v = t, t + 256, ... in order).
        if (t < 256) {
            for (uint32_t v = t; v < k / 8; v += 256) {
                const h8v x = *reinterpret_cast<const h8v*>(a.act + a.input_offset + 8 * v);
                const h8v w = *reinterpret_cast<const h8v*>(a.w_norms + a.w_norm_off + 8 * v);
                h8v r;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const float xf = static_cast<float>(x[i]);
                    ssq = ssq + xf * xf;
                    r[i] = x[i] * w[i];
                }
                stage8(x_sh, 8 * v, r);
            }
        }
    }
    float inv_rms = 1.0f;
    if constexpr (kMode == 2) {
        // Sum over the 256 threads: xor butterfly in each wave, then waves 0..3 in order.
        if (wave < 4) {
            ssq = wave_sum(ssq);
            if (lane == 0) red_sh[wave] = ssq;
        }
        __syncthreads();
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; w++) total += red_sh[w];
        inv_rms = 1.0f / sqrtf(total / static_cast<float>(k) + a.eps);
    } else {
        __syncthreads();
    }

    // ---- pass 2: block terms (weights of the next tile loaded ahead) --------------
    const uint32_t h = lane & 1;
    while (pos.tile < n_tiles) {
        TilePos nxt_pos = pos;
        tile_step(nxt_pos, n_wave, tcols);
        const WTile nxt = load_tile(a, nxt_pos, n_tiles, nb, n_here, rbase, d_off, qs_off, lane);
        const uint32_t r = pos.rq * 8 + (lane >> 3), b = min(pos.col * 4 + ((lane >> 1) & 3), nb - 1);
        const uint32_t q[4] = {cur.q.x, cur.q.y, cur.q.z, cur.q.w};
        // both lanes of a pair are valid or invalid together; the lane exchange is
        // executed by all lanes
        const h2v c = q1_half(q, x_sh + b * kBlockHalves + h * kHalfStride, h);
        const h2v c23 = __builtin_bit_cast(h2v, lane_xor<1>(__builtin_bit_cast(uint32_t, c)));
        if (cur.ok && h == 0) {
            const _Float16 sum = ((c.x + c.y) + c23.x) + c23.y;   // f16 adds, in this order
            float d = static_cast<float>(__builtin_bit_cast(_Float16, cur.d));
            if constexpr (kMode == 2) d = d * inv_rms;
            terms[r * nb + b] = d * static_cast<float>(sum);
        }
        cur = nxt;
        pos = nxt_pos;
    }
    __syncthreads();

    // ---- pass 3: the 8 ordered lane sums of each row, then the butterfly ----------
    if (t < static_cast<int>(rows * 8)) {
        const uint32_t r = t >> 3, bt = t & 7;
        float acc = 0.0f;
        if (r < n_here)
            for (uint32_t b = bt; b < nb; b += 8) acc = acc + terms[r * nb + b];
        acc = acc + lane_xor<1>(acc);
        acc = acc + lane_xor<2>(acc);
        acc = acc + lane_xor<4>(acc);
        if (bt == 0 && r < n_here) {
            uint16_t* y = a.act + out_off + rbase + r;
            if (kMode != 2 && a.accumulate) *y = f2h(h2f(*y) + acc);
            else *y = f2h(acc);
        }
    }
}

}  // namespace

hipError_t launch_matvec_q1_0(const MatvecArgs& args, int mode, hipStream_t s) {
    MatvecArgs a = args;
    const uint32_t nb = a.k / kQ1Block, tcols = (nb + 3) / 4;
    // Rows per workgroup and waves: one tile per wave while the whole grid
    // fits on the GPU at once (8192 waves); else two per wave. The silu matvec
    // stages an expensive x, so it shares each staging among 16 rows. The
    // normed sum of squares is defined over 256 threads (4 waves at least).
    auto plan = [&](uint32_t rows, uint32_t tiles_per_wave) {
        a.rows_per_wg = rows;
        const uint32_t tiles = rows / 8 * tcols;
        uint32_t w = (tiles + tiles_per_wave - 1) / tiles_per_wave;
        w = w > 16 ? 16 : w;
        return mode == 2 && w < 4 ? 4u : w;
    };
    uint32_t waves;
    if (mode == 1) {
        waves = plan(16, 1);
    } else {
        waves = plan(8, 1);
        if (((a.n_total + 7) / 8) * waves > 8192) waves = plan(16, 2);
    }
    const uint32_t n_wg = (a.n_total + a.rows_per_wg - 1) / a.rows_per_wg;
    const size_t lds = static_cast<size_t>(nb) * kBlockHalves * 2 + static_cast<size_t>(a.rows_per_wg) * nb * 4;
    const dim3 block(64 * waves);
    if (mode == 0)
        hipLaunchKernelGGL(matvec_q1_0_kernel<0>, dim3(n_wg), block, lds, s, a);
    else if (mode == 1)
        hipLaunchKernelGGL(matvec_q1_0_kernel<1>, dim3(n_wg), block, lds, s, a);
    else
        hipLaunchKernelGGL(matvec_q1_0_kernel<2>, dim3(n_wg), block, lds, s, a);
    return hipGetLastError();
}

uint32_t matvec_max_k() { return 16384; }

}  // namespace bp
