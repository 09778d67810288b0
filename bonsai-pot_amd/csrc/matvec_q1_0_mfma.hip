// Q1_0 decode matvecs on the i8 matrix cores (gfx950): y = W x with 1-bit
// weights (bit e of a block's 128-bit qs selects +x[e] or -x[e]) and one f16
// scale d per 128-weight block. Same operations as src/shaders/matvec_q1_0.wgsl,
// matvec_q1_0_silu.wgsl and matvec_q1_0_fused_normed.wgsl (reference
// repository): the staged x, the accumulate / fused-norm / silu semantics and
// the output rounding are the reference's; the sums run in exact integers and
// f32 instead of the reference's f16 adds.
//
// Per block b of x (128 elements), with a = max |x|: x is split as
//   x[e] ~= (a / 16383) * (128 * hi[e] + lo[e]),  hi in [-128, 127], lo in [0, 127]
// (x rounded to 15 bits of the block maximum). For a row's block with sign
// bits s[e] in {0, 1}, the exact integer P = sum_e s[e] (128 hi[e] + lo[e]) and
// S = sum_e (128 hi[e] + lo[e]) give the block's sum of +-x as
// (a / 16383) * (2P - S), and the row sums d * that over its blocks in f32.
//
// Matrix-core form: one v_mfma_i32_16x16x64_i8 takes 64 of the x bytes of 8
// blocks (A, 16 rows = (block of the 8, hi or lo)) times 16 weight rows (B:
// sign bits as 0/1 bytes). Lane group g of B holds blocks g and g + 4 of its
// weight row (8 bytes each); A row (block j, hi/lo) is nonzero only in the 8
// bytes that face block j. 16 such MFMAs cover the 8 blocks, and the result
// holds P_hi / P_lo of every (block, weight row), exact; lane (g, row) gets
// those of blocks 2g and 2g + 1. The A fragments depend
// only on x, so each workgroup builds them once in LDS (16 bytes per lane and
// MFMA, zero halves included).
//
// A byte order within a block: MFMA s (0..15) takes qs word w = s / 4 and bit
// planes p0 = 2 (s % 4), p0 + 1; byte (p % 2) * 4 + kk of the 8 holds bit
// 32 w + 8 kk + p of the block ((q >> p) & 0x01010101 gives 4 of them at once).
#include "bp_device.hpp"
#include "bp_kernels.hpp"

namespace bp {
namespace {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef int i4v __attribute__((ext_vector_type(4)));

constexpr int kMfMaxThreads = 1024;
constexpr int kQ1Block = 128;
constexpr int kGroupBlocks = 8;               // blocks per MFMA column set
constexpr int kFragBytes = 16;                // one lane's B operand
// (hi, lo) x 16 MFMAs per block; each run of 16 fragments is padded by 16
// bytes so that the 16 live lanes of one MFMA (16 different runs) read 16
// different bank groups
constexpr int kRunBytes = 16 * kFragBytes + 16;
constexpr int kBlockFragBytes = 2 * kRunBytes;
constexpr int kZeroBytes = 16 * kFragBytes;   // B of lanes outside their block pair
constexpr float kQMax = 16383.0f;

struct MfLayout {   // byte offsets into dynamic LDS
    uint32_t frag, zero, s_int, scl, part, bytes;
};
__host__ __device__ inline MfLayout mf_layout(uint32_t nb, uint32_t n_groups, uint32_t tiles) {
    MfLayout L;
    L.frag = 0;
    L.zero = n_groups * kGroupBlocks * kBlockFragBytes;
    L.s_int = L.zero + kZeroBytes;
    L.scl = L.s_int + 4 * n_groups * kGroupBlocks;
    L.part = L.scl + 4 * n_groups * kGroupBlocks;
    L.bytes = L.part + 4 * tiles * n_groups * 16;
    return L;
}

// Rows of one 16-row tile (global tile index T: rows 16T .. 16T + 15 over
// all ranges; ranges are multiples of 16 rows, so a tile lies in one range).
struct TileRows {
    uint32_t rbase;    // first row of the tile within its range
    uint32_t n_here;   // rows of the tile that exist (0..16)
    uint32_t d_off, qs_off, out_off;
};

template <int kMode>
__device__ __forceinline__ TileRows tile_rows(const MatvecArgs& a, uint32_t T) {
    TileRows tr;
    uint32_t row = 16 * T;
    tr.n_here = row < a.n_total ? min(16u, a.n_total - row) : 0u;
    tr.d_off = a.range[0].d_offset; tr.qs_off = a.range[0].qs_offset; tr.out_off = a.range[0].output_offset;
    if constexpr (kMode == 2) {
        if (row >= a.range[0].n) {
            row -= a.range[0].n;
            tr.d_off = a.range[1].d_offset; tr.qs_off = a.range[1].qs_offset; tr.out_off = a.range[1].output_offset;
            if (row >= a.range[1].n) {
                row -= a.range[1].n;
                tr.d_off = a.range[2].d_offset; tr.qs_off = a.range[2].qs_offset; tr.out_off = a.range[2].output_offset;
            }
        }
    }
    tr.rbase = row;
    return tr;
}

// One unit's weights for this lane (row c of the tile): the qs of blocks
// 8 grp + g and 8 grp + g + 4 (so that the 4 lanes of a row read 64 contiguous
// bytes per load) and the scales d of blocks 8 grp + 2g, + 1 (the blocks whose
// sums the lane's MFMA results hold). Zeros for rows / blocks that do not exist.
struct UnitW {
    uint4 qa, qb;
    uint16_t da, db;
};

__device__ __forceinline__ UnitW load_unit(const MatvecArgs& a, const TileRows& tr, uint32_t grp, uint32_t nb,
                                           uint32_t g, uint32_t c) {
    UnitW w;
    w.qa = make_uint4(0u, 0u, 0u, 0u);
    w.qb = w.qa;
    w.da = w.db = 0;
    const uint32_t b0 = kGroupBlocks * grp;
    if (c < tr.n_here) {
        const uint64_t r0 = static_cast<uint64_t>(tr.rbase + c) * nb + b0;
        const uint8_t* q = a.weights + tr.qs_off + 16 * r0;
        const uint8_t* d = a.weights + tr.d_off + 2 * r0;
        if (b0 + g < nb) w.qa = *reinterpret_cast<const uint4*>(q + 16 * g);
        if (b0 + g + 4 < nb) w.qb = *reinterpret_cast<const uint4*>(q + 16 * (g + 4));
        if (b0 + 2 * g < nb) w.da = *reinterpret_cast<const uint16_t*>(d + 4 * g);
        if (b0 + 2 * g + 1 < nb) w.db = *reinterpret_cast<const uint16_t*>(d + 4 * g + 2);
    }
    return w;
}

// kMode: 0 plain (x = act), 1 silu (x = f16(silu(gate)) * up), 2 normed
// (x = act * w_norm, scale d * inv_rms, up to 3 row ranges).
//
// Pass 1 stages x as MFMA fragments. Pass 2 runs units (16-row tile, group of
// 8 blocks): 16 MFMAs plus the f32 epilogue, one partial per row.
//  * kStream false: a workgroup owns `tiles_per_wg` tiles and its waves share
//    their units; the partials go through LDS and pass 3 adds a row's groups
//    in order and stores.
//  * kStream true (many rows): each wave walks whole tiles T = its global wave
//    index + i * (all waves), all groups of a tile in order, and stores the
//    rows itself; x is staged once per workgroup for all of its tiles.
// Each wave's weights are loaded one unit (stream: two units) ahead of its
// MFMAs.
template <int kMode, bool kStream>
__global__ __launch_bounds__(kMfMaxThreads) __attribute__((amdgpu_waves_per_eu(kStream ? 4 : 6))) void matvec_q1_0_mfma_kernel(MatvecArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sh[];
    __shared__ float red_sh[kMfMaxThreads / 64];
    const int t = threadIdx.x, n_thr = blockDim.x;
    const int lane = t & 63, n_wave = n_thr >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);   // wave-uniform (scalar registers)
    const uint32_t k = a.k, nb = k / kQ1Block;
    const uint32_t n_groups = (nb + kGroupBlocks - 1) / kGroupBlocks;
    const uint32_t tiles = kStream ? 0u : a.rows_per_wg / 16;
    const MfLayout L = mf_layout(nb, n_groups, tiles);
    int32_t* s_int = reinterpret_cast<int32_t*>(sh + L.s_int);
    float* scl = reinterpret_cast<float*>(sh + L.scl);
    float* part = reinterpret_cast<float*>(sh + L.part);   // [tile][group][16]
    const uint32_t n_tiles_all = (a.n_total + 15) / 16;
    const uint32_t g = lane >> 4, c = lane & 15;

    // This wave's unit sequence: (tile, group) pairs.
    //  split: u = wave, wave + n_wave, .. < tiles * n_groups of this workgroup
    //  stream: tile T = wave_id + i * total waves, groups 0 .. n_groups - 1
    const uint32_t wave_id = blockIdx.x * n_wave + wave, wave_stride = gridDim.x * n_wave;
    auto unit_tile = [&](uint32_t u) -> uint32_t {   // global tile of unit step u of this wave
        if constexpr (kStream) return wave_id + (u / n_groups) * wave_stride;
        else return blockIdx.x * tiles + (wave + u * n_wave) / n_groups;
    };
    auto unit_grp = [&](uint32_t u) -> uint32_t {
        if constexpr (kStream) return u % n_groups;
        else return (wave + u * n_wave) % n_groups;
    };
    auto unit_ok = [&](uint32_t u) -> bool {
        if constexpr (kStream) return unit_tile(u) < n_tiles_all;
        else return wave + u * n_wave < tiles * n_groups && unit_tile(u) < n_tiles_all;
    };

    // x of this thread's first 8 elements, then the first unit's weights, are
    // loaded before anything else (x first: pass 1 waits only for it)
    struct XIn {
        h8v p, q;   // plain / normed: x and w_norm; silu: gate and up
    };
    auto load_x = [&](uint32_t v) {
        XIn r;
        const uint32_t e = 8 * v;
        if constexpr (kMode == 1) {
            r.p = *reinterpret_cast<const h8v*>(a.act + a.gate_offset + e);
            r.q = *reinterpret_cast<const h8v*>(a.act + a.up_offset + e);
        } else {
            r.p = *reinterpret_cast<const h8v*>(a.act + a.input_offset + e);
            if constexpr (kMode == 2) r.q = *reinterpret_cast<const h8v*>(a.w_norms + a.w_norm_off + e);
        }
        return r;
    };
    // this thread's first two groups of 8 (all of x for k <= 16 * blockDim.x)
    XIn x0{}, x1{};
    if (static_cast<uint32_t>(t) < k / 8) x0 = load_x(t);
    if (static_cast<uint32_t>(t + n_thr) < k / 8) x1 = load_x(t + n_thr);
    if constexpr (kStream) {
        // x arrives before this wave's weight requests go out (behind the weight
        // requests of the whole grid, the small x loads would wait for them)
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_sched_barrier(0);
    }
    auto unit_rows = [&](uint32_t u) {
        TileRows tr = tile_rows<kMode>(a, unit_ok(u) ? unit_tile(u) : 0u);
        if (!unit_ok(u)) tr.n_here = 0;
        return tr;
    };
    // weights of this wave's first unit (stream: first two units) in flight
    // during pass 1
    TileRows cur_tr = unit_rows(0), nx1_tr = cur_tr;
    UnitW cur = load_unit(a, cur_tr, unit_grp(0), nb, g, c), nx1{};
    if constexpr (kStream) {
        nx1_tr = unit_rows(1);
        nx1 = load_unit(a, nx1_tr, unit_grp(1), nb, g, c);
    }

    // ---- pass 1: x -> per-block (hi, lo) bytes in fragment order ----------------------
    // Thread v holds elements 8v .. 8v + 7: block v / 16, word w, byte kk of
    // each bit plane p = 0..7.
    float ssq = 0.0f;
    for (uint32_t v = t, it = 0; v < k / 8; v += n_thr, it++) {
        const XIn xin = it == 0 ? x0 : it == 1 ? x1 : load_x(v);
        h8v xv;
        if constexpr (kMode == 0) {
            xv = xin.p;
        } else if constexpr (kMode == 1) {
            // matvec_q1_0_silu.wgsl:86-102: silu in f32, then f16(silu) * up in f16.
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float gf = static_cast<float>(xin.p[i]);
                const float sl = gf / (1.0f + expf(-gf));
                xv[i] = static_cast<_Float16>(sl) * xin.q[i];
            }
        } else {
            // matvec_q1_0_fused_normed.wgsl:102-121: x * w_norm in f16; sum of x^2 in f32.
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float xf = static_cast<float>(xin.p[i]);
                ssq = ssq + xf * xf;
                xv[i] = xin.p[i] * xin.q[i];
            }
        }
        float xf[8], amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            xf[i] = static_cast<float>(xv[i]);
            amax = fmaxf(amax, fabsf(xf[i]));
        }
        // the 16 threads of a block are 16 consecutive lanes
        amax = fmaxf(amax, lane_xor<1>(amax));
        amax = fmaxf(amax, lane_xor<2>(amax));
        amax = fmaxf(amax, lane_xor<4>(amax));
        amax = fmaxf(amax, lane_xor<8>(amax));
        const float qs = amax > 0.0f ? kQMax / amax : 0.0f;
        const uint32_t b = v / 16, w = (v % 16) / 4, kk = v % 4;
        uint8_t* fb = sh + L.frag + b * kBlockFragBytes;   // [h][s][16]
        const uint32_t half = ((b % kGroupBlocks) / 4) * 8;   // block j of a group: K slot j % 4, half j / 4
        int32_t sum = 0;
#pragma unroll
        for (int p = 0; p < 8; p++) {
            const int32_t xi = static_cast<int32_t>(rintf(xf[p] * qs));
            sum += xi;
            const uint32_t s = 4 * w + p / 2, at = s * kFragBytes + half + (p % 2) * 4 + kk;
            fb[at] = static_cast<uint8_t>(xi >> 7);                    // hi
            fb[kRunBytes + at] = static_cast<uint8_t>(xi & 127);       // lo
        }
        if (kk == 0) {   // the other half of this thread's 8 fragments
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int s2 = 0; s2 < 4; s2++)
                    *reinterpret_cast<uint2*>(fb + h * kRunBytes + (4 * w + s2) * kFragBytes + (8 - half)) =
                        make_uint2(0u, 0u);
        }
        sum += static_cast<int32_t>(lane_xor<1>(static_cast<uint32_t>(sum)));
        sum += static_cast<int32_t>(lane_xor<2>(static_cast<uint32_t>(sum)));
        sum += static_cast<int32_t>(lane_xor<4>(static_cast<uint32_t>(sum)));
        sum += static_cast<int32_t>(lane_xor<8>(static_cast<uint32_t>(sum)));
        if ((v % 16) == 0) {
            s_int[b] = sum;
            scl[b] = amax / kQMax;
        }
    }
    for (uint32_t i = t; i < kZeroBytes / 4; i += n_thr) reinterpret_cast<uint32_t*>(sh + L.zero)[i] = 0u;
    float inv_rms = 1.0f;
    if constexpr (kMode == 2) {
        // sum of squares: xor butterfly in each wave, then the waves in order
        ssq = wave_sum(ssq);
        if (lane == 0) red_sh[wave] = ssq;
        __syncthreads();
        float total = 0.0f;
        for (int w = 0; w < n_wave; w++) total += red_sh[w];
        inv_rms = 1.0f / sqrtf(total / static_cast<float>(k) + a.eps);
    } else {
        __syncthreads();
    }

    // ---- pass 2: units (tile, group) -------------------------------------------------
    // this lane's x fragment: A row c = (block c / 2 of the group, hi/lo c % 2), real
    // data only in K slot (c / 2) % 4, the one that holds that block
    const bool b_live = ((c >> 1) & 3) == g;
    float row_acc = 0.0f;   // stream: this tile's groups so far (weight row c)
    for (uint32_t u = 0; unit_ok(u); u++) {
        const uint32_t grp = unit_grp(u);
        // next load: unit u + 2 (stream) or u + 1 (split)
        const TileRows nx2_tr = unit_rows(kStream ? u + 2 : u + 1);
        const UnitW nx2 = load_unit(a, nx2_tr, unit_grp(kStream ? u + 2 : u + 1), nb, g, c);
        const uint8_t* bsrc = b_live ? sh + L.frag + (kGroupBlocks * grp + c / 2) * kBlockFragBytes +
                                           (c & 1) * kRunBytes
                                     : sh + L.zero;
        // two accumulator chains (even / odd MFMAs)
        i4v acc0 = {0, 0, 0, 0}, acc1 = acc0;
        const uint32_t qa4[4] = {cur.qa.x, cur.qa.y, cur.qa.z, cur.qa.w}, qb4[4] = {cur.qb.x, cur.qb.y, cur.qb.z, cur.qb.w};
        // x fragments read 8 at a time ahead of their MFMAs (one LDS latency per 8)
#pragma unroll
        for (int h8 = 0; h8 < 2; h8++) {
            i4v bf[8];
#pragma unroll
            for (int i = 0; i < 8; i++) bf[i] = *reinterpret_cast<const i4v*>(bsrc + (8 * h8 + i) * kFragBytes);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int s = 8 * h8 + i, w = s / 4, p0 = 2 * (s % 4);
                i4v av;
                av[0] = static_cast<int>((qa4[w] >> p0) & 0x01010101u);
                av[1] = static_cast<int>((qa4[w] >> (p0 + 1)) & 0x01010101u);
                av[2] = static_cast<int>((qb4[w] >> p0) & 0x01010101u);
                av[3] = static_cast<int>((qb4[w] >> (p0 + 1)) & 0x01010101u);
                // x fragments as the A operand (rows = (block, hi/lo)), weights as
                // B (columns = the 16 weight rows)
                if (s % 2 == 0) acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[i], av, acc0, 0, 0, 0);
                else acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf[i], av, acc1, 0, 0, 0);
            }
        }
        // acc[jj] = (P_hi, P_lo, P_hi, P_lo) of blocks 8 grp + 2g, + 1 for weight row c
        const i4v acc = acc0 + acc1;
        float rowp = 0.0f;
#pragma unroll
        for (int bb = 0; bb < 2; bb++) {
            const uint32_t be = kGroupBlocks * grp + 2 * g + bb;
            const int32_t ph = acc[2 * bb], pl = acc[2 * bb + 1];
            const int32_t P = 128 * ph + pl;
            float dd = h2f(bb == 0 ? cur.da : cur.db);
            if constexpr (kMode == 2) dd = dd * inv_rms;
            if (be < nb) rowp = rowp + static_cast<float>(2 * P - s_int[be]) * (scl[be] * dd);
        }
        // the 4 lane groups hold the 8 blocks of the group
        rowp = sum_xor16(rowp);
        rowp = sum_xor32(rowp);
        if constexpr (kStream) {
            row_acc = row_acc + rowp;
            if (grp == n_groups - 1) {
                if (g == 0 && c < cur_tr.n_here) {
                    uint16_t* dst = a.act + cur_tr.out_off + cur_tr.rbase + c;
                    if (kMode != 2 && a.accumulate) *dst = f2h(h2f(*dst) + row_acc);
                    else *dst = f2h(row_acc);
                }
                row_acc = 0.0f;
            }
        } else {
            const uint32_t tl = unit_tile(u) - blockIdx.x * tiles;
            if (g == 0) part[(tl * n_groups + grp) * 16 + c] = rowp;
        }
        if constexpr (kStream) {
            cur = nx1;
            cur_tr = nx1_tr;
            nx1 = nx2;
            nx1_tr = nx2_tr;
        } else {
            cur = nx2;
            cur_tr = nx2_tr;
        }
    }
    if constexpr (kStream) return;
    __syncthreads();

    // ---- pass 3 (split): group partials of each row in order ------------------------------
    for (uint32_t r = t; r < tiles * 16; r += n_thr) {
        const uint32_t tl = r / 16;
        const TileRows tr = tile_rows<kMode>(a, blockIdx.x * tiles + tl);
        if (blockIdx.x * tiles + tl >= n_tiles_all || (r % 16) >= tr.n_here) continue;
        float y = 0.0f;
        for (uint32_t gi = 0; gi < n_groups; gi++) y = y + part[(tl * n_groups + gi) * 16 + (r % 16)];
        uint16_t* dst = a.act + tr.out_off + tr.rbase + (r % 16);
        if (kMode != 2 && a.accumulate) *dst = f2h(h2f(*dst) + y);
        else *dst = f2h(y);
    }
}

}  // namespace

hipError_t launch_matvec_q1_0_mfma(const MatvecArgs& args, int mode, hipStream_t s) {
    MatvecArgs a = args;
    const uint32_t nb = a.k / kQ1Block;
    const uint32_t n_groups = (nb + kGroupBlocks - 1) / kGroupBlocks;
    const uint32_t n_tiles = (a.n_total + 15) / 16;
    // Many rows (stream_min_tiles tiles or more): stream (4-wave workgroups,
    // about 2 tiles per wave, at most 4 workgroups per CU). Else split: 32 rows
    // (two tiles) per workgroup while that keeps one wave per unit within 16
    // waves, else 16 rows; 4 waves at least.
    const bool stream = n_tiles >= a.stream_min_tiles;
    uint32_t waves, n_wg, tiles;
    if (stream) {
        waves = 4;
        tiles = 0;
        n_wg = (n_tiles + 2 * waves - 1) / (2 * waves);
        if (n_wg > 4 * a.cu_count) n_wg = 4 * a.cu_count;   // all resident at once
        a.rows_per_wg = 0;
    } else {
        // (a workgroup's rows must lie in one range: ranges of the normed matvec
        // are multiples of 16 rows, 32 allows two tiles)
        bool ranges32 = true;
        if (mode == 2)
            for (int i = 0; i < 3; i++) ranges32 = ranges32 && a.range[i].n % 32 == 0;
        a.rows_per_wg = 2 * n_groups <= 16 && ranges32 ? 32 : 16;
        tiles = a.rows_per_wg / 16;
        waves = tiles * n_groups;
        if (waves > 16) waves = 16;
        if (waves < 4) waves = 4;
        n_wg = (a.n_total + a.rows_per_wg - 1) / a.rows_per_wg;
    }
    const MfLayout L = mf_layout(nb, n_groups, tiles);
    const dim3 block(64 * waves);
#define BP_MF_LAUNCH(M, S) hipLaunchKernelGGL((matvec_q1_0_mfma_kernel<M, S>), dim3(n_wg), block, L.bytes, s, a)
    if (stream) {
        if (mode == 0) BP_MF_LAUNCH(0, true);
        else if (mode == 1) BP_MF_LAUNCH(1, true);
        else BP_MF_LAUNCH(2, true);
    } else {
        if (mode == 0) BP_MF_LAUNCH(0, false);
        else if (mode == 1) BP_MF_LAUNCH(1, false);
        else BP_MF_LAUNCH(2, false);
    }
#undef BP_MF_LAUNCH
    return hipGetLastError();
}

}  // namespace bp
