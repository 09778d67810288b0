// Single-token decode attention over the Q8_0 KV cache (gfx950).
//
// Same result as src/shaders/attention_split.wgsl + attention_merge.wgsl
// (reference repository): scores s_t = (q . k_t) / sqrt(128) over rows
// t in [0, n_keys), softmax in f32, o = sum p_t v_t, f16 output. The work
// decomposition is MI355X-first instead of the reference's 16-row chunks:
//
//  * grid = (n_splits, n_kv_head); one 256-thread workgroup owns one KV head
//    (its 4 GQA query heads) and `split_len` consecutive rows; n_splits is
//    chosen so the launch covers the 256 CUs about twice.
//  * Each wave streams its own rows with no workgroup barrier in the main
//    loop: a wave "round" is 8 rows, lane (slot = lane>>3, seg = lane&7)
//    reading the 16 contiguous qs bytes of dims [16 seg, 16 seg + 16) of its
//    row plus that block's FP32 scale — eight full 128-byte row segments per
//    load instruction. Waves interleave rounds (wave w takes rounds w, w+4,..)
//    and the loads of the next batch of 2 rounds are issued before the current
//    batch is consumed (register double buffering).
//  * int8 -> f32 uses the unsigned-byte converts on bytes xor 0x80
//    (u = q + 128); the +128 bias is removed algebraically:
//      q.k = sum q_i u_i - 128 sum q_i,   sum_t p_t v_t = sum_t p_t u_t - 128 sum_t p_t.
//  * Online softmax in the exp2 domain; the row max is shared by the whole
//    wave (3 xor shuffles), so the per-lane running sums need no reduction
//    until the end, and O is rescaled only when some max moved.
//  * End of split: shuffles reduce O over the 8 row slots, LDS merges the 4
//    waves (log-sum-exp), and with more than one split the last workgroup of a
//    KV head to finish (atomic ticket) merges all splits in parallel and resets
//    the ticket (attention_merge.wgsl:85-129), so one launch does the decode.
#include "bp_device.hpp"
#include "bp_kernels.hpp"

namespace bp {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kRounds = 2;                 // rounds (8 rows each) per wave batch
constexpr int kPartStride = kHeadDim + 2;  // o[128], m, l
constexpr int kMaxMergeSplits = 256;

struct alignas(16) Q16 { uint32_t w[4]; };

struct Batch {
    Q16 kq[kRounds], vq[kRounds];
    float kd[kRounds], vd[kRounds];
};

__device__ __forceinline__ float ub(uint32_t w, int i) {   // v_cvt_f32_ubyte{i}
    return static_cast<float>((w >> (8 * i)) & 0xffu);
}

__global__ __launch_bounds__(kThreads, 2) void decode_kernel(DecodeArgs a) {
    __shared__ float o_sh[kWaves][kGroup][kHeadDim];
    __shared__ float ml_sh[kWaves][kGroup][2];
    __shared__ float ms_sh[kGroup][kMaxMergeSplits];
    __shared__ float ls_sh[kGroup][kMaxMergeSplits];
    __shared__ uint32_t last_sh;

    const int t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int seg = lane & 7;              // dims [16*seg, 16*seg+16)
    const int slot = lane >> 3;            // row within a round
    const uint32_t g = blockIdx.y;
    const uint32_t split = blockIdx.x;
    const uint32_t row0 = split * a.split_len;
    const uint32_t row_end = min(row0 + a.split_len, a.n_keys);
    const float c2 = a.scale * 1.4426950408889634f;   // scores in log2 units

    // Query slice of the 4 heads, and its per-lane sums (for the +128 bias).
    float qf[kGroup][16], qsum[kGroup];
#pragma unroll
    for (int h = 0; h < kGroup; h++) {
        const uint16_t* qp = a.q + (static_cast<uint64_t>(g) * kGroup + h) * kHeadDim + 16 * seg;
        const Q16 r0 = *reinterpret_cast<const Q16*>(qp);
        const Q16 r1 = *reinterpret_cast<const Q16*>(qp + 8);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            qf[h][2 * i] = h2f(r0.w[i] & 0xffffu);
            qf[h][2 * i + 1] = h2f(r0.w[i] >> 16);
            qf[h][8 + 2 * i] = h2f(r1.w[i] & 0xffffu);
            qf[h][8 + 2 * i + 1] = h2f(r1.w[i] >> 16);
        }
#pragma unroll
        for (int i = 0; i < 16; i++) s += qf[h][i];
        qsum[h] = 128.0f * s;
    }

    float o[kGroup][16], bsum[kGroup], lsum[kGroup], m_run[kGroup];
#pragma unroll
    for (int h = 0; h < kGroup; h++) {
        bsum[h] = 0.0f; lsum[h] = 0.0f; m_run[h] = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; i++) o[h][i] = 0.0f;
    }

    const uint64_t kv_dim = a.kv_dim;
    const uint32_t nb_row = a.kv_dim / kBlock;
    const uint32_t col = g * kHeadDim + 16 * seg;
    const uint32_t dcol = g * (kHeadDim / kBlock) + (seg >> 1);
    // Row of (batch b, round r) for this lane: row0 + 32*(kRounds*b + r) + 8*wave + slot.
    auto row_of = [&](uint32_t b, int r) {
        return row0 + 32u * (kRounds * b + r) + 8u * wave + slot;
    };
    auto load = [&](Batch& B, uint32_t b) {
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            const uint32_t row = row_of(b, r);
            const bool ok = row < row_end;
            B.kq[r] = ok ? *reinterpret_cast<const Q16*>(a.k.qs + row * kv_dim + col) : Q16{{0, 0, 0, 0}};
            B.kd[r] = ok ? a.k.d[static_cast<uint64_t>(row) * nb_row + dcol] : 0.0f;
            B.vq[r] = ok ? *reinterpret_cast<const Q16*>(a.v.qs + row * kv_dim + col) : Q16{{0, 0, 0, 0}};
            B.vd[r] = ok ? a.v.d[static_cast<uint64_t>(row) * nb_row + dcol] : 0.0f;
        }
    };
    auto consume = [&](const Batch& B, uint32_t b) {
        float s[kRounds][kGroup];
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            Q16 k;
#pragma unroll
            for (int i = 0; i < 4; i++) k.w[i] = B.kq[r].w[i] ^ 0x80808080u;
            float dot[kGroup];
#pragma unroll
            for (int h = 0; h < kGroup; h++) {
                float acc = -qsum[h];
#pragma unroll
                for (int i = 0; i < 16; i++) acc = __builtin_fmaf(qf[h][i], ub(k.w[i >> 2], i & 3), acc);
                dot[h] = acc * B.kd[r];
            }
#pragma unroll
            for (int off = 1; off <= 4; off <<= 1)
#pragma unroll
                for (int h = 0; h < kGroup; h++) dot[h] += __shfl_xor(dot[h], off);
            const bool ok = row_of(b, r) < row_end;
#pragma unroll
            for (int h = 0; h < kGroup; h++) s[r][h] = ok ? dot[h] * c2 : -INFINITY;
        }
        float alpha[kGroup];
        bool moved = false;
#pragma unroll
        for (int h = 0; h < kGroup; h++) {
            float bm = s[0][h];
#pragma unroll
            for (int r = 1; r < kRounds; r++) bm = fmaxf(bm, s[r][h]);
            bm = fmaxf(bm, __shfl_xor(bm, 8));
            bm = fmaxf(bm, __shfl_xor(bm, 16));
            bm = fmaxf(bm, __shfl_xor(bm, 32));
            const float m_new = fmaxf(m_run[h], bm);
            alpha[h] = __builtin_amdgcn_exp2f(m_run[h] - m_new);   // 0 on the first batch
            moved |= m_new != m_run[h];
            m_run[h] = m_new;
        }
        if (moved) {   // wave-uniform: m_run is identical in all lanes
#pragma unroll
            for (int h = 0; h < kGroup; h++) {
                lsum[h] *= alpha[h];
                bsum[h] *= alpha[h];
#pragma unroll
                for (int i = 0; i < 16; i++) o[h][i] *= alpha[h];
            }
        }
#pragma unroll
        for (int r = 0; r < kRounds; r++) {
            Q16 v;
#pragma unroll
            for (int i = 0; i < 4; i++) v.w[i] = B.vq[r].w[i] ^ 0x80808080u;
            float vf[16];
#pragma unroll
            for (int i = 0; i < 16; i++) vf[i] = ub(v.w[i >> 2], i & 3);
#pragma unroll
            for (int h = 0; h < kGroup; h++) {
                const float p = __builtin_amdgcn_exp2f(s[r][h] - m_run[h]);   // 0 for masked rows
                lsum[h] += p;
                const float pv = p * B.vd[r];
                bsum[h] += pv;
#pragma unroll
                for (int i = 0; i < 16; i++) o[h][i] = __builtin_fmaf(pv, vf[i], o[h][i]);
            }
        }
    };

    // Batches this wave has rows in: rows of batch b start at row_of(b, 0) (slot 0).
    const uint32_t n_rows = row_end - row0;
    const uint32_t n_batches = n_rows > 8u * wave ? (n_rows - 8u * wave + 32u * kRounds - 1) / (32u * kRounds) : 0u;
    if (n_batches > 0) {
        Batch A, Bb;
        load(A, 0);
        uint32_t b = 0;
        while (true) {
            if (b + 1 < n_batches) load(Bb, b + 1);
            consume(A, b);
            if (++b >= n_batches) break;
            if (b + 1 < n_batches) load(A, b + 1);
            consume(Bb, b);
            if (++b >= n_batches) break;
        }
    }

    // ---- per-wave totals: O over the 8 row slots, l over row slots ----------
#pragma unroll
    for (int h = 0; h < kGroup; h++) {
#pragma unroll
        for (int i = 0; i < 16; i++) o[h][i] -= 128.0f * bsum[h];
#pragma unroll
        for (int off = 8; off <= 32; off <<= 1) {
            lsum[h] += __shfl_xor(lsum[h], off);
#pragma unroll
            for (int i = 0; i < 16; i++) o[h][i] += __shfl_xor(o[h][i], off);
        }
    }
    if (slot == 0) {
#pragma unroll
        for (int h = 0; h < kGroup; h++)
#pragma unroll
            for (int i = 0; i < 16; i++) o_sh[wave][h][16 * seg + i] = o[h][i];
    }
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < kGroup; h++) { ml_sh[wave][h][0] = m_run[h]; ml_sh[wave][h][1] = lsum[h]; }
    }
    __syncthreads();

    // ---- merge the 4 waves; thread t -> head t>>6, dims 2*(t&63), +1 -------
    const int fh = t >> 6, fd = 2 * (t & 63);
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; w++) M = fmaxf(M, ml_sh[w][fh][0]);
    float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) {
        const float mw = ml_sh[w][fh][0];
        const float e = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);   // waves without rows
        L = __builtin_fmaf(e, ml_sh[w][fh][1], L);
        o0 = __builtin_fmaf(e, o_sh[w][fh][fd], o0);
        o1 = __builtin_fmaf(e, o_sh[w][fh][fd + 1], o1);
    }
    const uint32_t qh = g * kGroup + fh;
    uint32_t* out = reinterpret_cast<uint32_t*>(a.out + static_cast<uint64_t>(qh) * kHeadDim + fd);
    if (a.n_splits == 1) {
        const float inv_l = 1.0f / L;
        *out = static_cast<uint32_t>(f2h(o0 * inv_l)) | (static_cast<uint32_t>(f2h(o1 * inv_l)) << 16);
        return;
    }
    float* part = a.partials + (static_cast<uint64_t>(qh) * a.n_splits + split) * kPartStride;
    *reinterpret_cast<float2*>(part + fd) = make_float2(o0, o1);
    if ((t & 63) == 0) { part[kHeadDim] = M; part[kHeadDim + 1] = L; }

    // ---- the last workgroup of this KV head merges all splits --------------
    __threadfence();
    __syncthreads();
    if (t == 0) last_sh = atomicAdd(&a.tickets[g], 1u) == a.n_splits - 1 ? 1u : 0u;
    __syncthreads();
    if (last_sh == 0) return;
    __threadfence();
    const uint32_t ns = a.n_splits;
    const float* pg = a.partials + static_cast<uint64_t>(g) * kGroup * ns * kPartStride;
    for (uint32_t i = t; i < kGroup * ns; i += kThreads) {
        const uint32_t h = i / ns, s = i % ns;
        const float* ps = pg + (static_cast<uint64_t>(h) * ns + s) * kPartStride;
        ms_sh[h][s] = __builtin_nontemporal_load(ps + kHeadDim);
        ls_sh[h][s] = __builtin_nontemporal_load(ps + kHeadDim + 1);
    }
    __syncthreads();
    {   // wave h: global max and weights of head h
        float mx = -INFINITY;
        for (uint32_t s = lane; s < ns; s += 64) mx = fmaxf(mx, ms_sh[wave][s]);
        mx = wave_max(mx);
        float l = 0.0f;
        for (uint32_t s = lane; s < ns; s += 64) {
            const float w = __builtin_amdgcn_exp2f(ms_sh[wave][s] - mx);
            ms_sh[wave][s] = w;
            l = __builtin_fmaf(w, ls_sh[wave][s], l);
        }
        l = wave_sum(l);
        if (lane == 0) ls_sh[wave][0] = l;   // slot 0 reused for the total (read after the barrier)
    }
    __syncthreads();
    const float* ph = pg + static_cast<uint64_t>(fh) * ns * kPartStride + fd;
    float a0 = 0.0f, a1 = 0.0f;
    uint32_t s = 0;
    for (; s + 4 <= ns; s += 4) {
        float2 v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            v[j].x = __builtin_nontemporal_load(ph + (s + j) * kPartStride);
            v[j].y = __builtin_nontemporal_load(ph + (s + j) * kPartStride + 1);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float w = ms_sh[fh][s + j];
            a0 = __builtin_fmaf(w, v[j].x, a0);
            a1 = __builtin_fmaf(w, v[j].y, a1);
        }
    }
    for (; s < ns; s++) {
        const float w = ms_sh[fh][s];
        a0 = __builtin_fmaf(w, __builtin_nontemporal_load(ph + s * kPartStride), a0);
        a1 = __builtin_fmaf(w, __builtin_nontemporal_load(ph + s * kPartStride + 1), a1);
    }
    const float inv_l = 1.0f / ls_sh[fh][0];
    *out = static_cast<uint32_t>(f2h(a0 * inv_l)) | (static_cast<uint32_t>(f2h(a1 * inv_l)) << 16);
    if (t == 0) atomicExch(&a.tickets[g], 0u);
}

}  // namespace

void decode_plan(uint32_t n_keys, uint32_t n_kv_head, int cu_count, uint32_t* split_len,
                 uint32_t* n_splits) {
    // ~2 workgroups per CU; rows per split a multiple of 32 (one round of all
    // 4 waves), at least 64, and at most kMaxMergeSplits splits.
    const uint32_t target = static_cast<uint32_t>(cu_count > 0 ? cu_count : 256) * 2;
    uint32_t want = (target + n_kv_head - 1) / n_kv_head;
    if (want < 1) want = 1;
    uint32_t len = (n_keys + want - 1) / want;
    len = (len + 31) / 32 * 32;
    if (len < 64) len = 64;
    const uint32_t min_len = (n_keys + kMaxMergeSplits - 1) / kMaxMergeSplits;
    if (len < min_len) len = (min_len + 31) / 32 * 32;
    *split_len = len;
    *n_splits = (n_keys + len - 1) / len;
}

hipError_t launch_decode(const DecodeArgs& a, uint32_t n_kv_head, hipStream_t s) {
    hipLaunchKernelGGL(decode_kernel, dim3(a.n_splits, n_kv_head), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace bp
