// Top-k of the f16 logits (gfx950), with the same values AND indices as
// src/shaders/topk_reduce.wgsl (reference repository), ties included.
//
// The reference runs one 256-thread workgroup: thread t keeps a 32-entry
// min-heap over the f16 pairs at words t, t+256, ... (strict > insertion,
// entries start at -1e30 / index 0), heap-sorts it to descending order, and
// the 256 lists are then merged pairwise (list p absorbs list p + s for s =
// 128, 64, .., 1) by one compare stage against the reversed partner and a
// 5-stage bitonic sort. Which of several equal logits survives, and in which
// order, follows from that exact sequence of steps.
//
// This kernel gets the same result without running 256 sequential heaps. Call
// an element "big" if its value is >= V, the 32nd-largest insertable value
// (insertable: > -1e30, i.e. not NaN and not -inf), and every other list
// entry "small". Every compare of the heaps and of the merge network between a
// big and a small is decided by the values alone, and compares between smalls
// only move smalls among the slots that smalls occupy. So the final top 32 (all
// bigs) do not depend on the smalls' values or order, only on which list slots
// hold smalls. In a reference thread whose bigs have pairwise different values,
// the heap-sorted list holds those bigs in descending order in its first slots
// and smalls in the rest; that list can be written directly, with -1e30 /
// index 0 as the smalls. Only threads with two equal bigs need their heap
// replayed step by step.
//
// One 1024-thread workgroup:
//  1. every thread takes the maximum of its share of the logits (16-byte
//     loads, all in flight together) and keeps its groups' maxima; tau = the
//     32nd largest of these 1024 maxima, by a two-round radix select on 16-bit
//     order keys (so at least 32 elements are >= tau): LDS-atomic histograms,
//     a DPP prefix scan over the bins;
//  2. the elements >= tau (a few dozen on real logits) are gathered in LDS,
//     only by threads whose maximum reaches tau and only from groups whose
//     maximum does (f16 compares with tau's value); among them V (exact) and
//     the bigs follow by counting, and each big's slot in its reference
//     thread's list by counting the larger bigs of that thread (one wave when
//     there are at most 64, comparing only bigs whose thread holds two or
//     more); equal bigs in one thread mark it "replay";
//  3. the replayed threads run the reference heap, one wave per thread (heap
//     in lanes 0..31, sifts by uniform readlanes), reading the logits again;
//     more than kCap gathered elements (massive ties) replay all 256;
//  4. the merge tree on the 256 lists in LDS: list p in lanes 0..31, list
//     p + s in lanes 32..63, the reversed compare and the stride-16 exchange
//     by row swaps, strides 1-8 by DPP, with the reference's strict
//     compare-swap. Merges whose second list is pure fill are skipped (lists
//     are sorted descending, so they are no-ops); merges of two one-entry
//     lists (or of an empty and a one-entry list) are closed-form; the rest
//     run the network, two per wave side by side.
#include <climits>

#include "bp_device.hpp"
#include "bp_kernels.hpp"

namespace bp {
namespace {

constexpr uint32_t kLanes = 256;    // reference workgroup size
constexpr uint32_t kK = 32;         // K_MAX
constexpr uint32_t kThreads = 1024;
constexpr uint32_t kWaves = kThreads / 64;
constexpr uint32_t kCap = 2048;     // gathered elements >= tau
constexpr uint32_t kRegGroups = 19; // 16-byte groups per thread loaded together
constexpr uint32_t kGmaxCap = kRegGroups * 1024;   // group maxima kept in LDS
constexpr float kEmpty = -1e30f;    // the reference's initial heap value

__device__ __forceinline__ float rl(float v, uint32_t lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ uint32_t rl(uint32_t v, uint32_t lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}
// writelane: `x` in lane `lane` (uniform), `old` elsewhere
__device__ __forceinline__ float wl(float x, uint32_t lane, float old) { return __lane_id() == lane ? x : old; }
__device__ __forceinline__ uint32_t wl(uint32_t x, uint32_t lane, uint32_t old) {
    return __lane_id() == lane ? x : old;
}

// Min-heap sift-down of heap[0 .. len) held in lanes 0..len-1 (the left child
// wins ties; a strictly smaller child moves up), topk_reduce.wgsl:42-55.
__device__ __forceinline__ void sift(float& hv, uint32_t& hi, uint32_t len) {
    uint32_t i = 0;
    const float vi = rl(hv, 0);
    for (;;) {
        const uint32_t l = 2 * i + 1, r = l + 1;
        uint32_t m = i;
        float vm = vi;
        if (l < len) {
            const float vl = rl(hv, l);
            if (vl < vm) { m = l; vm = vl; }
        }
        if (r < len) {
            const float vr = rl(hv, r);
            if (vr < vm) { m = r; vm = vr; }
        }
        if (m == i) return;
        const uint32_t ii = rl(hi, i), im = rl(hi, m);
        hv = wl(vm, i, hv);
        hv = wl(vi, m, hv);
        hi = wl(im, i, hi);
        hi = wl(ii, m, hi);
        i = m;   // the sifted value vi moves down with i
    }
}

// The reference thread t's heap (topk_reduce.wgsl:65-115), replayed by one
// wave: lanes 0..31 end with its list, descending.
__device__ void replay_thread(const uint32_t* words, uint32_t n, uint32_t t, float& hv, uint32_t& hi) {
    const uint32_t lane = __lane_id();
    const uint32_t n_words = (n + 1) / 2;
    hv = kEmpty;
    hi = 0;
    float root = kEmpty;
    // words t + 256 (64 c + lane) for chunk c, visited in order
    for (uint32_t base = t; base < n_words; base += kLanes * 64) {
        const uint32_t w = base + kLanes * lane;
        const bool ok0 = w < n_words;
        const bool ok1 = ok0 && 2 * w + 1 < n;
        const uint32_t pair = ok0 ? words[w] : 0u;
        const float v0 = h2f(static_cast<uint16_t>(pair & 0xFFFFu));
        const float v1 = h2f(static_cast<uint16_t>(pair >> 16));
        uint32_t cursor = 0;   // next element (2 lane + h) of this chunk to visit
        for (;;) {
            const bool c0 = ok0 && 2 * lane >= cursor && v0 > root;
            const bool c1 = ok1 && 2 * lane + 1 >= cursor && v1 > root;
            const uint64_t mask = __ballot(c0 || c1);
            if (mask == 0) break;
            const uint32_t j = __builtin_ctzll(mask);
            const uint32_t h = rl(static_cast<uint32_t>(c0 ? 0u : 1u), j);
            const float val = h ? rl(v1, j) : rl(v0, j);
            const uint32_t e = 2 * rl(w, j) + h;
            hv = wl(val, 0, hv);
            hi = wl(e, 0, hi);
            sift(hv, hi, kK);
            root = rl(hv, 0);
            cursor = 2 * j + h + 1;
        }
    }
    for (uint32_t last = kK - 1; last > 0; last--) {   // heap sort, :98-115
        const float v0 = rl(hv, 0), vl = rl(hv, last);
        const uint32_t i0 = rl(hi, 0), il = rl(hi, last);
        hv = wl(vl, 0, hv);
        hv = wl(v0, last, hv);
        hi = wl(il, 0, hi);
        hi = wl(i0, last, hi);
        sift(hv, hi, last);
    }
}

// Value of lane (lane ^ 16) / (lane ^ 32): v_permlane16/32_swap of a
// register with itself leaves the partner's value in one of its two results,
// which one depending on the lane's 16-lane (32-lane) row.
__device__ __forceinline__ uint32_t xor16_lane(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return (__lane_id() & 16) ? r0 : r1;
}
__device__ __forceinline__ uint32_t xor32_lane(uint32_t v) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    const uint32_t r0 = r[0], r1 = r[1];
    return (__lane_id() & 32) ? r0 : r1;
}
// Value of lane 63 - lane: DPP row mirror (15 - lane within 16 lanes), then
// the rows reversed (lane ^ 48).
__device__ __forceinline__ uint32_t rev_lane(uint32_t v) {
    const uint32_t m = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), 0x140, 0xF, 0xF, true));
    return xor16_lane(xor32_lane(m));
}

// Value of lane (lane ^ S): DPP lane moves for S = 1, 2, 4, 8 (quad
// permutes, half-row mirror + quad permute, row rotation by 8), a row swap
// for 16.
template <int S>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
    const int x = static_cast<int>(v);
    // (every source lane exists: bound_ctrl, no old value to preset)
    if constexpr (S == 1) return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true));
    else if constexpr (S == 2) return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true));
    else if constexpr (S == 4) {
        const int m = __builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, true);   // lane ^ 7
        return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(m, 0x1B, 0xF, 0xF, true));   // ^ 3
    } else if constexpr (S == 8) return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true));
    else return xor16_lane(v);
}

// One strict compare-swap stage of stride S (lanes l, l ^ S) on N lists.
template <int S, int N>
__device__ __forceinline__ void merge_stages(float (&v)[N], uint32_t (&ix)[N], uint32_t lane) {
    const float sgn = (lane & S) == 0 ? 1.0f : -1.0f;
#pragma unroll
    for (int u = 0; u < N; u++) {
        const float pv = __builtin_bit_cast(float, xor_lane<S>(__builtin_bit_cast(uint32_t, v[u])));
        const uint32_t pi = xor_lane<S>(ix[u]);
        // reference: if v[hi] > v[lo] swap, i.e. take the partner's entry if
        // it is strictly larger (lo lane) or strictly smaller (hi lane). As one
        // compare of the signed difference: list values are f16 values, +-inf
        // or the -1e30 fill, so pv - v is 0 or NaN (inf - inf) exactly when no
        // swap is due and never rounds to 0 otherwise.
        const bool take = (pv - v[u]) * sgn > 0.0f;
        v[u] = take ? pv : v[u];
        ix[u] = take ? pi : ix[u];
    }
}

// N merges of one tree level run side by side by one wave, so that their
// lane-exchange chains overlap: list p[u] absorbs list p[u] + s (list p in
// lanes 0..31, list p + s in lanes 32..63).
// (merge_lists_loaded: the lane's entries of the two lists already loaded)
template <int N>
__device__ __forceinline__ void merge_lists_loaded(uint2* lists, const uint32_t (&p)[N], const uint2 (&xv)[N],
                                                   uint32_t s, uint32_t lane, uint32_t* result, uint32_t out_offset,
                                                   uint32_t kk) {
    float v[N];
    uint32_t ix[N];
#pragma unroll
    for (int u = 0; u < N; u++) {
        v[u] = __builtin_bit_cast(float, xv[u].x);
        ix[u] = xv[u].y;
    }
#pragma unroll
    for (int u = 0; u < N; u++) {
        // stage 0: a[i] = b[31 - i] if strictly greater (b[31 - i] sits in lane 63 - i)
        const float bv = __builtin_bit_cast(float, rev_lane(__builtin_bit_cast(uint32_t, v[u])));
        const uint32_t bi = rev_lane(ix[u]);
        const bool take = bv > v[u];
        v[u] = take ? bv : v[u];
        ix[u] = take ? bi : ix[u];
    }
    merge_stages<16, N>(v, ix, lane);
    merge_stages<8, N>(v, ix, lane);
    merge_stages<4, N>(v, ix, lane);
    merge_stages<2, N>(v, ix, lane);
    merge_stages<1, N>(v, ix, lane);
#pragma unroll
    for (int u = 0; u < N; u++) {
        if (s > 1) {
            if (lane < kK) lists[p[u] * kK + lane] = make_uint2(__builtin_bit_cast(uint32_t, v[u]), ix[u]);
        } else if (lane < kk) {
            result[out_offset + lane] = __builtin_bit_cast(uint32_t, v[u]);
            result[out_offset + kk + lane] = ix[u];
        }
    }
}

template <int N>
__device__ __forceinline__ void merge_lists(uint2* lists, const uint32_t (&p)[N], uint32_t s, uint32_t lane,
                                            uint32_t* result, uint32_t out_offset, uint32_t kk) {
    uint2 xv[N];
#pragma unroll
    for (int u = 0; u < N; u++) xv[u] = lists[(lane < kK ? p[u] : p[u] + s) * kK + (lane & (kK - 1))];
    merge_lists_loaded<N>(lists, p, xv, s, lane, result, out_offset, kk);
}

// 16-bit key with the order of the f16 values (-0 and +0 share a key).
__device__ __forceinline__ uint32_t hkey(uint16_t h) {
    if (h == 0x8000u) h = 0;
    return (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
}
__device__ __forceinline__ uint16_t unkey16(uint32_t k) {   // inverse of hkey (+0 for key 0x8000)
    return static_cast<uint16_t>((k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu));
}
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
// Packed maximum of the 8 f16 values of a 16-byte group (as 2 lanes).
__device__ __forceinline__ h2 group_max(const uint4& q) {
    const h2 a = __builtin_elementwise_max(__builtin_bit_cast(h2, q.x), __builtin_bit_cast(h2, q.y));
    const h2 b = __builtin_elementwise_max(__builtin_bit_cast(h2, q.z), __builtin_bit_cast(h2, q.w));
    return __builtin_elementwise_max(a, b);
}
__device__ __forceinline__ bool insertable(uint16_t h) {   // > -1e30 as f32: not NaN, not -inf
    return (h & 0x7FFFu) <= 0x7C00u && h != 0xFC00u;
}

struct TopKShared {
    uint2 lists[kLanes * kK];   // {f32 bits, index}
    uint32_t hist[256];
    _Float16 gmax[kGmaxCap];    // maximum of each 16-byte group (maxNum: NaN-free unless all NaN)
    uint2 cand[kCap];
    uint32_t cand_big[kCap];    // 1 if a big
    uint32_t cand_slot[kCap];   // a big's slot in its thread's list
    uint32_t replay[kLanes];    // per reference thread: 1 = replay its heap
    uint32_t replay_ids[kLanes];
    uint32_t dirty[kLanes];     // list holds anything but the -1e30 / 0 fill
    uint32_t multi[kLanes];     // list holds two or more entries (merge tree)
    uint32_t tcnt[kLanes];      // bigs per reference thread (one-wave case)
    float cval[64];             // candidate values (one-wave case)
    uint32_t n_cand, n_replay, sel_hi, sel_rank, tau_key;
};

// Inclusive prefix sum over the 64 lanes: within each 16-lane row by DPP row
// shifts (lanes without a source add 0), then the totals of the rows below
// (read from lanes 15, 31, 47) added per row.
__device__ __forceinline__ uint32_t wave_incl_sum(uint32_t v) {
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xF, 0xF, true));   // row_shr:1
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xF, 0xF, true));   // row_shr:2
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xF, 0xF, true));   // row_shr:4
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xF, 0xF, true));   // row_shr:8
    const uint32_t t0 = rl(v, 15), t1 = rl(v, 31), t2 = rl(v, 47);
    const uint32_t row = __lane_id() >> 4;
    const uint32_t below = (row >= 1 ? t0 : 0u) + (row >= 2 ? t1 : 0u) + (row >= 3 ? t2 : 0u);
    return v + below;
}

// Key of the rank-th largest (0-based) of the 1024 keys held one per thread
// (0 = no value), by two 8-bit radix rounds; 0 if fewer than rank + 1 keys.
__device__ uint32_t select_key(TopKShared& sh, uint32_t key, uint32_t rank) {
    const uint32_t tid = threadIdx.x;
    for (int round = 0; round < 2; round++) {
        if (tid < 256) sh.hist[tid] = 0;
        __syncthreads();
        const bool in = key != 0 && (round == 0 || (key >> 8) == sh.sel_hi);
        const uint32_t bin = round == 0 ? key >> 8 : key & 0xFFu;
        if (in) atomicAdd(&sh.hist[bin], 1u);   // same-bin lanes serialize inside the LDS
        __syncthreads();
        if (tid < 64) {   // one wave scans the bins from the top
            const uint32_t want = round == 0 ? rank : sh.sel_rank;
            uint32_t c[4], tot = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) { c[i] = sh.hist[255 - (4 * tid + i)]; tot += c[i]; }
            const uint32_t incl = wave_incl_sum(tot);   // inclusive prefix over lanes (bins from the top)
            uint32_t run = incl - tot;
            bool found = false;
            uint32_t bin = 0, above = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (!found && run + c[i] > want) { found = true; bin = 255 - (4 * tid + i); above = run; }
                run += c[i];
            }
            const uint64_t fm = __ballot(found);
            if (fm == 0) {
                if (tid == 0) { sh.sel_hi = 0xFFFFFFFFu; sh.tau_key = 0; }
            } else if (tid == __builtin_ctzll(fm)) {
                if (round == 0) { sh.sel_hi = bin; sh.sel_rank = want - above; }
                else sh.tau_key = (sh.sel_hi << 8) | bin;
            }
        }
        __syncthreads();
        if (sh.sel_hi == 0xFFFFFFFFu) return 0;
    }
    return sh.tau_key;
}

__global__ __launch_bounds__(kThreads) void topk_kernel(TopKArgs a) {
    __shared__ TopKShared sh;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint16_t* x = a.logits + (a.in_offset & ~1u);
    const uint32_t* words = reinterpret_cast<const uint32_t*>(x);
    const uint32_t n = a.n;
    // 16-byte groups of 8 elements from the first 16-byte boundary; the
    // elements before it (head, < 8) and after the last group (tail) are
    // visited one by one.
    const uint32_t head = min(static_cast<uint32_t>(((16u - (reinterpret_cast<uintptr_t>(x) & 15u)) & 15u) / 2u), n);
    const uint32_t n_groups = (n - head) / 8;
    const uint32_t tail0 = head + 8 * n_groups;
    const uint4* groups = reinterpret_cast<const uint4*>(x + head);
    auto single = [&](uint32_t i) -> uint16_t { return i < n ? x[i] : static_cast<uint16_t>(0xFC00u); };

    if (tid == 0) { sh.n_cand = 0; sh.n_replay = 0; }
    for (uint32_t i = tid; i < kLanes * kK; i += kThreads)
        sh.lists[i] = make_uint2(__builtin_bit_cast(uint32_t, kEmpty), 0u);
    if (tid < kLanes) { sh.replay[tid] = 0; sh.dirty[tid] = 0; sh.tcnt[tid] = 0; }

    // ---- 1. per-thread maximum key of the insertable values. The groups are
    // taken kRegGroups per thread at a time into registers (all loads in
    // flight together); with n up to kRegGroups * 8192 the gather below reuses
    // them instead of reading again.
    const uint32_t per_round = kRegGroups * kThreads;
    const uint32_t n_rounds = (n_groups + per_round - 1) / per_round;
    uint4 q[kRegGroups];
    auto load_round = [&](uint32_t r) __attribute__((always_inline)) {
        // unconditional loads of clamped groups (n_groups >= 1 here), so that
        // all of them are in flight before the first is used
#pragma unroll
        for (uint32_t u = 0; u < kRegGroups; u++) {
            const uint32_t g = r * per_round + u * kThreads + tid;
            q[u] = groups[min(g, n_groups - 1)];
        }
#pragma unroll
        for (uint32_t u = 0; u < kRegGroups; u++) {
            const uint32_t g = r * per_round + u * kThreads + tid;
            if (g >= n_groups) q[u] = make_uint4(0xFC00FC00u, 0xFC00FC00u, 0xFC00FC00u, 0xFC00FC00u);
        }
    };
    // packed f16 maximum (maxNum: NaN operands drop out; -inf is the identity)
    h2 hm = {-INFINITY, -INFINITY};
    _Float16 gmx[kRegGroups];   // group maxima of the last round (the gather's first test)
    for (uint32_t r = 0; r < n_rounds; r++) {
        load_round(r);
#pragma unroll
        for (uint32_t u = 0; u < kRegGroups; u++) {
            const h2 gm = group_max(q[u]);
            hm = __builtin_elementwise_max(hm, gm);
            const uint32_t g = r * per_round + u * kThreads + tid;
            const _Float16 g0 = gm.x, g1 = gm.y;   // (scalars before the cast)
            gmx[u] = g0 > g1 ? g0 : g1;
            if (n_rounds > 1 && g < kGmaxCap) sh.gmax[g] = gmx[u];
        }
    }
    uint32_t mk = 0;
    auto take_max = [&](uint16_t h) { if (insertable(h)) mk = max(mk, hkey(h)); };
    {   // copied to scalars before the bit casts (a bit cast of a vector element
        // directly compiles to element 0)
        const _Float16 m0 = hm.x, m1 = hm.y;
        take_max(__builtin_bit_cast(uint16_t, m0));
        take_max(__builtin_bit_cast(uint16_t, m1));
    }
    if (tid < 8) take_max(single(tid < head ? tid : n));
    else if (tid < 16) take_max(single(tail0 + tid - 8));
    // tau: the 32nd largest maximum (at least 32 elements are >= tau); with
    // fewer than 32 maxima, every insertable element is gathered
    uint32_t tau = select_key(sh, mk, kK - 1);
    if (tau == 0) tau = hkey(0xFBFFu);   // -65504, the smallest insertable value

    // ---- 2. gather the elements >= tau (few on real logits): one LDS atomic
    // per 8-element group that holds any; past kCap every heap is replayed
    // (an f16 compare with tau's value is the same test: NaN fails it, and -inf
    // is below every tau; -0 and +0 compare equal as their keys do)
    const _Float16 tau_h = __builtin_bit_cast(_Float16, unkey16(tau));
    auto take = [&](uint16_t h) { return __builtin_bit_cast(_Float16, h) >= tau_h; };
    // groups whose maximum reaches tau (maxima from LDS up to kGmaxCap groups,
    // recomputed beyond), then their elements
    auto gather_group = [&](const uint4& qg, uint32_t g) __attribute__((always_inline)) {
        const uint32_t w[4] = {qg.x, qg.y, qg.z, qg.w};
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) m |= take(static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)))) ? 1u << e : 0u;
        uint32_t slot = atomicAdd(&sh.n_cand, static_cast<uint32_t>(__popc(m)));
#pragma unroll 1
        for (; m; m &= m - 1, slot++) {
            const int e = __builtin_ctz(m);
            const uint16_t h = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
            if (slot < kCap) sh.cand[slot] = make_uint2(__builtin_bit_cast(uint32_t, h2f(h)), head + 8 * g + e);
        }
    };
    auto gmax_h = [](const uint4& qg) {   // maxNum: NaN only for an all-NaN group
        const h2 gm = group_max(qg);
        const _Float16 g0 = gm.x, g1 = gm.y;
        return g0 > g1 ? g0 : g1;
    };
    if (n_rounds == 1) {
        // the only round is still in registers (groups past the end hold -inf)
        if (mk >= tau) {   // only threads whose maximum key reaches tau hold any
#pragma unroll
            for (uint32_t u = 0; u < kRegGroups; u++)
                if (gmx[u] >= tau_h) gather_group(q[u], u * kThreads + tid);
        }
    } else {
#pragma unroll 1
        for (uint32_t g = tid; g < n_groups; g += kThreads) {
            const _Float16 gm = g < kGmaxCap ? sh.gmax[g] : gmax_h(groups[g]);
            if (gm >= tau_h) gather_group(groups[g], g);
        }
    }
    if (wave == 0) {   // head and tail elements
        const uint32_t i = lane < 8 ? lane : tail0 + lane - 8;
        const bool ok = lane < 8 ? lane < head : (lane < 16 && i < n);
        if (ok && take(x[i])) {
            const uint32_t slot = atomicAdd(&sh.n_cand, 1u);
            if (slot < kCap) sh.cand[slot] = make_uint2(__builtin_bit_cast(uint32_t, h2f(x[i])), i);
        }
    }
    __syncthreads();
    const uint32_t n_cand = sh.n_cand;
    const bool overflow = n_cand > kCap;
    if (!overflow && n_cand <= 64) {
        // one wave: lane i holds candidate i
        if (wave == 0) {
            const bool live = lane < n_cand;
            const uint2 c = live ? sh.cand[lane] : make_uint2(__builtin_bit_cast(uint32_t, kEmpty), 0u);
            const float vi = __builtin_bit_cast(float, c.x);
            const uint32_t ti = (c.y >> 1) & (kLanes - 1);
            // g = the number of larger candidates, from the 64 values (padded
            // with -1e30, which is below every candidate) broadcast from LDS
            sh.cval[lane] = vi;
            __builtin_amdgcn_s_waitcnt(0);
            __builtin_amdgcn_wave_barrier();
            uint32_t gp[4] = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 64; j++) gp[j & 3] += sh.cval[j] > vi;
            const uint32_t g = (gp[0] + gp[1]) + (gp[2] + gp[3]);
            const bool big = live && g < kK;
            // r = the larger bigs of the same reference thread; only threads
            // holding two or more bigs (counted in LDS) need the comparison
            if (big) atomicAdd(&sh.tcnt[ti], 1u);
            __builtin_amdgcn_s_waitcnt(0);
            __builtin_amdgcn_wave_barrier();
            const bool coll = big && sh.tcnt[ti] > 1;
            uint64_t collm = __ballot(coll);
            uint32_t r = 0;
            bool dup = false;
            while (collm) {
                const uint32_t j = __builtin_ctzll(collm);
                collm &= collm - 1;
                const float vj = rl(vi, j);
                const uint32_t tj = rl(ti, j);
                if (coll && j != lane && tj == ti) {
                    r += vj > vi;
                    dup = dup || vj == vi;
                }
            }
            if (big && (dup || r >= kK)) sh.replay[ti] = 1;
            __builtin_amdgcn_s_waitcnt(0);
            __builtin_amdgcn_wave_barrier();
            if (big && r < kK && !sh.replay[ti]) { sh.lists[ti * kK + r] = c; sh.dirty[ti] = 1; }
        }
        __syncthreads();   // the replay flags are read by waves 0-3 below
    } else if (!overflow) {
        // V = the 32nd largest gathered value; bigs = gathered values >= V,
        // i.e. fewer than 32 gathered values above them
        for (uint32_t i = tid; i < n_cand; i += kThreads) {
            const float vi = __builtin_bit_cast(float, sh.cand[i].x);
            uint32_t g = 0;
            for (uint32_t j = 0; j < n_cand; j++) g += __builtin_bit_cast(float, sh.cand[j].x) > vi;
            sh.cand_big[i] = g < kK ? 1u : 0u;
        }
        __syncthreads();
        // slot of each big in its reference thread's list; equal bigs -> replay
        for (uint32_t i = tid; i < n_cand; i += kThreads) {
            if (!sh.cand_big[i]) continue;
            const float vi = __builtin_bit_cast(float, sh.cand[i].x);
            const uint32_t ti = (sh.cand[i].y >> 1) & (kLanes - 1);
            uint32_t r = 0;
            bool dup = false;
            for (uint32_t j = 0; j < n_cand; j++) {
                if (j == i || !sh.cand_big[j]) continue;
                if (((sh.cand[j].y >> 1) & (kLanes - 1)) != ti) continue;
                const float vj = __builtin_bit_cast(float, sh.cand[j].x);
                r += vj > vi;
                dup = dup || vj == vi;
            }
            if (dup || r >= kK) sh.replay[ti] = 1;
            sh.cand_slot[i] = r;
        }
        __syncthreads();
        for (uint32_t i = tid; i < n_cand; i += kThreads) {
            if (!sh.cand_big[i]) continue;
            const uint32_t r = sh.cand_slot[i];
            const uint32_t ti = (sh.cand[i].y >> 1) & (kLanes - 1);
            if (r < kK && !sh.replay[ti]) { sh.lists[ti * kK + r] = sh.cand[i]; sh.dirty[ti] = 1; }
        }
    }
    if (tid < kLanes && (overflow || sh.replay[tid])) sh.replay_ids[atomicAdd(&sh.n_replay, 1u)] = tid;
    __syncthreads();

    // ---- 3. replay the reference heaps that the shortcut cannot write
    const uint32_t n_replay = sh.n_replay;
    for (uint32_t e = wave; e < n_replay; e += kWaves) {
        const uint32_t t = sh.replay_ids[e];
        float hv;
        uint32_t hi;
        replay_thread(words, n, t, hv, hi);
        if (lane < kK) sh.lists[t * kK + lane] = make_uint2(__builtin_bit_cast(uint32_t, hv), hi);
        if (lane == 0) sh.dirty[t] = 1;
    }
    __syncthreads();

    // ---- 4. merge tree (topk_reduce.wgsl:117-184). Lists are always sorted
    // descending, so a merge whose second list is pure fill (-1e30 / 0, which
    // never wins the strict compares) leaves the first one unchanged and is
    // skipped. A wave runs its merges of a level (up to 8) side by side so that
    // their lane-exchange chains overlap.
    // Per list: dirty (anything but fill) and multi (two or more entries;
    // lists are sorted descending, so "slot 1 is not fill"), in LDS.
    const uint32_t fill_bits = __builtin_bit_cast(uint32_t, kEmpty);
    if (tid < kLanes) sh.multi[tid] = sh.dirty[tid] != 0 && sh.lists[tid * kK + 1].x != fill_bits ? 1u : 0u;
    __syncthreads();
    const uint32_t wv = __builtin_amdgcn_readfirstlane(wave);
    const uint32_t kk = a.k < kK ? a.k : kK;
#pragma unroll 1
    for (uint32_t s = kLanes / 2; s > 0; s /= 2) {
        if (wv >= s) return;   // no merges left for this wave (ended waves leave the barriers)
        // Lane u < 8 looks at merge u of this wave: list p = wave + 16 u
        // absorbs list p + s. With list p + s dirty it runs the network if
        // either list holds two or more entries, and is closed-form otherwise
        // (one entry on each side, or none in list p): the reference network
        // leaves [x, y] if y <= x and [y, x] if y > x (x = list p's entry or
        // fill, y = list p + s's entry). At s = 1 the network always runs (it
        // writes the result).
        // (from s = 16 on a wave has one merge, p = wave: its lists are read
        // in the same round trip as the flags)
        uint2 pre[1];
        if (s <= kWaves) pre[0] = sh.lists[(lane < kK ? wv : wv + s) * kK + (lane & (kK - 1))];
        const uint32_t pu = wv + kWaves * lane;
        const bool valid = lane < 8 && pu < s;
        const uint32_t dp = valid ? sh.dirty[pu] : 0u, di = valid ? sh.dirty[pu + s] : 0u;
        const uint32_t mp = valid ? sh.multi[pu] : 0u, mi = valid ? sh.multi[pu + s] : 0u;
        const bool merge = di != 0 || (s == 1 && valid);
        const bool use_net = merge && (mp != 0 || mi != 0 || s == 1);
        uint32_t net = static_cast<uint32_t>(__ballot(use_net)) & 0xFFu;
        if (merge && !use_net) {   // closed-form
            const uint2 x = sh.lists[pu * kK], y = sh.lists[(pu + s) * kK];
            if (__builtin_bit_cast(float, y.x) > __builtin_bit_cast(float, x.x)) {
                sh.lists[pu * kK] = y;
                sh.lists[pu * kK + 1] = x;
            } else {
                sh.lists[pu * kK + 1] = y;
            }
        }
        if (merge) {   // flags of the merged list (list p + s is not read again)
            sh.dirty[pu] = 1u;
            sh.multi[pu] = mp != 0 || mi != 0 || dp != 0 ? 1u : 0u;
        }
        if (s <= kWaves) {
            if (net) {
                const uint32_t ps[1] = {wv};
                merge_lists_loaded<1>(sh.lists, ps, pre, s, lane, a.result, a.out_offset, kk);
            }
            net = 0;
        }
        // network merges two at a time (one if one is left)
#pragma unroll 1
        while (net) {
            const uint32_t u0 = __builtin_ctz(net);
            net &= net - 1;
            if (net) {
                const uint32_t u1 = __builtin_ctz(net);
                net &= net - 1;
                const uint32_t ps[2] = {wv + kWaves * u0, wv + kWaves * u1};
                merge_lists<2>(sh.lists, ps, s, lane, a.result, a.out_offset, kk);
            } else {
                const uint32_t ps[1] = {wv + kWaves * u0};
                merge_lists<1>(sh.lists, ps, s, lane, a.result, a.out_offset, kk);
            }
        }
        __syncthreads();
    }
}

}  // namespace

hipError_t launch_topk_reduce(const TopKArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(topk_kernel, dim3(1), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace bp
