// Top-k of the f16 logits (gfx950), with the same values AND indices as
// src/shaders/topk_reduce.wgsl (reference repository), ties included.
//
// The reference runs one 256-thread workgroup: thread t keeps a 32-entry
// min-heap over the f16 pairs at words t, t+256, ... (strict > insertion,
// entries start at -1e30 / index 0), heap-sorts it to descending order, and
// the 256 lists are then merged pairwise (list p absorbs list p + s for s =
// 128, 64, .., 1) by one compare stage against the reversed partner and a
// 5-stage bitonic sort. Which of several equal logits survives depends on
// exactly that sequence of heap and network steps, so both are kept; what
// changes is where they run:
//
//  * topk_lane_kernel: one wave per reference thread t (256 waves, one per
//    CU). The heap lives in lanes 0..31 of two VGPRs (value, index); a sift
//    is a chain of uniform-index readlane steps and lane-selects, so nothing goes
//    through LDS. The wave loads 64 of its words at a time (64 elements x 2),
//    and a ballot of "v > heap minimum, at or after the cursor" finds the next
//    element that the reference's loop would insert; the rejected elements
//    cost nothing beyond that one compare. Each wave writes its sorted list
//    (32 x {value, index}) to the scratch buffer.
//  * topk_merge_kernel: one 1024-thread workgroup runs the 8 merge levels on
//    the 256 lists in LDS. One merge is one wave: list p in lanes 0..31, list
//    p + s in lanes 32..63; the compare against the reversed partner is one
//    lane permute (lane i reads lane 63 - i), the bitonic stages are xor
//    shuffles of stride 16 .. 1 with the reference's strict compare-swap.
#include "bp_device.hpp"
#include "bp_kernels.hpp"

namespace bp {
namespace {

constexpr uint32_t kLanes = 256;   // reference workgroup size
constexpr uint32_t kK = 32;        // K_MAX

__device__ __forceinline__ float rl(float v, uint32_t lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ uint32_t rl(uint32_t v, uint32_t lane) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}
// writelane: `x` in lane `lane` (uniform), `old` elsewhere
__device__ __forceinline__ float wl(float x, uint32_t lane, float old) {
    return __lane_id() == lane ? x : old;
}
__device__ __forceinline__ uint32_t wl(uint32_t x, uint32_t lane, uint32_t old) {
    return __lane_id() == lane ? x : old;
}

// Min-heap sift-down of heap[0 .. len) held in lanes 0..len-1 (the left child
// wins ties; a strictly smaller child moves up), topk_reduce.wgsl:42-55.
__device__ __forceinline__ void sift(float& hv, uint32_t& hi, uint32_t len) {
    uint32_t i = 0;
    float vi = rl(hv, 0);
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
        i = m;   // vi (the sifted value) is unchanged
    }
}

__global__ __launch_bounds__(64) void topk_lane_kernel(TopKArgs a) {
    const uint32_t t = blockIdx.x;   // reference thread
    const uint32_t lane = threadIdx.x;
    const uint32_t* words = reinterpret_cast<const uint32_t*>(a.logits + (a.in_offset & ~1u));
    const uint32_t n_words = (a.n + 1) / 2;
    float hv = -1e30f;
    uint32_t hi = 0;
    float root = -1e30f;
    // words t + 256 (64 c + lane), chunk c
    for (uint32_t base = t; base < n_words; base += kLanes * 64) {
        const uint32_t w = base + kLanes * lane;
        const bool ok0 = w < n_words;
        const bool ok1 = ok0 && 2 * w + 1 < a.n;
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
    // heap sort to descending (topk_reduce.wgsl:98-115)
    for (uint32_t last = kK - 1; last > 0; last--) {
        const float v0 = rl(hv, 0), vl = rl(hv, last);
        const uint32_t i0 = rl(hi, 0), il = rl(hi, last);
        hv = wl(vl, 0, hv);
        hv = wl(v0, last, hv);
        hi = wl(il, 0, hi);
        hi = wl(i0, last, hi);
        sift(hv, hi, last);
    }
    if (lane < kK) a.lists[t * kK + lane] = make_uint2(__builtin_bit_cast(uint32_t, hv), hi);
}

// One strict compare-swap stage of stride s across lanes (lane ^ s).
__device__ __forceinline__ void cswap(float& v, uint32_t& ix, uint32_t lane, int s) {
    const float pv = __shfl_xor(v, s);
    const uint32_t pi = __shfl_xor(ix, s);
    const bool lo = (lane & s) == 0;
    // reference: if v[hi] > v[lo] swap
    const bool take = lo ? (pv > v) : (v > pv);
    if (take) { v = pv; ix = pi; }
}

__global__ __launch_bounds__(1024) void topk_merge_kernel(TopKArgs a) {
    __shared__ uint2 lists[kLanes * kK];   // 64 KB
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (uint32_t i = tid; i < kLanes * kK; i += 1024) lists[i] = a.lists[i];
    __syncthreads();
    for (uint32_t s = kLanes / 2; s > 0; s /= 2) {
        for (uint32_t p = wave; p < s; p += 16) {
            const uint2 x = lists[(lane < kK ? p : p + s) * kK + (lane & (kK - 1))];
            float v = __builtin_bit_cast(float, x.x);
            uint32_t ix = x.y;
            // stage 0: a[i] = b[31 - i] if strictly greater (b[31 - i] sits in lane 63 - i)
            const float bv = __shfl(v, 63 - lane);
            const uint32_t bi = __shfl(ix, 63 - lane);
            if (bv > v) { v = bv; ix = bi; }
#pragma unroll
            for (int st = kK / 2; st >= 1; st >>= 1) cswap(v, ix, lane, st);
            if (s > 1) {
                if (lane < kK) lists[p * kK + lane] = make_uint2(__builtin_bit_cast(uint32_t, v), ix);
            } else {
                const uint32_t kk = a.k < kK ? a.k : kK;
                if (lane < kk) {
                    a.result[a.out_offset + lane] = __builtin_bit_cast(uint32_t, v);
                    a.result[a.out_offset + kk + lane] = ix;
                }
            }
        }
        __syncthreads();
    }
}

}  // namespace

uint64_t topk_scratch_bytes() { return static_cast<uint64_t>(kLanes) * kK * sizeof(uint2); }

hipError_t launch_topk_reduce(const TopKArgs& a, hipStream_t s) {
    hipLaunchKernelGGL(topk_lane_kernel, dim3(kLanes), dim3(64), 0, s, a);
    hipLaunchKernelGGL(topk_merge_kernel, dim3(1), dim3(1024), 0, s, a);
    return hipGetLastError();
}

}  // namespace bp
