// Internal interface between the host layer (bp_api.cpp) and the gfx950
// kernels. Every launcher checks nothing: argument validation is the host
// layer's job, and it has been done by the time a launcher runs.
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace bp {

constexpr uint32_t kHeadDim = 128;   // Bonsai head_dim (src/model.rs:1179-1183)
constexpr uint32_t kGroup = 4;       // Q heads per KV head (attention_split.wgsl:150)
constexpr uint32_t kBlock = 32;      // Q8_0 block (src/forward.rs:40-47)
constexpr uint32_t kPrefillTileTok = 32;   // query tokens per prefill tile
// Default split-K plan of decode_plan: fewest rows per split, and the row
// count from which the split pass reads 4 KV heads per workgroup.
constexpr uint32_t kDecodeMinSplitRows = 128;
constexpr uint32_t kDecodeWideMinRows = 8192;

// One (layer, kind) view of a Q8_0 KV buffer: FP32 scales at d (index
// (row*kv_dim + e)/32), int8 quants at qs (index row*kv_dim + e).
struct KvView {
    const float* d;
    const int8_t* qs;
};

// q_norm_rope_fused / kv_writeback_fused share the per-head norm+rope stage.
struct QNormRopeArgs {
    uint16_t* act;            // f16 bits
    const uint16_t* w_norms;  // f16 bits
    const uint16_t* rope_cs;  // f16 bits, [max_seq][64][(cos, sin)]
    uint64_t q_off;           // element offset of Q (token 0, head 0)
    uint64_t w_off;           // element offset of w_q_norm
    uint32_t pos_base;
    uint32_t q_dim;           // n_head * 128
    float eps;
    uint32_t n_head, n_items;   // set by launch_q_norm_rope (m_tokens * n_head items)
    uint32_t head_shift;        // set by launch_q_norm_rope: log2(n_head) if a power of two, else 32
};

struct KvWritebackArgs {
    const uint16_t* act;
    const uint16_t* w_norms;
    const uint16_t* rope_cs;
    float* k_d;               // layer base of kv_k's d-section
    int8_t* k_qs;             // layer base of kv_k's qs-section
    float* v_d;
    int8_t* v_qs;
    uint64_t k_cur_off, v_cur_off, w_off;
    uint32_t pos_base;
    uint32_t kv_dim;          // n_kv_head * 128
    float eps;
    uint32_t n_kv_head, n_pairs;   // set by launch_kv_writeback (m_tokens * n_kv_head pairs)
    uint32_t head_shift;           // set by launch_kv_writeback: log2(n_kv_head) if a power of two, else 32
};

struct DecodeArgs {
    const uint16_t* q;        // act + q_off: [n_head][128] (raw, un-normalized q when fused)
    uint16_t* out;            // act + out_off: [n_head][128]
    KvView k, v;              // layer bases
    float* partials;          // n_head * n_splits * decode_partial_stride() floats: o rows, then (m, l)
    uint32_t kv_dim;
    uint32_t n_rows;          // rows streamed by the split pass: [0, n_rows)
    uint32_t split_len;       // rows per workgroup, multiple of 32
    uint32_t n_splits;        // >= 1
    uint32_t heads_per_wg;    // split-pass layout: 1 or 4 KV heads per workgroup
    float scale;
    // Fused decode step only (q_norm_rope + kv_writeback of row `pos` + attention
    // over rows [0, pos]): the split pass normalizes q itself and writes cache row
    // `pos`; the merge pass adds that row and stores the normalized q into act.
    uint16_t* q_act;          // act + q_off (receives the normalized q)
    uint16_t* q_norm;         // scratch [n_head][128] f16
    const uint16_t* k_cur;    // act + k_cur_off: [n_kv_head][128]
    const uint16_t* v_cur;    // act + v_cur_off
    const uint16_t* w_norms;
    const uint16_t* rope_cs;
    uint64_t w_q_off, w_k_off;
    uint32_t pos;
    float eps;
};

struct PrefillArgs {
    const uint16_t* q;        // act + q_off: [m][n_head][128]
    uint16_t* out;            // act + out_off
    KvView k, v;
    uint32_t kv_dim;
    uint32_t q_stride;        // n_head * 128
    uint32_t m_tokens;
    uint32_t pos;             // first query's RoPE/cache position when causal
    uint32_t causal;          // 1: token m sees rows [0, pos+m]; 0: rows [0, pos)
    uint32_t n_tiles;         // ceil(m_tokens / kPrefillTileTok)
    uint32_t heads_per_wave;  // 2: prefill32_kernel (4 heads x 32 tokens per role); 1: prefill_kernel (two or four workgroups per tile pair)
    uint32_t wg_waves;        // with 1 head per wave: 8 (two head sets) or 4 (four, one head each)
    // Key split (short chunks over long caches, with direct = 1): n_ksplit > 1
    // workgroups of prefill_split_kernel per (KV head, tile pair), each over
    // split_chunks 64-row chunks of the pair's key range, write partial (O, m,
    // l) to kpart, [m][n_head][n_ksplit] x 132 floats (O, m, l, pad);
    // prefill_merge_kernel combines them.
    uint32_t n_ksplit;
    uint32_t split_chunks;
    float* kpart;
    float scale;
    // Image of the layer's K and V, written by the dequantization pass for
    // rows [0, n_rows) (zeros up to the next 64-row chunk), per KV head g:
    // K   at k16  + (g * ws_chunks + c) * 64 * 128: f16 rows of chunk c, row-major;
    // V^T at vt16 + (g * ws_chunks + c) * 128 * 64: f16 dims of chunk c, slot-major;
    // K residual at kl8 + (g * ws_chunks + c) * 64 * 128 bytes: per row and
    //   32-element block, 2^11 * (k - f16(k)) as fp6 (e2m3) with a power-of-two
    //   block scale (32 bytes: 6 words of fp6, the scale in word 6), so that
    //   f16 + residual carry the f32 key to about 15 bits.
    uint16_t* k16;
    uint16_t* vt16;
    uint8_t* kl8;
    uint32_t ws_chunks;       // 64-row chunks per KV head in the image
    uint32_t vt_order;        // key order of V^T: 0 for prefill_kernel, 1 for prefill32_kernel
    uint32_t n_rows;          // rows the queries attend: cur of the last token
    // 1: the key split runs prefill_split_kernel, which reads the cache's
    // Q8_0 rows itself: no image is written (the dequantization pass is
    // skipped and the preparation pass only writes the new rows and q).
    uint32_t direct;
};
// Fused prefill step (q_norm_rope + kv_writeback + attention for the
// m_tokens tokens at cache rows [pos, pos + m_tokens)): what the preparation
// pass reads and writes besides PrefillArgs. All act / w_norms offsets are
// multiples of 8 elements and the bases 16-byte aligned.
struct PrefillStepArgs {
    uint16_t* q_act;          // act + q_off: [m][n_head][128], normalized in place
    const uint16_t* k_cur;    // act + k_cur_off: [m][kv_dim]
    const uint16_t* v_cur;    // act + v_cur_off
    const uint16_t* w_norms;
    const uint16_t* rope_cs;  // [max_seq][64][(cos, sin)]
    uint64_t w_q_off, w_k_off;
    float* k_d;               // writable layer bases of the cache (the KvViews of PrefillArgs)
    int8_t* k_qs;
    float* v_d;
    int8_t* v_qs;
    float eps;
};
// Token x split products the key-split partials are sized for (the host
// picks n_ksplit within it).
constexpr uint32_t kPrefillSplitTok = 2048;
// Bytes of the K/V image for max_seq rows (one layer): f16 K, f16 V^T and
// the K residual, 640 bytes per (row, KV head).
inline uint64_t prefill_image_bytes(uint32_t n_kv_head, uint32_t max_seq) {
    return 5ull * n_kv_head * ((max_seq + 63) / 64) * 64 * 128;
}

// Q1_0 matvec family (matvec_q1_0*.wgsl). Byte offsets into `weights`,
// f16-element offsets into `act` / `w_norms` (inputs 8-element aligned).
struct MatvecRange {
    uint32_t d_offset, qs_offset, n, output_offset;
};
struct MatvecArgs {
    const uint8_t* weights;
    uint16_t* act;
    const uint16_t* w_norms;  // normed mode only
    uint32_t k;               // multiple of 128, <= matvec_max_k()
    uint32_t n_total;         // rows over all ranges
    uint32_t input_offset;    // plain / normed input x
    uint32_t gate_offset, up_offset;   // silu mode input silu(gate) * up
    uint32_t w_norm_off;
    float eps;
    uint32_t accumulate;      // plain / silu: y = f16(f32(y) + acc)
    MatvecRange range[3];     // plain / silu: range[0] only; normed: multiples of 32 rows
    uint32_t rows_per_wg;     // set by the launchers
    uint32_t stream_min_tiles;   // MFMA matvec: rows / 16 from which waves stream whole tiles
    uint32_t cu_count;
};
// mode 0: matvec_q1_0, 1: matvec_q1_0_silu, 2: matvec_q1_0_fused_normed.
hipError_t launch_matvec_q1_0(const MatvecArgs& a, int mode, hipStream_t s);
hipError_t launch_matvec_q1_0_mfma(const MatvecArgs& a, int mode, hipStream_t s);
uint32_t matvec_max_k();

// Prefill projections (quantize_q8_0 / matmul_q1_0_q8_0).
struct QuantArgs {
    const uint16_t* act;      // f16 activations
    uint8_t* out;             // Q8_0 buffer (bytes)
    uint32_t k, m;            // k multiple of 32
    uint32_t input_offset;    // f16 elements
    uint32_t d_offset, qs_offset;   // bytes, multiples of 4
};
struct MatmulArgs {
    const uint8_t* weights;   // Q1_0 weight buffer (bytes)
    const uint8_t* acts;      // Q8_0 activation buffer (bytes)
    uint16_t* y;              // f16 output buffer
    uint32_t k, n, m;         // k multiple of 128
    uint32_t w_d_offset, w_qs_offset, a_d_offset, a_qs_offset;   // bytes
    uint32_t out_offset;      // f16 elements
    uint32_t accumulate;
};
struct TopKArgs {
    const uint16_t* logits;   // f16 activation buffer
    uint32_t* result;         // u32 result buffer
    uint32_t n, in_offset, out_offset, k;   // in_offset: f16 elements (rounded down to even)
};
hipError_t launch_topk_reduce(const TopKArgs& a, hipStream_t s);
hipError_t launch_quantize_act_q8_0(const QuantArgs& a, hipStream_t s);
hipError_t launch_matmul_q1_0_q8_0(const MatmulArgs& a, hipStream_t s);

hipError_t launch_q_norm_rope(const QNormRopeArgs& a, uint32_t n_head, uint32_t m_tokens,
                              hipStream_t s);
hipError_t launch_kv_writeback(const KvWritebackArgs& a, uint32_t n_kv_head, uint32_t m_tokens,
                               hipStream_t s);
// Split-K plan of a decode over n_rows rows (1 <= n_splits <= decode_max_splits())
// and the split pass's layout (heads_per_wg = 4 from wide_min_rows rows on).
void decode_plan(uint32_t n_rows, uint32_t n_kv_head, int cu_count, uint32_t min_split_rows,
                 uint32_t wide_min_rows, uint32_t* split_len, uint32_t* n_splits, uint32_t* heads_per_wg);
uint32_t decode_max_splits();
uint32_t decode_partial_stride();   // floats per (head, split) partial
// Plain decode (q already normalized, cache row already written): one launch
// when n_splits == 1, else split pass + merge pass.
hipError_t launch_decode(const DecodeArgs& a, uint32_t n_kv_head, hipStream_t s);
// Fused decode step: split pass (with q norm + row writeback) + merge pass.
hipError_t launch_decode_step(const DecodeArgs& a, uint32_t n_kv_head, hipStream_t s);
hipError_t launch_prefill(const PrefillArgs& a, uint32_t n_kv_head, hipStream_t s);
// Whether the launches of launch_prefill (step = false) or launch_prefill_step
// (step = true) for these arguments fit HIP's grid limits (y, z <= 65535).
bool prefill_grid_fits(const PrefillArgs& a, bool step);
// The fused prefill step: preparation pass (in place of the dequantization
// pass) and attention, 2 launches; with prep_only the first launch alone.
hipError_t launch_prefill_step(const PrefillArgs& a, const PrefillStepArgs& w, uint32_t n_kv_head, hipStream_t s,
                               bool prep_only);

}  // namespace bp
