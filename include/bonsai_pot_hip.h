/*
 * bonsai_pot_hip.h — C ABI of the MI355X (gfx950) attention hot path of
 * bonsai-pot: Q/K RMSNorm + NEOX RoPE, Q8_0 KV-cache writeback, split-K
 * decode attention and causal (chunked) prefill attention.
 *
 * The entry points replace the reference's crate-private dispatch helpers
 * (paths relative to the reference repository root) one for one:
 *
 *   bp_dispatch_q_norm_rope_fused    <- dispatch_q_norm_rope_fused   src/forward.rs:392-413
 *   bp_dispatch_kv_writeback_fused   <- dispatch_kv_writeback_fused  src/forward.rs:359-388
 *   bp_dispatch_attention_decode     <- split+merge block in layer_post_kv_in_pass
 *                                       src/forward.rs:820-857
 *   bp_dispatch_attention_decode_step <- the three above for one token (fused, 2 launches)
 *   bp_dispatch_attention            <- dispatch_attention           src/forward.rs:501-532
 *   bp_dispatch_attention_prefill_step <- q_norm_rope + kv_writeback + attention for m tokens (fused, 2 launches)
 *   bp_dispatch_matvec_q1_0          <- dispatch_matvec_q1_0         src/forward.rs:212-241
 *   bp_dispatch_matvec_q1_0_silu     <- dispatch_matvec_q1_0_silu    src/forward.rs:243-282
 *   bp_dispatch_matvec_q1_0_fused_normed <- dispatch_matvec_q1_0_fused_normed
 *                                       src/forward.rs:284-334
 *   bp_dispatch_quantize_act         <- dispatch_quantize_act        src/forward.rs:415-441
 *   bp_dispatch_matmul_q1_0          <- dispatch_matmul_q1_0         src/forward.rs:443-472
 *   bp_dispatch_topk_reduce          <- dispatch_topk_reduce         src/forward.rs:336-354
 *   bp_topk_readback                 <- wait_topk_readback           src/forward.rs:542-568
 *   bp_model_create / _destroy       <- KV / RoPE / partials part of Model::load_with_options
 *                                       src/model.rs:1148-1248
 *   bp_kv_snapshot_capture / _apply  <- kv_snapshot::capture / apply src/kv_snapshot.rs:203-372
 *   bp_check_device                  <- Model::check_device          src/model.rs:1733-1741
 *   bp_debug_lose_device             <- Model::__destroy_device_for_test src/model.rs:1746-1751
 *
 * Conventions (the same as the reference's Params structs):
 *   - `act` is one f16 buffer; *_off arguments are f16-ELEMENT offsets into it.
 *   - `w_norms` is the f16 norm-weight buffer; w_*_norm_off are element offsets.
 *   - kv_k / kv_v are owned by the model and keep the reference byte layout
 *     (src/forward.rs:40-58, src/model.rs:1167-1215):
 *       [d-section: n_layer*max_seq*(kv_dim/32) f32][qs-section: n_layer*max_seq*kv_dim i8]
 *   - All calls are asynchronous on the model's stream, stream-ordered, and
 *     never allocate device memory. One model is driven by one host thread at
 *     a time (src/session.rs:67-88).
 *   - Every call returns a bp_status; nothing unwinds across the ABI. After a
 *     device fault the model latches "lost" and every later call returns
 *     BP_ERR_DEVICE_LOST (src/model.rs:1087-1098, :1733-1741).
 */
#ifndef BONSAI_POT_HIP_H
#define BONSAI_POT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t bp_status;
/* Status codes; each maps onto a PotError variant (src/error.rs:8-38). */
#define BP_OK                    0
#define BP_ERR_CONFIG           -1  /* PotError::Config */
#define BP_ERR_CONTEXT_OVERFLOW -2  /* PotError::ContextOverflow */
#define BP_ERR_INVALID_ARG      -3  /* PotError::Config (bad pointer / offset) */
#define BP_ERR_HIP              -4  /* runtime error other than device loss */
#define BP_ERR_DEVICE_LOST      -5  /* PotError::DeviceLost */
#define BP_ERR_OUT_OF_MEMORY    -6  /* allocation at model creation failed */
#define BP_ERR_NO_DEVICE        -7  /* PotError::NoAdapter */

/* Attention-side subset of Config (src/model.rs:568-656). */
typedef struct bp_config {
    uint32_t n_layer;
    uint32_t n_head;         /* query heads (32 for Bonsai 4B/8B) */
    uint32_t n_kv_head;      /* KV heads (8); n_head/n_kv_head must be 4 */
    uint32_t head_dim;       /* must be 128 (src/model.rs:1179-1183) */
    float rms_eps;           /* 1e-6 for Bonsai */
    float rope_freq_base;    /* 1e6 for Bonsai */
} bp_config;

typedef struct bp_model bp_model;

/* Creates the device-side state the attention path owns: kv_k, kv_v (zeroed),
 * the f16 RoPE table for positions [0, max_seq) and the split-K partials
 * scratch. `device` is a HIP device ordinal. BP_ERR_CONFIG when
 * max_seq * kv_dim exceeds 2^32 (the kernels' per-layer offsets are 32-bit). */
bp_status bp_model_create(const bp_config* cfg, uint32_t max_seq, int device, bp_model** out);
void bp_model_destroy(bp_model* model);

/* Stream all later calls are ordered on (a hipStream_t; NULL = the null stream).
 * Switching to another stream first waits for the device to drain (all work
 * queued so far, on any stream), since the model's scratch buffers are shared
 * by all launches; the old stream's handle is not used, so it may already be
 * destroyed. Not to be called while a stream of this device is being captured
 * into a graph. */
bp_status bp_model_set_stream(bp_model* model, void* stream);
/* Blocks until the model's stream is idle; latches device loss on failure. */
bp_status bp_model_synchronize(bp_model* model);

/* Device pointers and sizes of the model-owned buffers (for snapshotting,
 * tests and the caller's own bookkeeping). Any out-pointer may be NULL. */
bp_status bp_model_kv_buffers(const bp_model* model, void** kv_k, void** kv_v, uint64_t* bytes_each);
bp_status bp_model_rope_table(const bp_model* model, const void** rope_cs_f16);
uint32_t bp_model_max_seq(const bp_model* model);

/* Layer base offsets inside kv_k / kv_v: (u32-word offset of the d-section,
 * byte offset of the qs-section) — src/forward.rs:48-58 (u64 here). */
bp_status bp_kv_layer_offsets(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq, uint32_t il,
                              uint64_t* d_word_offset, uint64_t* qs_byte_offset);
/* Bytes of one KV buffer: n_layer*max_seq*(kv_dim/32)*4 + n_layer*max_seq*kv_dim
 * (src/model.rs:1184-1187). */
uint64_t bp_kv_buffer_bytes(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq);

/* q_norm_rope_fused (src/shaders/q_norm_rope_fused.wgsl): for m_tokens tokens
 * starting at RoPE position pos_base, RMSNorm each 128-wide Q head, multiply by
 * w_q_norm, apply NEOX RoPE, and write f16 back in place at act[q_off...]. */
bp_status bp_dispatch_q_norm_rope_fused(bp_model* model, void* act, const void* w_norms,
                                        uint32_t q_off, uint32_t w_q_norm_off,
                                        uint32_t pos_base, uint32_t m_tokens);

/* kv_writeback_fused (src/shaders/kv_writeback_fused.wgsl): for m_tokens
 * tokens written at cache rows [pos_base, pos_base+m_tokens) of layer
 * layer_il: K = RoPE(RMSNorm(k)*w_k_norm), V = v; both Q8_0-quantized
 * (d = amax/127 FP32, q = clamp(rne(x*(1/d)), +-127)) into kv_k / kv_v. */
bp_status bp_dispatch_kv_writeback_fused(bp_model* model, const void* act, const void* w_norms,
                                         uint32_t k_cur_off, uint32_t v_cur_off,
                                         uint32_t w_k_norm_off, uint32_t layer_il,
                                         uint32_t pos_base, uint32_t m_tokens);

/* Single-token decode attention at step position `pos`: the query at
 * act[q_off] ([n_head][128] f16) attends cache rows [0, pos] of layer
 * layer_il (pos+1 rows, src/forward.rs:822), split-K over the sequence with a
 * log-sum-exp merge; writes f16 [n_head][128] at act[out_off]. */
bp_status bp_dispatch_attention_decode(bp_model* model, void* act, uint32_t q_off,
                                       uint32_t out_off, uint32_t layer_il, uint32_t pos);

/* One whole attention decode step for one layer at step position `pos`, in
 * two launches instead of the reference's four dispatches: the same results as
 *   bp_dispatch_q_norm_rope_fused(act, w_norms, q_off, w_q_norm_off, pos, 1)
 *   bp_dispatch_kv_writeback_fused(act, w_norms, k_cur_off, v_cur_off, w_k_norm_off, layer_il, pos, 1)
 *   bp_dispatch_attention_decode(act, q_off, out_off, layer_il, pos)
 * i.e. src/forward.rs:796-804 + :618-628 + :820-857 for one token. act[q_off]
 * holds the raw (pre-norm) query and receives the normalized one; cache row
 * `pos` receives the new K/V; act[out_off] receives the attention output. */
bp_status bp_dispatch_attention_decode_step(bp_model* model, void* act, const void* w_norms,
                                            uint32_t q_off, uint32_t k_cur_off, uint32_t v_cur_off,
                                            uint32_t out_off, uint32_t w_q_norm_off,
                                            uint32_t w_k_norm_off, uint32_t layer_il, uint32_t pos);

/* Batched attention (src/shaders/attention.wgsl, src/forward.rs:501-532) over
 * m_tokens query tokens at act[q_off] ([m][n_head][128] f16), writing
 * act[out_off] ([m][n_head][128] f16). Token m attends cache rows
 * [0, cur) with cur = is_prefill ? pos + m + 1 : pos. With pos == 0 and
 * is_prefill != 0 this is the reference's causal prefill from an empty cache;
 * pos > 0 is causal chunked prefill over an existing cache (the reference
 * reaches that result only one token at a time, src/forward.rs:914-967).
 * BP_ERR_CONFIG when the cache rows or tokens exceed the kernels' grid limits
 * (more than 65535 64-row chunks, or 65535 pairs of 32-token tiles). */
bp_status bp_dispatch_attention(bp_model* model, void* act, uint32_t q_off, uint32_t out_off,
                                uint32_t layer_il, uint32_t pos, uint32_t m_tokens,
                                uint32_t is_prefill);

/* One whole causal prefill-attention step for one layer: m_tokens tokens at
 * cache rows [pos, pos+m_tokens), in two launches instead of four, with the
 * same results as
 *   bp_dispatch_q_norm_rope_fused(act, w_norms, q_off, w_q_norm_off, pos, m_tokens)
 *   bp_dispatch_kv_writeback_fused(act, w_norms, k_cur_off, v_cur_off, w_k_norm_off, layer_il, pos, m_tokens)
 *   bp_dispatch_attention(act, q_off, out_off, layer_il, pos, m_tokens, 1)
 * i.e. src/forward.rs:392-413 + :359-388 + :501-532 as the prefill layer
 * calls them (src/forward.rs:1141-1172). act[q_off] holds the raw
 * queries and receives the normalized ones; cache rows [pos, pos+m_tokens)
 * receive the new K/V; act[out_off] receives the attention output. q_off and
 * out_off must be multiples of 8; when the other offsets are not (or act /
 * w_norms are not 16-byte aligned) the call runs the three dispatches above.
 * BP_ERR_CONFIG when the preparation pass's grid would exceed 65535 in y
 * (2 per 64-row chunk of the cache rows plus 4 per 32-row half holding the new
 * rows: about 2 million rows), or as bp_dispatch_attention. */
bp_status bp_dispatch_attention_prefill_step(bp_model* model, void* act, const void* w_norms,
                                             uint32_t q_off, uint32_t k_cur_off, uint32_t v_cur_off,
                                             uint32_t out_off, uint32_t w_q_norm_off,
                                             uint32_t w_k_norm_off, uint32_t layer_il, uint32_t pos,
                                             uint32_t m_tokens);

/* Q1_0 decode matvec family (src/shaders/matvec_q1_0*.wgsl). `weights` is the
 * device weight buffer; w_d / w_qs are BYTE offsets of a Q1_0 tensor in it
 * (d: n x (k/128) f16, then qs: n x (k/128) x 16 bytes, 4-byte aligned,
 * src/model.rs:784-804). k is a multiple of 128, at most 16384; activation
 * offsets are f16-element offsets into `act` and must be multiples of 8.
 * y[out_off + r] = f16(sum_b d[r][b] * sum_e (+-x[e])) (or, with accumulate,
 * f16(f32(y) + that)). Arithmetic (environment BP_MATVEC_ARITH at
 * bp_model_create): "f16" = the reference's f16 block sums, bit for bit;
 * "mfma" = exact integer sums of x rounded to 15 bits of each block's max |x|,
 * f32 scaling; default "auto" = f16 below 32768 rows, mfma from there on. */
bp_status bp_dispatch_matvec_q1_0(bp_model* model, const void* weights, void* act, uint32_t k,
                                  uint32_t n, uint32_t w_d, uint32_t w_qs, uint32_t in_off,
                                  uint32_t out_off, uint32_t accumulate);
/* x = f16(silu(gate)) * up (silu in f32), gate / up at act[gate_off] / act[up_off]
 * (src/shaders/matvec_q1_0_silu.wgsl, src/forward.rs:243-282). */
bp_status bp_dispatch_matvec_q1_0_silu(bp_model* model, const void* weights, void* act, uint32_t k,
                                       uint32_t n, uint32_t w_d, uint32_t w_qs, uint32_t gate_off,
                                       uint32_t up_off, uint32_t out_off, uint32_t accumulate);
/* One Q1_0 row range of the fused normed matvec: (d_offset, qs_offset, n, output_offset)
 * (the ranges tuple of src/forward.rs:284-334). */
typedef struct {
    uint32_t d_offset, qs_offset, n, output_offset;
} bp_matvec_range;
/* rms_norm(x) * w_norm followed by 2 or 3 Q1_0 matvecs sharing x
 * (src/shaders/matvec_q1_0_fused_normed.wgsl, src/forward.rs:284-334); every
 * range's n is a multiple of 16, 1 to 3 ranges. */
bp_status bp_dispatch_matvec_q1_0_fused_normed(bp_model* model, const void* weights, void* act,
                                               const void* w_norms, uint32_t k, uint32_t in_off,
                                               uint32_t w_norm_off, uint32_t n_ranges,
                                               const bp_matvec_range* ranges);

/* Prefill projections (src/shaders/quantize_q8_0.wgsl, matmul_q1_0_q8_0.wgsl).
 * quantize: act[in_off + t*k ..] (f16, t < n_tokens) to Q8_0 in the byte
 * buffer acts_q8: f32 d of block (t, b) at d_off + 4*(t*k/32 + b), qs at
 * qs_off + t*k + 32*b; k a multiple of 32, offsets multiples of 4
 * (src/forward.rs:415-441 uses d_off = 0, qs_off = n_tokens*k/32*4). */
bp_status bp_dispatch_quantize_act(bp_model* model, const void* act, void* acts_q8, uint32_t k,
                                   uint32_t n_tokens, uint32_t in_off, uint32_t d_off, uint32_t qs_off);
/* y[out_off + t*n + r] = f16(sum over 128-blocks b, then 32-blocks s, of
 * (a_d * w_d) * f32(sumi)) in f32, bit for bit the reference's arithmetic
 * (sumi: exact sum of +-q); with accumulate f16(f32(y) + that). Weights as in
 * the matvecs (byte offsets w_d / w_qs), activations as written by
 * bp_dispatch_quantize_act (byte offsets a_d / a_qs); k a multiple of 128
 * (src/forward.rs:443-472). */
bp_status bp_dispatch_matmul_q1_0(bp_model* model, const void* weights, const void* acts_q8, void* act,
                                  uint32_t k, uint32_t n, uint32_t n_tokens, uint32_t w_d, uint32_t w_qs,
                                  uint32_t a_d, uint32_t a_qs, uint32_t out_off, uint32_t accumulate);

/* Top-k of n f16 logits at act[in_off ..] (in_off even), same values and
 * indices as src/shaders/topk_reduce.wgsl, ties included (the reference's
 * per-thread heaps and bitonic merge tree are kept step for step):
 * result[out_off + i] = f32 bits of the i-th largest value (descending),
 * result[out_off + kk + i] = its index, kk = min(k, 32); if fewer than kk
 * logits exceed -1e30 the rest are -1e30 / index 0. `result` is a u32 device
 * buffer. Replaces dispatch_topk_reduce (src/forward.rs:336-354). */
bp_status bp_dispatch_topk_reduce(bp_model* model, const void* act, void* result, uint32_t n, uint32_t k,
                                  uint32_t in_off, uint32_t out_off);
/* Waits for the model's stream, then copies the k values (f32) and k indices
 * written by bp_dispatch_topk_reduce (with the same k <= 32) to host memory.
 * Replaces wait_topk_readback (src/forward.rs:542-568). */
bp_status bp_topk_readback(bp_model* model, const void* result, uint32_t out_off, uint32_t k, float* values,
                           uint32_t* indices);

/* BONSAIKV v1 payload (src/kv_snapshot.rs:8-20): for kind in {K, V}, for each
 * layer: pos*(kv_dim/32)*4 bytes of d, then pos*kv_dim bytes of qs.
 * `payload` is host memory of exactly bp_kv_snapshot_payload_bytes(). Both
 * calls synchronize the model's stream. */
uint64_t bp_kv_snapshot_payload_bytes(uint32_t n_layer, uint32_t kv_dim, uint32_t pos);
bp_status bp_kv_snapshot_capture(bp_model* model, uint32_t pos, void* payload, uint64_t payload_bytes);
bp_status bp_kv_snapshot_apply(bp_model* model, uint32_t pos, const void* payload, uint64_t payload_bytes);

/* Device-loss latch (src/model.rs:1733-1741) and its test hook
 * (src/model.rs:1746-1751; host-side only: marks the model lost without
 * touching the GPU). */
bp_status bp_check_device(const bp_model* model);
bp_status bp_debug_lose_device(bp_model* model);

/* Allocation-free single-token decode. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same result
 * and kernels as bp_dispatch_attention_decode — rows [0, pos] of layer
 * `layer_il`, q already normalized at act[q_off], output at act[out_off] —
 * but it needs no bp_model: the caller passes its own kv_k / kv_v buffers (the
 * reference byte layout for cfg->n_layer x max_seq), and the split-K partials
 * live in a fixed 4.0625 MiB device array inside the library (one per GPU, kept
 * until the process ends), so the call never allocates. Launches on `stream`
 * on the current device. BP_ERR_CONFIG when n_head x the split count of
 * pos + 1 rows does not fit that array (it fits every context at n_head <= 64).
 * Calls that overlap on one GPU share the array and race: serialize them
 * (one stream, or events between streams). Nothing in the array needs to
 * start at zero: every partial is written before it is read. */
bp_status bp_attention_decode_noalloc(const bp_config* cfg, void* kv_k, void* kv_v, uint32_t max_seq, void* act,
                                      uint32_t q_off, uint32_t out_off, uint32_t layer_il, uint32_t pos,
                                      void* stream);

/* Message of the last failing call on this thread ("" if none). */
const char* bp_last_error(void);
const char* bp_status_name(bp_status status);

#ifdef __cplusplus
}
#endif
#endif /* BONSAI_POT_HIP_H */
