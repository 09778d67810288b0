/*
 * bp_oracle.h — CPU restatement of bonsai-pot's attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing on the product path may include, link or
 * call this code; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker.
 *
 * Every function restates one reference kernel or host helper (paths are
 * relative to the reference repository root). The Params structs have the
 * same field order and meaning as the reference's #[repr(C)] structs, so an
 * oracle call reads like the reference's dispatch.
 */
#ifndef BP_ORACLE_H
#define BP_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- f16 helpers (IEEE binary16, round-to-nearest-even) ------------------ */
uint16_t bpo_f32_to_f16(float v);
float bpo_f16_to_f32(uint16_t h);
void bpo_f32_to_f16_array(const float* in, uint16_t* out, size_t n);
void bpo_f16_to_f32_array(const uint16_t* in, float* out, size_t n);

/* ---- RoPE table: src/model.rs:1756-1769 (+ f16 downcast :1148-1149) ------- */
void bpo_build_rope_table(uint32_t head_dim, float rope_freq_base, uint32_t max_seq,
                          float* out_f32 /* [max_seq*head_dim] or NULL */,
                          uint16_t* out_f16 /* [max_seq*head_dim] or NULL */);

/* ---- KV layout: src/forward.rs:48-58 -------------------------------------- */
uint64_t bpo_kv_qs_byte_base(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq);
void bpo_kv_layer_offsets(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq, uint32_t il,
                          uint64_t* d_word, uint64_t* qs_byte);
uint64_t bpo_kv_buffer_bytes(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq);

/* ---- Snapshot payload layout: src/kv_snapshot.rs:145-180 ------------------ */
uint64_t bpo_snapshot_payload_bytes(uint32_t n_layer, uint32_t kv_dim, uint32_t pos);
uint64_t bpo_snapshot_payload_offset(uint32_t n_layer, uint32_t kv_dim, uint32_t pos,
                                     uint32_t kind, uint32_t il, uint32_t sect);
/* capture: kv buffers (host copies) -> payload; apply: payload -> kv buffers
 * (src/kv_snapshot.rs:204-372). */
void bpo_snapshot_capture(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq, uint32_t pos,
                          const uint8_t* kv_k, const uint8_t* kv_v, uint8_t* payload);
void bpo_snapshot_apply(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq, uint32_t pos,
                        const uint8_t* payload, uint8_t* kv_k, uint8_t* kv_v);

/* ---- Q8_0 block quantizer: src/shaders/kv_writeback_fused.wgsl:159-166,
 *      src/shaders/quantize_q8_0.wgsl:67-70 -------------------------------- */
void bpo_quantize_q8_0_block(const float x[32], float* d, int8_t q[32]);

/* ---- kv_writeback_fused: src/shaders/kv_writeback_fused.wgsl:53-201 ------- */
typedef struct {            /* KvWritebackFusedParams, src/model.rs:265-276 */
    uint32_t k_cur_off, v_cur_off, w_k_norm_off, rope_offset;
    uint32_t dst_d_word_offset, dst_qs_byte_offset, pos_base, kv_dim, nb_per_row;
    float eps;
} bpo_kv_writeback_params;

void bpo_kv_writeback_fused(const bpo_kv_writeback_params* p, const uint16_t* act,
                            const uint16_t* w_norms, const uint16_t* rope_cs,
                            uint8_t* kv_k, uint8_t* kv_v, uint32_t n_kv_head, uint32_t m_tokens);

/* ---- q_norm_rope_fused: src/shaders/q_norm_rope_fused.wgsl:38-96 ---------- */
typedef struct {            /* QNormRopeFusedParams, src/model.rs:255-262 */
    uint32_t q_off, w_q_norm_off, rope_offset, pos_base, q_dim;
    float eps;
} bpo_q_norm_rope_params;

void bpo_q_norm_rope_fused(const bpo_q_norm_rope_params* p, uint16_t* act,
                           const uint16_t* w_norms, const uint16_t* rope_cs,
                           uint32_t n_head, uint32_t m_tokens);

/* ---- decode attention: attention_split.wgsl:112-199 + attention_merge.wgsl:70-130
 *      host: src/forward.rs:820-857 ----------------------------------------- */
typedef struct {            /* AttnSplitParams, src/model.rs:213-226 (+ merge out_offset) */
    uint32_t head_dim, n_head, n_kv_head, pos, kv_stride, q_offset;
    uint32_t k_d_word_offset, k_qs_byte_offset, v_d_word_offset, v_qs_byte_offset;
    uint32_t n_chunks_active;
    float scale;
    uint32_t out_offset;    /* AttnMergeParams.out_offset, src/model.rs:229-234 */
} bpo_attn_split_params;

/* Writes f16 output into act at out_offset (if act_out != NULL) and the
 * pre-rounding f32 output [n_head*head_dim] into out_f32 (if not NULL). */
void bpo_attention_split_merge(const bpo_attn_split_params* p, const uint16_t* act,
                               const uint8_t* kv_k, const uint8_t* kv_v,
                               uint16_t* act_out, float* out_f32);

/* ---- batched attention: src/shaders/attention.wgsl:120-214, host forward.rs:501-532 */
typedef struct {            /* AttnParams, src/model.rs:195-210 */
    uint32_t head_dim, n_head, n_kv_head, pos, kv_stride, q_offset;
    uint32_t k_d_word_offset, k_qs_byte_offset, v_d_word_offset, v_qs_byte_offset;
    uint32_t out_offset;
    float scale;
    uint32_t m_tokens, is_prefill;
} bpo_attn_params;

/* Rows attended by token m: is_prefill ? pos + m + 1 : pos. With pos == 0 this
 * is exactly attention.wgsl:263 (cur_pos = m_tok + 1); pos > 0 is the chunked
 * prefill extension (same result as the reference's one-token-at-a-time route,
 * src/forward.rs:914-967). `tokens` selects which m to compute (NULL = all
 * m_tokens); out_f32 is [n_tokens][n_head*head_dim]. */
void bpo_attention(const bpo_attn_params* p, const uint16_t* act, const uint8_t* kv_k,
                   const uint8_t* kv_v, const uint32_t* tokens, uint32_t n_tokens,
                   uint16_t* act_out, float* out_f32);

/* ---- Q1_0 decode matvecs: src/shaders/matvec_q1_0.wgsl, matvec_q1_0_silu.wgsl,
 *      matvec_q1_0_fused_normed.wgsl; host src/forward.rs:212-334 ----------- */
/* f16 add / multiply of two f16 values, rounded once (RNE, subnormals kept). */
uint16_t bpo_f16_add(uint16_t a, uint16_t b);
uint16_t bpo_f16_mul(uint16_t a, uint16_t b);

typedef struct {            /* MatvecParams, src/model.rs:105-114 (no dispatch_x_dim) */
    uint32_t k, n, d_offset, qs_offset, input_offset, output_offset, accumulate;
} bpo_matvec_params;
typedef struct {            /* MatvecSiluParams, src/model.rs:117-127 */
    uint32_t k, n, d_offset, qs_offset, gate_offset, up_offset, output_offset, accumulate;
} bpo_matvec_silu_params;
typedef struct {            /* MatvecFusedNormedParams, src/model.rs:150-169 */
    uint32_t k, input_offset, w_norm_off;
    float eps;
    uint32_t n_ranges;
    uint32_t d_offset[3], qs_offset[3], n[3], output_offset[3];
} bpo_matvec_fused_normed_params;

/* In place on act (f16 bits); `weights` is the weight buffer (byte offsets). */
void bpo_matvec_q1_0(const bpo_matvec_params* p, const uint8_t* weights, uint16_t* act);
void bpo_matvec_q1_0_silu(const bpo_matvec_silu_params* p, const uint8_t* weights, uint16_t* act);
/* The sum of squares is taken in the GPU kernel's fixed order (256 threads,
 * 8-element groups, wave butterflies, 4 waves in order); the reference's
 * subgroupAdd order is backend-defined. */
void bpo_matvec_q1_0_fused_normed(const bpo_matvec_fused_normed_params* p, const uint8_t* weights,
                                  uint16_t* act, const uint16_t* w_norms);

/* ---- prefill projections: Q8_0 activations x Q1_0 weights ----------------- */
typedef struct {            /* QuantParams, src/model.rs:172-179 (no dispatch_x_dim) */
    uint32_t k, m, input_offset, d_offset, qs_offset;
} bpo_quant_params;
/* src/shaders/quantize_q8_0.wgsl: act[input_offset + m*k ..] (f16 elements) to
 * Q8_0 in `outbuf` (bytes): f32 d of block (row, b) at d_offset + 4*(row*k/32 + b),
 * qs at qs_offset + row*k + 32*b. */
void bpo_quantize_act_q8_0(const bpo_quant_params* p, const uint16_t* act, uint8_t* outbuf);

typedef struct {            /* MatmulParams, src/model.rs:182-192 */
    uint32_t k, n, m, w_d_offset, w_qs_offset, a_d_offset, a_qs_offset, out_offset, accumulate;
} bpo_matmul_params;
/* src/shaders/matmul_q1_0_q8_0.wgsl: y[out_offset + row*n + col] (f16) =
 * sum over 128-blocks b, then 32-blocks s of (a_d * w_d) * f32(sumi), in f32,
 * sumi the exact integer sum of +-q over the 32 elements. */
void bpo_matmul_q1_0_q8_0(const bpo_matmul_params* p, const uint8_t* weights, const uint8_t* acts,
                          uint16_t* y);

/* ---- top-k of the logits: src/shaders/topk_reduce.wgsl -------------------- */
typedef struct {            /* TopKParams, src/forward.rs:343-348 field order */
    uint32_t n, in_offset, out_offset, k;
} bpo_topk_params;
/* The reference's single-workgroup network, restated step for step so that
 * ties resolve to the same indices: 256 lanes, lane t owns the f16 pairs at
 * words t, t+256, ...; per lane a 32-entry min-heap (strict > insertion,
 * -1e30 / index 0 initial), heap sort to descending, then the pairwise
 * bitonic tree merge (lists p and p+s, s = 128 .. 1). Writes
 * result[out_offset + i] = f32 bits of value i and
 * result[out_offset + kk + i] = its index, kk = min(k, 32). */
void bpo_topk_reduce(const bpo_topk_params* p, const uint16_t* act, uint32_t* result);

/* ---- seeded synthetic inputs (splitmix64 + Box-Muller) -------------------- */
void bpo_fill_normal_f16(uint64_t seed, float mean, float stddev, uint16_t* out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
