/*
 * bp_oracle.c — CPU restatement of bonsai-pot's Q8_0-KV GQA attention path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the thing measured or shipped).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math:
 * every f32 operation below is a single IEEE-rounded op, in the order written).
 *
 * Reference files restated (paths relative to the reference repository root):
 *   src/shaders/kv_writeback_fused.wgsl   bpo_kv_writeback_fused
 *   src/shaders/q_norm_rope_fused.wgsl    bpo_q_norm_rope_fused
 *   src/shaders/attention_split.wgsl +
 *   src/shaders/attention_merge.wgsl      bpo_attention_split_merge
 *   src/shaders/attention.wgsl            bpo_attention
 *   src/model.rs:1756-1769                bpo_build_rope_table
 *   src/forward.rs:48-58                  bpo_kv_layer_offsets
 *   src/kv_snapshot.rs:145-372            bpo_snapshot_*
 *
 * Reduction order. The reference sums squares for RMSNorm with subgroupAdd,
 * whose association order the WGSL spec leaves to the implementation. This
 * oracle fixes one order, the one a 64-lane wavefront gets from an xor
 * butterfly when lane j holds elements j and j+64:
 *     a[j] = x[j]*x[j] + x[j+64]*x[j+64]           (j < 64)
 *     for off in 32,16,8,4,2,1:  a[j] = a[j] + a[j+off]   (j < off)
 *     total = a[0]
 * The HIP kernels use the same order, so K-cache bytes are bit-exact between
 * them. Against the reference's own (unknown) order a byte can differ by one
 * only where x*(1/d) lies within an ULP or so of a .5 tie.
 *
 * inverseSqrt (kv_writeback_fused.wgsl:86) is restated as the correctly
 * rounded 1/sqrt: one IEEE sqrt followed by one IEEE divide.
 */
#include "bp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------- */
/* f16 conversion (RNE, subnormals kept) — half::f16::from_f32 semantics,     */
/* used by the reference for the RoPE table (src/model.rs:1149) and by WGSL's  */
/* f16(...) casts.                                                             */
/* ------------------------------------------------------------------------- */
static uint32_t f32_bits(float v) { uint32_t x; memcpy(&x, &v, 4); return x; }
static float bits_f32(uint32_t x) { float v; memcpy(&v, &x, 4); return v; }

static uint32_t rne_shift(uint32_t m, uint32_t shift) {
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q += 1u;
    return q;
}

uint16_t bpo_f32_to_f16(float v) {
    uint32_t x = f32_bits(v);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x1ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 -> inf */
    uint32_t e = ax >> 23;
    if (e < 113u) {                                /* below 2^-14: f16 subnormal */
        if (e < 102u) return (uint16_t)sign;       /* < 2^-25 rounds to zero */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        return (uint16_t)(sign | rne_shift(m, 126u - e));
    }
    uint32_t q = ((e - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
}

float bpo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    if (e == 0x1fu) return bits_f32(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return bits_f32(sign);
        float f = (float)m * (1.0f / 16777216.0f);  /* m * 2^-24, exact */
        return sign ? -f : f;
    }
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

void bpo_f32_to_f16_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = bpo_f32_to_f16(in[i]);
}
void bpo_f16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = bpo_f16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------- */
/* RoPE table — src/model.rs:1756-1769: theta_j = base^(-2j/head_dim) in f64,  */
/* (cos, sin)(p*theta_j) in f64 -> f32, interleaved; then f16 (model.rs:1149). */
/* ------------------------------------------------------------------------- */
void bpo_build_rope_table(uint32_t head_dim, float rope_freq_base, uint32_t max_seq,
                          float* out_f32, uint16_t* out_f16) {
    uint32_t half = head_dim / 2;
    for (uint32_t p = 0; p < max_seq; p++) {
        for (uint32_t j = 0; j < half; j++) {
            double theta = pow((double)rope_freq_base, -2.0 * (double)j / (double)head_dim);
            double angle = (double)p * theta;
            float c = (float)cos(angle);
            float s = (float)sin(angle);
            size_t i = (size_t)p * head_dim + 2 * j;
            if (out_f32) { out_f32[i] = c; out_f32[i + 1] = s; }
            if (out_f16) { out_f16[i] = bpo_f32_to_f16(c); out_f16[i + 1] = bpo_f32_to_f16(s); }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* KV layout — src/forward.rs:48-58 (u64 here; the reference's u32 values are  */
/* the same numbers wherever they fit).                                        */
/* ------------------------------------------------------------------------- */
uint64_t bpo_kv_qs_byte_base(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq) {
    return (uint64_t)n_layer * max_seq * (kv_dim / 32) * 4;
}
void bpo_kv_layer_offsets(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq, uint32_t il,
                          uint64_t* d_word, uint64_t* qs_byte) {
    *d_word = (uint64_t)il * max_seq * (kv_dim / 32);
    *qs_byte = bpo_kv_qs_byte_base(n_layer, kv_dim, max_seq) + (uint64_t)il * max_seq * kv_dim;
}
uint64_t bpo_kv_buffer_bytes(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq) {
    /* src/model.rs:1184-1187: d_total + qs_total */
    return (uint64_t)n_layer * max_seq * (kv_dim / 32) * 4 + (uint64_t)n_layer * max_seq * kv_dim;
}

/* ------------------------------------------------------------------------- */
/* Snapshot payload — src/kv_snapshot.rs:145-180, capture :203-304, apply      */
/* :306-372.                                                                    */
/* ------------------------------------------------------------------------- */
uint64_t bpo_snapshot_payload_bytes(uint32_t n_layer, uint32_t kv_dim, uint32_t pos) {
    uint64_t d_layer = (uint64_t)pos * (kv_dim / 32) * 4;
    uint64_t qs_layer = (uint64_t)pos * kv_dim;
    return 2ull * n_layer * (d_layer + qs_layer);
}
uint64_t bpo_snapshot_payload_offset(uint32_t n_layer, uint32_t kv_dim, uint32_t pos,
                                     uint32_t kind, uint32_t il, uint32_t sect) {
    uint64_t d_layer = (uint64_t)pos * (kv_dim / 32) * 4;
    uint64_t qs_layer = (uint64_t)pos * kv_dim;
    uint64_t layer_bytes = d_layer + qs_layer;
    uint64_t base = (uint64_t)kind * n_layer * layer_bytes + (uint64_t)il * layer_bytes;
    return sect == 0 ? base : base + d_layer;
}
static void snapshot_copy(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq, uint32_t pos,
                          uint8_t* payload, uint8_t* kv_k, uint8_t* kv_v, int to_payload) {
    uint64_t d_size = (uint64_t)pos * (kv_dim / 32) * 4;
    uint64_t qs_size = (uint64_t)pos * kv_dim;
    for (uint32_t kind = 0; kind < 2; kind++) {
        uint8_t* buf = kind == 0 ? kv_k : kv_v;
        for (uint32_t il = 0; il < n_layer; il++) {
            uint64_t dw, qb;
            bpo_kv_layer_offsets(n_layer, kv_dim, max_seq, il, &dw, &qb);
            uint8_t* pd = payload + bpo_snapshot_payload_offset(n_layer, kv_dim, pos, kind, il, 0);
            uint8_t* pq = payload + bpo_snapshot_payload_offset(n_layer, kv_dim, pos, kind, il, 1);
            if (to_payload) {
                memcpy(pd, buf + dw * 4, d_size);
                memcpy(pq, buf + qb, qs_size);
            } else {
                memcpy(buf + dw * 4, pd, d_size);
                memcpy(buf + qb, pq, qs_size);
            }
        }
    }
}
void bpo_snapshot_capture(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq, uint32_t pos,
                          const uint8_t* kv_k, const uint8_t* kv_v, uint8_t* payload) {
    snapshot_copy(n_layer, kv_dim, max_seq, pos, payload, (uint8_t*)kv_k, (uint8_t*)kv_v, 1);
}
void bpo_snapshot_apply(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq, uint32_t pos,
                        const uint8_t* payload, uint8_t* kv_k, uint8_t* kv_v) {
    snapshot_copy(n_layer, kv_dim, max_seq, pos, (uint8_t*)payload, kv_k, kv_v, 0);
}

/* ------------------------------------------------------------------------- */
/* Q8_0 block quantizer — kv_writeback_fused.wgsl:118-166:                    */
/*   d = amax/127; inv_d = d > 0 ? 1/d : 0; q = clamp(rne(x*inv_d), -127, 127) */
/* ------------------------------------------------------------------------- */
void bpo_quantize_q8_0_block(const float x[32], float* d_out, int8_t q[32]) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) {
        float a = fabsf(x[i]);
        amax = a > amax ? a : amax;
    }
    float d = amax / 127.0f;
    float inv_d = d > 0.0f ? 1.0f / d : 0.0f;
    for (int i = 0; i < 32; i++) {
        /* WGSL round() is half-to-even; clamp with IEEE min/max (a NaN
         * operand yields the other operand, as v_max_f32/v_min_f32 do). */
        float r = fminf(fmaxf(rintf(x[i] * inv_d), -127.0f), 127.0f);
        q[i] = (int8_t)r;
    }
    *d_out = d;
}

/* Sum of squares of a 128-element head in the fixed butterfly order above. */
static float head_sumsq(const float x[128]) {
    float a[64];
    for (int j = 0; j < 64; j++) {
        float lo = x[j] * x[j];
        float hi = x[j + 64] * x[j + 64];
        a[j] = lo + hi;
    }
    for (int off = 32; off >= 1; off >>= 1)
        for (int j = 0; j < off; j++) a[j] = a[j] + a[j + off];
    return a[0];
}

/* RMSNorm * weight then NEOX RoPE on one 128-wide head (kv_writeback_fused.wgsl
 * :69-108, q_norm_rope_fused.wgsl:53-93). `x` is the raw head, `w` the f16
 * norm weights, `cs` the (cos, sin) row of the table for this position. */
static void norm_rope_head(const float x[128], const uint16_t* w, const uint16_t* cs,
                           float eps, float out[128]) {
    float total = head_sumsq(x);
    float inv_h = 1.0f / sqrtf(total / 128.0f + eps);
    float xn[128];
    for (int i = 0; i < 128; i++) {
        float t = x[i] * inv_h;
        xn[i] = t * bpo_f16_to_f32(w[i]);
    }
    for (int j = 0; j < 64; j++) {
        float c = bpo_f16_to_f32(cs[2 * j]);
        float s = bpo_f16_to_f32(cs[2 * j + 1]);
        float a = xn[j] * c, b = xn[j + 64] * s;
        out[j] = a - b;                          /* :102 */
        float e = xn[j] * s, f = xn[j + 64] * c;
        out[j + 64] = e + f;                     /* :107 */
    }
}

static void store_q8_head(uint8_t* buf, uint64_t d_word, uint64_t qs_byte, const float x[128]) {
    for (int b = 0; b < 4; b++) {
        float d;
        int8_t q[32];
        bpo_quantize_q8_0_block(x + 32 * b, &d, q);
        memcpy(buf + (d_word + (uint64_t)b) * 4, &d, 4);   /* FP32 d, little endian */
        memcpy(buf + qs_byte + 32u * (uint64_t)b, q, 32);
    }
}

void bpo_kv_writeback_fused(const bpo_kv_writeback_params* p, const uint16_t* act,
                            const uint16_t* w_norms, const uint16_t* rope_cs,
                            uint8_t* kv_k, uint8_t* kv_v, uint32_t n_kv_head, uint32_t m_tokens) {
    for (uint32_t tok = 0; tok < m_tokens; tok++) {
        for (uint32_t head = 0; head < n_kv_head; head++) {
            uint64_t tok_off = (uint64_t)tok * p->kv_dim + (uint64_t)head * 128;
            float k[128], v[128], kr[128];
            for (int i = 0; i < 128; i++) {
                k[i] = bpo_f16_to_f32(act[p->k_cur_off + tok_off + i]);
                v[i] = bpo_f16_to_f32(act[p->v_cur_off + tok_off + i]);
            }
            uint64_t pos_abs = (uint64_t)p->pos_base + tok;
            const uint16_t* cs = rope_cs + p->rope_offset + pos_abs * 128;
            norm_rope_head(k, w_norms + p->w_k_norm_off, cs, p->eps, kr);
            uint64_t d_word = p->dst_d_word_offset + pos_abs * p->nb_per_row + (uint64_t)head * 4;
            uint64_t qs_byte = p->dst_qs_byte_offset + pos_abs * p->kv_dim + (uint64_t)head * 128;
            store_q8_head(kv_k, d_word, qs_byte, kr);
            store_q8_head(kv_v, d_word, qs_byte, v);
        }
    }
}

void bpo_q_norm_rope_fused(const bpo_q_norm_rope_params* p, uint16_t* act,
                           const uint16_t* w_norms, const uint16_t* rope_cs,
                           uint32_t n_head, uint32_t m_tokens) {
    for (uint32_t tok = 0; tok < m_tokens; tok++) {
        for (uint32_t head = 0; head < n_head; head++) {
            uint64_t base = (uint64_t)p->q_off + (uint64_t)tok * p->q_dim + (uint64_t)head * 128;
            float q[128], qr[128];
            for (int i = 0; i < 128; i++) q[i] = bpo_f16_to_f32(act[base + i]);
            uint64_t pos_abs = (uint64_t)p->pos_base + tok;
            norm_rope_head(q, w_norms + p->w_q_norm_off, rope_cs + p->rope_offset + pos_abs * 128,
                           p->eps, qr);
            for (int i = 0; i < 128; i++) act[base + i] = bpo_f32_to_f16(qr[i]);   /* :95 */
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Attention                                                                    */
/* ------------------------------------------------------------------------- */
/* Dequantized cache row (attention_split.wgsl:183-205 load_k/load_v). */
static void load_row(const uint8_t* buf, uint32_t d_word_off, uint32_t qs_byte_off,
                     uint32_t kv_stride, uint32_t t, uint32_t e0, uint32_t hd, float* out) {
    for (uint32_t d = 0; d < hd; d++) {
        uint64_t elem = (uint64_t)t * kv_stride + e0 + d;
        float scale;
        memcpy(&scale, buf + ((uint64_t)d_word_off + (elem >> 5)) * 4, 4);
        int8_t q = (int8_t)buf[(uint64_t)qs_byte_off + elem];
        out[d] = scale * (float)q;
    }
}

/* One online-softmax update (attention_split.wgsl:252-265, attention.wgsl
 * :298-308). */
static void online_update(float score, const float* v, uint32_t hd,
                          float* m, float* l, float* o) {
    float m_new = *m > score ? *m : score;
    float corr = expf(*m - m_new);
    float w = expf(score - m_new);
    *l = *l * corr + w;
    *m = m_new;
    for (uint32_t d = 0; d < hd; d++) {
        float a = o[d] * corr;
        float b = w * v[d];
        o[d] = a + b;
    }
}

static float dot_f32(const float* a, const float* b, uint32_t n) {
    float s = 0.0f;
    for (uint32_t i = 0; i < n; i++) { float t = a[i] * b[i]; s = s + t; }
    return s;
}

#define ORACLE_CHUNK 16u   /* ATTN_CHUNK_SIZE, src/model.rs:511 */

void bpo_attention_split_merge(const bpo_attn_split_params* p, const uint16_t* act,
                               const uint8_t* kv_k, const uint8_t* kv_v,
                               uint16_t* act_out, float* out_f32) {
    uint32_t hd = p->head_dim, group = p->n_head / p->n_kv_head;
    uint32_t n = p->n_chunks_active;
    float* part = (float*)malloc((size_t)n * (hd + 2) * sizeof(float));
    float* q = (float*)malloc(hd * sizeof(float));
    float* k = (float*)malloc(hd * sizeof(float));
    float* v = (float*)malloc(hd * sizeof(float));
    for (uint32_t h = 0; h < p->n_head; h++) {
        uint32_t g = h / group;
        for (uint32_t d = 0; d < hd; d++) q[d] = bpo_f16_to_f32(act[p->q_offset + h * hd + d]);
        /* attention_split.wgsl:215-294: partial (o, m, l) per 16-row chunk */
        for (uint32_t c = 0; c < n; c++) {
            float* o = part + (size_t)c * (hd + 2);
            float m = -1e30f, l = 0.0f;
            for (uint32_t d = 0; d < hd; d++) o[d] = 0.0f;
            uint32_t start = c * ORACLE_CHUNK;
            uint32_t end = start + ORACLE_CHUNK < p->pos ? start + ORACLE_CHUNK : p->pos;
            for (uint32_t t = start; t < end; t++) {
                load_row(kv_k, p->k_d_word_offset, p->k_qs_byte_offset, p->kv_stride, t, g * hd, hd, k);
                float score = dot_f32(q, k, hd) * p->scale;
                load_row(kv_v, p->v_d_word_offset, p->v_qs_byte_offset, p->kv_stride, t, g * hd, hd, v);
                online_update(score, v, hd, &m, &l, o);
            }
            o[hd] = m;
            o[hd + 1] = l;
        }
        /* attention_merge.wgsl:85-129 */
        float mg = -1e30f;
        for (uint32_t c = 0; c < n; c++) {
            float mc = part[(size_t)c * (hd + 2) + hd];
            mg = mc > mg ? mc : mg;
        }
        float lg = 0.0f;
        for (uint32_t c = 0; c < n; c++) {
            float* pc = part + (size_t)c * (hd + 2);
            float w = expf(pc[hd] - mg);
            pc[hd] = w;                               /* weights_sh[c] */
            float t = pc[hd + 1] * w;
            lg = lg + t;
        }
        float inv_l = 1.0f / lg;
        for (uint32_t d = 0; d < hd; d++) {
            float acc = 0.0f;
            for (uint32_t c = 0; c < n; c++) {
                float* pc = part + (size_t)c * (hd + 2);
                float t = pc[d] * pc[hd];
                acc = acc + t;
            }
            float r = acc * inv_l;
            if (out_f32) out_f32[h * hd + d] = r;
            if (act_out) act_out[p->out_offset + h * hd + d] = bpo_f32_to_f16(r);
        }
    }
    free(part); free(q); free(k); free(v);
}

void bpo_attention(const bpo_attn_params* p, const uint16_t* act, const uint8_t* kv_k,
                   const uint8_t* kv_v, const uint32_t* tokens, uint32_t n_tokens,
                   uint16_t* act_out, float* out_f32) {
    uint32_t hd = p->head_dim, group = p->n_head / p->n_kv_head;
    uint32_t q_stride = p->n_head * hd;
    uint32_t count = tokens ? n_tokens : p->m_tokens;
    float* q = (float*)malloc(hd * sizeof(float));
    float* k = (float*)malloc(hd * sizeof(float));
    float* v = (float*)malloc(hd * sizeof(float));
    float* o = (float*)malloc(hd * sizeof(float));
    for (uint32_t i = 0; i < count; i++) {
        uint32_t m_tok = tokens ? tokens[i] : i;
        /* attention.wgsl:263 (pos_base extension: see header) */
        uint32_t cur_pos = p->is_prefill ? p->pos + m_tok + 1u : p->pos;
        for (uint32_t h = 0; h < p->n_head; h++) {
            uint32_t g = h / group;
            uint64_t q_base = (uint64_t)p->q_offset + (uint64_t)m_tok * q_stride + h * hd;
            for (uint32_t d = 0; d < hd; d++) { q[d] = bpo_f16_to_f32(act[q_base + d]); o[d] = 0.0f; }
            float m = -1e30f, l = 0.0f;
            for (uint32_t t = 0; t < cur_pos; t++) {
                load_row(kv_k, p->k_d_word_offset, p->k_qs_byte_offset, p->kv_stride, t, g * hd, hd, k);
                float score = dot_f32(q, k, hd) * p->scale;
                load_row(kv_v, p->v_d_word_offset, p->v_qs_byte_offset, p->kv_stride, t, g * hd, hd, v);
                online_update(score, v, hd, &m, &l, o);
            }
            float inv_l = 1.0f / l;                                  /* :339 */
            for (uint32_t d = 0; d < hd; d++) {
                float r = o[d] * inv_l;
                if (out_f32) out_f32[(size_t)i * q_stride + h * hd + d] = r;
                if (act_out)
                    act_out[(uint64_t)p->out_offset + (uint64_t)m_tok * q_stride + h * hd + d] =
                        bpo_f32_to_f16(r);
            }
        }
    }
    free(q); free(k); free(v); free(o);
}

/* ------------------------------------------------------------------------- */
/* Seeded inputs: splitmix64 -> uniform (53-bit) -> Box-Muller -> f16.        */
/* ------------------------------------------------------------------------- */
/* ---- Q1_0 decode matvecs ------------------------------------------------ */
/* f64 -> f16, round to nearest even, subnormals kept. A sum or product of two
 * f16 values is exact in f64, so f16 ops below round once, like the GPU's. */
static uint16_t f64_to_f16(double v) {
    const uint16_t sign = signbit(v) ? 0x8000u : 0u;
    const double a = fabs(v);
    if (isnan(v)) return sign | 0x7E00u;
    if (a >= 65520.0) return sign | 0x7C00u;      /* the 65504 / 65536 tie goes to inf */
    if (a < 6.103515625e-05) {                     /* below 2^-14: quantum 2^-24 */
        const double r = nearbyint(a * 16777216.0);
        return sign | (uint16_t)r;                 /* r = 1024 is the smallest normal */
    }
    int e;
    (void)frexp(a, &e);                            /* a = m * 2^e, m in [0.5, 1) */
    double r = nearbyint(ldexp(a, 11 - e));        /* [1024, 2048] */
    if (r == 2048.0) { r = 1024.0; e += 1; }
    const int E = e - 1 + 15;
    if (E >= 31) return sign | 0x7C00u;
    return (uint16_t)(sign | (uint16_t)(E << 10) | (uint16_t)((uint32_t)r - 1024u));
}
uint16_t bpo_f16_add(uint16_t a, uint16_t b) {
    return f64_to_f16((double)bpo_f16_to_f32(a) + (double)bpo_f16_to_f32(b));
}
uint16_t bpo_f16_mul(uint16_t a, uint16_t b) {
    return f64_to_f16((double)bpo_f16_to_f32(a) * (double)bpo_f16_to_f32(b));
}

/* matvec_q1_0.wgsl:88-111: one block, four f16 accumulators (component
 * e mod 4, elements in increasing order), then f32(((c0 + c1) + c2) + c3). */
static float q1_block_sum(const uint8_t* qs16, const uint16_t* x) {
    uint16_t c[4] = {0, 0, 0, 0};
    for (int w = 0; w < 4; w++) {
        uint32_t q;
        memcpy(&q, qs16 + 4 * w, 4);
        for (int i = 0; i < 8; i++)
            for (int cc = 0; cc < 4; cc++) {
                const int e = 32 * w + 4 * i + cc;
                const uint16_t xv = x[e];
                const uint16_t v = ((q >> (4 * i + cc)) & 1u) ? xv : (uint16_t)(xv ^ 0x8000u);
                c[cc] = bpo_f16_add(c[cc], v);
            }
    }
    return bpo_f16_to_f32(bpo_f16_add(bpo_f16_add(bpo_f16_add(c[0], c[1]), c[2]), c[3]));
}

/* One row: lane t = block mod 8 accumulates acc_t = acc_t + d * sum over its
 * blocks in order, then the xor 1, 2, 4 butterfly (matvec_q1_0.wgsl:112-123).
 * dscale multiplies each block's f32 scale first (the fused normed inv_rms). */
static float q1_row(const uint8_t* weights, uint32_t d_off, uint32_t qs_off, uint32_t k, uint32_t row,
                    const uint16_t* x, int use_dscale, float dscale) {
    const uint32_t nb = k / 128;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t b = 0; b < nb; b++) {
        uint16_t dh;
        memcpy(&dh, weights + d_off + ((uint64_t)row * nb + b) * 2, 2);
        float d = bpo_f16_to_f32(dh);
        if (use_dscale) d = d * dscale;
        const float sum = q1_block_sum(weights + qs_off + ((uint64_t)row * nb + b) * 16, x + 128 * b);
        const float term = d * sum;
        acc[b % 8] = acc[b % 8] + term;
    }
    float s1[8], s2[8];
    for (int t = 0; t < 8; t++) s1[t] = acc[t] + acc[t ^ 1];
    for (int t = 0; t < 8; t++) s2[t] = s1[t] + s1[t ^ 2];
    return s2[0] + s2[4];
}

static void q1_store(uint16_t* act, uint32_t yi, float acc, uint32_t accumulate) {
    act[yi] = accumulate ? bpo_f32_to_f16(bpo_f16_to_f32(act[yi]) + acc) : bpo_f32_to_f16(acc);
}

void bpo_matvec_q1_0(const bpo_matvec_params* p, const uint8_t* weights, uint16_t* act) {
    uint16_t* x = (uint16_t*)malloc((size_t)p->k * 2);
    memcpy(x, act + p->input_offset, (size_t)p->k * 2);
    for (uint32_t r = 0; r < p->n; r++)
        q1_store(act, p->output_offset + r, q1_row(weights, p->d_offset, p->qs_offset, p->k, r, x, 0, 1.0f),
                 p->accumulate);
    free(x);
}

void bpo_matvec_q1_0_silu(const bpo_matvec_silu_params* p, const uint8_t* weights, uint16_t* act) {
    uint16_t* x = (uint16_t*)malloc((size_t)p->k * 2);
    for (uint32_t i = 0; i < p->k; i++) {                /* matvec_q1_0_silu.wgsl:86-102 */
        const float g = bpo_f16_to_f32(act[p->gate_offset + i]);
        const float s = g / (1.0f + expf(-g));
        x[i] = bpo_f16_mul(bpo_f32_to_f16(s), act[p->up_offset + i]);
    }
    for (uint32_t r = 0; r < p->n; r++)
        q1_store(act, p->output_offset + r, q1_row(weights, p->d_offset, p->qs_offset, p->k, r, x, 0, 1.0f),
                 p->accumulate);
    free(x);
}

void bpo_matvec_q1_0_fused_normed(const bpo_matvec_fused_normed_params* p, const uint8_t* weights,
                                  uint16_t* act, const uint16_t* w_norms) {
    const uint32_t k = p->k;
    uint16_t* x = (uint16_t*)malloc((size_t)k * 2);
    float thr[256];
    for (int t = 0; t < 256; t++) thr[t] = 0.0f;
    for (uint32_t v = 0; v < k / 8; v++)                 /* thread v mod 256 */
        for (int i = 0; i < 8; i++) {
            const uint32_t e = 8 * v + i;
            const uint16_t xh = act[p->input_offset + e];
            const float xf = bpo_f16_to_f32(xh);
            thr[v % 256] = thr[v % 256] + xf * xf;
            x[e] = bpo_f16_mul(xh, w_norms[p->w_norm_off + e]);   /* :102-121 */
        }
    float total = 0.0f;
    for (int w = 0; w < 4; w++) {                        /* each wave: xor butterfly 32 .. 1 */
        float v[64], nv[64];
        for (int l = 0; l < 64; l++) v[l] = thr[64 * w + l];
        for (int off = 32; off >= 1; off >>= 1) {
            for (int l = 0; l < 64; l++) nv[l] = v[l] + v[l ^ off];
            memcpy(v, nv, sizeof v);
        }
        total = total + v[0];
    }
    const float inv_rms = 1.0f / sqrtf(total / (float)k + p->eps);
    for (uint32_t g = 0; g < p->n_ranges; g++)
        for (uint32_t r = 0; r < p->n[g]; r++)
            q1_store(act, p->output_offset[g] + r,
                     q1_row(weights, p->d_offset[g], p->qs_offset[g], k, r, x, 1, inv_rms), 0);
    free(x);
}

/* quantize_q8_0.wgsl:49-86: one workgroup per (row, 32-block); the quantizer
 * is the one of kv_writeback (amax / 127, RNE, clamp +-127). */
void bpo_quantize_act_q8_0(const bpo_quant_params* p, const uint16_t* act, uint8_t* outbuf) {
    const uint32_t nb = p->k / 32;
    for (uint32_t row = 0; row < p->m; row++)
        for (uint32_t b = 0; b < nb; b++) {
            float x[32], d;
            int8_t q[32];
            for (int i = 0; i < 32; i++)
                x[i] = bpo_f16_to_f32(act[p->input_offset + (uint64_t)row * p->k + 32u * b + (uint32_t)i]);
            bpo_quantize_q8_0_block(x, &d, q);
            memcpy(outbuf + p->d_offset + 4 * ((uint64_t)row * nb + b), &d, 4);
            memcpy(outbuf + p->qs_offset + (uint64_t)row * p->k + 32u * b, q, 32);
        }
}

/* matmul_q1_0_q8_0.wgsl:78-262: for each (row, col): acc over 128-blocks b
 * (outer) and their four 32-blocks s (inner) of (a_d * w_d) * f32(sumi), where
 * sumi = sum of (bit ? +q : -q) over the 32 elements (exact); then the f16
 * store, or f16(f32(y) + acc) with accumulate. */
void bpo_matmul_q1_0_q8_0(const bpo_matmul_params* p, const uint8_t* weights, const uint8_t* acts,
                          uint16_t* y) {
    const uint32_t nb1 = p->k / 128, nb8 = p->k / 32;
    for (uint32_t row = 0; row < p->m; row++)
        for (uint32_t col = 0; col < p->n; col++) {
            float acc = 0.0f;
            for (uint32_t b = 0; b < nb1; b++) {
                uint16_t wdh;
                memcpy(&wdh, weights + p->w_d_offset + 2 * ((uint64_t)col * nb1 + b), 2);
                const float wd = bpo_f16_to_f32(wdh);
                const uint8_t* bits = weights + p->w_qs_offset + ((uint64_t)col * nb1 + b) * 16;
                for (uint32_t s = 0; s < 4; s++) {
                    float ad;
                    memcpy(&ad, acts + p->a_d_offset + 4 * ((uint64_t)row * nb8 + 4 * b + s), 4);
                    const int8_t* q = (const int8_t*)(acts + p->a_qs_offset + (uint64_t)row * p->k + 128u * b + 32u * s);
                    int32_t sumi = 0;
                    for (uint32_t e = 0; e < 32; e++) {
                        const uint32_t bit = (bits[(32 * s + e) / 8] >> ((32 * s + e) % 8)) & 1u;
                        sumi += bit ? q[e] : -q[e];
                    }
                    const float scale = ad * wd;
                    const float v = scale * (float)sumi;
                    acc = acc + v;
                }
            }
            const uint64_t yi = p->out_offset + (uint64_t)row * p->n + col;
            y[yi] = p->accumulate ? bpo_f32_to_f16(bpo_f16_to_f32(y[yi]) + acc) : bpo_f32_to_f16(acc);
        }
}

static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
void bpo_fill_normal_f16(uint64_t seed, float mean, float stddev, uint16_t* out, size_t n) {
    uint64_t s = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = bpo_f32_to_f16((float)(mean + stddev * r * cos(two_pi * u2)));
        if (i + 1 < n) out[i + 1] = bpo_f32_to_f16((float)(mean + stddev * r * sin(two_pi * u2)));
    }
}

/* ---- src/shaders/topk_reduce.wgsl ----------------------------------------- */
#define TOPK_LANES 256u   /* WG, topk_reduce.wgsl:34 */
#define TOPK_KMAX 32u     /* K_MAX, topk_reduce.wgsl:35 */

/* Min-heap sift-down over heap[0 .. len) (topk_reduce.wgsl:42-55, :103-113):
 * the left child wins ties, a strictly smaller child is swapped up. */
static void topk_sift(float* v, uint32_t* ix, uint32_t len) {
    uint32_t i = 0;
    for (;;) {
        const uint32_t l = 2 * i + 1, r = l + 1;
        uint32_t m = i;
        if (l < len && v[l] < v[m]) m = l;
        if (r < len && v[r] < v[m]) m = r;
        if (m == i) return;
        const float tv = v[i]; v[i] = v[m]; v[m] = tv;
        const uint32_t ti = ix[i]; ix[i] = ix[m]; ix[m] = ti;
        i = m;
    }
}

void bpo_topk_reduce(const bpo_topk_params* p, const uint16_t* act, uint32_t* result) {
    float* v = malloc(sizeof(float) * TOPK_LANES * TOPK_KMAX);
    uint32_t* ix = malloc(sizeof(uint32_t) * TOPK_LANES * TOPK_KMAX);
    if (!v || !ix) abort();
    const uint32_t n_words = (p->n + 1) / 2;
    const uint16_t* x = act + (p->in_offset & ~1u);
    /* phase 1 (:65-96) and 2a (:98-115): independent per lane */
    for (uint32_t t = 0; t < TOPK_LANES; t++) {
        float* hv = v + t * TOPK_KMAX;
        uint32_t* hi = ix + t * TOPK_KMAX;
        for (uint32_t i = 0; i < TOPK_KMAX; i++) { hv[i] = -1e30f; hi[i] = 0; }
        for (uint32_t w = t; w < n_words; w += TOPK_LANES) {
            for (uint32_t h = 0; h < 2; h++) {
                const uint32_t e = 2 * w + h;
                if (h == 1 && e >= p->n) break;
                const float val = bpo_f16_to_f32(x[e]);
                if (val > hv[0]) { hv[0] = val; hi[0] = e; topk_sift(hv, hi, TOPK_KMAX); }
            }
        }
        for (uint32_t last = TOPK_KMAX - 1; last > 0; last--) {
            const float tv = hv[0]; hv[0] = hv[last]; hv[last] = tv;
            const uint32_t ti = hi[0]; hi[0] = hi[last]; hi[last] = ti;
            topk_sift(hv, hi, last);
        }
    }
    /* phase 2b (:117-184): list p absorbs list p + s, s = 128, 64, .., 1 */
    for (uint32_t s = TOPK_LANES / 2; s > 0; s /= 2) {
        for (uint32_t pr = 0; pr < s; pr++) {
            float* av = v + pr * TOPK_KMAX;
            uint32_t* ai = ix + pr * TOPK_KMAX;
            const float* bv = v + (pr + s) * TOPK_KMAX;
            const uint32_t* bi = ix + (pr + s) * TOPK_KMAX;
            for (uint32_t i = 0; i < TOPK_KMAX; i++) {   /* stage 0: a[i] vs b[31-i] */
                const uint32_t j = TOPK_KMAX - 1 - i;
                if (bv[j] > av[i]) { av[i] = bv[j]; ai[i] = bi[j]; }
            }
            for (uint32_t stride = TOPK_KMAX / 2; stride > 0; stride /= 2) {
                for (uint32_t lo = 0; lo < TOPK_KMAX; lo++) {
                    if (lo & stride) continue;
                    const uint32_t hi = lo | stride;
                    if (av[hi] > av[lo]) {
                        const float tv = av[lo]; av[lo] = av[hi]; av[hi] = tv;
                        const uint32_t ti = ai[lo]; ai[lo] = ai[hi]; ai[hi] = ti;
                    }
                }
            }
        }
    }
    const uint32_t kk = p->k < TOPK_KMAX ? p->k : TOPK_KMAX;
    for (uint32_t i = 0; i < kk; i++) {   /* :187-195 */
        uint32_t bits;
        memcpy(&bits, &v[i], 4);
        result[p->out_offset + i] = bits;
        result[p->out_offset + kk + i] = ix[i];
    }
    free(v);
    free(ix);
}
