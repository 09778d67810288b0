// Host layer of the MI355X attention path: the C ABI declared in
// include/bonsai_pot_hip.h.
//
// It restates, for HIP, the parts of the reference's host code (paths relative
// to the reference repository root) that the attention path needs:
//   - Model::load_with_options, KV / RoPE / partials part (src/model.rs:1148-1248):
//     bp_model_create, with the same config validation (head_dim == 128,
//     kv_dim % 32 == 0) and the same KV byte layout;
//   - the dispatch helpers of src/forward.rs (:48-58, :359-413, :501-532,
//     :820-857): bp_kv_layer_offsets and bp_dispatch_*;
//   - kv_snapshot::capture / apply (src/kv_snapshot.rs:203-372);
//   - the device-loss latch (src/model.rs:1087-1098, :1733-1751).
// Kernels never allocate: everything a launch touches is created here once.
#include "../../include/bonsai_pot_hip.h"
#ifdef BP_BENCH_HOOKS
#include "../../include/bonsai_pot_hip_bench.h"
#endif

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "bp_kernels.hpp"

struct bp_model {
    bp_config cfg;
    uint32_t kv_dim, q_dim, nb_per_row, max_seq;
    int device;
    int cu_count;
    hipStream_t stream;
    uint8_t* kv_k;
    uint8_t* kv_v;
    uint64_t kv_bytes;
    uint16_t* rope_cs;
    float* partials;
    uint64_t partials_floats;
    uint16_t* kv16;       // prefill: image of one layer's K and V (prefill_image_bytes)
    uint16_t* q_norm;     // decode-step scratch: normalized q, [n_head][128] f16
    uint32_t decode_min_split_rows;
    uint32_t decode_wide_min_rows;
    uint32_t prefill_hpw;   // 0 = by grid size; 2 = prefill32_kernel, 1 = the one-head 16x16 kernels
    uint32_t prefill_waves; // 0 = by grid size, else 4 or 8 waves per workgroup at 1 head per wave
    uint32_t prefill_ksplit;   // 0 = by grid size, else the key split count of the 4-wave layout
    int matvec_arith;        // Q1_0 matvecs: 0 auto, 1 (default) f16 sums in the reference's order, 2 i8 MFMA
    uint32_t matvec_stream_min_tiles;
    bool lost;
    std::string lost_message;
};

namespace {

thread_local std::string g_last_error;

bp_status fail(bp_status code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

// Errors after which the context (and every later call) is unusable.
bool is_device_fatal(hipError_t e) {
    switch (e) {
        case hipErrorIllegalAddress:
        case hipErrorLaunchFailure:
        case hipErrorLaunchTimeOut:
        case hipErrorECCNotCorrectable:
        case hipErrorAssert:
        case hipErrorContextIsDestroyed:
            return true;
        default:
            return false;
    }
}

bp_status hip_check(bp_model* m, hipError_t e, const char* what) {
    if (e == hipSuccess) return BP_OK;
    if (m && is_device_fatal(e)) {
        m->lost = true;
        m->lost_message = std::string(what) + ": " + hipGetErrorString(e);
        return fail(BP_ERR_DEVICE_LOST, "device lost: %s", m->lost_message.c_str());
    }
    return fail(BP_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bp_status check_model(const bp_model* m) {
    if (!m) return fail(BP_ERR_INVALID_ARG, "model is NULL");
    if (m->lost) return fail(BP_ERR_DEVICE_LOST, "device lost: %s", m->lost_message.c_str());
    return BP_OK;
}

// Makes the model's device current for this thread.
// Floats per prefill key-split partial (O, m, l, 2 pad), as attn_prefill.hip.
constexpr uint64_t kPrefillSplitStride = 132;

bp_status enter(bp_model* m) {
    bp_status st = check_model(m);
    if (st != BP_OK) return st;
    return hip_check(m, hipSetDevice(m->device), "hipSetDevice");
}

// half::f16::from_f32 semantics (round to nearest even), for the RoPE table.
uint16_t host_f32_to_f16(float v) {
    _Float16 h = static_cast<_Float16>(v);
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}

// src/model.rs:1756-1769: theta_j = base^(-2j/head_dim) in f64, (cos, sin)
// of p*theta_j in f64 -> f32, interleaved per j; uploaded as f16 (:1149).
std::vector<uint16_t> build_rope_table(const bp_config& cfg, uint32_t max_seq) {
    const uint32_t hd = cfg.head_dim, half = hd / 2;
    std::vector<uint16_t> out(static_cast<size_t>(max_seq) * hd);
    std::vector<double> theta(half);
    for (uint32_t j = 0; j < half; j++)
        theta[j] = std::pow(static_cast<double>(cfg.rope_freq_base),
                            -2.0 * static_cast<double>(j) / static_cast<double>(hd));
    for (uint32_t p = 0; p < max_seq; p++) {
        for (uint32_t j = 0; j < half; j++) {
            const double angle = static_cast<double>(p) * theta[j];
            out[static_cast<size_t>(p) * hd + 2 * j] = host_f32_to_f16(static_cast<float>(std::cos(angle)));
            out[static_cast<size_t>(p) * hd + 2 * j + 1] = host_f32_to_f16(static_cast<float>(std::sin(angle)));
        }
    }
    return out;
}

uint64_t kv_d_word(const bp_model* m, uint32_t il) {
    return static_cast<uint64_t>(il) * m->max_seq * m->nb_per_row;
}
uint64_t kv_qs_byte(const bp_model* m, uint32_t il) {
    return static_cast<uint64_t>(m->cfg.n_layer) * m->max_seq * m->nb_per_row * 4 +
           static_cast<uint64_t>(il) * m->max_seq * m->kv_dim;
}
bp::KvView kv_view(const bp_model* m, const uint8_t* buf, uint32_t il) {
    bp::KvView v;
    v.d = reinterpret_cast<const float*>(buf) + kv_d_word(m, il);
    v.qs = reinterpret_cast<const int8_t*>(buf + kv_qs_byte(m, il));
    return v;
}

constexpr uint32_t kMaxGridY = 65535;

bp::DecodeArgs decode_args(const bp_model* m, void* act, uint32_t q_off, uint32_t out_off, uint32_t il,
                           uint32_t n_rows) {
    bp::DecodeArgs a{};
    a.q = static_cast<const uint16_t*>(act) + q_off;
    a.out = static_cast<uint16_t*>(act) + out_off;
    a.k = kv_view(m, m->kv_k, il);
    a.v = kv_view(m, m->kv_v, il);
    a.partials = m->partials;
    a.kv_dim = m->kv_dim;
    a.n_rows = n_rows;
    bp::decode_plan(n_rows, m->cfg.n_kv_head, m->cu_count, m->decode_min_split_rows,
                    m->decode_wide_min_rows, &a.split_len, &a.n_splits, &a.heads_per_wg);
    a.scale = 1.0f / std::sqrt(static_cast<float>(m->cfg.head_dim));   // src/forward.rs:838
    return a;
}

}  // namespace

extern "C" {

const char* bp_last_error(void) { return g_last_error.c_str(); }

const char* bp_status_name(bp_status s) {
    switch (s) {
        case BP_OK: return "BP_OK";
        case BP_ERR_CONFIG: return "BP_ERR_CONFIG";
        case BP_ERR_CONTEXT_OVERFLOW: return "BP_ERR_CONTEXT_OVERFLOW";
        case BP_ERR_INVALID_ARG: return "BP_ERR_INVALID_ARG";
        case BP_ERR_HIP: return "BP_ERR_HIP";
        case BP_ERR_DEVICE_LOST: return "BP_ERR_DEVICE_LOST";
        case BP_ERR_OUT_OF_MEMORY: return "BP_ERR_OUT_OF_MEMORY";
        case BP_ERR_NO_DEVICE: return "BP_ERR_NO_DEVICE";
        default: return "BP_ERR_UNKNOWN";
    }
}

uint64_t bp_kv_buffer_bytes(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq) {
    const uint64_t rows = static_cast<uint64_t>(n_layer) * max_seq;
    return rows * (kv_dim / 32) * 4 + rows * kv_dim;
}

bp_status bp_kv_layer_offsets(uint32_t n_layer, uint32_t kv_dim, uint32_t max_seq, uint32_t il,
                              uint64_t* d_word_offset, uint64_t* qs_byte_offset) {
    if (il >= n_layer) return fail(BP_ERR_INVALID_ARG, "layer %u >= n_layer %u", il, n_layer);
    if (kv_dim % 32 != 0) return fail(BP_ERR_CONFIG, "kv_dim must be a multiple of 32 (Q8_0 block size)");
    const uint64_t nb = kv_dim / 32;
    if (d_word_offset) *d_word_offset = static_cast<uint64_t>(il) * max_seq * nb;
    if (qs_byte_offset)
        *qs_byte_offset = static_cast<uint64_t>(n_layer) * max_seq * nb * 4 +
                          static_cast<uint64_t>(il) * max_seq * kv_dim;
    return BP_OK;
}

uint64_t bp_kv_snapshot_payload_bytes(uint32_t n_layer, uint32_t kv_dim, uint32_t pos) {
    const uint64_t d_layer = static_cast<uint64_t>(pos) * (kv_dim / 32) * 4;
    const uint64_t qs_layer = static_cast<uint64_t>(pos) * kv_dim;
    return 2ull * n_layer * (d_layer + qs_layer);
}

bp_status bp_model_create(const bp_config* cfg, uint32_t max_seq, int device, bp_model** out) {
    if (!cfg || !out) return fail(BP_ERR_INVALID_ARG, "cfg/out is NULL");
    *out = nullptr;
    // Validation mirrors src/model.rs:1174-1183 plus the kernels' fixed shapes.
    if (cfg->head_dim != bp::kHeadDim)
        return fail(BP_ERR_CONFIG, "head_dim must be 128 (got %u)", cfg->head_dim);
    if (cfg->n_kv_head == 0 || cfg->n_head != cfg->n_kv_head * bp::kGroup)
        return fail(BP_ERR_CONFIG, "n_head must be 4 * n_kv_head (got %u, %u)", cfg->n_head,
                    cfg->n_kv_head);
    if (cfg->n_layer == 0) return fail(BP_ERR_CONFIG, "n_layer must be > 0");
    if (max_seq == 0) return fail(BP_ERR_CONFIG, "max_seq must be > 0");
    // The kernels address a row inside one layer's section with 32-bit
    // offsets (row * kv_dim + column): one layer's qs section must stay below
    // 4 GiB. The reference keeps whole-buffer offsets in u32
    // (src/forward.rs:48-58) and rejects caches above the adapter's buffer
    // limit with PotError::Config (src/model.rs:1189-1198).
    if (static_cast<uint64_t>(max_seq) * cfg->n_kv_head * cfg->head_dim > 0xFFFFFFFFull)
        return fail(BP_ERR_CONFIG, "max_seq %u x kv_dim %u exceeds the 32-bit per-layer cache offsets; reduce max_seq",
                    max_seq, cfg->n_kv_head * cfg->head_dim);
    if (!(cfg->rms_eps >= 0.0f) || !(cfg->rope_freq_base > 0.0f))
        return fail(BP_ERR_CONFIG, "rms_eps must be >= 0 and rope_freq_base > 0");
    int n_dev = 0;
    if (hipGetDeviceCount(&n_dev) != hipSuccess || n_dev == 0)
        return fail(BP_ERR_NO_DEVICE, "no HIP device available");
    if (device < 0 || device >= n_dev)
        return fail(BP_ERR_INVALID_ARG, "device %d out of range (%d devices)", device, n_dev);

    bp_model* m = new bp_model();
    m->cfg = *cfg;
    m->kv_dim = cfg->n_kv_head * cfg->head_dim;
    m->q_dim = cfg->n_head * cfg->head_dim;
    m->nb_per_row = m->kv_dim / 32;
    m->max_seq = max_seq;
    m->device = device;
    m->stream = nullptr;
    m->lost = false;
    bp_status st = BP_OK;
    auto bail = [&](bp_status s) { bp_model_destroy(m); return s; };
    if ((st = hip_check(nullptr, hipSetDevice(device), "hipSetDevice")) != BP_OK) return bail(st);
    hipDeviceProp_t prop;
    if ((st = hip_check(nullptr, hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties")) != BP_OK)
        return bail(st);
    m->cu_count = prop.multiProcessorCount;

    m->kv_bytes = bp_kv_buffer_bytes(cfg->n_layer, m->kv_dim, max_seq);
    // Split-K partials: n_head x (at most decode_max_splits()) x stride floats.
    m->decode_min_split_rows = bp::kDecodeMinSplitRows;
    if (const char* env = std::getenv("BP_DECODE_MIN_SPLIT_ROWS")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v >= 32 && v <= (1 << 20)) m->decode_min_split_rows = static_cast<uint32_t>(v);
    }
    // Rows from which the split pass reads 4 KV heads per workgroup.
    m->decode_wide_min_rows = bp::kDecodeWideMinRows;
    if (const char* env = std::getenv("BP_DECODE_WIDE_MIN_ROWS")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v >= 0) m->decode_wide_min_rows = static_cast<uint32_t>(v);
    }
    m->prefill_hpw = 0;
    if (const char* env = std::getenv("BP_PREFILL_HEADS_PER_WAVE")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v == 1 || v == 2) m->prefill_hpw = static_cast<uint32_t>(v);
    }
    m->prefill_ksplit = 0;
    if (const char* env = std::getenv("BP_PREFILL_KSPLIT")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v >= 1 && v <= 64) m->prefill_ksplit = static_cast<uint32_t>(v);
    }
    m->prefill_waves = 0;
    if (const char* env = std::getenv("BP_PREFILL_WG_WAVES")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v == 4 || v == 8) m->prefill_waves = static_cast<uint32_t>(v);
    }
    // Q1_0 matvec arithmetic. Default "f16": the reference's f16 block sums in
    // its order, bit for bit (VALU-bound), so logits and hence top-k token
    // choices equal the reference's. Opt-in "mfma": exact integer sums of x
    // rounded to 15 bits per block on the i8 matrix cores (closer to the
    // exact product, not the reference's bits); "auto": f16 below the
    // streaming size, MFMA from it on (the LM head, 2.2x faster there).
    m->matvec_arith = 1;
    if (const char* env = std::getenv("BP_MATVEC_ARITH")) {
        if (std::strcmp(env, "auto") == 0) m->matvec_arith = 0;
        else if (std::strcmp(env, "mfma") == 0) m->matvec_arith = 2;
    }
    // MFMA matvec: 16-row tiles from which each wave streams whole tiles.
    m->matvec_stream_min_tiles = 2048;
    if (const char* env = std::getenv("BP_MATVEC_STREAM_MIN_TILES")) {
        const long v = std::strtol(env, nullptr, 10);
        if (v >= 1) m->matvec_stream_min_tiles = static_cast<uint32_t>(v);
    }
    // Split-K partials, shared (stream order) by decode (n_head x its splits)
    // and the prefill key split (token x split products up to
    // kPrefillSplitTok, 132 floats each per query head).
    m->partials_floats = std::max<uint64_t>(
        static_cast<uint64_t>(cfg->n_head) * bp::decode_max_splits() * bp::decode_partial_stride(),
        static_cast<uint64_t>(cfg->n_head) * bp::kPrefillSplitTok * kPrefillSplitStride);
    const size_t rope_elems = static_cast<size_t>(max_seq) * cfg->head_dim;
    if (hipMalloc(&m->kv_k, m->kv_bytes) != hipSuccess || hipMalloc(&m->kv_v, m->kv_bytes) != hipSuccess ||
        hipMalloc(&m->rope_cs, rope_elems * 2) != hipSuccess ||
        hipMalloc(&m->partials, m->partials_floats * 4) != hipSuccess ||
        hipMalloc(&m->q_norm, static_cast<size_t>(cfg->n_head) * cfg->head_dim * 2) != hipSuccess ||
        hipMalloc(&m->kv16, bp::prefill_image_bytes(cfg->n_kv_head, max_seq)) != hipSuccess) {
        (void)hipGetLastError();
        return bail(fail(BP_ERR_OUT_OF_MEMORY, "hipMalloc failed for KV cache of %llu bytes x2",
                         static_cast<unsigned long long>(m->kv_bytes)));
    }
    std::vector<uint16_t> rope = build_rope_table(*cfg, max_seq);
    if ((st = hip_check(m, hipMemcpy(m->rope_cs, rope.data(), rope_elems * 2, hipMemcpyHostToDevice),
                        "upload rope table")) != BP_OK ||
        (st = hip_check(m, hipMemset(m->kv_k, 0, m->kv_bytes), "zero kv_k")) != BP_OK ||
        (st = hip_check(m, hipMemset(m->kv_v, 0, m->kv_bytes), "zero kv_v")) != BP_OK ||
        (st = hip_check(m, hipDeviceSynchronize(), "model create sync")) != BP_OK)
        return bail(st);
    *out = m;
    return BP_OK;
}

void bp_model_destroy(bp_model* m) {
    if (!m) return;
    if (hipSetDevice(m->device) == hipSuccess) {
        if (!m->lost && m->stream) (void)hipStreamSynchronize(m->stream);
        if (m->kv_k) (void)hipFree(m->kv_k);
        if (m->kv_v) (void)hipFree(m->kv_v);
        if (m->rope_cs) (void)hipFree(m->rope_cs);
        if (m->partials) (void)hipFree(m->partials);
        if (m->kv16) (void)hipFree(m->kv16);
        if (m->q_norm) (void)hipFree(m->q_norm);
    }
    (void)hipGetLastError();
    delete m;
}

bp_status bp_model_set_stream(bp_model* m, void* stream) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    // The model's scratch (split-K partials, normalized q, the prefill f16
    // image) is shared by every launch: work still queued on the old stream
    // must finish before the new stream may reuse it. The whole device is
    // drained, so that the old stream's handle is never used again (its owner
    // may already have destroyed it).
    if (m->stream != static_cast<hipStream_t>(stream) &&
        (st = hip_check(m, hipDeviceSynchronize(), "set_stream: drain the device")) != BP_OK)
        return st;
    m->stream = static_cast<hipStream_t>(stream);
    return BP_OK;
}

bp_status bp_model_synchronize(bp_model* m) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    return hip_check(m, hipStreamSynchronize(m->stream), "hipStreamSynchronize");
}

bp_status bp_model_kv_buffers(const bp_model* m, void** kv_k, void** kv_v, uint64_t* bytes_each) {
    if (!m) return fail(BP_ERR_INVALID_ARG, "model is NULL");
    if (kv_k) *kv_k = m->kv_k;
    if (kv_v) *kv_v = m->kv_v;
    if (bytes_each) *bytes_each = m->kv_bytes;
    return BP_OK;
}

bp_status bp_model_rope_table(const bp_model* m, const void** rope_cs) {
    if (!m || !rope_cs) return fail(BP_ERR_INVALID_ARG, "model/rope_cs is NULL");
    *rope_cs = m->rope_cs;
    return BP_OK;
}

uint32_t bp_model_max_seq(const bp_model* m) { return m ? m->max_seq : 0; }

bp_status bp_check_device(const bp_model* m) { return check_model(m); }

bp_status bp_debug_lose_device(bp_model* m) {
    if (!m) return fail(BP_ERR_INVALID_ARG, "model is NULL");
    m->lost = true;
    m->lost_message = "device destroyed by bp_debug_lose_device";
    return BP_OK;
}

bp_status bp_dispatch_q_norm_rope_fused(bp_model* m, void* act, const void* w_norms, uint32_t q_off,
                                        uint32_t w_q_norm_off, uint32_t pos_base, uint32_t m_tokens) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!act || !w_norms) return fail(BP_ERR_INVALID_ARG, "act/w_norms is NULL");
    if (m_tokens == 0) return BP_OK;
    if (static_cast<uint64_t>(pos_base) + m_tokens > m->max_seq)
        return fail(BP_ERR_CONTEXT_OVERFLOW, "context overflow: pos %u + tokens %u > max_seq %u",
                    pos_base, m_tokens, m->max_seq);
    for (uint32_t t0 = 0; t0 < m_tokens; t0 += kMaxGridY) {
        const uint32_t n = std::min(kMaxGridY, m_tokens - t0);
        bp::QNormRopeArgs a;
        a.act = static_cast<uint16_t*>(act);
        a.w_norms = static_cast<const uint16_t*>(w_norms);
        a.rope_cs = m->rope_cs;
        a.q_off = static_cast<uint64_t>(q_off) + static_cast<uint64_t>(t0) * m->q_dim;
        a.w_off = w_q_norm_off;
        a.pos_base = pos_base + t0;
        a.q_dim = m->q_dim;
        a.eps = m->cfg.rms_eps;
        if ((st = hip_check(m, bp::launch_q_norm_rope(a, m->cfg.n_head, n, m->stream), "q_norm_rope launch")) != BP_OK)
            return st;
    }
    return BP_OK;
}

bp_status bp_dispatch_kv_writeback_fused(bp_model* m, const void* act, const void* w_norms,
                                         uint32_t k_cur_off, uint32_t v_cur_off, uint32_t w_k_norm_off,
                                         uint32_t layer_il, uint32_t pos_base, uint32_t m_tokens) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!act || !w_norms) return fail(BP_ERR_INVALID_ARG, "act/w_norms is NULL");
    if (layer_il >= m->cfg.n_layer)
        return fail(BP_ERR_INVALID_ARG, "layer %u >= n_layer %u", layer_il, m->cfg.n_layer);
    if (m_tokens == 0) return BP_OK;
    if (static_cast<uint64_t>(pos_base) + m_tokens > m->max_seq)
        return fail(BP_ERR_CONTEXT_OVERFLOW, "context overflow: pos %u + tokens %u > max_seq %u",
                    pos_base, m_tokens, m->max_seq);
    const bp::KvView kv = kv_view(m, m->kv_k, layer_il), vv = kv_view(m, m->kv_v, layer_il);
    for (uint32_t t0 = 0; t0 < m_tokens; t0 += kMaxGridY) {
        const uint32_t n = std::min(kMaxGridY, m_tokens - t0);
        bp::KvWritebackArgs a;
        a.act = static_cast<const uint16_t*>(act);
        a.w_norms = static_cast<const uint16_t*>(w_norms);
        a.rope_cs = m->rope_cs;
        a.k_d = const_cast<float*>(kv.d);
        a.k_qs = const_cast<int8_t*>(kv.qs);
        a.v_d = const_cast<float*>(vv.d);
        a.v_qs = const_cast<int8_t*>(vv.qs);
        a.k_cur_off = static_cast<uint64_t>(k_cur_off) + static_cast<uint64_t>(t0) * m->kv_dim;
        a.v_cur_off = static_cast<uint64_t>(v_cur_off) + static_cast<uint64_t>(t0) * m->kv_dim;
        a.w_off = w_k_norm_off;
        a.pos_base = pos_base + t0;
        a.kv_dim = m->kv_dim;
        a.eps = m->cfg.rms_eps;
        if ((st = hip_check(m, bp::launch_kv_writeback(a, m->cfg.n_kv_head, n, m->stream),
                            "kv_writeback launch")) != BP_OK)
            return st;
    }
    return BP_OK;
}

bp_status bp_dispatch_attention_decode(bp_model* m, void* act, uint32_t q_off, uint32_t out_off,
                                       uint32_t layer_il, uint32_t pos) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!act) return fail(BP_ERR_INVALID_ARG, "act is NULL");
    if (layer_il >= m->cfg.n_layer)
        return fail(BP_ERR_INVALID_ARG, "layer %u >= n_layer %u", layer_il, m->cfg.n_layer);
    if (pos >= m->max_seq)
        return fail(BP_ERR_CONTEXT_OVERFLOW, "context overflow: pos %u + tokens 1 > max_seq %u", pos,
                    m->max_seq);
    if ((q_off & 7u) || (out_off & 3u))
        return fail(BP_ERR_INVALID_ARG, "q_off must be a multiple of 8 and out_off of 4 (aligned f16 rows)");
    bp::DecodeArgs a = decode_args(m, act, q_off, out_off, layer_il, pos + 1);   // src/forward.rs:822
    if (static_cast<uint64_t>(a.n_splits) * m->cfg.n_head * bp::decode_partial_stride() > m->partials_floats)
        return fail(BP_ERR_CONFIG, "internal: partials scratch too small for %u splits", a.n_splits);
    return hip_check(m, bp::launch_decode(a, m->cfg.n_kv_head, m->stream), "attention_decode launch");
}

bp_status bp_dispatch_attention_decode_step(bp_model* m, void* act, const void* w_norms, uint32_t q_off,
                                            uint32_t k_cur_off, uint32_t v_cur_off, uint32_t out_off,
                                            uint32_t w_q_norm_off, uint32_t w_k_norm_off, uint32_t layer_il,
                                            uint32_t pos) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!act || !w_norms) return fail(BP_ERR_INVALID_ARG, "act/w_norms is NULL");
    if (layer_il >= m->cfg.n_layer)
        return fail(BP_ERR_INVALID_ARG, "layer %u >= n_layer %u", layer_il, m->cfg.n_layer);
    if (pos >= m->max_seq)
        return fail(BP_ERR_CONTEXT_OVERFLOW, "context overflow: pos %u + tokens 1 > max_seq %u", pos,
                    m->max_seq);
    if ((out_off & 3u))
        return fail(BP_ERR_INVALID_ARG, "out_off must be a multiple of 4 (8-byte aligned f16 rows)");
    // The split pass streams rows [0, pos); row `pos` is written and added in-kernel.
    bp::DecodeArgs a = decode_args(m, act, q_off, out_off, layer_il, pos);
    a.q_act = static_cast<uint16_t*>(act) + q_off;
    a.q_norm = m->q_norm;
    a.k_cur = static_cast<const uint16_t*>(act) + k_cur_off;
    a.v_cur = static_cast<const uint16_t*>(act) + v_cur_off;
    a.w_norms = static_cast<const uint16_t*>(w_norms);
    a.rope_cs = m->rope_cs;
    a.w_q_off = w_q_norm_off;
    a.w_k_off = w_k_norm_off;
    a.pos = pos;
    a.eps = m->cfg.rms_eps;
    if (static_cast<uint64_t>(a.n_splits) * m->cfg.n_head * bp::decode_partial_stride() > m->partials_floats)
        return fail(BP_ERR_CONFIG, "internal: partials scratch too small for %u splits", a.n_splits);
    return hip_check(m, bp::launch_decode_step(a, m->cfg.n_kv_head, m->stream), "attention_decode_step launch");
}

// Validates a batched-attention call (src/forward.rs:501-532) and fills its
// PrefillArgs; BP_OK with a.m_tokens == 0 means there is nothing to do.
static bp_status prefill_args(bp_model* m, void* act, uint32_t q_off, uint32_t out_off, uint32_t layer_il,
                              uint32_t pos, uint32_t m_tokens, uint32_t is_prefill, bp::PrefillArgs& a) {
    a.m_tokens = 0;
    if (!act) return fail(BP_ERR_INVALID_ARG, "act is NULL");
    if (layer_il >= m->cfg.n_layer)
        return fail(BP_ERR_INVALID_ARG, "layer %u >= n_layer %u", layer_il, m->cfg.n_layer);
    if (m_tokens == 0) return BP_OK;
    if ((q_off | out_off) & 7u)
        return fail(BP_ERR_INVALID_ARG, "q_off/out_off must be multiples of 8 (16-byte aligned f16 rows)");
    const uint64_t rows = is_prefill ? static_cast<uint64_t>(pos) + m_tokens : pos;
    if (rows > m->max_seq)
        return fail(BP_ERR_CONTEXT_OVERFLOW, "context overflow: pos %u + tokens %u > max_seq %u", pos,
                    m_tokens, m->max_seq);
    if (rows == 0) return fail(BP_ERR_INVALID_ARG, "attention over zero cache rows (pos 0, is_prefill 0)");
    a.q = static_cast<const uint16_t*>(act) + q_off;
    a.out = static_cast<uint16_t*>(act) + out_off;
    a.k = kv_view(m, m->kv_k, layer_il);
    a.v = kv_view(m, m->kv_v, layer_il);
    a.kv_dim = m->kv_dim;
    a.q_stride = m->q_dim;
    a.m_tokens = m_tokens;
    a.pos = pos;
    a.causal = is_prefill ? 1u : 0u;
    a.n_tiles = (m_tokens + bp::kPrefillTileTok - 1) / bp::kPrefillTileTok;
    {
        // The one-head 16x16 kernels (two 8-wave workgroups per tile pair and KV
        // head, each wave 16 tokens of one query head) while that grid still
        // fits the compute units at one workgroup each, else prefill32_kernel
        // (one 8-wave workgroup per tile pair and KV head; at 64-1024 tokens it
        // measured 12.0-32.5 us against 10.1-27.3 us for the 16x16 kernels).
        // Then 4-wave workgroups (four per tile pair and KV head) while those
        // fit. BP_PREFILL_HEADS_PER_WAVE and BP_PREFILL_WG_WAVES force a layout.
        const uint32_t pairs = (a.n_tiles + 1) / 2;
        const uint32_t cus = static_cast<uint32_t>(m->cu_count > 0 ? m->cu_count : 256);
        a.heads_per_wave = m->prefill_hpw != 0 ? m->prefill_hpw : (2 * pairs * m->cfg.n_kv_head <= cus ? 1u : 2u);
        a.wg_waves = 8;
        if (a.heads_per_wave == 1)
            a.wg_waves = m->prefill_waves != 0 ? m->prefill_waves : (4 * pairs * m->cfg.n_kv_head <= cus ? 4u : 8u);
        // Key split for short chunks over long caches (where the 4-wave
        // layout would be chosen): split every tile pair's key range over
        // n_ksplit workgroups (fewer splits when the partials would not fit),
        // then merge. BP_PREFILL_KSPLIT forces a split count (within the
        // partials).
        a.n_ksplit = 1;
        a.split_chunks = 0;
        a.kpart = m->partials;
        a.direct = 0;
        const uint32_t chunks = static_cast<uint32_t>((rows + 63) / 64);   // the last tile's key chunks
        if (a.heads_per_wave == 1 && a.wg_waves == 4 && is_prefill &&
            (m->prefill_ksplit != 0 || chunks >= 4 * a.n_tiles)) {
            // prefill_split_kernel for few tiles over a long cache (at least 4
            // key chunks per tile): one 8-wave workgroup per (KV head, key
            // split, tile pair) reading the cache rows itself; enough splits
            // to give every CU a workgroup, at least 2 chunks each.
            const uint32_t wgs = pairs * m->cfg.n_kv_head;                   // workgroups per split
            uint32_t ns = m->prefill_ksplit != 0
                              ? m->prefill_ksplit
                              : std::min<uint32_t>(std::max<uint32_t>((cus + wgs - 1) / wgs, 1u), chunks / 2);
            const uint64_t cap = m->partials_floats / (static_cast<uint64_t>(m->cfg.n_head) * kPrefillSplitStride);
            ns = std::min<uint32_t>(ns, 64);   // prefill_merge_kernel: one split per lane
            while (ns > 1 && static_cast<uint64_t>(m_tokens) * ns > cap) --ns;
            if (ns > 1) {
                a.n_ksplit = ns;
                a.split_chunks = (chunks + ns - 1) / ns;
                a.direct = 1;
            }
        }
    }
    // The 32x32 kernel serves the two-heads layout; its V^T image keys are in
    // its own MFMA order.
    a.vt_order = a.heads_per_wave == 2 ? 1u : 0u;
    a.scale = 1.0f / std::sqrt(static_cast<float>(m->cfg.head_dim));   // src/forward.rs:524
    a.ws_chunks = (m->max_seq + 63) / 64;
    const uint64_t image_elems = static_cast<uint64_t>(m->cfg.n_kv_head) * a.ws_chunks * 64 * 128;
    a.k16 = m->kv16;
    a.vt16 = m->kv16 + image_elems;
    a.kl8 = reinterpret_cast<uint8_t*>(m->kv16 + 2 * image_elems);
    a.n_rows = static_cast<uint32_t>(rows);
    return BP_OK;
}

bp_status bp_dispatch_attention(bp_model* m, void* act, uint32_t q_off, uint32_t out_off, uint32_t layer_il,
                                uint32_t pos, uint32_t m_tokens, uint32_t is_prefill) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    bp::PrefillArgs a;
    if ((st = prefill_args(m, act, q_off, out_off, layer_il, pos, m_tokens, is_prefill, a)) != BP_OK ||
        a.m_tokens == 0)
        return st;
    if (!bp::prefill_grid_fits(a, false))
        return fail(BP_ERR_CONFIG, "attention: %u rows / %u tokens exceed the kernels' grid limits", a.n_rows, m_tokens);
    return hip_check(m, bp::launch_prefill(a, m->cfg.n_kv_head, m->stream), "attention launch");
}

// The fused prefill step, or (prep_only, a measurement aid) its first launch.
static bp_status prefill_step(bp_model* m, void* act, const void* w_norms, uint32_t q_off, uint32_t k_cur_off,
                              uint32_t v_cur_off, uint32_t out_off, uint32_t w_q_norm_off, uint32_t w_k_norm_off,
                              uint32_t layer_il, uint32_t pos, uint32_t m_tokens, bool prep_only) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!act || !w_norms) return fail(BP_ERR_INVALID_ARG, "act/w_norms is NULL");
    bp::PrefillArgs a;
    if ((st = prefill_args(m, act, q_off, out_off, layer_il, pos, m_tokens, 1, a)) != BP_OK || a.m_tokens == 0)
        return st;
    // The preparation pass moves 16-byte vectors only; other offsets take the
    // three separate dispatches (same results).
    const bool vec = ((k_cur_off | v_cur_off | w_q_norm_off | w_k_norm_off) & 7u) == 0 &&
                     (reinterpret_cast<uintptr_t>(act) & 15u) == 0 && (reinterpret_cast<uintptr_t>(w_norms) & 15u) == 0;
    if (!vec && prep_only)
        return fail(BP_ERR_INVALID_ARG, "prefill_prep: offsets must be multiples of 8, act/w_norms 16-byte aligned");
    if (!vec) {
        if ((st = bp_dispatch_q_norm_rope_fused(m, act, w_norms, q_off, w_q_norm_off, pos, m_tokens)) != BP_OK ||
            (st = bp_dispatch_kv_writeback_fused(m, act, w_norms, k_cur_off, v_cur_off, w_k_norm_off, layer_il, pos,
                                                 m_tokens)) != BP_OK)
            return st;
        return bp_dispatch_attention(m, act, q_off, out_off, layer_il, pos, m_tokens, 1);
    }
    if (!bp::prefill_grid_fits(a, true))
        return fail(BP_ERR_CONFIG, "attention_prefill_step: %u rows / %u tokens exceed the kernels' grid limits",
                    a.n_rows, m_tokens);
    bp::PrefillStepArgs w;
    w.q_act = static_cast<uint16_t*>(act) + q_off;
    w.k_cur = static_cast<const uint16_t*>(act) + k_cur_off;
    w.v_cur = static_cast<const uint16_t*>(act) + v_cur_off;
    w.w_norms = static_cast<const uint16_t*>(w_norms);
    w.rope_cs = m->rope_cs;
    w.w_q_off = w_q_norm_off;
    w.w_k_off = w_k_norm_off;
    w.k_d = const_cast<float*>(a.k.d);
    w.k_qs = const_cast<int8_t*>(a.k.qs);
    w.v_d = const_cast<float*>(a.v.d);
    w.v_qs = const_cast<int8_t*>(a.v.qs);
    w.eps = m->cfg.rms_eps;
    return hip_check(m, bp::launch_prefill_step(a, w, m->cfg.n_kv_head, m->stream, prep_only),
                     "attention_prefill_step launch");
}

bp_status bp_dispatch_attention_prefill_step(bp_model* m, void* act, const void* w_norms, uint32_t q_off,
                                             uint32_t k_cur_off, uint32_t v_cur_off, uint32_t out_off,
                                             uint32_t w_q_norm_off, uint32_t w_k_norm_off, uint32_t layer_il,
                                             uint32_t pos, uint32_t m_tokens) {
    return prefill_step(m, act, w_norms, q_off, k_cur_off, v_cur_off, out_off, w_q_norm_off, w_k_norm_off, layer_il,
                        pos, m_tokens, false);
}

#ifdef BP_BENCH_HOOKS
bp_status bp_debug_prefill_prep(bp_model* m, void* act, const void* w_norms, uint32_t q_off, uint32_t k_cur_off,
                                uint32_t v_cur_off, uint32_t out_off, uint32_t w_q_norm_off, uint32_t w_k_norm_off,
                                uint32_t layer_il, uint32_t pos, uint32_t m_tokens) {
    return prefill_step(m, act, w_norms, q_off, k_cur_off, v_cur_off, out_off, w_q_norm_off, w_k_norm_off, layer_il,
                        pos, m_tokens, true);
}
#endif

static bp_status matvec_common(bp_model* m, const void* weights, void* act, uint32_t k,
                               bp::MatvecArgs& a) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!weights || !act) return fail(BP_ERR_INVALID_ARG, "weights/act is NULL");
    if (k == 0 || k % 128 != 0 || k > bp::matvec_max_k())
        return fail(BP_ERR_INVALID_ARG, "matvec k = %u must be a positive multiple of 128 <= %u", k,
                    bp::matvec_max_k());
    a.weights = static_cast<const uint8_t*>(weights);
    a.act = static_cast<uint16_t*>(act);
    a.k = k;
    a.eps = m->cfg.rms_eps;
    a.stream_min_tiles = m->matvec_stream_min_tiles;
    a.cu_count = static_cast<uint32_t>(m->cu_count);
    return BP_OK;
}

static bp_status matvec_check_tensor(uint32_t w_d, uint32_t w_qs) {
    if ((w_d & 1u) || (w_qs & 3u))
        return fail(BP_ERR_INVALID_ARG, "Q1_0 offsets: d must be 2-byte, qs 4-byte aligned (%u, %u)", w_d, w_qs);
    return BP_OK;
}

static hipError_t launch_matvec(const bp_model* m, const bp::MatvecArgs& a, int mode) {
    const bool mfma = m->matvec_arith == 2 ||
                      (m->matvec_arith == 0 && (a.n_total + 15) / 16 >= m->matvec_stream_min_tiles);
    return mfma ? bp::launch_matvec_q1_0_mfma(a, mode, m->stream) : bp::launch_matvec_q1_0(a, mode, m->stream);
}

bp_status bp_dispatch_matvec_q1_0(bp_model* m, const void* weights, void* act, uint32_t k, uint32_t n,
                                  uint32_t w_d, uint32_t w_qs, uint32_t in_off, uint32_t out_off,
                                  uint32_t accumulate) {
    bp::MatvecArgs a{};
    bp_status st = matvec_common(m, weights, act, k, a);
    if (st != BP_OK) return st;
    if (n == 0) return BP_OK;
    if ((st = matvec_check_tensor(w_d, w_qs)) != BP_OK) return st;
    if (in_off & 7u) return fail(BP_ERR_INVALID_ARG, "matvec in_off %u must be a multiple of 8", in_off);
    a.n_total = n;
    a.input_offset = in_off;
    a.accumulate = accumulate ? 1u : 0u;
    a.range[0] = {w_d, w_qs, n, out_off};
    return hip_check(m, launch_matvec(m, a, 0), "matvec_q1_0 launch");
}

bp_status bp_dispatch_matvec_q1_0_silu(bp_model* m, const void* weights, void* act, uint32_t k, uint32_t n,
                                       uint32_t w_d, uint32_t w_qs, uint32_t gate_off, uint32_t up_off,
                                       uint32_t out_off, uint32_t accumulate) {
    bp::MatvecArgs a{};
    bp_status st = matvec_common(m, weights, act, k, a);
    if (st != BP_OK) return st;
    if (n == 0) return BP_OK;
    if ((st = matvec_check_tensor(w_d, w_qs)) != BP_OK) return st;
    if ((gate_off | up_off) & 7u)
        return fail(BP_ERR_INVALID_ARG, "matvec gate/up offsets (%u, %u) must be multiples of 8", gate_off, up_off);
    a.n_total = n;
    a.gate_offset = gate_off;
    a.up_offset = up_off;
    a.accumulate = accumulate ? 1u : 0u;
    a.range[0] = {w_d, w_qs, n, out_off};
    return hip_check(m, launch_matvec(m, a, 1), "matvec_q1_0_silu launch");
}

bp_status bp_dispatch_matvec_q1_0_fused_normed(bp_model* m, const void* weights, void* act, const void* w_norms,
                                               uint32_t k, uint32_t in_off, uint32_t w_norm_off,
                                               uint32_t n_ranges, const bp_matvec_range* ranges) {
    bp::MatvecArgs a{};
    bp_status st = matvec_common(m, weights, act, k, a);
    if (st != BP_OK) return st;
    if (!w_norms || !ranges) return fail(BP_ERR_INVALID_ARG, "w_norms/ranges is NULL");
    if (n_ranges < 1 || n_ranges > 3) return fail(BP_ERR_INVALID_ARG, "n_ranges %u not in 1..3", n_ranges);
    if ((in_off | w_norm_off) & 7u)
        return fail(BP_ERR_INVALID_ARG, "matvec in_off / w_norm_off (%u, %u) must be multiples of 8", in_off, w_norm_off);
    uint64_t total = 0;
    for (uint32_t i = 0; i < n_ranges; i++) {
        if (ranges[i].n % 16 != 0)
            return fail(BP_ERR_INVALID_ARG, "fused normed matvec range %u: n = %u not a multiple of 16", i, ranges[i].n);
        if ((st = matvec_check_tensor(ranges[i].d_offset, ranges[i].qs_offset)) != BP_OK) return st;
        a.range[i] = {ranges[i].d_offset, ranges[i].qs_offset, ranges[i].n, ranges[i].output_offset};
        total += ranges[i].n;
    }
    if (total == 0) return BP_OK;
    a.w_norms = static_cast<const uint16_t*>(w_norms);
    a.n_total = static_cast<uint32_t>(total);
    a.input_offset = in_off;
    a.w_norm_off = w_norm_off;
    return hip_check(m, launch_matvec(m, a, 2), "matvec_q1_0_fused_normed launch");
}

bp_status bp_dispatch_quantize_act(bp_model* m, const void* act, void* acts_q8, uint32_t k, uint32_t n_tokens,
                                   uint32_t in_off, uint32_t d_off, uint32_t qs_off) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!act || !acts_q8) return fail(BP_ERR_INVALID_ARG, "act/acts_q8 is NULL");
    if (k == 0 || k % 32 != 0) return fail(BP_ERR_INVALID_ARG, "quantize k = %u must be a positive multiple of 32", k);
    if ((d_off | qs_off) & 3u)
        return fail(BP_ERR_INVALID_ARG, "quantize d/qs offsets (%u, %u) must be multiples of 4", d_off, qs_off);
    if (n_tokens == 0) return BP_OK;
    if (static_cast<uint64_t>(n_tokens) * (k / 32) > 0xFFFFFFFFull / 8)
        return fail(BP_ERR_INVALID_ARG, "quantize: %u x %u too large", n_tokens, k);
    bp::QuantArgs a{};
    a.act = static_cast<const uint16_t*>(act);
    a.out = static_cast<uint8_t*>(acts_q8);
    a.k = k;
    a.m = n_tokens;
    a.input_offset = in_off;
    a.d_offset = d_off;
    a.qs_offset = qs_off;
    return hip_check(m, bp::launch_quantize_act_q8_0(a, m->stream), "quantize_act_q8_0 launch");
}

bp_status bp_dispatch_matmul_q1_0(bp_model* m, const void* weights, const void* acts_q8, void* act, uint32_t k,
                                  uint32_t n, uint32_t n_tokens, uint32_t w_d, uint32_t w_qs, uint32_t a_d,
                                  uint32_t a_qs, uint32_t out_off, uint32_t accumulate) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!weights || !acts_q8 || !act) return fail(BP_ERR_INVALID_ARG, "weights/acts_q8/act is NULL");
    if (k == 0 || k % 128 != 0) return fail(BP_ERR_INVALID_ARG, "matmul k = %u must be a positive multiple of 128", k);
    if ((w_d & 1u) || (w_qs & 3u) || (a_d & 3u) || (a_qs & 3u))
        return fail(BP_ERR_INVALID_ARG, "matmul offsets: w_d 2-byte, w_qs / a_d / a_qs 4-byte aligned (%u, %u, %u, %u)",
                    w_d, w_qs, a_d, a_qs);
    if (n == 0 || n_tokens == 0) return BP_OK;
    if ((n_tokens + 31) / 32 > 65535) return fail(BP_ERR_INVALID_ARG, "matmul: %u tokens too many", n_tokens);
    bp::MatmulArgs a{};
    a.weights = static_cast<const uint8_t*>(weights);
    a.acts = static_cast<const uint8_t*>(acts_q8);
    a.y = static_cast<uint16_t*>(act);
    a.k = k;
    a.n = n;
    a.m = n_tokens;
    a.w_d_offset = w_d;
    a.w_qs_offset = w_qs;
    a.a_d_offset = a_d;
    a.a_qs_offset = a_qs;
    a.out_offset = out_off;
    a.accumulate = accumulate ? 1u : 0u;
    return hip_check(m, bp::launch_matmul_q1_0_q8_0(a, m->stream), "matmul_q1_0_q8_0 launch");
}

bp_status bp_dispatch_topk_reduce(bp_model* m, const void* act, void* result, uint32_t n, uint32_t k,
                                  uint32_t in_off, uint32_t out_off) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!act || !result) return fail(BP_ERR_INVALID_ARG, "act/result is NULL");
    if (in_off & 1u) return fail(BP_ERR_INVALID_ARG, "topk in_offset %u must be even (f16 pairs)", in_off);
    if (static_cast<uint64_t>(n) + in_off > 0xFFFFFFFFull)
        return fail(BP_ERR_INVALID_ARG, "topk: n %u + in_offset %u overflows u32", n, in_off);
    bp::TopKArgs a{};
    a.logits = static_cast<const uint16_t*>(act);
    a.result = static_cast<uint32_t*>(result);
    a.n = n;
    a.in_offset = in_off;
    a.out_offset = out_off;
    a.k = k;
    return hip_check(m, bp::launch_topk_reduce(a, m->stream), "topk_reduce launch");
}

bp_status bp_topk_readback(bp_model* m, const void* result, uint32_t out_off, uint32_t k, float* values,
                           uint32_t* indices) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (!result || (k && (!values || !indices))) return fail(BP_ERR_INVALID_ARG, "result/values/indices is NULL");
    if (k > 32) return fail(BP_ERR_INVALID_ARG, "topk readback k = %u exceeds 32", k);
    if ((st = hip_check(m, hipStreamSynchronize(m->stream), "topk readback sync")) != BP_OK) return st;
    if (k == 0) return BP_OK;
    const uint32_t* src = static_cast<const uint32_t*>(result) + out_off;
    if ((st = hip_check(m, hipMemcpy(values, src, 4ull * k, hipMemcpyDeviceToHost), "topk readback values")) != BP_OK)
        return st;
    return hip_check(m, hipMemcpy(indices, src + k, 4ull * k, hipMemcpyDeviceToHost), "topk readback indices");
}

static bp_status snapshot_copy(bp_model* m, uint32_t pos, uint8_t* payload, uint64_t payload_bytes,
                               bool to_host) {
    bp_status st = enter(m);
    if (st != BP_OK) return st;
    if (pos > m->max_seq)
        return fail(BP_ERR_CONTEXT_OVERFLOW, "context overflow: pos 0 + tokens %u > max_seq %u", pos,
                    m->max_seq);
    const uint64_t need = bp_kv_snapshot_payload_bytes(m->cfg.n_layer, m->kv_dim, pos);
    if (payload_bytes != need)
        return fail(BP_ERR_CONFIG, "KvSnapshot payload length %llu does not match %llu",
                    static_cast<unsigned long long>(payload_bytes), static_cast<unsigned long long>(need));
    if (pos == 0) return BP_OK;   // src/kv_snapshot.rs:212-221, :310-312
    if (!payload) return fail(BP_ERR_INVALID_ARG, "payload is NULL");
    const uint64_t d_size = static_cast<uint64_t>(pos) * m->nb_per_row * 4;
    const uint64_t qs_size = static_cast<uint64_t>(pos) * m->kv_dim;
    const uint64_t layer_bytes = d_size + qs_size;
    const uint32_t nl = m->cfg.n_layer;
    for (uint32_t kind = 0; kind < 2; kind++) {
        uint8_t* buf = kind == 0 ? m->kv_k : m->kv_v;
        for (uint32_t il = 0; il < nl; il++) {
            // payload_offset, src/kv_snapshot.rs:158-169
            uint8_t* pd = payload + static_cast<uint64_t>(kind) * nl * layer_bytes + il * layer_bytes;
            uint8_t* pq = pd + d_size;
            uint8_t* bd = buf + kv_d_word(m, il) * 4;
            uint8_t* bq = buf + kv_qs_byte(m, il);
            hipError_t e1 = to_host ? hipMemcpyAsync(pd, bd, d_size, hipMemcpyDeviceToHost, m->stream)
                                    : hipMemcpyAsync(bd, pd, d_size, hipMemcpyHostToDevice, m->stream);
            if ((st = hip_check(m, e1, "snapshot copy (d)")) != BP_OK) return st;
            hipError_t e2 = to_host ? hipMemcpyAsync(pq, bq, qs_size, hipMemcpyDeviceToHost, m->stream)
                                    : hipMemcpyAsync(bq, pq, qs_size, hipMemcpyHostToDevice, m->stream);
            if ((st = hip_check(m, e2, "snapshot copy (qs)")) != BP_OK) return st;
        }
    }
    return hip_check(m, hipStreamSynchronize(m->stream), "snapshot sync");
}

// ---- allocation-free decode ---------------------------------------------------
// Split-K partials for bp_attention_decode_noalloc live in this file-scope
// device array instead of memory the library allocates: 64 query heads x 128
// splits (the most decode_plan makes) x 130 floats per partial = 4.0625 MiB, so
// every context fits at n_head <= 64. Every GPU holds its own copy until the
// process ends.
// In host code `scratch` is only a stand-in for the symbol: kernels get the
// device address from hipGetSymbolAddress, looked up once per device.
constexpr uint64_t kNoAllocScratchFloats = 64ull * 128 * 130;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

constexpr int kNoAllocMaxDevices = 64;
struct NoAllocDevice {
    std::once_flag once;
    hipError_t status = hipSuccess;
    float* ptr = nullptr;   // device address of `scratch` on this device
    int cu_count = 0;
};
static NoAllocDevice g_noalloc[kNoAllocMaxDevices];

// Once per device, with that device current: the device address of this
// device's `scratch` and its CU count (for the split plan).
static NoAllocDevice* noalloc_setup(int dev) {
    NoAllocDevice* d = &g_noalloc[dev];
    std::call_once(d->once, [d, dev]() {
        void* p = nullptr;
        d->status = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (d->status == hipSuccess)
            d->status = hipDeviceGetAttribute(&d->cu_count, hipDeviceAttributeMultiprocessorCount, dev);
        d->ptr = static_cast<float*>(p);
    });
    return d;
}

bp_status bp_attention_decode_noalloc(const bp_config* cfg, void* kv_k, void* kv_v, uint32_t max_seq, void* act,
                                      uint32_t q_off, uint32_t out_off, uint32_t layer_il, uint32_t pos,
                                      void* stream) {
    if (!cfg || !kv_k || !kv_v || !act) return fail(BP_ERR_INVALID_ARG, "cfg/kv_k/kv_v/act is NULL");
    if (cfg->head_dim != bp::kHeadDim)
        return fail(BP_ERR_CONFIG, "head_dim must be 128 (got %u)", cfg->head_dim);
    if (cfg->n_kv_head == 0 || cfg->n_head != cfg->n_kv_head * bp::kGroup)
        return fail(BP_ERR_CONFIG, "n_head must be 4 * n_kv_head (got %u, %u)", cfg->n_head, cfg->n_kv_head);
    if (layer_il >= cfg->n_layer) return fail(BP_ERR_INVALID_ARG, "layer %u >= n_layer %u", layer_il, cfg->n_layer);
    const uint32_t kv_dim = cfg->n_kv_head * cfg->head_dim;
    if (static_cast<uint64_t>(max_seq) * kv_dim > 0xFFFFFFFFull)
        return fail(BP_ERR_CONFIG, "max_seq %u x kv_dim %u exceeds the 32-bit per-layer cache offsets", max_seq, kv_dim);
    if (pos >= max_seq)
        return fail(BP_ERR_CONTEXT_OVERFLOW, "context overflow: pos %u + tokens 1 > max_seq %u", pos, max_seq);
    if ((q_off & 7u) || (out_off & 3u))
        return fail(BP_ERR_INVALID_ARG, "q_off must be a multiple of 8 and out_off of 4 (aligned f16 rows)");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(BP_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kNoAllocMaxDevices) return fail(BP_ERR_INVALID_ARG, "device %d out of range", dev);
    NoAllocDevice* d = noalloc_setup(dev);
    if (d->status != hipSuccess)
        return fail(BP_ERR_HIP, "scratch symbol lookup on device %d: %s", dev, hipGetErrorString(d->status));

    bp::DecodeArgs a{};
    a.q = static_cast<const uint16_t*>(act) + q_off;
    a.out = static_cast<uint16_t*>(act) + out_off;
    const uint64_t nb = kv_dim / 32;
    const uint64_t d_word = static_cast<uint64_t>(layer_il) * max_seq * nb;
    const uint64_t qs_byte = static_cast<uint64_t>(cfg->n_layer) * max_seq * nb * 4 +
                             static_cast<uint64_t>(layer_il) * max_seq * kv_dim;
    a.k.d = static_cast<const float*>(kv_k) + d_word;
    a.k.qs = static_cast<const int8_t*>(kv_k) + qs_byte;
    a.v.d = static_cast<const float*>(kv_v) + d_word;
    a.v.qs = static_cast<const int8_t*>(kv_v) + qs_byte;
    a.partials = d->ptr;
    a.kv_dim = kv_dim;
    a.n_rows = pos + 1;   // src/forward.rs:822
    bp::decode_plan(a.n_rows, cfg->n_kv_head, d->cu_count, bp::kDecodeMinSplitRows, bp::kDecodeWideMinRows,
                    &a.split_len, &a.n_splits, &a.heads_per_wg);
    a.scale = 1.0f / std::sqrt(static_cast<float>(cfg->head_dim));   // src/forward.rs:838
    if (static_cast<uint64_t>(a.n_splits) * cfg->n_head * bp::decode_partial_stride() > kNoAllocScratchFloats)
        return fail(BP_ERR_CONFIG, "noalloc decode: %u query heads x %u splits exceed the %llu-float scratch",
                    cfg->n_head, a.n_splits, static_cast<unsigned long long>(kNoAllocScratchFloats));
    e = bp::launch_decode(a, cfg->n_kv_head, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return fail(BP_ERR_HIP, "attention_decode_noalloc launch: %s", hipGetErrorString(e));
    return BP_OK;
}

bp_status bp_kv_snapshot_capture(bp_model* m, uint32_t pos, void* payload, uint64_t payload_bytes) {
    return snapshot_copy(m, pos, static_cast<uint8_t*>(payload), payload_bytes, true);
}

bp_status bp_kv_snapshot_apply(bp_model* m, uint32_t pos, const void* payload, uint64_t payload_bytes) {
    return snapshot_copy(m, pos, static_cast<uint8_t*>(const_cast<void*>(payload)), payload_bytes, false);
}

}  // extern "C"
