/* A plain-C caller of the C ABI: it includes only include/bonsai_pot_hip.h
 * (plus the HIP runtime API for device memory, as any host program needs) and
 * links libbonsai_pot_hip.so, standing in for the Rust -sys crate a
 * bonsai-pot maintainer would write. It runs one layer of one decode step,
 * the sequence src/forward.rs issues per token:
 *   bp_dispatch_q_norm_rope_fused, bp_dispatch_kv_writeback_fused,
 *   bp_dispatch_attention_decode (rows [0, pos]),
 * and, on a second model with the same inputs, the fused
 *   bp_dispatch_attention_decode_step,
 * then writes both resulting act buffers and KV buffers to a file, which
 * tests/test_capi_client.py compares with the CPU oracle.
 *
 * Input file (little-endian): u32 n_layer, max_seq, layer_il, pos, n_act,
 * n_w, then u16 act[n_act], u16 w_norms[n_w], u8 kv_k[bytes], u8 kv_v[bytes]
 * (bytes = bp_kv_buffer_bytes(...)). Offsets are fixed: q at 0, k_cur at
 * 4096, v_cur at 5120, out at 6144; w_q_norm at 0, w_k_norm at 128.
 * Output file: for each of the two runs, act then kv_k then kv_v. */
#include "bonsai_pot_hip.h"

#include <hip/hip_runtime_api.h>

#include <stdio.h>
#include <stdlib.h>

#define CHECK_BP(call)                                                              \
    do {                                                                            \
        bp_status s_ = (call);                                                      \
        if (s_ != BP_OK) {                                                          \
            fprintf(stderr, "%s failed: %s (%s)\n", #call, bp_status_name(s_),      \
                    bp_last_error());                                               \
            return 2;                                                               \
        }                                                                           \
    } while (0)
#define CHECK_HIP(call)                                                             \
    do {                                                                            \
        hipError_t e_ = (call);                                                     \
        if (e_ != hipSuccess) {                                                     \
            fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));       \
            return 3;                                                               \
        }                                                                           \
    } while (0)

static int read_all(FILE* f, void* dst, size_t n) { return fread(dst, 1, n, f) == n ? 0 : 1; }

static int run(int fused, const bp_config* cfg, uint32_t max_seq, uint32_t il, uint32_t pos,
               const uint16_t* act_h, uint32_t n_act, const uint16_t* w_h, uint32_t n_w,
               const uint8_t* k_h, const uint8_t* v_h, uint64_t kv_bytes, FILE* out) {
    bp_model* m = NULL;
    CHECK_BP(bp_model_create(cfg, max_seq, 0, &m));
    void *kv_k = NULL, *kv_v = NULL;
    uint64_t bytes = 0;
    CHECK_BP(bp_model_kv_buffers(m, &kv_k, &kv_v, &bytes));
    if (bytes != kv_bytes) {
        fprintf(stderr, "kv buffer size %llu != %llu\n", (unsigned long long)bytes,
                (unsigned long long)kv_bytes);
        return 4;
    }
    void *act = NULL, *w = NULL;
    CHECK_HIP(hipMalloc(&act, (size_t)n_act * 2));
    CHECK_HIP(hipMalloc(&w, (size_t)n_w * 2));
    CHECK_HIP(hipMemcpy(act, act_h, (size_t)n_act * 2, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(w, w_h, (size_t)n_w * 2, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(kv_k, k_h, kv_bytes, hipMemcpyHostToDevice));
    CHECK_HIP(hipMemcpy(kv_v, v_h, kv_bytes, hipMemcpyHostToDevice));
    const uint32_t q_off = 0, k_off = 4096, v_off = 5120, out_off = 6144, wq = 0, wk = 128;
    if (fused) {
        CHECK_BP(bp_dispatch_attention_decode_step(m, act, w, q_off, k_off, v_off, out_off, wq, wk, il, pos));
    } else {
        CHECK_BP(bp_dispatch_q_norm_rope_fused(m, act, w, q_off, wq, pos, 1));
        CHECK_BP(bp_dispatch_kv_writeback_fused(m, act, w, k_off, v_off, wk, il, pos, 1));
        CHECK_BP(bp_dispatch_attention_decode(m, act, q_off, out_off, il, pos));
    }
    CHECK_BP(bp_model_synchronize(m));
    uint16_t* a_out = (uint16_t*)malloc((size_t)n_act * 2);
    uint8_t* kv_out = (uint8_t*)malloc(kv_bytes);
    if (!a_out || !kv_out) return 5;
    CHECK_HIP(hipMemcpy(a_out, act, (size_t)n_act * 2, hipMemcpyDeviceToHost));
    fwrite(a_out, 2, n_act, out);
    CHECK_HIP(hipMemcpy(kv_out, kv_k, kv_bytes, hipMemcpyDeviceToHost));
    fwrite(kv_out, 1, kv_bytes, out);
    CHECK_HIP(hipMemcpy(kv_out, kv_v, kv_bytes, hipMemcpyDeviceToHost));
    fwrite(kv_out, 1, kv_bytes, out);
    free(a_out);
    free(kv_out);
    CHECK_HIP(hipFree(act));
    CHECK_HIP(hipFree(w));
    bp_model_destroy(m);
    return 0;
}

int main(int argc, char** argv) {
    if (argc != 3) {
        fprintf(stderr, "usage: %s input.bin output.bin\n", argv[0]);
        return 1;
    }
    FILE* in = fopen(argv[1], "rb");
    if (!in) return 1;
    uint32_t hdr[6];
    if (read_all(in, hdr, sizeof hdr)) return 1;
    const bp_config cfg = {hdr[0], 32, 8, 128, 1e-6f, 1e6f};
    const uint32_t max_seq = hdr[1], il = hdr[2], pos = hdr[3], n_act = hdr[4], n_w = hdr[5];
    const uint64_t kv_bytes = bp_kv_buffer_bytes(cfg.n_layer, 1024, max_seq);
    uint16_t* act = (uint16_t*)malloc((size_t)n_act * 2);
    uint16_t* w = (uint16_t*)malloc((size_t)n_w * 2);
    uint8_t* k = (uint8_t*)malloc(kv_bytes);
    uint8_t* v = (uint8_t*)malloc(kv_bytes);
    if (!act || !w || !k || !v) return 1;
    if (read_all(in, act, (size_t)n_act * 2) || read_all(in, w, (size_t)n_w * 2) || read_all(in, k, kv_bytes) ||
        read_all(in, v, kv_bytes))
        return 1;
    fclose(in);
    FILE* out = fopen(argv[2], "wb");
    if (!out) return 1;
    for (int fused = 0; fused < 2; fused++) {
        const int rc = run(fused, &cfg, max_seq, il, pos, act, n_act, w, n_w, k, v, kv_bytes, out);
        if (rc != 0) return rc;
    }
    fclose(out);
    printf("capi_client ok: layer %u pos %u\n", il, pos);
    return 0;
}
