/* Measurement hooks of bench.py: no counterpart in the reference and not
 * part of the attention path. They are exported only by the bench build of
 * the library, lib/libbonsai_pot_hip_bench.so (the same objects as
 * lib/libbonsai_pot_hip.so, with bp_api.cpp compiled with BP_BENCH_HOOKS and
 * the read-floor kernel linked in); the product library lacks them. */
#ifndef BONSAI_POT_HIP_BENCH_H
#define BONSAI_POT_HIP_BENCH_H

#include "bonsai_pot_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Measurement aid, no counterpart in the reference and not part of the
 * attention path: reads `bytes` (a multiple of 16) of device memory at `src`
 * once with independent 16-byte loads over `n_workgroups` workgroups of 256
 * threads and writes one word per workgroup to `sink` (n_workgroups x 4 bytes),
 * on `stream`. bench.py times it as the streaming-read floor of a decode's
 * byte count. */
bp_status bp_debug_read_floor(const void* src, uint64_t bytes, void* sink, uint32_t n_workgroups, void* stream);

/* Measurement aid, no counterpart in the reference and not part of the
 * attention path: `iters` x 4 back-to-back v_mfma_f32_32x32x16_f16 per wave
 * on random f16 operands, `n_workgroups` workgroups of 4 waves, on `stream`;
 * writes one float per thread to `sink` (n_workgroups x 1 KB). That is
 * n_workgroups x 4 x iters x 4 x 32768 flops; bench.py times it as the f16
 * matrix rate the GPU sustains on real (random) data. */
bp_status bp_debug_mfma_rate(void* sink, uint32_t iters, uint32_t n_workgroups, uint32_t seed, void* stream);

/* Measurement aid, no counterpart in the reference: the first of the two
 * launches of bp_dispatch_attention_prefill_step alone (q norm + RoPE, the
 * K/V writeback and the attention kernel's f16 image of the layer's rows),
 * same arguments; every act / w_norms offset must be a multiple of 8.
 * bench.py times it to split the step's time between its two kernels. */
bp_status bp_debug_prefill_prep(bp_model* model, void* act, const void* w_norms, uint32_t q_off,
                                uint32_t k_cur_off, uint32_t v_cur_off, uint32_t out_off,
                                uint32_t w_q_norm_off, uint32_t w_k_norm_off, uint32_t layer_il,
                                uint32_t pos, uint32_t m_tokens);

#ifdef __cplusplus
}
#endif

#endif /* BONSAI_POT_HIP_BENCH_H */
