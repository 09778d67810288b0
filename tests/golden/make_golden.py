"""Writes tests/golden/attn_small.npz: seeded inputs and the CPU oracle's
outputs for one small end-to-end case of the attention path.

Case (one layer, Bonsai head shapes, max_seq 48, w_q_norm/w_k_norm ~ N(1, 0.1)):
  1. kv_writeback_fused of 32 tokens at rows [0, 32)        -> kv_k, kv_v
  2. q_norm_rope_fused of 4 query tokens at pos_base 32      -> q (f16 bits)
  3. kv_writeback_fused of those 4 tokens at rows [32, 36)   -> kv_k, kv_v
  4. causal chunked prefill attention of the 4 tokens at pos 32 (rows [0, 33+i))
  5. split/merge decode of query token 0 at step position 35 (rows [0, 35])

The bytes are produced by the oracle (the restatement of the reference
shaders), so the fixture pins the oracle against later edits and gives the
HIP path a fixed target. Regenerate with: python3 tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "bonsai-pot_amd"), os.path.join(ROOT, "tests")):
    sys.path.insert(0, p)

from bonsai_pot_amd import layout  # noqa: E402
from helpers import Scenario  # noqa: E402

PATH = os.path.join(HERE, "attn_small.npz")
MAX_SEQ, N_CACHE, M_Q = 48, 32, 4


def build():
    cfg = layout.Config(n_layer=1)
    pre = Scenario(cfg, MAX_SEQ, N_CACHE, seed=11, w_std=0.1, with_q=False)
    sc = Scenario(cfg, MAX_SEQ, M_Q, seed=12, w_std=0.1)
    sc.w_norms = pre.w_norms.copy()
    inputs = {"pre_act": pre.act.copy(), "act": sc.act.copy(), "w_norms": sc.w_norms.copy()}
    pre.oracle_writeback(0, 0)
    sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v
    sc.oracle_q_norm_rope(N_CACHE)
    sc.oracle_writeback(0, N_CACHE)
    prefill = sc.oracle_attention(0, N_CACHE, is_prefill=True)
    dec_bits, dec = sc.oracle_decode(0, N_CACHE + M_Q - 1)
    out = {
        **inputs,
        "q_normed": sc.act[sc.q_off:sc.q_off + M_Q * cfg.q_dim].copy(),
        "kv_k": sc.kv_k.copy(), "kv_v": sc.kv_v.copy(),
        "prefill_out": np.asarray(prefill, np.float32),
        "decode_out": np.asarray(dec, np.float32),
        "decode_out_f16": np.asarray(dec_bits, np.uint16),
    }
    return cfg, out


if __name__ == "__main__":
    _, out = build()
    np.savez_compressed(PATH, **out)
    print("wrote", PATH, os.path.getsize(PATH), "bytes")
