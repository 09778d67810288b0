"""bp_attention_decode_noalloc (the allocation-free decode: split-K partials
in the library's fixed device array, no bp_model) against
bp_dispatch_attention_decode on the same cache and query: identical f16
output bits, and both within the attention tolerance of the oracle. Two calls
in a row, the second with fewer cache rows (a smaller input), so the array's
reuse with a different split count is covered; a too-large configuration is
rejected without launching."""
import ctypes
import sys

import numpy as np
import pytest

import bonsai_pot_amd as bp
from bonsai_pot_amd import errors, layout
from bonsai_pot_amd.model import _Config
from helpers import DeviceScenario, Scenario, assert_attn_close

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def test_noalloc_decode_matches_model_decode(cuda):
    import torch
    cfg = layout.Config(n_layer=3)
    max_seq, il = 33000, 2
    sc = Scenario(cfg, max_seq=max_seq, m_tokens=1, seed=4242)
    pre = Scenario(cfg, max_seq, 32768, seed=4243, with_q=False)
    pre.kv_k, pre.kv_v = sc.kv_k, sc.kv_v
    pre.oracle_writeback(il, 0)
    sc.oracle_q_norm_rope(32768)
    dev = DeviceScenario(sc, upload_kv=True)
    c = _Config(cfg.n_layer, cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.rms_eps, cfg.rope_freq_base)
    stream = torch.cuda.current_stream().cuda_stream
    a = dev.act.data_ptr()
    for pos in (32767, 1000):   # second call: smaller input (fewer rows and splits)
        _say(f"[noalloc] layer {il} pos {pos}")
        dev.decode(il, pos)
        want_bits = dev.act_host()[sc.out_off:sc.out_off + cfg.q_dim].copy()
        dev.act[sc.out_off:sc.out_off + cfg.q_dim] = 0
        rc = bp.lib.bp_attention_decode_noalloc(ctypes.byref(c), dev.kv_k, dev.kv_v, max_seq, a, sc.q_off,
                                                sc.out_off, il, pos, stream)
        assert rc == 0, bp.lib.bp_last_error()
        torch.cuda.synchronize()
        got_bits = dev.act_host()[sc.out_off:sc.out_off + cfg.q_dim]
        assert np.array_equal(got_bits, want_bits), f"pos {pos}: noalloc output differs from the model entry point"
        _, want = sc.oracle_decode(il, pos)
        assert_attn_close(got_bits.view(np.float16).astype(np.float32), want, f"noalloc decode pos {pos}")
    # rejected before any launch: n_head * splits beyond the fixed array
    # (4096 KV heads: one split each, 16384 x 130 floats > 64 x 128 x 130)
    big = _Config(1, 16384, 4096, 128, 1e-6, 1e6)
    rc = bp.lib.bp_attention_decode_noalloc(ctypes.byref(big), dev.kv_k, dev.kv_v, 64, a, 0, 0, 0, 10, stream)
    assert rc == errors.BP_ERR_CONFIG and b"scratch" in bp.lib.bp_last_error()
    rc = bp.lib.bp_attention_decode_noalloc(ctypes.byref(c), dev.kv_k, dev.kv_v, max_seq, a, 0, 0, 0, max_seq, stream)
    assert rc == errors.BP_ERR_CONTEXT_OVERFLOW
    dev.model.close()
