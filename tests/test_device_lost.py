"""Device-loss latch (src/model.rs:1087-1098, :1733-1751; the reference's
tests/gpu_integration.rs:268-336): after bp_debug_lose_device — the
reference's __destroy_device_for_test — every call that would touch the
device returns BP_ERR_DEVICE_LOST without launching anything, snapshot
capture / apply fail the same way, and a freshly created model is healthy and
passes a decode parity check. The latch is host-side only: no kernel faults."""
import ctypes
import sys

import numpy as np
import pytest

import bonsai_pot_amd as bp
from bonsai_pot_amd import errors, layout
from helpers import DeviceScenario, Scenario, assert_attn_close

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _fresh_decode_parity(seed):
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=96, m_tokens=1, seed=seed)
    pre = Scenario(cfg, max_seq=96, m_tokens=40, seed=seed + 1, with_q=False)
    pre.oracle_writeback(1, 0)
    sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v
    dev = DeviceScenario(sc, upload_kv=True)
    assert not dev.model.is_device_lost()
    dev.decode_step(1, 40)
    sc.oracle_q_norm_rope(40)
    sc.oracle_writeback(1, 40)
    _, want = sc.oracle_decode(1, 40)
    err = assert_attn_close(dev.out_f32(1)[0], want, "decode after recovery")
    return dev, err


def test_device_lost_latch_and_recovery(cuda):
    import torch
    _say("[device_lost] healthy model, snapshot, lose device")
    dev, _ = _fresh_decode_parity(seed=71)
    m = dev.model
    snap_payload = m.snapshot_payload(8)   # healthy: capture works
    m._destroy_device_for_test()
    assert m.is_device_lost()
    h = m.handle
    L = bp.lib
    a = dev.act.data_ptr()
    w = dev.w.data_ptr()
    scratch = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    s = scratch.data_ptr()
    calls = {
        "bp_check_device": lambda: L.bp_check_device(h),
        "bp_model_synchronize": lambda: L.bp_model_synchronize(h),
        "bp_model_set_stream": lambda: L.bp_model_set_stream(h, None),
        "bp_dispatch_q_norm_rope_fused": lambda: L.bp_dispatch_q_norm_rope_fused(h, a, w, 0, 0, 8, 1),
        "bp_dispatch_kv_writeback_fused": lambda: L.bp_dispatch_kv_writeback_fused(h, a, w, 0, 0, 128, 0, 8, 1),
        "bp_dispatch_attention_decode": lambda: L.bp_dispatch_attention_decode(h, a, 0, 0, 0, 8),
        "bp_dispatch_attention_decode_step": lambda: L.bp_dispatch_attention_decode_step(
            h, a, w, 0, 0, 0, 0, 0, 128, 0, 8),
        "bp_dispatch_attention": lambda: L.bp_dispatch_attention(h, a, 0, 0, 0, 0, 4, 1),
        "bp_dispatch_attention_prefill_step": lambda: L.bp_dispatch_attention_prefill_step(
            h, a, w, 0, 0, 0, 0, 0, 128, 0, 0, 4),
        "bp_dispatch_matvec_q1_0": lambda: L.bp_dispatch_matvec_q1_0(h, s, a, 128, 16, 0, 64, 0, 128, 0),
        "bp_dispatch_matvec_q1_0_silu": lambda: L.bp_dispatch_matvec_q1_0_silu(h, s, a, 128, 16, 0, 64, 0, 128, 256, 0),
        "bp_dispatch_matvec_q1_0_fused_normed": lambda: L.bp_dispatch_matvec_q1_0_fused_normed(
            h, s, a, w, 128, 0, 0, 1, ctypes.byref(bp.model.MatvecRange(0, 64, 16, 128))),
        "bp_dispatch_quantize_act": lambda: L.bp_dispatch_quantize_act(h, a, s, 32, 1, 0, 0, 4),
        "bp_dispatch_matmul_q1_0": lambda: L.bp_dispatch_matmul_q1_0(h, s, s, a, 128, 16, 1, 0, 64, 0, 4, 0, 0),
        "bp_dispatch_topk_reduce": lambda: L.bp_dispatch_topk_reduce(h, a, s, 64, 8, 0, 0),
    }
    for name, call in calls.items():
        rc = call()
        assert rc == errors.BP_ERR_DEVICE_LOST, f"{name} returned {rc} after device loss"
        assert b"device lost" in L.bp_last_error(), name
    vals = np.zeros(8, np.float32)
    idx = np.zeros(8, np.uint32)
    assert L.bp_topk_readback(h, s, 0, 8, vals.ctypes.data_as(ctypes.c_void_p),
                              idx.ctypes.data_as(ctypes.c_void_p)) == errors.BP_ERR_DEVICE_LOST
    # snapshot() and restore() are guarded too
    with pytest.raises(bp.DeviceLostError):
        m.snapshot_payload(8)
    with pytest.raises(bp.DeviceLostError):
        m.apply_payload(8, snap_payload)
    # the Python mirror raises the matching error class
    with pytest.raises(bp.DeviceLostError):
        m.dispatch_attention_decode(a, 0, 0, 0, 8)
    torch.cuda.synchronize()
    m.close()

    _say("[device_lost] fresh model after loss: decode parity")
    dev2, err = _fresh_decode_parity(seed=72)
    _say(f"[device_lost] recovered decode max_abs {err[0]:.2e} rel_l2 {err[1]:.2e}")
    dev2.model.close()
