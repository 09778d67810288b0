"""Golden fixture tests (tests/golden/attn_small.npz, written by
tests/golden/make_golden.py from the CPU oracle).

CPU: the oracle still reproduces every committed bit (pins the oracle).
GPU: the HIP path on the fixture's inputs gives bit-identical cache bytes and
normalized q, and attention outputs within the tolerance of the fixture's.
"""
import os

import numpy as np
import pytest

from helpers import DeviceScenario, Scenario, assert_attn_close

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "attn_small.npz")


def _fixture():
    with np.load(FIXTURE, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_oracle_reproduces_golden_fixture():
    from golden.make_golden import build
    _, got = build()
    want = _fixture()
    assert sorted(got) == sorted(want)
    for k in want:
        assert got[k].dtype == want[k].dtype and got[k].shape == want[k].shape, k
        assert np.array_equal(got[k].view(np.uint8), want[k].view(np.uint8)), f"{k} differs"


@pytest.mark.gpu
def test_hip_path_matches_golden_fixture(cuda):
    from bonsai_pot_amd import layout
    from golden.make_golden import MAX_SEQ, M_Q, N_CACHE
    fx = _fixture()
    cfg = layout.Config(n_layer=1)
    pre = Scenario(cfg, MAX_SEQ, N_CACHE, with_q=False)
    pre.act[:] = fx["pre_act"]
    pre.w_norms[:] = fx["w_norms"]
    dpre = DeviceScenario(pre)
    dpre.writeback(0, 0)
    k_pre, v_pre = dpre.kv_host()

    sc = Scenario(cfg, MAX_SEQ, M_Q)
    sc.act[:] = fx["act"]
    sc.w_norms[:] = fx["w_norms"]
    sc.kv_k[:], sc.kv_v[:] = k_pre, v_pre
    dev = DeviceScenario(sc, upload_kv=True)
    dev.q_norm_rope(N_CACHE)
    dev.writeback(0, N_CACHE)
    k, v = dev.kv_host()
    assert np.array_equal(k, fx["kv_k"]) and np.array_equal(v, fx["kv_v"]), "cache bytes differ"
    act = dev.act_host()
    assert np.array_equal(act[sc.q_off:sc.q_off + M_Q * cfg.q_dim], fx["q_normed"]), "q_norm_rope differs"
    dev.attention(0, N_CACHE, is_prefill=True)
    assert_attn_close(dev.out_f32(), fx["prefill_out"], "golden prefill")
    dev.decode(0, N_CACHE + M_Q - 1)
    assert_attn_close(dev.out_f32(1)[0], fx["decode_out"], "golden decode")
