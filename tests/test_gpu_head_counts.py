"""Other head counts than Bonsai's 8 KV heads (n_head = 4 n_kv_head, the only
grouping the reference accepts: src/model.rs:672), HIP path vs CPU oracle.

The kernels take the head count from the model: grids, the decode layouts (four
KV heads per workgroup only when n_kv_head is a multiple of 4) and the XCD
order of the prefill grid all follow it. Same bars as test_gpu_parity.py:
cache bytes and normalized q bit-exact, attention within max-abs 2e-3 and
rel-L2 1e-3 of the oracle.
"""
import sys

import numpy as np
import pytest

from bonsai_pot_amd import layout
from helpers import DeviceScenario, Scenario, assert_attn_close

pytestmark = pytest.mark.gpu

KV_HEADS = [1, 2, 4, 12]


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _cfg(kv):
    return layout.Config(n_layer=2, n_head=4 * kv, n_kv_head=kv)


def _prefill_cache(sc, il, n_rows, seed):
    if n_rows == 0:
        return
    pre = Scenario(sc.cfg, sc.max_seq, n_rows, seed=seed, with_q=False)
    pre.oracle_writeback(il, 0)
    sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v


@pytest.mark.parametrize("kv", KV_HEADS)
def test_writeback_and_q_norm_rope(cuda, kv):
    _say(f"[heads] writeback n_kv_head={kv}")
    sc = Scenario(_cfg(kv), max_seq=64, m_tokens=5, seed=10 + kv, w_std=0.1)
    dev = DeviceScenario(sc)
    dev.writeback(il=1, pos_base=10)
    dev.q_norm_rope(10)
    sc.oracle_writeback(il=1, pos_base=10)
    sc.oracle_q_norm_rope(10)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k) and np.array_equal(v, sc.kv_v), "cache bytes differ"
    assert np.array_equal(dev.act_host(), sc.act), "q_norm_rope output differs"


@pytest.mark.parametrize("kv", KV_HEADS)
@pytest.mark.parametrize("pos", [300, 9000])
def test_decode_step(cuda, kv, pos):
    """The fused step; at 9000 rows the wide layout runs when n_kv_head % 4 == 0."""
    _say(f"[heads] decode step n_kv_head={kv} pos={pos}")
    cfg = _cfg(kv)
    sc = Scenario(cfg, max_seq=pos + 4, m_tokens=1, seed=20 + kv + pos)
    _prefill_cache(sc, 1, pos, seed=30 + kv + pos)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.decode_step(1, pos)
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(1, pos)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k) and np.array_equal(v, sc.kv_v), "cache bytes differ"
    _, want = sc.oracle_decode(1, pos)
    assert_attn_close(dev.out_f32(1)[0], want, f"decode step n_kv_head={kv} pos={pos}")


@pytest.mark.parametrize("kv", KV_HEADS)
@pytest.mark.parametrize("m,pos_base", [(70, 0), (33, 100)])
@pytest.mark.parametrize("hpw", ["1", "1w4", "2"])
def test_prefill(cuda, monkeypatch, kv, m, pos_base, hpw):
    monkeypatch.setenv("BP_PREFILL_HEADS_PER_WAVE", hpw[0])
    monkeypatch.setenv("BP_PREFILL_WG_WAVES", "4" if hpw.endswith("w4") else "8")
    _say(f"[heads] prefill n_kv_head={kv} m={m} pos_base={pos_base} heads_per_wave={hpw}")
    cfg = _cfg(kv)
    sc = Scenario(cfg, max_seq=pos_base + m + 3, m_tokens=m, seed=40 + kv + m + pos_base)
    _prefill_cache(sc, 0, pos_base, seed=50 + kv + pos_base)
    sc.oracle_q_norm_rope(pos_base)
    sc.oracle_writeback(0, pos_base)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.attention(0, pos_base, is_prefill=True)
    want = sc.oracle_attention(0, pos_base, is_prefill=True)
    assert_attn_close(dev.out_f32(), want, f"prefill n_kv_head={kv} m={m} pos_base={pos_base}")


@pytest.mark.parametrize("kv", KV_HEADS)
@pytest.mark.parametrize("m,pos", [(70, 0), (33, 100)])
def test_prefill_step(cuda, kv, m, pos):
    """The fused prefill step (preparation pass over (KV head, chunk, part)
    grids of this head count): cache bytes and normalized q bit-exact,
    attention within tolerance."""
    _say(f"[heads] prefill step n_kv_head={kv} m={m} pos={pos}")
    cfg = _cfg(kv)
    sc = Scenario(cfg, max_seq=pos + m + 3, m_tokens=m, seed=60 + kv + m + pos, w_std=0.1)
    _prefill_cache(sc, 1, pos, seed=70 + kv + pos)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.model.dispatch_attention_prefill_step(dev.act.data_ptr(), dev.w.data_ptr(), sc.q_off, sc.k_off,
                                              sc.v_off, sc.out_off, sc.w_q_off, sc.w_k_off, 1, pos, m)
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(1, pos)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k) and np.array_equal(v, sc.kv_v), "cache bytes differ"
    act = dev.act_host()
    q = slice(sc.q_off, sc.q_off + m * cfg.q_dim)
    assert np.array_equal(act[q], sc.act[q]), "normalized q differs"
    want = sc.oracle_attention(1, pos, is_prefill=True)
    assert_attn_close(dev.out_f32(), want, f"prefill step n_kv_head={kv} m={m} pos={pos}")


@pytest.mark.parametrize("kv", KV_HEADS)
def test_prefill_key_split(cuda, monkeypatch, kv):
    """The key-split 4-wave layout (grid y = splits x 4 head sets) at this head count."""
    monkeypatch.setenv("BP_PREFILL_HEADS_PER_WAVE", "1")
    monkeypatch.setenv("BP_PREFILL_WG_WAVES", "4")
    monkeypatch.setenv("BP_PREFILL_KSPLIT", "3")
    _say(f"[heads] prefill key split n_kv_head={kv}")
    cfg = _cfg(kv)
    m, pos = 40, 1500
    sc = Scenario(cfg, max_seq=pos + m + 3, m_tokens=m, seed=80 + kv)
    _prefill_cache(sc, 0, pos, seed=90 + kv)
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(0, pos)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.attention(0, pos, is_prefill=True)
    want = sc.oracle_attention(0, pos, is_prefill=True)
    assert_attn_close(dev.out_f32(), want, f"prefill key split n_kv_head={kv}")
