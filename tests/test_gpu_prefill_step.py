"""bp_dispatch_attention_prefill_step (the fused causal prefill step: q norm +
RoPE, K/V writeback and attention in two launches) against the three separate
dispatches it replaces and against the CPU oracle, through the C ABI.

Bars: normalized q, the whole act buffer and the Q8_0 cache bytes bit-exact
against the separate dispatches (whose image and attention arithmetic the
step shares); against the oracle, cache bytes and q bit-exact and attention
within max-abs 2e-3 and rel-L2 1e-3.
"""
import sys

import numpy as np
import pytest

from bonsai_pot_amd import layout
from helpers import DeviceScenario, Scenario, assert_attn_close

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _scenario(m, pos, seed, w_std=0.1, n_layer=2, il=1):
    cfg = layout.Config(n_layer=n_layer)
    sc = Scenario(cfg, max_seq=pos + m + 5, m_tokens=m, seed=seed, w_std=w_std)
    if pos:
        pre = Scenario(cfg, sc.max_seq, pos, seed=seed + 1, with_q=False)
        pre.oracle_writeback(il, 0)
        sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v
    return sc


def _step(dev, il, pos):
    sc = dev.sc
    dev.model.dispatch_attention_prefill_step(dev.act.data_ptr(), dev.w.data_ptr(), sc.q_off, sc.k_off,
                                              sc.v_off, sc.out_off, sc.w_q_off, sc.w_k_off, il, pos, sc.m)


def _unfused(dev, il, pos):
    dev.q_norm_rope(pos)
    dev.writeback(il, pos)
    dev.attention(il, pos, is_prefill=True)


def _same(dev_a, dev_b, what):
    ka, va = dev_a.kv_host()
    kb, vb = dev_b.kv_host()
    assert np.array_equal(ka, kb), f"{what}: K cache bytes differ at {np.flatnonzero(ka != kb)[:8]}"
    assert np.array_equal(va, vb), f"{what}: V cache bytes differ at {np.flatnonzero(va != vb)[:8]}"
    aa, ab = dev_a.act_host(), dev_b.act_host()
    assert np.array_equal(aa, ab), f"{what}: act differs at {np.flatnonzero(aa != ab)[:8]}"


@pytest.mark.parametrize("m,pos", [(1, 0), (33, 0), (64, 0), (70, 0), (512, 0), (100, 5), (33, 31),
                                   (130, 1000), (200, 900), (64, 64), (300, 64), (1, 4095),
                                   (2048, 0), (2048, 2048)])
def test_prefill_step_matches_separate_dispatches(cuda, m, pos):
    """Chunks wholly before pos, chunks mixing cache rows and new rows (pos not
    a multiple of 64), new rows ending inside a chunk, and the full-size
    configurations: same bits as q_norm_rope + kv_writeback + attention."""
    _say(f"[prefill-step] m={m} pos={pos}")
    sc = _scenario(m, pos, seed=1000 + m + pos)
    dev_a = DeviceScenario(sc, upload_kv=True)
    dev_b = DeviceScenario(sc, upload_kv=True)
    _step(dev_a, 1, pos)
    _unfused(dev_b, 1, pos)
    _same(dev_a, dev_b, f"m={m} pos={pos}")


@pytest.mark.parametrize("hpw", ["1", "1w4", "2"])
@pytest.mark.parametrize("m,pos", [(17, 0), (100, 5), (200, 900)])
def test_prefill_step_vs_oracle(cuda, monkeypatch, m, pos, hpw):
    """The fused step against the oracle directly, in both attention layouts."""
    monkeypatch.setenv("BP_PREFILL_HEADS_PER_WAVE", hpw[0])
    monkeypatch.setenv("BP_PREFILL_WG_WAVES", "4" if hpw.endswith("w4") else "8")
    _say(f"[prefill-step] oracle m={m} pos={pos} heads_per_wave={hpw}")
    sc = _scenario(m, pos, seed=2000 + m + pos)
    dev = DeviceScenario(sc, upload_kv=True)
    _step(dev, 1, pos)
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(1, pos)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k), f"K cache bytes differ at {np.flatnonzero(k != sc.kv_k)[:8]}"
    assert np.array_equal(v, sc.kv_v), f"V cache bytes differ at {np.flatnonzero(v != sc.kv_v)[:8]}"
    act = dev.act_host()
    q = slice(sc.q_off, sc.q_off + m * sc.cfg.q_dim)
    assert np.array_equal(act[q], sc.act[q]), "normalized q differs"
    want = sc.oracle_attention(1, pos, is_prefill=True)
    assert_attn_close(dev.out_f32(), want, f"prefill step m={m} pos={pos}")


@pytest.mark.parametrize("m", [9, 70])
def test_prefill_step_unaligned_offsets(cuda, m):
    """Offsets that are not multiples of 8 take the separate dispatches inside
    the call: same bits as calling them."""
    _say(f"[prefill-step] unaligned offsets m={m}")
    sc = _scenario(m, 40, seed=3000 + m)
    sc.k_off, sc.v_off = sc.k_off + 5, sc.v_off + 7
    sc.w_q_off, sc.w_k_off = 1, 127
    dev_a = DeviceScenario(sc, upload_kv=True)
    dev_b = DeviceScenario(sc, upload_kv=True)
    _step(dev_a, 1, 40)
    _unfused(dev_b, 1, 40)
    _same(dev_a, dev_b, f"unaligned m={m}")


def test_prefill_step_then_decode_steps(cuda):
    """A prompt through the fused prefill step, then fused decode steps that
    attend its rows, on layers 0 and 1 of one model: the same bits as the
    separate dispatches for the whole sequence."""
    _say("[prefill-step] prompt then decode")
    import torch
    m, pos0 = 150, 0
    sc = _scenario(m, pos0, seed=4000, n_layer=2, il=0)
    dev_a = DeviceScenario(sc, upload_kv=True)
    dev_b = DeviceScenario(sc, upload_kv=True)
    for il in (0, 1):
        _step(dev_a, il, pos0)
        _unfused(dev_b, il, pos0)
    _same(dev_a, dev_b, "prompt")
    rng = np.random.default_rng(4)
    for step in range(3):
        pos = pos0 + m + step
        raw = rng.standard_normal(sc.cfg.q_dim + 2 * sc.cfg.kv_dim).astype(np.float16).view(np.uint16)
        for dev in (dev_a, dev_b):
            dev.act[:raw.size] = torch.from_numpy(raw.view(np.int16).copy()).cuda()
            for il in (0, 1):
                dev.decode_step(il, pos)
        _same(dev_a, dev_b, f"decode step {step}")


@pytest.mark.parametrize("m,pos", [(16, 3000), (70, 2500)])
def test_prefill_step_key_split(cuda, m, pos):
    """The fused step where the attention splits each tile's keys (short chunk,
    long cache: chosen by grid size): same bits as the separate dispatches."""
    _say(f"[prefill-step] key split m={m} pos={pos}")
    sc = _scenario(m, pos, seed=5000 + m + pos)
    dev_a = DeviceScenario(sc, upload_kv=True)
    dev_b = DeviceScenario(sc, upload_kv=True)
    _step(dev_a, 1, pos)
    _unfused(dev_b, 1, pos)
    _same(dev_a, dev_b, f"key split m={m} pos={pos}")
