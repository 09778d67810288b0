"""HIP path vs CPU oracle, through the C ABI (bonsai_pot_amd -> libbonsai_pot_hip.so).

Bars: Q8_0 cache bytes and q_norm_rope f16 outputs bit-exact; attention outputs
within max-abs 2e-3 and rel-L2 1e-3 of the oracle's f32-softmax result.
"""
import sys

import numpy as np
import pytest

import oracle as orc
from bonsai_pot_amd import layout
from helpers import DeviceScenario, Scenario, assert_attn_close

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _prefill_cache(sc: Scenario, il: int, n_rows: int, seed: int):
    """Oracle-written cache rows [0, n_rows) of layer il (from an independent
    seeded K/V scenario), copied into sc's KV buffers."""
    if n_rows == 0:
        return
    pre = Scenario(sc.cfg, sc.max_seq, n_rows, seed=seed, with_q=False)
    pre.oracle_writeback(il, 0)
    sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v


@pytest.mark.parametrize("m,pos_base,w_std", [(1, 0, 0.0), (1, 512, 0.1), (7, 33, 0.1),
                                              (512, 0, 0.0), (300, 1700, 0.1)])
def test_writeback_and_q_norm_rope_bit_exact(cuda, m, pos_base, w_std):
    _say(f"[writeback] m={m} pos_base={pos_base} w_std={w_std}")
    cfg = layout.Config(n_layer=3)
    sc = Scenario(cfg, max_seq=2048, m_tokens=m, seed=m + pos_base, w_std=w_std)
    dev = DeviceScenario(sc)
    dev.writeback(il=2, pos_base=pos_base)
    dev.q_norm_rope(pos_base)
    sc.oracle_writeback(il=2, pos_base=pos_base)
    sc.oracle_q_norm_rope(pos_base)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k), f"K cache bytes differ at {np.flatnonzero(k != sc.kv_k)[:8]}"
    assert np.array_equal(v, sc.kv_v), f"V cache bytes differ at {np.flatnonzero(v != sc.kv_v)[:8]}"
    act = dev.act_host()
    assert np.array_equal(act, sc.act), "q_norm_rope f16 output differs"


def test_writeback_special_values(cuda):
    """All-zero heads (d = 0 path), tiny subnormal f16 V values, +-max f16."""
    _say("[writeback] special values")
    cfg = layout.Config(n_layer=1)
    sc = Scenario(cfg, max_seq=16, m_tokens=4, seed=3)
    a16 = sc.act.view(np.float16)
    kv = cfg.kv_dim
    a16[sc.k_off:sc.k_off + kv] = 0                     # token 0: K all zero
    a16[sc.v_off:sc.v_off + kv] = 0                     # token 0: V all zero
    a16[sc.v_off + kv:sc.v_off + 2 * kv] = np.float16(2.0**-24)   # token 1: min subnormal V
    a16[sc.v_off + kv + 5] = np.float16(-2.0**-24)
    a16[sc.v_off + 2 * kv:sc.v_off + 3 * kv] = np.float16(65504)  # token 2: max f16 V
    a16[sc.k_off + 2 * kv:sc.k_off + 3 * kv] = np.float16(-65504)
    dev = DeviceScenario(sc)
    dev.writeback(0, 0)
    sc.oracle_writeback(0, 0)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k) and np.array_equal(v, sc.kv_v)


@pytest.mark.parametrize("pos", [0, 1, 31, 512, 4096])
def test_decode_vs_oracle(cuda, pos):
    _say(f"[decode] pos={pos}")
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=pos + 8, m_tokens=1, seed=100 + pos)
    _prefill_cache(sc, 1, pos, seed=200 + pos)
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(1, pos)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.decode(1, pos)
    _, want = sc.oracle_decode(1, pos)
    assert_attn_close(dev.out_f32(1)[0], want, f"decode pos={pos}")


def test_decode_ctx32k_with_outlier_rows(cuda):
    """Config 5: ctx 32768 (32769 rows), 1% of key rows x8 before quantization
    (x8 = a w_k_norm of 8.0 for those rows, exact in f16)."""
    _say("[decode] ctx32k outliers")
    cfg = layout.Config(n_layer=1)
    pos = 32768
    sc = Scenario(cfg, max_seq=pos + 1, m_tokens=1, seed=5)
    pre = Scenario(cfg, max_seq=pos + 1, m_tokens=pos, seed=6, with_q=False)
    pre.oracle_writeback(0, 0)
    rng = np.random.default_rng(7)
    rows = rng.choice(pos, size=pos // 100, replace=False)
    w8 = np.concatenate([pre.w_norms, np.full(128, np.float16(8.0)).view(np.uint16)])
    big = Scenario(cfg, max_seq=pos + 1, m_tokens=1, seed=0)
    for r in rows:   # rewrite those rows with K scaled x8
        big.act[big.k_off:big.k_off + cfg.kv_dim] = pre.act[pre.k_off + r * cfg.kv_dim:
                                                            pre.k_off + (r + 1) * cfg.kv_dim]
        big.act[big.v_off:big.v_off + cfg.kv_dim] = pre.act[pre.v_off + r * cfg.kv_dim:
                                                            pre.v_off + (r + 1) * cfg.kv_dim]
        big.w_norms = w8
        big.kv_k, big.kv_v = pre.kv_k, pre.kv_v
        big.oracle_writeback(0, int(r), m=1, w_k_off=256)
    sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(0, pos)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.decode(0, pos)
    _, want = sc.oracle_decode(0, pos)
    assert_attn_close(dev.out_f32(1)[0], want, "decode ctx32k")


@pytest.mark.parametrize("m,pos_base", [(1, 0), (17, 0), (64, 0), (65, 0), (100, 5), (512, 0),
                                        (130, 1000), (33, 31)])
def test_prefill_vs_oracle(cuda, m, pos_base):
    _say(f"[prefill] m={m} pos_base={pos_base}")
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=pos_base + m + 3, m_tokens=m, seed=300 + m + pos_base)
    _prefill_cache(sc, 0, pos_base, seed=400 + pos_base)
    sc.oracle_q_norm_rope(pos_base)
    sc.oracle_writeback(0, pos_base)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.attention(0, pos_base, is_prefill=True)
    want = sc.oracle_attention(0, pos_base, is_prefill=True)
    assert_attn_close(dev.out_f32(), want, f"prefill m={m} pos_base={pos_base}")


def test_attention_non_causal_multi_token(cuda):
    """is_prefill = 0: every token sees rows [0, pos) (attention.wgsl:263)."""
    _say("[prefill] non-causal")
    cfg = layout.Config(n_layer=1)
    sc = Scenario(cfg, max_seq=300, m_tokens=40, seed=9)
    _prefill_cache(sc, 0, 250, seed=10)
    sc.oracle_q_norm_rope(250)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.attention(0, 250, is_prefill=False)
    want = sc.oracle_attention(0, 250, is_prefill=False)
    assert_attn_close(dev.out_f32(), want, "non-causal")


@pytest.mark.parametrize("m,pos_base", [(2048, 0), (2048, 2048)])
def test_prefill_full_size_sampled_rows(cuda, m, pos_base):
    """pp2048 (metric) and config 4 (2048-token chunk over a 2048-row cache):
    the whole output is computed on the GPU, the oracle checks sampled tokens
    spread over every 64-token tile, including first/last rows."""
    _say(f"[prefill-full] m={m} pos_base={pos_base}")
    cfg = layout.Config(n_layer=1)
    sc = Scenario(cfg, max_seq=pos_base + m, m_tokens=m, seed=m + pos_base)
    _prefill_cache(sc, 0, pos_base, seed=77)
    sc.oracle_q_norm_rope(pos_base)
    sc.oracle_writeback(0, pos_base)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.attention(0, pos_base, is_prefill=True)
    rng = np.random.default_rng(1)
    tokens = np.unique(np.concatenate([[0, 1, 15, 16, 63, 64, m - 1],
                                       np.arange(0, m, 64) + rng.integers(0, 64, m // 64)]))
    want = sc.oracle_attention(0, pos_base, is_prefill=True, tokens=tokens)
    got = dev.out_f32()[tokens]
    assert_attn_close(got, want, f"prefill m={m} pos_base={pos_base}")
