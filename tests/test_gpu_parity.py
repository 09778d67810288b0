"""HIP path vs CPU oracle, through the C ABI (bonsai_pot_amd -> libbonsai_pot_hip.so).

Bars: Q8_0 cache bytes and q_norm_rope f16 outputs bit-exact; attention outputs
within max-abs 2e-3 and rel-L2 1e-3 of the oracle's f32-softmax result.
"""
import sys

import numpy as np
import pytest

import oracle as orc
from bonsai_pot_amd import layout
from helpers import DeviceScenario, Scenario, assert_attn_close, write_outlier_rows

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
                                              (512, 0, 0.0), (300, 1700, 0.1), (2048, 2048, 0.1)])
def test_writeback_and_q_norm_rope_bit_exact(cuda, m, pos_base, w_std):
    _say(f"[writeback] m={m} pos_base={pos_base} w_std={w_std}")
    cfg = layout.Config(n_layer=3)
    sc = Scenario(cfg, max_seq=4096, m_tokens=m, seed=m + pos_base, w_std=w_std)
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


@pytest.mark.parametrize("m", [1, 9, 64])
def test_writeback_and_q_norm_rope_unaligned_offsets(cuda, m):
    """Element offsets that are not multiples of 8 (the kernels then use 2-byte
    loads and stores instead of 16-byte vectors): same bits as the oracle."""
    _say(f"[writeback] unaligned offsets m={m}")
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=256, m_tokens=m, seed=100 + m, w_std=0.1)
    sc.q_off, sc.k_off, sc.v_off = 3, sc.k_off + 5, sc.v_off + 7
    sc.w_q_off, sc.w_k_off = 1, 127
    dev = DeviceScenario(sc)
    dev.writeback(il=1, pos_base=40)
    dev.q_norm_rope(40)
    sc.oracle_writeback(il=1, pos_base=40)
    sc.oracle_q_norm_rope(40)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k), f"K cache bytes differ at {np.flatnonzero(k != sc.kv_k)[:8]}"
    assert np.array_equal(v, sc.kv_v), f"V cache bytes differ at {np.flatnonzero(v != sc.kv_v)[:8]}"
    assert np.array_equal(dev.act_host(), sc.act), "q_norm_rope f16 output differs"


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


# The split pass has two layouts (1 or 4 KV heads per workgroup), chosen by
# context length; BP_DECODE_WIDE_MIN_ROWS forces either one at model creation.
LAYOUTS = {"narrow": str(2**31), "wide": "0"}


@pytest.mark.parametrize("layout_name", sorted(LAYOUTS))
@pytest.mark.parametrize("pos", [0, 1, 31, 512, 4096])
def test_decode_vs_oracle(cuda, monkeypatch, pos, layout_name):
    monkeypatch.setenv("BP_DECODE_WIDE_MIN_ROWS", LAYOUTS[layout_name])
    _say(f"[decode] pos={pos} layout={layout_name}")
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=pos + 8, m_tokens=1, seed=100 + pos)
    _prefill_cache(sc, 1, pos, seed=200 + pos)
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(1, pos)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.decode(1, pos)
    _, want = sc.oracle_decode(1, pos)
    assert_attn_close(dev.out_f32(1)[0], want, f"decode pos={pos}")


@pytest.mark.parametrize("pos", [65536, 99999])
def test_decode_long_context(cuda, pos):
    """Past 128 x 256 rows the split plan keeps 128 splits and lengthens them
    (65536: 512 rows each, 16 batches per wave; 99999: 800 rows, an odd 25
    batches per wave and a short last split): the plain decode and the fused
    step against the oracle."""
    _say(f"[decode] long context pos={pos}")
    cfg = layout.Config(n_layer=1)
    sc = Scenario(cfg, max_seq=pos + 1, m_tokens=1, seed=300 + pos % 1000)
    _prefill_cache(sc, 0, pos, seed=400 + pos % 1000)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.decode_step(0, pos)
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(0, pos)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k) and np.array_equal(v, sc.kv_v), "cache bytes differ"
    _, want = sc.oracle_decode(0, pos)
    assert_attn_close(dev.out_f32(1)[0], want, f"decode step pos={pos}")
    dev.decode(0, pos)   # plain entry point on the normalized q the step left in act
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
                                        (130, 1000), (33, 31), (200, 900)])
@pytest.mark.parametrize("hpw", ["1", "1w4", "2"])
def test_prefill_vs_oracle(cuda, monkeypatch, m, pos_base, hpw):
    """Every prefill_kernel layout (1 query head per wave in 8- or 4-wave
    workgroups, or 2 per wave; by default the grid size picks one), forced
    through BP_PREFILL_HEADS_PER_WAVE and BP_PREFILL_WG_WAVES. (200, 900)
    gives second-half units whose first chunk lies wholly past some tokens'
    last row (all scores masked while the running max is still unset)."""
    monkeypatch.setenv("BP_PREFILL_HEADS_PER_WAVE", hpw[0])
    monkeypatch.setenv("BP_PREFILL_WG_WAVES", "4" if hpw.endswith("w4") else "8")
    _say(f"[prefill] m={m} pos_base={pos_base} heads_per_wave={hpw}")
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


@pytest.mark.parametrize("m,pos_base", [(2048, 0), (2048, 2048), (64, 16384)])
def test_prefill_full_size_sampled_rows(cuda, m, pos_base):
    """pp2048 (metric), config 4 (2048-token chunk over a 2048-row cache) and
    the bench's chat-turn shape (64 tokens over 16384 rows: the key-split
    kernel at its default 32 splits): the whole output is computed on the
    GPU, the oracle checks sampled tokens spread over every 64-token tile,
    including first/last rows."""
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
    tokens = tokens[tokens < m] if m > 128 else np.arange(m)   # short chunks: every token
    want = sc.oracle_attention(0, pos_base, is_prefill=True, tokens=tokens)
    got = dev.out_f32()[tokens]
    assert_attn_close(got, want, f"prefill m={m} pos_base={pos_base}")


@pytest.mark.parametrize("m,pos_base", [(100, 30000), (1000, 8000), (2048, 6000)])
def test_prefill_long_cache_sampled_rows(cuda, m, pos_base):
    """Chunks over long caches in each layout the library picks by default:
    100 tokens on 30000 rows (the key split), 1000 on 8000 (the one-head
    8-wave kernel over the image) and 2048 on 6000 (prefill32_kernel); the
    oracle checks sampled tokens of every 64-token tile, first and last
    included."""
    _say(f"[prefill-long] m={m} pos_base={pos_base}")
    cfg = layout.Config(n_layer=1)
    sc = Scenario(cfg, max_seq=pos_base + m, m_tokens=m, seed=m + pos_base)
    _prefill_cache(sc, 0, pos_base, seed=78)
    sc.oracle_q_norm_rope(pos_base)
    sc.oracle_writeback(0, pos_base)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.attention(0, pos_base, is_prefill=True)
    rng = np.random.default_rng(2)
    tokens = np.unique(np.concatenate([[0, 1, 31, 32, m - 1], np.arange(0, m, 64) + rng.integers(0, 64, (m + 63) // 64)]))
    tokens = tokens[tokens < m]
    want = sc.oracle_attention(0, pos_base, is_prefill=True, tokens=tokens)
    assert_attn_close(dev.out_f32()[tokens], want, f"prefill m={m} pos_base={pos_base}")


def test_decode_repeated_calls_fresh_partials(cuda):
    """Back-to-back decodes on one model (different layers, positions and queries)
    reuse the split-K scratch and tickets; every output must match its own oracle
    result, so stale partials from an earlier launch would show up here."""
    _say("[decode] repeated calls")
    cfg = layout.Config(n_layer=3)
    max_seq = 6000
    sc = Scenario(cfg, max_seq=max_seq, m_tokens=1, seed=61)
    for il in range(3):
        pre = Scenario(cfg, max_seq, 5000, seed=62 + il, with_q=False)
        pre.kv_k, pre.kv_v = sc.kv_k, sc.kv_v
        pre.oracle_writeback(il, 0)
    dev = DeviceScenario(sc, upload_kv=True)
    rng = np.random.default_rng(5)
    for step, (il, pos) in enumerate([(0, 4999), (1, 3000), (2, 4095), (0, 700), (1, 4999), (2, 64)]):
        q = rng.standard_normal(cfg.q_dim).astype(np.float16).view(np.uint16)
        sc.act[sc.q_off:sc.q_off + cfg.q_dim] = q
        dev.act[sc.q_off:sc.q_off + cfg.q_dim] = __import__("torch").from_numpy(q.view(np.int16).copy()).cuda()
        dev.decode(il, pos)
        _, want = sc.oracle_decode(il, pos)
        assert_attn_close(dev.out_f32(1)[0], want, f"repeat step {step} layer {il} pos {pos}")


@pytest.mark.parametrize("layout_name", sorted(LAYOUTS))
@pytest.mark.parametrize("pos,w_std", [(0, 0.0), (1, 0.1), (40, 0.1), (4096, 0.0), (32768, 0.1)])
def test_fused_decode_step(cuda, monkeypatch, pos, w_std, layout_name):
    """bp_dispatch_attention_decode_step == q_norm_rope + kv_writeback + decode:
    normalized q and cache bytes bit-exact, attention output within tolerance."""
    monkeypatch.setenv("BP_DECODE_WIDE_MIN_ROWS", LAYOUTS[layout_name])
    _say(f"[decode-step] pos={pos} layout={layout_name}")
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=pos + 4, m_tokens=1, seed=700 + pos, w_std=w_std)
    _prefill_cache(sc, 1, pos, seed=800 + pos)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.decode_step(1, pos)
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(1, pos)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k) and np.array_equal(v, sc.kv_v), "cache bytes differ"
    act = dev.act_host()
    assert np.array_equal(act[:cfg.q_dim], sc.act[:cfg.q_dim]), "normalized q differs"
    _, want = sc.oracle_decode(1, pos)
    assert_attn_close(dev.out_f32(1)[0], want, f"decode step pos={pos}")


def test_fused_decode_step_sequence(cuda):
    """Eight consecutive fused steps (pos 300..307) across two layers on one model:
    each step's row is then attended by the next; matches the oracle every step."""
    _say("[decode-step] sequence")
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=320, m_tokens=1, seed=91)
    _prefill_cache(sc, 0, 300, seed=92)
    pre1 = Scenario(cfg, 320, 300, seed=93, with_q=False)
    pre1.kv_k, pre1.kv_v = sc.kv_k, sc.kv_v
    pre1.oracle_writeback(1, 0)
    dev = DeviceScenario(sc, upload_kv=True)
    import torch
    rng = np.random.default_rng(9)
    for step in range(8):
        pos = 300 + step
        raw = rng.standard_normal(cfg.q_dim + 2 * cfg.kv_dim).astype(np.float16).view(np.uint16)
        sc.act[:raw.size] = raw
        dev.act[:raw.size] = torch.from_numpy(raw.view(np.int16).copy()).cuda()
        for il in (0, 1):
            sc.act[:raw.size] = raw
            dev.act[:raw.size] = torch.from_numpy(raw.view(np.int16).copy()).cuda()
            dev.decode_step(il, pos)
            sc.oracle_q_norm_rope(pos)
            sc.oracle_writeback(il, pos)
            _, want = sc.oracle_decode(il, pos)
            assert_attn_close(dev.out_f32(1)[0], want, f"step {step} layer {il}")
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k) and np.array_equal(v, sc.kv_v)


@pytest.mark.parametrize("hpw", ["1", "1w4", "2"])
@pytest.mark.parametrize("m,pos_base", [(512, 0), (200, 900)])
def test_prefill_with_outlier_key_rows(cuda, monkeypatch, m, pos_base, hpw):
    """Causal prefill over a cache whose K rows are 1 % x8 (rows of the chunk
    itself and of the cached prefix): scores far above the running max drive
    the lazy rescale with P up to 2^8 in f16. The cache [0, pos_base + m) is
    written by the oracle; the device runs the attention only."""
    monkeypatch.setenv("BP_PREFILL_HEADS_PER_WAVE", hpw[0])
    monkeypatch.setenv("BP_PREFILL_WG_WAVES", "4" if hpw.endswith("w4") else "8")
    _say(f"[prefill-outliers] m={m} pos_base={pos_base} heads_per_wave={hpw}")
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=pos_base + m + 1, m_tokens=m, seed=1300 + m + pos_base)
    write_outlier_rows(sc, 1, pos_base + m, seed=1400 + m)
    sc.oracle_q_norm_rope(pos_base)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.attention(1, pos_base, is_prefill=True)
    want = sc.oracle_attention(1, pos_base, is_prefill=True)
    assert_attn_close(dev.out_f32(), want, f"prefill outliers m={m} pos={pos_base} hpw={hpw}")


def test_config1_real_cache_last_layer(cuda):
    """configs[1]'s real cache: n_layer 36, ctx 4096, the fused step on the last
    layer (35). Cache rows written by the oracle for layer 35 only; after the
    step layer 35 gains row 4096 and every other layer's bytes are untouched."""
    _say("[config1] n_layer=36 ctx=4096 layer 35")
    cfg = layout.Config(n_layer=36)
    pos = 4096
    sc = Scenario(cfg, max_seq=pos + 64, m_tokens=1, seed=4135)
    pre = Scenario(cfg, pos + 64, pos, seed=4136, with_q=False)
    pre.kv_k, pre.kv_v = sc.kv_k, sc.kv_v
    pre.oracle_writeback(35, 0)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.decode_step(35, pos)
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(35, pos)
    k, v = dev.kv_host()
    assert np.array_equal(k, sc.kv_k) and np.array_equal(v, sc.kv_v), "cache bytes differ"
    _, want = sc.oracle_decode(35, pos)
    assert_attn_close(dev.out_f32(1)[0], want, "config1 layer 35 decode step")
    # and the plain decode entry point on the same cache
    dev.decode(35, pos)
    assert_attn_close(dev.out_f32(1)[0], want, "config1 layer 35 decode")


@pytest.mark.parametrize("m,pos_base,ksplit", [(1, 4000, "auto"), (16, 3000, "auto"), (16, 3000, "3"),
                                               (70, 2500, "auto"), (70, 2500, "7"), (100, 5, "4"),
                                               (33, 31, "2"), (64, 640, "40")])
def test_prefill_key_split(cuda, monkeypatch, m, pos_base, ksplit):
    """Short chunks over long caches: prefill_split_kernel splits the keys over
    several workgroups, each reading the cache rows itself, and
    prefill_merge_kernel combines their partials (forced split counts include
    ones whose last splits lie past some tiles' keys, and one above the chunk
    count)."""
    monkeypatch.setenv("BP_PREFILL_HEADS_PER_WAVE", "1")
    monkeypatch.setenv("BP_PREFILL_WG_WAVES", "4")
    if ksplit != "auto":
        monkeypatch.setenv("BP_PREFILL_KSPLIT", ksplit)
    _say(f"[prefill-ksplit] m={m} pos_base={pos_base} ksplit={ksplit}")
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=pos_base + m + 3, m_tokens=m, seed=900 + m + pos_base)
    if pos_base >= 100:   # 1 % of the cache's K rows x8 (the lazy-rescale stress)
        write_outlier_rows(sc, 0, pos_base, seed=960 + m)
    else:
        _prefill_cache(sc, 0, pos_base, seed=950 + pos_base)
    sc.oracle_q_norm_rope(pos_base)
    sc.oracle_writeback(0, pos_base)
    dev = DeviceScenario(sc, upload_kv=True)
    dev.attention(0, pos_base, is_prefill=True)
    want = sc.oracle_attention(0, pos_base, is_prefill=True)
    assert_attn_close(dev.out_f32(), want, f"prefill key split m={m} pos_base={pos_base} ksplit={ksplit}")
