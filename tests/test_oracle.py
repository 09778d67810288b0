"""Pins the CPU oracle (oracle/bp_oracle.c) before anything is checked against it.

Each check is independent of the oracle's own code: the reference's unit-test
values, numpy's IEEE conversions, closed forms in float64, hand-built
known-answer vectors, brute-force float64 attention, and invariants.
"""
import math

import numpy as np
import pytest

import oracle as orc
from bonsai_pot_amd import layout
from helpers import Scenario

CFG = layout.Config()


# ---- f16 conversion: numpy's astype is IEEE round-to-nearest-even ---------------
def test_f32_to_f16_matches_numpy_random_bits():
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    want = x.astype(np.float16).view(np.uint16)
    got = orc.f32_to_f16_bits(x)
    assert np.array_equal(got, want)


def test_f32_to_f16_ties_and_edges():
    # every f16 value, its midpoints with the next value, and values just off them
    h = np.arange(0, 0x7c00, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)         # exact in f32
    cand = np.concatenate([lo.astype(np.float32), mids, np.nextafter(mids, 0, dtype=np.float32),
                           np.nextafter(mids, np.inf, dtype=np.float32),
                           np.array([65504, 65519.996, 65520, 1e-8, 2.0**-25, 2.0**-24], np.float32)])
    cand = np.concatenate([cand, -cand])
    assert np.array_equal(orc.f32_to_f16_bits(cand), cand.astype(np.float16).view(np.uint16))


def test_f16_to_f32_all_values():
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = orc.f16_bits_to_f32(h)
    ok = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert ok.all()


# ---- RoPE table: src/model.rs:2022-2045 and the closed form ----------------------
def test_rope_table_reference_unit_test_values():
    # The reference's own test: head_dim 8, base 1e4, max_seq 4.
    f, _ = orc.rope_table(8, 10_000.0, 4)
    assert f.shape == (32,)
    assert abs(f[0] - 1.0) < 1e-6 and abs(f[1]) < 1e-6
    assert abs(f[8] - np.float32(math.cos(1.0))) < 1e-5
    assert abs(f[9] - np.float32(math.sin(1.0))) < 1e-5


def test_rope_table_closed_form_bonsai():
    max_seq = 4097
    f, h = orc.rope_table(128, 1e6, max_seq)
    p = np.arange(max_seq, dtype=np.float64)[:, None]
    j = np.arange(64, dtype=np.float64)[None, :]
    ang = p * (1e6 ** (-2.0 * j / 128.0))
    want = np.empty((max_seq, 64, 2), np.float32)
    want[..., 0] = np.cos(ang).astype(np.float32)
    want[..., 1] = np.sin(ang).astype(np.float32)
    # f64 pow/cos/sin may differ from numpy's in the last f64 bit -> <= 1 f32 ulp
    assert np.max(np.abs(f.reshape(max_seq, 64, 2) - want)) <= 1.2e-7
    want16 = want.astype(np.float16).view(np.uint16).reshape(-1)
    assert np.mean(h == want16) > 0.9999
    assert np.max(np.abs(h.view(np.float16).astype(np.float32) - want.reshape(-1))) <= 2**-11


# ---- KV layout + snapshot payload: src/kv_snapshot.rs:376-521 --------------------
def test_snapshot_payload_sizes_reference_values():
    assert orc.snapshot_payload_bytes(36, 1024, 512) == 42_467_328
    assert orc.snapshot_payload_bytes(36, 1024, 32768) == 2_717_908_992
    assert orc.snapshot_payload_bytes(36, 1024, 0) == 0
    assert layout.snapshot_payload_bytes(36, 1024, 512) == 42_467_328


def test_snapshot_offsets_no_overlap():
    n_layer, kv_dim, pos = 36, 1024, 16
    for kind in range(2):
        for il in range(n_layer):
            d0 = orc.snapshot_payload_offset(n_layer, kv_dim, pos, kind, il, 0)
            q0 = orc.snapshot_payload_offset(n_layer, kv_dim, pos, kind, il, 1)
            assert d0 + pos * (kv_dim // 32) * 4 <= q0
            if il + 1 < n_layer:
                nd = orc.snapshot_payload_offset(n_layer, kv_dim, pos, kind, il + 1, 0)
                assert q0 + pos * kv_dim <= nd
            assert d0 == layout.snapshot_payload_offset(n_layer, kv_dim, pos, kind, il, 0)
            assert q0 == layout.snapshot_payload_offset(n_layer, kv_dim, pos, kind, il, 1)


def test_kv_layout_u32_range_at_36x32768():
    # SURVEY-derived: qs base 150,994,944 B; whole buffer 1,358,954,496 B < 2^32.
    d, q = orc.kv_layer_offsets(36, 1024, 32768, 0)
    assert (d, q) == (0, 150_994_944)
    assert orc.kv_buffer_bytes(36, 1024, 32768) == 1_358_954_496 < 2**32
    d35, q35 = orc.kv_layer_offsets(36, 1024, 32768, 35)
    assert d35 == 35 * 32768 * 32 and q35 == 150_994_944 + 35 * 32768 * 1024
    assert layout.kv_layer_offsets(36, 1024, 32768, 35) == (d35, q35)


def test_snapshot_capture_apply_roundtrip():
    rng = np.random.default_rng(3)
    n_layer, kv_dim, max_seq, pos = 3, 1024, 40, 17
    nbytes = orc.kv_buffer_bytes(n_layer, kv_dim, max_seq)
    k = rng.integers(0, 256, nbytes, dtype=np.uint8)
    v = rng.integers(0, 256, nbytes, dtype=np.uint8)
    payload = orc.snapshot_capture(n_layer, kv_dim, max_seq, pos, k, v)
    # independent decode of the payload: K block for layer 1, row 5, block 7
    d_word, qs_byte = layout.kv_layer_offsets(n_layer, kv_dim, max_seq, 1)
    off_d = layout.snapshot_payload_offset(n_layer, kv_dim, pos, 0, 1, 0)
    assert payload[off_d + (5 * 32 + 7) * 4: off_d + (5 * 32 + 8) * 4].tobytes() == \
        k[(d_word + 5 * 32 + 7) * 4:(d_word + 5 * 32 + 8) * 4].tobytes()
    off_q = layout.snapshot_payload_offset(n_layer, kv_dim, pos, 1, 2, 1)
    d2, q2 = layout.kv_layer_offsets(n_layer, kv_dim, max_seq, 2)
    assert payload[off_q + 16 * 1024: off_q + 17 * 1024].tobytes() == \
        v[q2 + 16 * 1024: q2 + 17 * 1024].tobytes()
    # restore into a bigger max_seq: snapshot is independent of max_seq (kv_snapshot.rs:19-20)
    max2 = 64
    k2 = np.zeros(orc.kv_buffer_bytes(n_layer, kv_dim, max2), np.uint8)
    v2 = np.zeros_like(k2)
    orc.snapshot_apply(n_layer, kv_dim, max2, pos, payload, k2, v2)
    assert np.array_equal(orc.snapshot_capture(n_layer, kv_dim, max2, pos, k2, v2), payload)


# ---- Q8_0 quantizer: hand-built known answers -------------------------------------
def test_quantize_known_answers():
    d, q = orc.quantize_block(np.zeros(32))
    assert d == 0.0 and not q.any()
    # amax 127 -> d = 1, inv_d = 1: q = rne(x); ties go to even
    x = np.zeros(32, np.float32)
    x[:8] = [127, -127, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5]
    d, q = orc.quantize_block(x)
    assert d == 1.0
    assert list(q[:8]) == [127, -127, 2, 4, -2, 0, 0, 2]
    # +-amax maps to +-127 for arbitrary scales; d is an f32 division
    rng = np.random.default_rng(0)
    for _ in range(200):
        x = rng.standard_normal(32).astype(np.float32) * np.float32(rng.uniform(1e-3, 1e3))
        d, q = orc.quantize_block(x)
        amax = np.max(np.abs(x))
        assert np.float32(d) == np.float32(amax) / np.float32(127)
        assert q[np.argmax(np.abs(x))] == (127 if x[np.argmax(np.abs(x))] > 0 else -127)
        inv = np.float32(1) / np.float32(d)
        want = np.clip(np.rint(x * inv), -127, 127).astype(np.int8)
        assert np.array_equal(q, want)


def test_quantize_tiny_amax():
    # f16's smallest subnormal: d is a normal f32, the element quantizes to 127
    x = np.zeros(32, np.float32)
    x[3] = np.float32(2.0**-24)
    d, q = orc.quantize_block(x)
    assert d == np.float32(2.0**-24) / np.float32(127) and q[3] == 127 and q.sum() == 127
    x[3] = np.float32(-1e-30)
    d, q = orc.quantize_block(x)
    assert d > 0 and q[3] == -127 and np.count_nonzero(q) == 1


# ---- kv_writeback / q_norm_rope vs float64 ideal --------------------------------
def _ideal_norm_rope(x16, w16, rope16, pos, eps):
    x = x16.astype(np.float64)
    w = w16.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x) + eps)
    n = x * inv * w
    cs = rope16[pos * 128:(pos + 1) * 128].view(np.float16).astype(np.float64).reshape(64, 2)
    c, s = cs[:, 0], cs[:, 1]
    out = np.empty(128)
    out[:64] = n[:64] * c - n[64:] * s
    out[64:] = n[:64] * s + n[64:] * c
    return out


def _dequant_rows(buf, cfg, max_seq, il, rows):
    d_word, qs_byte = layout.kv_layer_offsets(cfg.n_layer, cfg.kv_dim, max_seq, il)
    nb = cfg.kv_dim // 32
    d = buf[d_word * 4:(d_word + max_seq * nb) * 4].view(np.float32).reshape(max_seq, nb)
    qs = buf[qs_byte:qs_byte + max_seq * cfg.kv_dim].view(np.int8).reshape(max_seq, cfg.kv_dim)
    return d[rows], qs[rows]


@pytest.mark.parametrize("w_std", [0.0, 0.1])
def test_kv_writeback_matches_f64_ideal(w_std):
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=300, m_tokens=40, seed=11, w_std=w_std)
    pos_base = 250
    sc.oracle_writeback(il=1, pos_base=pos_base)
    rows = np.arange(pos_base, pos_base + sc.m)
    kd, kq = _dequant_rows(sc.kv_k, cfg, sc.max_seq, 1, rows)
    vd, vq = _dequant_rows(sc.kv_v, cfg, sc.max_seq, 1, rows)
    act16 = sc.act.view(np.float16)
    w_k = sc.w_norms.view(np.float16)[128:256]
    near_tie = total = 0
    for t in range(sc.m):
        for h in range(cfg.n_kv_head):
            k = act16[sc.k_off + t * cfg.kv_dim + h * 128: sc.k_off + t * cfg.kv_dim + (h + 1) * 128]
            ideal = _ideal_norm_rope(k, w_k, sc.rope, pos_base + t, cfg.rms_eps)
            v = act16[sc.v_off + t * cfg.kv_dim + h * 128: sc.v_off + t * cfg.kv_dim + (h + 1) * 128]
            for b in range(4):
                blk = slice(32 * b, 32 * b + 32)
                for x, d, q in ((ideal[blk], kd[t, 4 * h + b], kq[t, h * 128 + 32 * b: h * 128 + 32 * b + 32]),
                                (v[blk].astype(np.float64), vd[t, 4 * h + b],
                                 vq[t, h * 128 + 32 * b: h * 128 + 32 * b + 32])):
                    amax = np.max(np.abs(x))
                    assert abs(d - amax / 127) <= 4e-7 * amax / 127 + 1e-30
                    r = x / (amax / 127)
                    want = np.clip(np.rint(r), -127, 127)
                    frac = np.abs(np.abs(r - np.floor(r)) - 0.5)
                    diff = q.astype(np.int64) != want
                    # only values within 1e-3 of a .5 tie may round the other way
                    assert np.all(frac[diff] < 1e-3), (t, h, b)
                    assert np.all(np.abs(q.astype(np.int64) - want) <= 1)
                    near_tie += int(diff.sum())
                    total += 32
    assert near_tie <= total * 1e-3


def test_q_norm_rope_matches_f64_ideal():
    cfg = layout.Config(n_layer=1)
    sc = Scenario(cfg, max_seq=600, m_tokens=20, seed=5, w_std=0.1)
    raw = sc.act.copy()
    sc.oracle_q_norm_rope(pos_base=580)
    w_q = sc.w_norms.view(np.float16)[:128]
    for t in range(sc.m):
        for h in range(cfg.n_head):
            o = t * cfg.q_dim + h * 128
            ideal = _ideal_norm_rope(raw[o:o + 128].view(np.float16), w_q, sc.rope, 580 + t, cfg.rms_eps)
            got = sc.act[o:o + 128].view(np.float16).astype(np.float64)
            # <= 1 f16 ulp (plus f32 rounding of the intermediates)
            ulp = np.spacing(np.abs(ideal).astype(np.float16)).astype(np.float64)
            assert np.all(np.abs(got - ideal) <= ulp * 0.5 + 1e-6 * np.abs(ideal) + 1e-7)


# ---- attention vs float64 brute force ----------------------------------------------
def _brute_attention(sc, il, tokens, n_rows_of):
    cfg = sc.cfg
    rows = np.arange(sc.max_seq)
    kd, kq = _dequant_rows(sc.kv_k, cfg, sc.max_seq, il, rows)
    vd, vq = _dequant_rows(sc.kv_v, cfg, sc.max_seq, il, rows)
    K = (kq.reshape(sc.max_seq, -1, 32).astype(np.float64) * kd[..., None]).reshape(sc.max_seq, -1)
    V = (vq.reshape(sc.max_seq, -1, 32).astype(np.float64) * vd[..., None]).reshape(sc.max_seq, -1)
    q = sc.act[sc.q_off:sc.q_off + sc.m * cfg.q_dim].view(np.float16).astype(np.float64)
    q = q.reshape(sc.m, cfg.n_head, 128)
    out = np.zeros((len(tokens), cfg.q_dim))
    for i, t in enumerate(tokens):
        n = n_rows_of(t)
        for h in range(cfg.n_head):
            g = h // (cfg.n_head // cfg.n_kv_head)            # GQA: attention.wgsl:260
            s = K[:n, g * 128:(g + 1) * 128] @ q[t, h] / math.sqrt(128)
            p = np.exp(s - s.max())
            out[i, h * 128:(h + 1) * 128] = p @ V[:n, g * 128:(g + 1) * 128] / p.sum()
    return out


@pytest.mark.parametrize("pos_base,m", [(0, 37), (45, 20)])
def test_attention_oracle_matches_brute_force(pos_base, m):
    cfg = layout.Config(n_layer=2)
    sc = Scenario(cfg, max_seq=96, m_tokens=m, seed=7 + pos_base)
    if pos_base:
        pre = Scenario(cfg, max_seq=96, m_tokens=pos_base, seed=99, with_q=False)
        pre.oracle_writeback(il=1, pos_base=0)
        sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v
    sc.oracle_q_norm_rope(pos_base)
    sc.oracle_writeback(il=1, pos_base=pos_base)
    tokens = np.arange(m)
    got = sc.oracle_attention(1, pos_base, is_prefill=True)
    want = _brute_attention(sc, 1, tokens, lambda t: pos_base + t + 1)
    assert np.max(np.abs(got - want)) < 2e-6
    # non-causal form: every token sees rows [0, pos)
    pos = pos_base + m
    got_nc = sc.oracle_attention(1, pos, is_prefill=False)
    want_nc = _brute_attention(sc, 1, tokens, lambda t: pos)
    assert np.max(np.abs(got_nc - want_nc)) < 2e-6


def test_decode_split_merge_matches_brute_force_and_direct():
    cfg = layout.Config(n_layer=1)
    sc = Scenario(cfg, max_seq=200, m_tokens=1, seed=21)
    pre = Scenario(cfg, max_seq=200, m_tokens=150, seed=22, with_q=False)
    pre.oracle_writeback(il=0, pos_base=0)
    sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v
    pos = 150
    sc.oracle_q_norm_rope(pos)
    sc.oracle_writeback(il=0, pos_base=pos)
    out16, out32 = sc.oracle_decode(0, pos)
    want = _brute_attention(sc, 0, [0], lambda t: pos + 1)[0]
    assert np.max(np.abs(out32 - want)) < 2e-6
    direct = sc.oracle_attention(0, pos + 1, is_prefill=False)[0]
    assert np.max(np.abs(out32 - direct)) < 2e-6
    assert np.array_equal(out16, orc.f32_to_f16_bits(out32))


def test_chunked_prefill_equals_token_by_token_decode():
    """pos_base > 0 batched causal attention == the reference's one-token-at-a-time
    route (src/forward.rs:914-967): token i decoded at step pos_base + i."""
    cfg = layout.Config(n_layer=1)
    P, M = 70, 12
    sc = Scenario(cfg, max_seq=128, m_tokens=M, seed=31)
    pre = Scenario(cfg, max_seq=128, m_tokens=P, seed=32, with_q=False)
    pre.oracle_writeback(il=0, pos_base=0)
    sc.kv_k[:], sc.kv_v[:] = pre.kv_k, pre.kv_v
    sc.oracle_q_norm_rope(P)
    sc.oracle_writeback(il=0, pos_base=P)
    batched = sc.oracle_attention(0, P, is_prefill=True)
    for i in range(M):
        one = Scenario(cfg, max_seq=128, m_tokens=1, seed=0)
        one.kv_k, one.kv_v = sc.kv_k, sc.kv_v
        one.act[:cfg.q_dim] = sc.act[i * cfg.q_dim:(i + 1) * cfg.q_dim]
        _, out32 = one.oracle_decode(0, P + i)
        assert np.max(np.abs(out32 - batched[i])) < 2e-6


def test_attention_row_permutation_invariance():
    """Permuting whole cache rows (K and V together) leaves non-causal output unchanged."""
    cfg = layout.Config(n_layer=1)
    sc = Scenario(cfg, max_seq=64, m_tokens=64, seed=41)
    sc.oracle_writeback(il=0, pos_base=0)
    sc.oracle_q_norm_rope(0)
    base = sc.oracle_attention(0, 64, is_prefill=False, tokens=[0, 5, 63])
    perm = np.random.default_rng(0).permutation(64)
    nb = cfg.kv_dim // 32
    for buf in (sc.kv_k, sc.kv_v):
        d = buf[:64 * nb * 4].view(np.float32).reshape(64, nb)
        qs = buf[64 * nb * 4:].view(np.int8).reshape(64, cfg.kv_dim)
        d[:] = d[perm]
        qs[:] = qs[perm]
    permuted = sc.oracle_attention(0, 64, is_prefill=False, tokens=[0, 5, 63])
    assert np.max(np.abs(base - permuted)) < 2e-6
