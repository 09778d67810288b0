"""Q1_0 decode matvecs (src/forward.rs:212-334, matvec_q1_0*.wgsl).

CPU part: the oracle's f16 arithmetic against numpy's IEEE binary16, and the
oracle's matvecs against an f64 brute force (exact where every partial sum is
representable, within an f16-accumulation bound otherwise).
GPU part: the HIP kernels through the C ABI against the oracle, bit-exact for
the plain and fused normed matvecs; the silu one within one f16 ulp of the
staged product's effect (the device expf may differ from libm's by an ulp).
"""
import sys

import numpy as np
import pytest

import oracle as orc

# Bonsai-4B per-layer matvec shapes (n rows, k)
HIDDEN, Q_DIM, KV_DIM, FFN = 2560, 4096, 1024, 9728


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _f16(a):
    return np.asarray(a, np.float16).view(np.uint16)


def _weights(rng, tensors, pad=256):
    """Concatenate Q1_0 tensors [(n, k), ...] into one byte buffer, each at a
    nonzero offset. Returns buf and [(d_off, qs_off), ...]."""
    parts, offs, at = [], [], pad
    for n, k in tensors:
        buf, d0, q0 = orc.q1_0_tensor(rng, n, k)
        offs.append((at + d0, at + q0))
        parts.append((at, buf))
        at = (at + buf.size + pad + 255) // 256 * 256
    out = rng.integers(0, 256, at, dtype=np.uint8)     # garbage between tensors
    for a, b in parts:
        out[a:a + b.size] = b
    return out, offs


def _decode(buf, d_off, qs_off, n, k):
    """(d [n, nb] f64, signs [n, k] +-1 f64) of a Q1_0 tensor."""
    nb = k // 128
    d = buf[d_off:d_off + 2 * n * nb].view(np.float16).astype(np.float64).reshape(n, nb)
    qs = buf[qs_off:qs_off + 16 * n * nb].reshape(n, nb, 16)
    bits = np.unpackbits(qs, axis=-1, bitorder="little").reshape(n, k).astype(np.int64)
    return d, (2 * bits - 1).astype(np.float64)


def _brute(buf, d_off, qs_off, n, k, x):
    d, s = _decode(buf, d_off, qs_off, n, k)
    blk = (s * x[None, :]).reshape(n, k // 128, 128).sum(-1)
    return (d * blk).sum(-1), (np.abs(d) * np.abs(x).reshape(k // 128, 128).sum(-1)[None, :]).sum(-1)


def _f16_sum_bound(buf, d_off, qs_off, n, k, x):
    """First-order bound on the oracle's rounding error: each f16 add of the
    four component chains and of the block combine errs by at most 2^-11 of
    its result; f32 terms by 2^-24 of theirs (with margin)."""
    d, s = _decode(buf, d_off, qs_off, n, k)
    t = (s * x[None, :]).reshape(n, k // 128, 32, 4)          # [row, block, step, component]
    chain = np.abs(np.cumsum(t, axis=2)).sum(axis=(2, 3))
    c = np.cumsum(t.sum(axis=2), axis=-1)
    comb = np.abs(c[..., 1:]).sum(-1)
    blk = (chain + comb) * 2.0**-11
    absterm = np.abs(d) * np.abs(c[..., 3])
    return (np.abs(d) * blk).sum(-1) + 2.0**-20 * absterm.sum(-1)


# ---------------------------------------------------------------- CPU: oracle pins
def test_oracle_f16_ops_match_ieee():
    rng = np.random.default_rng(0)
    a = rng.integers(0, 0x10000, 20000, dtype=np.uint32).astype(np.uint16)
    b = rng.integers(0, 0x10000, 20000, dtype=np.uint32).astype(np.uint16)
    # edge cases: zeros, subnormals, max, overflow ties, cancellation
    edge = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x3C00, 0xBC00,
                     0x7BFE, 0x0200, 0x3555, 0x7C00, 0xFC00], np.uint16)
    a = np.concatenate([a, np.repeat(edge, edge.size)])
    b = np.concatenate([b, np.tile(edge, edge.size)])
    fa, fb = a.view(np.float16), b.view(np.float16)
    keep = np.isfinite(fa) & np.isfinite(fb)
    with np.errstate(over="ignore", invalid="ignore"):
        want_add = (fa.astype(np.float64) + fb.astype(np.float64)).astype(np.float16).view(np.uint16)
        want_mul = (fa.astype(np.float64) * fb.astype(np.float64)).astype(np.float16).view(np.uint16)
    got_add = np.array([orc.f16_add(int(x), int(y)) for x, y in zip(a, b)], np.uint16)
    got_mul = np.array([orc.f16_mul(int(x), int(y)) for x, y in zip(a, b)], np.uint16)
    # compare finite operands; a zero result's sign: x + (-x) = +0 under RNE in both
    assert np.array_equal(got_add[keep], want_add[keep]), np.flatnonzero(got_add[keep] != want_add[keep])[:8]
    assert np.array_equal(got_mul[keep], want_mul[keep]), np.flatnonzero(got_mul[keep] != want_mul[keep])[:8]


def test_oracle_matvec_exact_cases():
    """Small-integer x and power-of-two d: every f16 and f32 partial sum is
    exact, so the result is the brute-force dot product rounded once to f16 by
    the store, whatever the order; this fixes the bit -> sign mapping, the
    block -> scale pairing and the row / offset indexing."""
    rng = np.random.default_rng(1)
    n, k = 40, 1024
    buf, [(d_off, qs_off)] = _weights(rng, [(n, k)])
    nb = k // 128
    d = (2.0 ** rng.integers(-4, 3, n * nb)).astype(np.float16)
    buf[d_off:d_off + 2 * n * nb] = d.view(np.uint8)
    x = rng.integers(-3, 4, k).astype(np.float16)
    act = np.zeros(64 + k + 64 + n, np.uint16)
    act[64:64 + k] = _f16(x)
    out_off = 64 + k + 64
    p = orc.MatvecParams(k=k, n=n, d_offset=d_off, qs_offset=qs_off, input_offset=64,
                         output_offset=out_off, accumulate=0)
    got = orc.matvec_q1_0(p, buf, act)
    want, _ = _brute(buf, d_off, qs_off, n, k, x.astype(np.float64))
    f16 = lambda v: np.asarray(v, np.float64).astype(np.float16).astype(np.float64)
    assert np.array_equal(got[out_off:].view(np.float16).astype(np.float64), f16(want))
    assert np.array_equal(got[:out_off], act[:out_off])      # nothing else written
    # all bits one / all zero: +-sum(x) per block
    buf2 = buf.copy()
    buf2[qs_off:qs_off + 16 * n * nb] = 0xFF
    got2 = orc.matvec_q1_0(p, buf2, act)[out_off:].view(np.float16).astype(np.float64)
    dd = d.astype(np.float64).reshape(n, nb)
    xs = x.astype(np.float64).reshape(nb, 128).sum(-1)
    assert np.array_equal(got2, f16((dd * xs).sum(-1)))
    buf2[qs_off:qs_off + 16 * n * nb] = 0x00
    got3 = orc.matvec_q1_0(p, buf2, act)[out_off:].view(np.float16).astype(np.float64)
    assert np.array_equal(got3, f16(-(dd * xs).sum(-1)))
    # accumulate adds to the f16 already there
    act4 = act.copy()
    act4[out_off:] = _f16(np.arange(n) * 0.5)
    p.accumulate = 1
    got4 = orc.matvec_q1_0(p, buf, act4)[out_off:].view(np.float16).astype(np.float64)
    assert np.array_equal(got4, f16(want + np.arange(n) * 0.5))


def test_oracle_matvec_random_within_f16_bound():
    rng = np.random.default_rng(2)
    n, k = 48, 2560
    buf, [(d_off, qs_off)] = _weights(rng, [(n, k)])
    x = rng.standard_normal(k).astype(np.float16)
    act = np.concatenate([_f16(x), np.zeros(n, np.uint16)])
    p = orc.MatvecParams(k=k, n=n, d_offset=d_off, qs_offset=qs_off, input_offset=0, output_offset=k,
                         accumulate=0)
    got = orc.matvec_q1_0(p, buf, act)[k:].view(np.float16).astype(np.float64)
    want, mag = _brute(buf, d_off, qs_off, n, k, x.astype(np.float64))
    bound = _f16_sum_bound(buf, d_off, qs_off, n, k, x.astype(np.float64))
    err = np.abs(got - want)
    assert np.all(err <= bound + 2.0**-11 * np.abs(want)), (err - bound).max()
    # the errors are far below what a dropped or sign-flipped block would make
    d, s = _decode(buf, d_off, qs_off, n, k)
    one_block = np.abs(d[:, 0] * (s[:, :128] * x[:128].astype(np.float64)).sum(-1))
    assert 20 * np.median(err) < np.median(one_block)


def test_oracle_silu_and_normed_vs_f64():
    rng = np.random.default_rng(3)
    n, k = 32, 2048
    buf, [(d_off, qs_off)] = _weights(rng, [(n, k)])
    g = rng.standard_normal(k).astype(np.float16)
    u = rng.standard_normal(k).astype(np.float16)
    act = np.concatenate([_f16(g), _f16(u), np.zeros(n, np.uint16)])
    p = orc.MatvecSiluParams(k=k, n=n, d_offset=d_off, qs_offset=qs_off, gate_offset=0, up_offset=k,
                             output_offset=2 * k, accumulate=0)
    got = orc.matvec_q1_0_silu(p, buf, act)[2 * k:].view(np.float16).astype(np.float64)
    g64 = g.astype(np.float64)
    x = g64 / (1 + np.exp(-g64)) * u.astype(np.float64)
    want, mag = _brute(buf, d_off, qs_off, n, k, x)
    assert np.all(np.abs(got - want) <= 40 * 2.0**-11 * mag + 2.0**-11 * np.abs(want) + 1e-6)

    # fused normed: two ranges (the q / k / v pattern), rms over the input
    buf, offs = _weights(rng, [(64, k), (32, k)])
    xin = (rng.standard_normal(k) * 3).astype(np.float16)
    wn = (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
    act = np.concatenate([_f16(xin), np.zeros(96, np.uint16)])
    eps = 1e-6
    pn = orc.MatvecFusedNormedParams(k=k, input_offset=0, w_norm_off=0, eps=eps, n_ranges=2)
    for i, ((d_o, q_o), (nn, oo)) in enumerate(zip(offs, [(64, k + 32), (32, k)])):
        pn.d_offset[i], pn.qs_offset[i], pn.n[i], pn.output_offset[i] = d_o, q_o, nn, oo
    got = orc.matvec_q1_0_fused_normed(pn, buf, act, _f16(wn))
    x64 = xin.astype(np.float64)
    inv = 1 / np.sqrt((x64 ** 2).mean() + eps)
    xn = x64 * wn.astype(np.float64)
    for (d_o, q_o), (nn, oo) in zip(offs, [(64, k + 32), (32, k)]):
        want, mag = _brute(buf, d_o, q_o, nn, k, xn)
        g_ = got[oo:oo + nn].view(np.float16).astype(np.float64)
        assert np.all(np.abs(g_ - want * inv) <= (40 * 2.0**-11 * mag + 2.0**-11 * np.abs(want)) * inv + 1e-5)


# ---------------------------------------------------------------- GPU: HIP vs oracle
def _dev(arr):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr).view(np.int8 if arr.dtype == np.uint8 else np.int16)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def _model():
    import torch
    from bonsai_pot_amd import Model, layout
    m = Model(layout.Config(n_layer=1), 64)
    m.set_stream(torch.cuda.current_stream().cuda_stream)
    return m


@pytest.mark.gpu
@pytest.mark.parametrize("n,k,acc", [(Q_DIM, HIDDEN, 0), (HIDDEN, Q_DIM, 1), (KV_DIM, HIDDEN, 0),
                                     (37, 128, 0), (1, 16384, 1), (HIDDEN, FFN, 0)])
def test_matvec_bit_exact(cuda, n, k, acc):
    _say(f"[matvec] n={n} k={k} acc={acc}")
    rng = np.random.default_rng(n + k)
    buf, [(d_off, qs_off)] = _weights(rng, [(n, k)])
    in_off, out_off = 8, 8 + k + 24
    act = _f16(rng.standard_normal(out_off + n + 8))
    p = orc.MatvecParams(k=k, n=n, d_offset=d_off, qs_offset=qs_off, input_offset=in_off,
                         output_offset=out_off, accumulate=acc)
    want = orc.matvec_q1_0(p, buf, act)
    w_d, a_d = _dev(buf), _dev(act)
    m = _model()
    m.dispatch_matvec_q1_0(w_d.data_ptr(), a_d.data_ptr(), k, n, d_off, qs_off, in_off, out_off, bool(acc))
    got = _host(a_d)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} f16 outputs differ, first at {bad[:8]}"


@pytest.mark.gpu
@pytest.mark.parametrize("n,k,acc", [(HIDDEN, FFN, 1), (HIDDEN, FFN, 0), (64, 1024, 0)])
def test_matvec_silu(cuda, n, k, acc):
    _say(f"[matvec_silu] n={n} k={k} acc={acc}")
    rng = np.random.default_rng(7 * n + k)
    buf, [(d_off, qs_off)] = _weights(rng, [(n, k)])
    gate_off, up_off, out_off = 0, k + 16, 2 * k + 32
    act = _f16(rng.standard_normal(out_off + n) * 2)
    p = orc.MatvecSiluParams(k=k, n=n, d_offset=d_off, qs_offset=qs_off, gate_offset=gate_off,
                             up_offset=up_off, output_offset=out_off, accumulate=acc)
    want = orc.matvec_q1_0_silu(p, buf, act)
    w_d, a_d = _dev(buf), _dev(act)
    m = _model()
    m.dispatch_matvec_q1_0_silu(w_d.data_ptr(), a_d.data_ptr(), k, n, d_off, qs_off, gate_off, up_off,
                                out_off, bool(acc))
    got = _host(a_d)
    assert np.array_equal(got[:out_off], act[:out_off])
    g = got[out_off:].view(np.float16).astype(np.float64)
    w = want[out_off:].view(np.float16).astype(np.float64)
    # an ulp of difference in silu(g) changes one f16 x; bound the row effect by
    # 2^-10 of the row's |d| . |x| plus one output ulp
    _, mag = _brute(buf, d_off, qs_off, n, k, np.abs(act[up_off:up_off + k].view(np.float16)).astype(np.float64) * 4)
    exact = np.mean(got[out_off:] == want[out_off:])
    _say(f"  bit-identical rows: {exact:.4f}")
    assert np.all(np.abs(g - w) <= 2.0**-10 * mag + 2.0**-10 * np.abs(w) + 1e-6)
    assert exact > 0.9


@pytest.mark.gpu
@pytest.mark.parametrize("ranges", [
    [(Q_DIM, 0), (KV_DIM, 1), (KV_DIM, 2)],          # q / k / v from attn_norm(x)
    [(FFN, 0), (FFN, 1)],                            # gate / up from ffn_norm(x)
    [(96, 0)],
])
def test_matvec_fused_normed_bit_exact(cuda, ranges):
    k = HIDDEN
    _say(f"[matvec_fused_normed] ranges={ranges}")
    rng = np.random.default_rng(len(ranges) * 11 + ranges[0][0])
    buf, offs = _weights(rng, [(n, k) for n, _ in ranges])
    total = sum(n for n, _ in ranges)
    in_off, w_norm_off = 0, 0
    act = np.concatenate([_f16(rng.standard_normal(k) * 4), np.zeros(total + 8, np.uint16)])
    wn = _f16(1 + 0.2 * rng.standard_normal(k + 16))
    w_norm_off = 16
    # output regions in a different order from the ranges
    outs, at = {}, k + 8
    for n, tag in sorted(ranges, key=lambda r: -r[1]):
        outs[tag] = at
        at += n
    eps = 1e-6     # the model's rms_eps
    pn = orc.MatvecFusedNormedParams(k=k, input_offset=in_off, w_norm_off=w_norm_off, eps=eps,
                                     n_ranges=len(ranges))
    r_list = []
    for i, ((n, tag), (d_o, q_o)) in enumerate(zip(ranges, offs)):
        pn.d_offset[i], pn.qs_offset[i], pn.n[i], pn.output_offset[i] = d_o, q_o, n, outs[tag]
        r_list.append((d_o, q_o, n, outs[tag]))
    want = orc.matvec_q1_0_fused_normed(pn, buf, act, wn)
    from bonsai_pot_amd import layout
    assert layout.Config(n_layer=1).rms_eps == eps
    w_d, a_d, n_d = _dev(buf), _dev(act), _dev(wn)
    m = _model()
    m.dispatch_matvec_q1_0_fused_normed(w_d.data_ptr(), a_d.data_ptr(), n_d.data_ptr(), k, in_off,
                                        w_norm_off, r_list)
    got = _host(a_d)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} f16 outputs differ, first at {bad[:8]}"


@pytest.mark.gpu
def test_matvec_rejects_bad_shapes(cuda):
    from bonsai_pot_amd.errors import PotError
    m = _model()
    import torch
    w = torch.zeros(1 << 16, dtype=torch.int8, device="cuda")
    a = torch.zeros(1 << 16, dtype=torch.int16, device="cuda")
    for k in (0, 100, 16384 + 128):
        with pytest.raises(PotError):
            m.dispatch_matvec_q1_0(w.data_ptr(), a.data_ptr(), k, 32, 0, 0, 0, 0, False)
    with pytest.raises(PotError):
        m.dispatch_matvec_q1_0(w.data_ptr(), a.data_ptr(), 256, 32, 1, 0, 0, 0, False)
    with pytest.raises(PotError):
        m.dispatch_matvec_q1_0_fused_normed(w.data_ptr(), a.data_ptr(), a.data_ptr(), 256, 0, 0,
                                            [(0, 0, 33, 0)])
