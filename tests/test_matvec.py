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
# Two arithmetics (BP_MATVEC_ARITH, read at model creation):
#  * "f16" (default): the reference's f16 sums in its order -> bit-exact with
#    the oracle;
#  * "mfma" (opt-in): x rounded to 15 bits of each block's max |x|, exact
#    integer sums, f32 scaling -> within the bound of _mfma_bound of the exact
#    f64 product of the staged x, and within that bound plus the oracle's own
#    f16-accumulation bound of the oracle. "mfma_stream" forces the MFMA
#    kernel's streaming schedule (each wave walks whole 16-row tiles), which it
#    otherwise takes from 2048 tiles on (BP_MATVEC_STREAM_MIN_TILES).
ARITHS = ["f16", "mfma", "mfma_stream"]


def _dev(arr):
    import torch
    return torch.from_numpy(np.ascontiguousarray(arr).view(np.int8 if arr.dtype == np.uint8 else np.int16)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def _model(monkeypatch, arith):
    import torch
    from bonsai_pot_amd import Model, layout
    monkeypatch.setenv("BP_MATVEC_ARITH", "mfma" if arith.startswith("mfma") else "f16")
    monkeypatch.setenv("BP_MATVEC_STREAM_MIN_TILES", "1" if arith.endswith("_stream") else "2048")
    m = Model(layout.Config(n_layer=1), 64)
    m.set_stream(torch.cuda.current_stream().cuda_stream)
    return m


def _mfma_bound(buf, d_off, qs_off, n, k, x, scale=1.0):
    """Bound on |mfma result - exact| before the f16 store: each x moves by at
    most half of its block's quantum max|x| / 16383, and f32 terms and sums by
    a few ulps."""
    d, _ = _decode(buf, d_off, qs_off, n, k)
    xb = np.abs(x).reshape(k // 128, 128)
    quant = 128 * xb.max(-1) / 32766 * 1.001
    f32 = 8 * 2.0**-24 * xb.sum(-1)
    return scale * (np.abs(d) * (quant + f32)[None, :]).sum(-1)


def _check(arith, got, want_oracle, out, n, exact, bound_mfma, bound_oracle, old=None, written=None):
    """got / want_oracle: whole act buffers (uint16); exact / bounds per row;
    written: every (offset, rows) output region of the call (default this one)."""
    if arith.startswith("f16"):
        bad = np.flatnonzero(got != want_oracle)
        assert bad.size == 0, f"{bad.size} f16 outputs differ, first at {bad[:8]}"
        return
    mask = np.ones(got.size, bool)
    for o_, n_ in (written or [(out, n)]):
        mask[o_:o_ + n_] = False
    assert np.array_equal(got[mask], want_oracle[mask]), "matvec wrote outside its output rows"
    y = got[out:out + n].view(np.float16).astype(np.float64)
    ref = exact if old is None else exact + old
    tol = bound_mfma + 2.0**-11 * np.abs(ref) + 2.0**-24
    err = np.abs(y - ref)
    assert np.all(err <= tol), f"vs exact: worst row {np.argmax(err - tol)}, excess {(err - tol).max():.3g}"
    yo = want_oracle[out:out + n].view(np.float16).astype(np.float64)
    tol2 = tol + bound_oracle + 2.0**-11 * np.abs(yo)
    assert np.all(np.abs(y - yo) <= tol2), "vs oracle outside the two bounds"
    _say(f"  max |gpu - exact| / bound = {(err / tol).max():.3f}; max |gpu - oracle| = {np.abs(y - yo).max():.3g}")


@pytest.mark.gpu
@pytest.mark.parametrize("arith", ARITHS)
@pytest.mark.parametrize("n,k,acc", [(Q_DIM, HIDDEN, 0), (HIDDEN, Q_DIM, 1), (KV_DIM, HIDDEN, 0),
                                     (37, 128, 0), (1, 16384, 1), (HIDDEN, FFN, 0), (70, 2432, 0)])
def test_matvec(cuda, monkeypatch, arith, n, k, acc):
    _say(f"[matvec] {arith} n={n} k={k} acc={acc}")
    rng = np.random.default_rng(n + k)
    buf, [(d_off, qs_off)] = _weights(rng, [(n, k)])
    in_off, out_off = 8, 8 + k + 24
    act = _f16(rng.standard_normal(out_off + n + 8))
    p = orc.MatvecParams(k=k, n=n, d_offset=d_off, qs_offset=qs_off, input_offset=in_off,
                         output_offset=out_off, accumulate=acc)
    want = orc.matvec_q1_0(p, buf, act)
    w_d, a_d = _dev(buf), _dev(act)
    m = _model(monkeypatch, arith)
    m.dispatch_matvec_q1_0(w_d.data_ptr(), a_d.data_ptr(), k, n, d_off, qs_off, in_off, out_off, bool(acc))
    got = _host(a_d)
    x = act[in_off:in_off + k].view(np.float16).astype(np.float64)
    exact, _ = _brute(buf, d_off, qs_off, n, k, x)
    old = act[out_off:out_off + n].view(np.float16).astype(np.float64) if acc else None
    _check(arith, got, want, out_off, n, exact, _mfma_bound(buf, d_off, qs_off, n, k, x),
           _f16_sum_bound(buf, d_off, qs_off, n, k, x), old)


@pytest.mark.gpu
@pytest.mark.parametrize("arith", ARITHS)
@pytest.mark.parametrize("n,k,acc", [(HIDDEN, FFN, 1), (HIDDEN, FFN, 0), (64, 1024, 0)])
def test_matvec_silu(cuda, monkeypatch, arith, n, k, acc):
    _say(f"[matvec_silu] {arith} n={n} k={k} acc={acc}")
    rng = np.random.default_rng(7 * n + k)
    buf, [(d_off, qs_off)] = _weights(rng, [(n, k)])
    gate_off, up_off, out_off = 0, k + 16, 2 * k + 32
    act = _f16(rng.standard_normal(out_off + n) * 2)
    p = orc.MatvecSiluParams(k=k, n=n, d_offset=d_off, qs_offset=qs_off, gate_offset=gate_off,
                             up_offset=up_off, output_offset=out_off, accumulate=acc)
    want = orc.matvec_q1_0_silu(p, buf, act)
    w_d, a_d = _dev(buf), _dev(act)
    m = _model(monkeypatch, arith)
    m.dispatch_matvec_q1_0_silu(w_d.data_ptr(), a_d.data_ptr(), k, n, d_off, qs_off, gate_off, up_off,
                                out_off, bool(acc))
    got = _host(a_d)
    assert np.array_equal(got[:out_off], act[:out_off])
    # staged x as the oracle forms it (libm expf; the device expf may differ by
    # an ulp, which can move one f16 x by one ulp: 2^-10 |x| per element)
    g = act[gate_off:gate_off + k].view(np.float16).astype(np.float32)
    u = act[up_off:up_off + k].view(np.float16)
    x = ((g / (np.float32(1) + np.exp(-g))).astype(np.float16) * u).astype(np.float64)
    exact, _ = _brute(buf, d_off, qs_off, n, k, x)
    d, _ = _decode(buf, d_off, qs_off, n, k)
    ulp_x = (np.abs(d) * (2.0**-10 * np.abs(x)).reshape(k // 128, 128).sum(-1)[None, :]).sum(-1)
    old = act[out_off:out_off + n].view(np.float16).astype(np.float64) if acc else None
    if arith.startswith("f16"):
        gg = got[out_off:].view(np.float16).astype(np.float64)
        ww = want[out_off:].view(np.float16).astype(np.float64)
        assert np.all(np.abs(gg - ww) <= ulp_x + 2.0**-10 * np.abs(ww) + 1e-6)
        _say(f"  bit-identical rows: {np.mean(got[out_off:] == want[out_off:]):.4f}")
        return
    _check(arith, got, want, out_off, n, exact, _mfma_bound(buf, d_off, qs_off, n, k, x) + ulp_x,
           _f16_sum_bound(buf, d_off, qs_off, n, k, x), old)


@pytest.mark.gpu
@pytest.mark.parametrize("arith", ARITHS)
@pytest.mark.parametrize("ranges", [
    [(Q_DIM, 0), (KV_DIM, 1), (KV_DIM, 2)],          # q / k / v from attn_norm(x)
    [(FFN, 0), (FFN, 1)],                            # gate / up from ffn_norm(x)
    [(96, 0)],
    [(48, 0), (16, 1), (80, 2)],                     # multiples of 16 only
])
def test_matvec_fused_normed(cuda, monkeypatch, arith, ranges):
    k = HIDDEN
    _say(f"[matvec_fused_normed] {arith} ranges={ranges}")
    rng = np.random.default_rng(len(ranges) * 11 + ranges[0][0])
    buf, offs = _weights(rng, [(n, k) for n, _ in ranges])
    total = sum(n for n, _ in ranges)
    in_off = 0
    act = np.concatenate([_f16(rng.standard_normal(k) * 4), np.zeros(total + 8, np.uint16)])
    wn = _f16(1 + 0.2 * rng.standard_normal(k + 16))
    w_norm_off = 16
    outs, at = {}, k + 8        # output regions in a different order from the ranges
    for n, tag in sorted(ranges, key=lambda r: -r[1]):
        outs[tag] = at
        at += n
    from bonsai_pot_amd import layout
    eps = layout.Config(n_layer=1).rms_eps
    pn = orc.MatvecFusedNormedParams(k=k, input_offset=in_off, w_norm_off=w_norm_off, eps=eps,
                                     n_ranges=len(ranges))
    r_list = []
    for i, ((n, tag), (d_o, q_o)) in enumerate(zip(ranges, offs)):
        pn.d_offset[i], pn.qs_offset[i], pn.n[i], pn.output_offset[i] = d_o, q_o, n, outs[tag]
        r_list.append((d_o, q_o, n, outs[tag]))
    want = orc.matvec_q1_0_fused_normed(pn, buf, act, wn)
    w_d, a_d, n_d = _dev(buf), _dev(act), _dev(wn)
    m = _model(monkeypatch, arith)
    m.dispatch_matvec_q1_0_fused_normed(w_d.data_ptr(), a_d.data_ptr(), n_d.data_ptr(), k, in_off,
                                        w_norm_off, r_list)
    got = _host(a_d)
    if arith.startswith("f16"):
        bad = np.flatnonzero(got != want)
        assert bad.size == 0, f"{bad.size} f16 outputs differ, first at {bad[:8]}"
        return
    xin = act[in_off:in_off + k].view(np.float16)
    x = (xin * wn[w_norm_off:w_norm_off + k].view(np.float16)).astype(np.float64)
    inv = 1 / np.sqrt((xin.astype(np.float64) ** 2).mean() + eps)
    for (n, tag), (d_o, q_o) in zip(ranges, offs):
        o = outs[tag]
        exact, _ = _brute(buf, d_o, q_o, n, k, x)
        mag = _mfma_bound(buf, d_o, q_o, n, k, x, inv) + 1e-5 * np.abs(exact * inv)   # inv_rms in f32
        _check(arith, got, want, o, n, exact * inv, mag, inv * _f16_sum_bound(buf, d_o, q_o, n, k, x),
               written=[(outs[tg], nn) for nn, tg in ranges])


@pytest.mark.gpu
@pytest.mark.parametrize("arith,min_tiles,want_exact", [(None, "2048", True), (None, "1", True),
                                                        ("auto", "2048", True), ("auto", "1", False)])
def test_matvec_default_and_auto_dispatch(cuda, monkeypatch, arith, min_tiles, want_exact):
    """Default arithmetic: the f16-order kernel (the reference's bits) at every
    size. "auto": the f16-order kernel below the streaming size, the MFMA
    kernel from it on."""
    import torch
    from bonsai_pot_amd import Model, layout
    if arith is None:
        monkeypatch.delenv("BP_MATVEC_ARITH", raising=False)
    else:
        monkeypatch.setenv("BP_MATVEC_ARITH", arith)
    monkeypatch.setenv("BP_MATVEC_STREAM_MIN_TILES", min_tiles)
    n, k = 512, 2560
    rng = np.random.default_rng(5)
    buf, [(d_off, qs_off)] = _weights(rng, [(n, k)])
    act = _f16(rng.standard_normal(k + n))
    p = orc.MatvecParams(k=k, n=n, d_offset=d_off, qs_offset=qs_off, input_offset=0, output_offset=k,
                         accumulate=0)
    want = orc.matvec_q1_0(p, buf, act)
    m = Model(layout.Config(n_layer=1), 64)
    m.set_stream(torch.cuda.current_stream().cuda_stream)
    w_d, a_d = _dev(buf), _dev(act)
    m.dispatch_matvec_q1_0(w_d.data_ptr(), a_d.data_ptr(), k, n, d_off, qs_off, 0, k, False)
    got = _host(a_d)
    assert np.array_equal(got, want) == want_exact
    x = act[:k].view(np.float16).astype(np.float64)
    exact, _ = _brute(buf, d_off, qs_off, n, k, x)
    _check("mfma", got, want, k, n, exact, _mfma_bound(buf, d_off, qs_off, n, k, x),
           _f16_sum_bound(buf, d_off, qs_off, n, k, x))


@pytest.mark.gpu
def test_matvec_lm_head_default_is_reference_bits(cuda, monkeypatch):
    """The LM head (151936 x 2560) on the default f16-order kernel: every logit
    bit-identical to the oracle's f16 sums, and the top-k
    of those logits identical to the oracle's top-k of the oracle's logits."""
    import torch
    from bonsai_pot_amd import Model, layout
    monkeypatch.delenv("BP_MATVEC_ARITH", raising=False)
    monkeypatch.delenv("BP_MATVEC_STREAM_MIN_TILES", raising=False)
    n, k = 151936, HIDDEN
    _say(f"[matvec] lm head default n={n} k={k}")
    rng = np.random.default_rng(151936)
    buf, [(d_off, qs_off)] = _weights(rng, [(n, k)])
    act = _f16(rng.standard_normal(k + n))
    p = orc.MatvecParams(k=k, n=n, d_offset=d_off, qs_offset=qs_off, input_offset=0, output_offset=k,
                         accumulate=0)
    want = orc.matvec_q1_0(p, buf, act)
    m = Model(layout.Config(n_layer=1), 64)
    m.set_stream(torch.cuda.current_stream().cuda_stream)
    w_d, a_d = _dev(buf), _dev(act)
    m.dispatch_matvec_q1_0(w_d.data_ptr(), a_d.data_ptr(), k, n, d_off, qs_off, 0, k, False)
    got = _host(a_d)
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} logits differ, first at {bad[:8]}"
    res = torch.zeros(64, dtype=torch.int32, device="cuda")
    m.dispatch_topk_reduce(a_d.data_ptr(), res.data_ptr(), n, 32, k, 0)
    vals, idx = m.wait_topk_readback(res.data_ptr(), 0, 32)
    ores = orc.topk_reduce(orc.TopKParams(n=n, in_offset=k, out_offset=0, k=32), want, np.zeros(72, np.uint32))
    assert np.array_equal(idx, ores[32:64]) and np.array_equal(vals.view(np.uint32), ores[:32])


@pytest.mark.gpu
def test_matvec_rejects_bad_shapes(cuda, monkeypatch):
    from bonsai_pot_amd.errors import PotError
    m = _model(monkeypatch, "mfma")
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
                                            [(0, 0, 24, 0)])
